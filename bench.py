"""Benchmark of the hot path: block-scaled FP8 GEMM (fp8_gemm_nt) on one MI355X.

Workload (BASELINE.json metric): D[4096, 7168] (bf16) = A[4096, 2048] (e4m3, 1x128 UE8M0
scales) . B[7168, 2048]^T (e4m3, 128x128 UE8M0 scales), from seeded N(0,1) data.  A "step"
is one fp8_gemm_nt call over that batch with inputs resident in HBM and the scale factors
already in the kernel's required layout (the reference times the GEMM kernel alone,
tests/common.py:226-228).

Prints ONE JSON line.  `roofline` uses the GEMM kernel's own average duration measured
with HIP events on the launch stream; `cpu_baseline` times the CPU oracle (dequantise ->
fp32 matmul -> bf16) on the host cores over a bounded sample of the same workload.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, 'deepgemm-ascend_amd'))
sys.path.insert(0, ROOT)

PEAK_FP8_TFLOPS = 5000.0      # MI355X dense FP8 MFMA (published)
PEAK_HBM_GBS = 8000.0
# The reference's published figure for this exact metric and shape (Ascend 950DT, README.md:132
# of the reference): 838 TFLOP/s.
REFERENCE_TFLOPS = 838.0
M, N, K = 4096, 7168, 2048
TRAFFIC_FILE = os.path.join(ROOT, 'profiles', 'fp8_gemm_nt_4096x7168x2048_traffic.json')


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=50)
    ap.add_argument('--warmup', type=int, default=10)
    ap.add_argument('--cpu-seconds', type=float, default=10.0, help='bounded CPU baseline sample')
    ap.add_argument('--no-cpu', action='store_true')
    ap.add_argument('--m', type=int, default=M)
    ap.add_argument('--n', type=int, default=N)
    ap.add_argument('--k', type=int, default=K)
    ap.add_argument('--suite', default=None,
                    help='comma list of dense,decode,bf16,bf16nn,fp4,grouped,kgrouped,einsum,host,ref: one JSON line per shape '
                         '(cold-L2 kernel times) instead of the north-star line')
    ap.add_argument('--calibrate-copy', action='store_true',
                    help='run only a 256 MiB device copy (reference kernel for FETCH_SIZE / WRITE_SIZE scaling)')
    ap.add_argument('--profile-case', choices=('north', 'north_tn', 'grouped', 'decode', 'gemv', 'fp4_north', 'fp4_4096'),
                    default=None,
                    help='launch one workload 20 times and exit (the command rocprofv3 wraps for the profiles/ '
                         'summaries): north = fp8_gemm_nt 4096x7168x2048, north_tn = fp8_gemm_tn at that shape (MN-major '
                         'A and B), grouped = m_grouped contiguous G=32 '
                         'N=4096 K=7168, decode = fp8_gemm_nt 128x2112x7168, fp4_north / fp4_4096 = fp8_fp4_gemm_nt '
                         '4096x7168x2048 / 4096x4096x7168 (e2m1 B, 1x32 scales)')
    return ap.parse_args()


def calibrate_copy():
    import torch
    n = 256 << 20
    src = torch.empty(n, dtype=torch.uint8, device='cuda').fill_(1)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({'calibration': 'device copy', 'bytes_read_per_launch': n, 'bytes_written_per_launch': n}))


PEAK_CLOCK_MHZ = 2400.0      # engine clock the published peaks are quoted at


def sustained_clock(step, seconds=1.0):
    """Shader clock and socket power while `step` runs back to back for `seconds` (the clock the
    chip holds under this load: MI355X is power-limited, so the published peak at 2.4 GHz is not
    reachable).  Sampled from the SMU metrics table through amdsmi every ~5 ms; the table refreshes
    more slowly, so distinct samples are a few per window.  None if amdsmi is unavailable."""
    import threading
    import torch
    try:
        import amdsmi
        amdsmi.amdsmi_init()
        h = amdsmi.amdsmi_get_processor_handles()[0]
        amdsmi.amdsmi_get_gpu_metrics_info(h)
    except Exception as e:   # noqa: BLE001 (no SMU access: report why)
        return {'error': f'amdsmi unavailable: {e!r}'[:200]}
    samples, stop = [], [False]

    def sampler():
        while not stop[0]:
            try:
                m = amdsmi.amdsmi_get_gpu_metrics_info(h)
                clks = [c for c in m.get('current_gfxclks', []) if isinstance(c, int)]
                if not clks:
                    c = m.get('current_gfxclk')
                    clks = [c] if isinstance(c, int) else []
                # (idle XCDs sit near 100 MHz; a sample taken before the clock ramps is not the
                # sustained clock)
                if clks and min(clks) >= 1000:
                    ts = m.get('system_clock_counter', m.get('firmware_timestamp'))
                    samples.append((sum(clks) / len(clks), m.get('current_socket_power'), ts))
            except Exception:   # noqa: BLE001
                pass
            time.sleep(0.005)

    for _ in range(50):
        step()
    torch.cuda.synchronize()
    th = threading.Thread(target=sampler, daemon=True)
    th.start()
    t_end = time.perf_counter() + seconds
    n = 0
    while time.perf_counter() < t_end:
        for _ in range(100):
            step()
        n += 100
        torch.cuda.synchronize()
    stop[0] = True
    th.join()
    try:
        amdsmi.amdsmi_shut_down()
    except Exception:   # noqa: BLE001
        pass
    # one sample per refresh of the metrics table (its timestamp), and only those taken under load: the
    # table can lag the workload, and a refresh from an idle moment reports a low clock at a fraction of
    # the loaded power
    seen, uniq = set(), []
    for c, p, ts in samples:
        key = ts if ts is not None else (c, p)
        if key not in seen:
            seen.add(key)
            uniq.append((c, p))
    pmax = max((p for _, p in uniq if isinstance(p, (int, float))), default=None)
    loaded = [(c, p) for c, p in uniq if pmax is None or (isinstance(p, (int, float)) and p >= 0.6 * pmax)]
    if not loaded:
        return {'error': 'no samples at a loaded clock (>= 1000 MHz on every XCD)'}
    clk = sorted(c for c, _ in loaded)
    pw = sorted(p for _, p in loaded if isinstance(p, (int, float)))
    return {'clock_mhz_median': round(clk[len(clk) // 2], 1), 'clock_mhz_min': round(clk[0], 1),
            'clock_mhz_max': round(clk[-1], 1), 'socket_power_w_median': pw[len(pw) // 2] if pw else None,
            'samples': len(loaded), 'samples_taken': len(samples), 'launches': n,
            'source': 'amdsmi gpu_metrics current_gfxclks (mean over XCDs), one sample per metrics refresh, '
                      'those at >= 60 % of the peak sampled socket power, while the step ran back to back'}


def make_inputs(m, n, k):
    import torch
    from oracle import quant
    g = torch.Generator().manual_seed(0)
    a, sfa, a_deq = quant.quantize_blockwise(torch.randn(m, k, generator=g), (1, 128), 'e4m3')
    b, sfb, b_deq = quant.quantize_blockwise(torch.randn(n, k, generator=g), (128, 128), 'e4m3')
    return a, sfa, a_deq, b, sfb, b_deq


def cpu_model() -> str:
    try:
        with open('/proc/cpuinfo') as f:
            for line in f:
                if line.startswith('model name'):
                    return line.split(':', 1)[1].strip()
    except OSError:
        pass
    return 'unknown'


def cpu_baseline_config1(runs=15):
    """BASELINE config 1 on the host: fp8_gemm_nt 128x256x512 through the oracle (per-block dequantise
    -> fp32 matmul -> bf16), seeded N(0,1) A / B with 1x128 / 128x128 UE8M0 scales; 3 warm-ups, median of
    `runs` timed calls."""
    import torch
    from oracle import quant, gemm as og
    m, n, k = 128, 256, 512
    g = torch.Generator().manual_seed(0)
    a, sfa, _ = quant.quantize_blockwise(torch.randn(m, k, generator=g), (1, 128), 'e4m3')
    b, sfb, _ = quant.quantize_blockwise(torch.randn(n, k, generator=g), (128, 128), 'e4m3')

    def run():
        a_deq = quant.decode(a) * quant.expand_sf(sfa, (m, k), (1, 128))
        b_deq = quant.decode(b) * quant.expand_sf(sfb, (n, k), (128, 128))
        return og.gemm_nt(a_deq, b_deq)

    for _ in range(3):
        run()
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    return {'config': 'fp8_gemm_nt 128x256x512 (BASELINE config 1)', 'median_us': round(med * 1e6, 1),
            'gflops': round(2.0 * m * n * k / med / 1e9, 2), 'runs': runs, 'threads': torch.get_num_threads(),
            'os_cpu_count': os.cpu_count(), 'cpu_model': cpu_model()}


def cpu_baseline(a, sfa, b, sfb, m, n, k, seconds):
    """Time the oracle (per-block dequant to fp32 -> torch.matmul -> bf16) on host cores."""
    import torch
    from oracle import quant, gemm as og

    def run():
        a_deq = quant.decode(a) * quant.expand_sf(sfa, (m, k), (1, 128))
        b_deq = quant.decode(b) * quant.expand_sf(sfb, (n, k), (128, 128))
        return og.gemm_nt(a_deq, b_deq)

    run()
    times = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    return {
        'value': round(2.0 * m * n * k / med / 1e12, 4), 'unit': 'TFLOP/s', 'cores': torch.get_num_threads(),
        'kind': 'port',
        'sample': f'full {m}x{n}x{k} fp8_gemm_nt oracle (dequant->fp32 matmul->bf16), median of {len(times)} '
                  f'runs ({med * 1e3:.1f} ms each), host os.cpu_count()={os.cpu_count()}, {cpu_model()}',
    }


# ----------------------------------------------------------------------------- shape suite
def _gpu_codes(shape, dev, gen):
    """Random e4m3 codes (every non-NaN code) generated on the device."""
    import torch
    raw = torch.randint(0, 254, shape, dtype=torch.uint8, device=dev, generator=gen)
    raw += (raw >= 0x7f).to(torch.uint8)
    return raw.view(torch.float8_e4m3fn)


def _gpu_sf(shape, dev, gen, lo=118, hi=122):
    """fp32 power-of-two scales 2^(e-127), e in [lo, hi)."""
    import torch
    e = torch.randint(lo, hi, shape, dtype=torch.int32, device=dev, generator=gen)
    return (e << 23).view(torch.float32)


_FLUSH = None


def _time_cold(fn, iters=20):
    """Median kernel time (µs) with the operands evicted from L2 and the 256 MB MALL before every
    launch (the reference times cold-L2 launches, tests/common.py:226-236); events bracket each
    launch on its stream.  The eviction READS 1 GiB: a write-based flush leaves the MALL full of
    dirty lines whose write-back then competes with the measured kernel (measured: a plain
    streaming read drops from 4.5 to 2.4 TB/s after a 512 MB memset)."""
    import torch
    global _FLUSH
    if _FLUSH is None:
        _FLUSH = torch.ones(1 << 28, dtype=torch.float32, device='cuda')
    fn()
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(iters)]
    sinks = []
    torch.cuda._sleep(int(2e7))
    for e0, e1 in evs:
        sinks.append(_FLUSH.sum())
        e0.record()
        fn()
        e1.record()
    torch.cuda.synchronize()
    ts = sorted(e0.elapsed_time(e1) * 1e3 for e0, e1 in evs)
    return ts[len(ts) // 2]


def _line(group, workload, us, flops, nbytes, peak_tflops=PEAK_FP8_TFLOPS, **extra):
    tflops = flops / (us * 1e-6) / 1e12
    roof_us = max(flops / (peak_tflops * 1e12), nbytes / (PEAK_HBM_GBS * 1e9)) * 1e6
    out = {'suite': group, 'workload': workload, 'kernel_us': round(us, 2), 'tflops': round(tflops, 1),
           'hbm_gbs': round(nbytes / (us * 1e-6) / 1e9, 1), 'bound': 'mfma' if flops / (peak_tflops * 1e12) * 1e6 >= roof_us - 1e-9 else 'hbm',
           'roofline_us': round(roof_us, 2), 'roofline_frac': round(roof_us / us, 4),
           'mfma_frac': round(tflops / peak_tflops, 4)}
    out.update(extra)
    print(json.dumps(out), flush=True)


def _routed_counts(num_tokens=8192, num_experts=256, topk=8, local=32, seed=0):
    """Per-expert token counts of one GPU's 32 experts: top-8 of N(0,1) logits over 256 experts."""
    import torch
    g = torch.Generator().manual_seed(seed)
    idx = torch.randn(num_tokens, num_experts, generator=g).topk(topk, dim=-1).indices.flatten()
    return torch.bincount(idx, minlength=num_experts)[:local].tolist()


def run_suite(groups):
    import torch
    import deep_gemm
    dev = torch.device('cuda:0')
    gen = torch.Generator(device=dev).manual_seed(0)
    NK = [(2112, 7168), (24576, 1536), (7168, 16384), (4096, 7168), (7168, 2048)]

    def fp8_operand(rows, k, gran_mn, batch=None):
        shape = (batch, rows, k) if batch else (rows, k)
        sf_shape = ((batch,) if batch else ()) + (-(-rows // gran_mn), -(-k // 128))
        return _gpu_codes(shape, dev, gen), _gpu_sf(sf_shape, dev, gen)

    if 'dense' in groups or 'decode' in groups:
        # ('decode': the M <= 4 rows alone, M = 1, 2, 4)
        for m in ((1, 64, 128, 4096) if 'dense' in groups else (1, 2, 4)):
            for n, k in NK:
                a, sfa = fp8_operand(m, k, 1)
                b, sfb = fp8_operand(n, k, 128)
                sfa = deep_gemm.transform_sf_into_required_layout(sfa, m, k, (1, 128), is_sfa=True)
                sfb = deep_gemm.transform_sf_into_required_layout(sfb, n, k, (128, 128), is_sfa=False)
                d = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
                us = _time_cold(lambda: deep_gemm.fp8_gemm_nt((a, sfa), (b, sfb), d))
                _line('dense', f'fp8_gemm_nt {m}x{n}x{k}', us, 2.0 * m * n * k,
                      m * k + n * k + 2 * m * n + (m + n) * (k // 64) * 2)
    if 'bf16' in groups or 'bf16nn' in groups:
        # config 3: bf16_gemm_nt and bf16_gemm_nn (B stored [K, N]) over config 2's grid
        for lay in [x for x in ('nt', 'nn') if ('bf16' if x == 'nt' else 'bf16nn') in groups]:
            for m in (1, 64, 128, 4096):
                for n, k in NK:
                    a = (torch.randn(m, k, device=dev, generator=gen) * 0.1).bfloat16()
                    b = (torch.randn(n, k, device=dev, generator=gen) * 0.1).bfloat16()
                    d = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
                    if lay == 'nt':
                        fn = lambda: deep_gemm.bf16_gemm_nt(a, b, d)
                    else:
                        b_kn = b.t().contiguous()
                        fn = lambda: deep_gemm.bf16_gemm_nn(a, b_kn, d)
                    us = _time_cold(fn)
                    _line('bf16' if lay == 'nt' else 'bf16nn', f'bf16_gemm_{lay} {m}x{n}x{k}', us, 2.0 * m * n * k,
                          2 * (m * k + n * k + m * n), peak_tflops=2500.0)
    if 'fp4' in groups:
        for m in (128, 4096):
            for n, k in ((7168, 2048), (4096, 7168)):
                a, sfa = fp8_operand(m, k, 1)
                b = torch.randint(-128, 128, (n, k // 2), dtype=torch.int8, device=dev, generator=gen)
                sfb = _gpu_sf((n, k // 32), dev, gen, 125, 128)
                sfa = deep_gemm.transform_sf_into_required_layout(sfa, m, k, (1, 128), is_sfa=True)
                sfb = deep_gemm.transform_sf_into_required_layout(sfb, n, k, (1, 32), is_sfa=False)
                d = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
                us = _time_cold(lambda: deep_gemm.fp8_fp4_gemm_nt((a, sfa), (b, sfb), d))
                _line('fp4', f'fp8_fp4_gemm_nt {m}x{n}x{k}', us, 2.0 * m * n * k,
                      m * k + n * k // 2 + 2 * m * n + (m + n) * (k // 64) * 2)
    if 'ref' in groups:
        # the reference's other published FP8 x FP4 shapes (its MX recipe: 1x32 UE8M0 scales on both
        # operands, e2m1 B packed two per byte): dense 4096x7168x16384, and M-grouped contiguous with 8
        # groups of 4096 rows at N=4096 K=2048 and N=7168 K=3072
        def fp4_b(rows, k, batch=None):
            shape = ((batch,) if batch else ()) + (rows, k // 2)
            sf = _gpu_sf(((batch,) if batch else ()) + (rows, k // 32), dev, gen, 125, 128)
            return torch.randint(-128, 128, shape, dtype=torch.int8, device=dev, generator=gen), sf
        m, n, k = 4096, 7168, 16384
        a = _gpu_codes((m, k), dev, gen)
        sfa = deep_gemm.transform_sf_into_required_layout(_gpu_sf((m, k // 32), dev, gen), m, k, (1, 32), is_sfa=True)
        b, sfb = fp4_b(n, k)
        sfb = deep_gemm.transform_sf_into_required_layout(sfb, n, k, (1, 32), is_sfa=False)
        d = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
        us = _time_cold(lambda: deep_gemm.fp8_fp4_gemm_nt((a, sfa), (b, sfb), d))
        _line('ref', f'fp8_fp4_gemm_nt {m}x{n}x{k} (1x32 / 1x32)', us, 2.0 * m * n * k,
              m * k + n * k // 2 + 2 * m * n + (m + n) * (k // 32))
        g_, rows = 8, 4096
        deep_gemm.set_mk_alignment_for_contiguous_layout(256)
        layout = torch.tensor([rows * (i + 1) for i in range(g_)], dtype=torch.int32, device=dev)
        for n, k in ((4096, 2048), (7168, 3072)):
            total = g_ * rows
            a = _gpu_codes((total, k), dev, gen)
            sfa = deep_gemm.transform_sf_into_required_layout(_gpu_sf((total, k // 32), dev, gen), total, k, (1, 32),
                                                               is_sfa=True, psum_layout=layout)
            b, sfb = fp4_b(n, k, batch=g_)
            sfb = deep_gemm.transform_sf_into_required_layout(sfb, n, k, (1, 32), num_groups=g_, is_sfa=False)
            d = torch.empty(total, n, dtype=torch.bfloat16, device=dev)
            us = _time_cold(lambda: deep_gemm.m_grouped_fp8_fp4_gemm_nt_contiguous((a, sfa), (b, sfb), d, layout))
            _line('ref', f'm_grouped_fp8_fp4_gemm_nt_contiguous G=8 x {rows} rows N={n} K={k} (1x32 / 1x32)', us,
                  2.0 * total * n * k, total * k + g_ * n * k // 2 + 2 * total * n + (total + g_ * n) * (k // 32))
    if 'grouped' in groups:
        counts = _routed_counts()
        align = 128
        deep_gemm.set_mk_alignment_for_contiguous_layout(align)
        total, psum = 0, []
        for c in counts:
            psum.append(total + c)
            total = -(-(total + c) // align) * align
        valid = sum(counts)
        for n, k in ((4096, 7168), (7168, 2048)):
            g_ = len(counts)
            a, sfa = fp8_operand(total, k, 1)
            b, sfb = fp8_operand(n, k, 128, batch=g_)
            layout = torch.tensor(psum, dtype=torch.int32, device=dev)
            sfa = deep_gemm.transform_sf_into_required_layout(sfa, total, k, (1, 128), is_sfa=True, psum_layout=layout)
            sfb = deep_gemm.transform_sf_into_required_layout(sfb, n, k, (128, 128), num_groups=g_, is_sfa=False)
            d = torch.empty(total, n, dtype=torch.bfloat16, device=dev)
            us = _time_cold(lambda: deep_gemm.m_grouped_fp8_gemm_nt_contiguous((a, sfa), (b, sfb), d, layout))
            _line('grouped', f'm_grouped_contiguous G=32 rows={total} (valid {valid}) N={n} K={k}', us,
                  2.0 * valid * n * k, total * k + g_ * n * k + 2 * total * n, padded_tflops=round(
                      2.0 * total * n * k / (us * 1e-6) / 1e12, 1))
            # the same rows with an m_indices layout (-1 on padding rows)
            idx = torch.full((total,), -1, dtype=torch.int32)
            start = 0
            for gi, ps in enumerate(psum):
                idx[start:ps] = gi
                start = -(-ps // align) * align
            idx = idx.to(dev)
            us = _time_cold(lambda: deep_gemm.m_grouped_fp8_gemm_nt_contiguous((a, sfa), (b, sfb), d, idx,
                                                                              use_psum_layout=False))
            _line('grouped', f'm_grouped_contiguous m_indices G=32 rows={total} (valid {valid}) N={n} K={k}', us,
                  2.0 * valid * n * k, total * k + g_ * n * k + 2 * total * n)
            mmax = 256
            masked = torch.tensor([min(c, mmax) for c in counts], dtype=torch.int32, device=dev)
            am, sfam = fp8_operand(mmax, k, 1, batch=g_)
            sfam = deep_gemm.transform_sf_into_required_layout(sfam, mmax, k, (1, 128), num_groups=g_, is_sfa=True)
            dm = torch.empty(g_, mmax, n, dtype=torch.bfloat16, device=dev)
            em = int(sum(min(c, mmax) for c in counts) / g_)
            us = _time_cold(lambda: deep_gemm.m_grouped_fp8_gemm_nt_masked((am, sfam), (b, sfb), dm, masked, em))
            vm = sum(min(c, mmax) for c in counts)
            _line('grouped', f'm_grouped_masked G=32 max_m={mmax} (valid {vm}) N={n} K={k}', us,
                  2.0 * vm * n * k, vm * k + g_ * n * k + 2 * vm * n)
        deep_gemm.set_mk_alignment_for_contiguous_layout(256)
    if 'kgrouped' in groups:
        import random
        rng = random.Random(0)
        for g_, m, n, ek in ((4, 4096, 7168, 8192), (4, 7168, 2048, 8192), (8, 4096, 7168, 4096),
                             (8, 7168, 2048, 4096), (16, 4096, 7168, 2048), (16, 7168, 2048, 2048)):
            ks = [max(1, int(ek * rng.uniform(0.7, 1.3))) for _ in range(g_)]
            total, psum = 0, []
            for kk in ks:
                psum.append(total + kk)
                total = -(-(total + kk) // 256) * 256
            a = _gpu_codes((total, m), dev, gen)
            b = _gpu_codes((total, n), dev, gen)
            sfa = _gpu_sf((total // 32, m), dev, gen)
            sfb = _gpu_sf((total // 32, n), dev, gen)
            layout = torch.tensor(psum, dtype=torch.int32, device=dev)
            d = torch.zeros(g_, m, n, dtype=torch.float32, device=dev)
            fn = lambda: deep_gemm.k_grouped_fp8_gemm_tn_contiguous((a, sfa), (b, sfb), d, ks, layout, c=d)
            us = _time_cold(fn)
            sk = sum(ks)
            _line('kgrouped', f'k_grouped_fp8_gemm_tn G={g_} M={m} N={n} sumK={sk} fp32 acc', us,
                  2.0 * m * n * sk, total * (m + n) + 8 * g_ * m * n, includes='MN->K-major operand copy and SF transform')
    if 'host' in groups:
        # Host time per call: `calls` launches queued behind a spin kernel (so the device never
        # pushes back), wall time / calls; through the C++ host path and through the Python path.
        from deep_gemm import _lib
        calls = 200
        for m, n, k in ((128, 2112, 7168), (4096, 7168, 2048)):
            a, sfa32 = fp8_operand(m, k, 1)
            b, sfb32 = fp8_operand(n, k, 128)
            sfa = deep_gemm.transform_sf_into_required_layout(sfa32, m, k, (1, 128), is_sfa=True)
            sfb = deep_gemm.transform_sf_into_required_layout(sfb32, n, k, (128, 128), is_sfa=False)
            d = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
            for sf_kind, (sa, sb) in (('packed', (sfa, sfb)), ('fp32', (sfa32, sfb32))):
                for path in ('cpp', 'python'):
                    saved = _lib.ext()
                    if path == 'python':
                        _lib._ext = None
                    try:
                        rec = dict(recipe_a=(1, 128), recipe_b=(128, 128)) if sf_kind == 'fp32' else {}
                        fn = lambda: deep_gemm.fp8_gemm_nt((a, sa), (b, sb), d, **rec)
                        for _ in range(5):
                            fn()
                        torch.cuda.synchronize()
                        torch.cuda._sleep(int(3e8))
                        t0 = time.perf_counter()
                        for _ in range(calls):
                            fn()
                        host_us = (time.perf_counter() - t0) / calls * 1e6
                        torch.cuda.synchronize()
                    finally:
                        _lib._ext = saved
                    print(json.dumps({'suite': 'host', 'workload': f'fp8_gemm_nt {m}x{n}x{k}', 'sf': sf_kind,
                                      'path': path, 'host_us_per_call': round(host_us, 2)}), flush=True)
    if 'einsum' in groups:
        h, r, dd = 8, 4096, 1024
        for bsz in (4096, 8192):
            a = _gpu_codes((h, bsz, r), dev, gen).permute(1, 0, 2)          # [b, h, r], r contiguous
            sfa = _gpu_sf((h, bsz, r // 32), dev, gen).permute(1, 0, 2)
            bw = _gpu_codes((h, dd, r), dev, gen)
            sfb = _gpu_sf((h, dd, r // 32), dev, gen)
            d = torch.empty(bsz, h, dd, dtype=torch.bfloat16, device=dev)
            us = _time_cold(lambda: deep_gemm.fp8_einsum('bhr,hdr->bhd', (a, sfa), (bw, sfb), d))
            _line('einsum', f"fp8_einsum bhr,hdr->bhd b={bsz} h={h} r={r} d={dd}", us, 2.0 * bsz * h * r * dd,
                  bsz * h * r + h * dd * r + 2 * bsz * h * dd, includes='SF transform')


def profile_case(case):
    """20 launches of one workload (warm), nothing else: the command the profiles/ summaries wrap."""
    import torch
    import deep_gemm
    dev = torch.device('cuda:0')
    gen = torch.Generator(device=dev).manual_seed(0)
    if case == 'north_tn':
        # the north-star shape as fp8_gemm_tn: A [K, M] and B [K, N] MN-major, read in place
        m, n, k = 4096, 7168, 2048
        a, sfa = _gpu_codes((k, m), dev, gen), _gpu_sf((k // 128, m), dev, gen)
        b, sfb = _gpu_codes((k, n), dev, gen), _gpu_sf((k // 128, -(-n // 128)), dev, gen)
        d = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
        fn = lambda: deep_gemm.fp8_gemm_tn((a, sfa), (b, sfb), d, recipe_a=(1, 128), recipe_b=(128, 128))
    elif case in ('fp4_north', 'fp4_4096'):
        # e4m3 A (1x128 scales) x e2m1 B packed two per byte (1x32 scales)
        m, n, k = (4096, 7168, 2048) if case == 'fp4_north' else (4096, 4096, 7168)
        a, sfa = _gpu_codes((m, k), dev, gen), _gpu_sf((m, k // 128), dev, gen)
        b = torch.randint(0, 256, (n, k // 2), dtype=torch.uint8, device=dev, generator=gen).view(torch.int8)
        sfb = _gpu_sf((n, k // 32), dev, gen)
        sfa = deep_gemm.transform_sf_into_required_layout(sfa, m, k, (1, 128), is_sfa=True)
        sfb = deep_gemm.transform_sf_into_required_layout(sfb, n, k, (1, 32), is_sfa=False)
        d = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
        fn = lambda: deep_gemm.fp8_fp4_gemm_nt((a, sfa), (b, sfb), d)
    elif case in ('north', 'decode', 'gemv'):
        m, n, k = {'north': (4096, 7168, 2048), 'decode': (128, 2112, 7168), 'gemv': (1, 2112, 7168)}[case]
        a, sfa = _gpu_codes((m, k), dev, gen), _gpu_sf((m, k // 128), dev, gen)
        b, sfb = _gpu_codes((n, k), dev, gen), _gpu_sf((-(-n // 128), k // 128), dev, gen)
        sfa = deep_gemm.transform_sf_into_required_layout(sfa, m, k, (1, 128), is_sfa=True)
        sfb = deep_gemm.transform_sf_into_required_layout(sfb, n, k, (128, 128), is_sfa=False)
        d = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
        fn = lambda: deep_gemm.fp8_gemm_nt((a, sfa), (b, sfb), d)
    else:
        counts = _routed_counts()
        align = 128
        deep_gemm.set_mk_alignment_for_contiguous_layout(align)
        total, psum = 0, []
        for c in counts:
            psum.append(total + c)
            total = -(-(total + c) // align) * align
        n, k, g_ = 4096, 7168, len(counts)
        a, sfa = _gpu_codes((total, k), dev, gen), _gpu_sf((total, k // 128), dev, gen)
        b, sfb = _gpu_codes((g_, n, k), dev, gen), _gpu_sf((g_, n // 128, k // 128), dev, gen)
        layout = torch.tensor(psum, dtype=torch.int32, device=dev)
        sfa = deep_gemm.transform_sf_into_required_layout(sfa, total, k, (1, 128), is_sfa=True, psum_layout=layout)
        sfb = deep_gemm.transform_sf_into_required_layout(sfb, n, k, (128, 128), num_groups=g_, is_sfa=False)
        d = torch.empty(total, n, dtype=torch.bfloat16, device=dev)
        fn = lambda: deep_gemm.m_grouped_fp8_gemm_nt_contiguous((a, sfa), (b, sfb), d, layout)
    for _ in range(20):
        fn()
    torch.cuda.synchronize()
    print(json.dumps({'profile_case': case, 'launches': 20}), flush=True)


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get('WORLD_SIZE', '1')) != 1:
        print(f'bench.py measures one GPU only (the hot path does not shard across GPUs in this build); '
              f'got --gpus {args.gpus}', file=sys.stderr)
        sys.exit(2)
    if args.calibrate_copy:
        calibrate_copy()
        return
    if args.suite:
        run_suite(set(args.suite.split(',')))
        return
    if args.profile_case:
        profile_case(args.profile_case)
        return
    import torch
    import deep_gemm
    from oracle import gemm as og

    m, n, k = args.m, args.n, args.k
    a, sfa, a_deq, b, sfb, b_deq = make_inputs(m, n, k)
    dev = torch.device('cuda:0')
    a_d, b_d = a.to(dev), b.to(dev)
    # scale factors transformed once, outside the timed region
    sfa_t = deep_gemm.transform_sf_into_required_layout(sfa.to(dev), m, k, (1, 128), is_sfa=True)
    sfb_t = deep_gemm.transform_sf_into_required_layout(sfb.to(dev), n, k, (128, 128), is_sfa=False)
    d = torch.empty(m, n, dtype=torch.bfloat16, device=dev)

    def step():
        deep_gemm.fp8_gemm_nt((a_d, sfa_t), (b_d, sfb_t), d)

    step()
    torch.cuda.synchronize()
    diff = og.calc_diff(d.cpu(), og.gemm_nt(a_deq, b_deq))
    if diff >= 1e-3:
        raise SystemExit(f'bench: result mismatch vs oracle, calc_diff={diff}')

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    # whole-job throughput: K back-to-back steps
    t0 = time.perf_counter()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(args.steps):
        step()
    stop.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_total = start.elapsed_time(stop)
    ms_per_step = ms_total / args.steps

    # per-launch kernel duration (events on the launch stream around each launch); a spin
    # kernel first keeps the GPU busy while the host queues every launch, so host-side call
    # overhead never lands between an event pair
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    torch.cuda._sleep(int(2e7))
    for e0, e1 in evs:
        e0.record()
        step()
        e1.record()
    torch.cuda.synchronize()
    kern_ms = sorted(e0.elapsed_time(e1) for e0, e1 in evs)
    kern_avg = sum(kern_ms) / len(kern_ms)
    # cold-L2 kernel time (operands evicted from L2 and the MALL before every launch, as the
    # reference times its kernels): the roofline's achieved rate
    cold_us = _time_cold(step, iters=max(10, min(args.steps, 40)))

    clock = sustained_clock(step, seconds=4.0)

    flops = 2.0 * m * n * k
    tflops = flops / (ms_per_step * 1e-3) / 1e12
    achieved = flops / (cold_us * 1e-6) / 1e12
    traffic = None
    if os.path.exists(TRAFFIC_FILE) and (m, n, k) == (M, N, K):
        with open(TRAFFIC_FILE) as f:
            traffic = json.load(f).get('hbm_bytes_per_launch')
    cfg = deep_gemm.select_config(m, n, k)
    out = {
        'metric': 'FP8 block-scaled GEMM TFLOPS @ M=4096,N=7168,K=2048 bf16-out; % FP8 MFMA peak',
        'value': round(tflops, 2), 'unit': 'TFLOP/s', 'n_gpus': 1, 'steps': args.steps, 'warmup': args.warmup,
        'ms_per_step': round(ms_per_step, 5), 'higher_is_better': True, 'scaling': 'weak', 'vs_baseline': round(tflops / REFERENCE_TFLOPS, 3),
        'vs_baseline_ref': 'reference published 838 TFLOP/s at this shape on Ascend 950DT',
        'dtype': 'fp8_e4m3 (UE8M0 block scales, fp32 accumulate, bf16 out)', 'data': 'synthetic',
        'config': {'workload': f'fp8_gemm_nt M={m} N={n} K={k} bf16-out, A 1x128 / B 128x128 UE8M0 scales '
                               f'(seeded N(0,1)), SF pre-transformed', 'm': m, 'n': n, 'k': k,
                   'tile': f'{cfg[0]}x{cfg[1]}', 'parallelism': 'single GPU'},
        'roofline': {'bound': 'mfma', 'achieved': round(achieved, 2), 'peak': PEAK_FP8_TFLOPS, 'unit': 'TFLOP/s',
                     'frac': round(achieved / PEAK_FP8_TFLOPS, 4), 'traffic': traffic,
                     'kernel_us_cold_median': round(cold_us, 3),
                     'kernel_avg_us_warm': round(kern_avg * 1e3, 3), 'kernel_min_us_warm': round(kern_ms[0] * 1e3, 3),
                     'clock': clock,
                     'peak_at_clock': (round(PEAK_FP8_TFLOPS * clock['clock_mhz_median'] / PEAK_CLOCK_MHZ, 1)
                                       if 'clock_mhz_median' in clock else None),
                     'frac_at_clock': (round(achieved / (PEAK_FP8_TFLOPS * clock['clock_mhz_median'] / PEAK_CLOCK_MHZ), 4)
                                       if 'clock_mhz_median' in clock else None),
                     'timing': 'achieved = 2MNK / cold-L2 kernel time (HIP events around each launch on its stream, '
                               '1 GiB read evicts L2 and the MALL before each); value = back-to-back warm steps'},
        'calc_diff': diff,
        'wall_s_timed': round(wall, 4),
    }
    if not args.no_cpu:
        out['cpu_baseline'] = cpu_baseline(a, sfa, b, sfb, m, n, k, args.cpu_seconds)
        out['cpu_baseline_config1'] = cpu_baseline_config1()
    print(json.dumps(out), flush=True)


if __name__ == '__main__':
    main()
