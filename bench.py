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
    ap.add_argument('--calibrate-copy', action='store_true',
                    help='run only a 256 MiB device copy (reference kernel for FETCH_SIZE / WRITE_SIZE scaling)')
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


def make_inputs(m, n, k):
    import torch
    from oracle import quant
    g = torch.Generator().manual_seed(0)
    a, sfa, a_deq = quant.quantize_blockwise(torch.randn(m, k, generator=g), (1, 128), 'e4m3')
    b, sfb, b_deq = quant.quantize_blockwise(torch.randn(n, k, generator=g), (128, 128), 'e4m3')
    return a, sfa, a_deq, b, sfb, b_deq


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
                  f'runs ({med * 1e3:.1f} ms each), host os.cpu_count()={os.cpu_count()}',
    }


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get('WORLD_SIZE', '1')) != 1:
        print(f'bench.py measures one GPU only (the hot path does not shard across GPUs in this build); '
              f'got --gpus {args.gpus}', file=sys.stderr)
        sys.exit(2)
    if args.calibrate_copy:
        calibrate_copy()
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

    flops = 2.0 * m * n * k
    tflops = flops / (ms_per_step * 1e-3) / 1e12
    achieved = flops / (kern_avg * 1e-3) / 1e12
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
                     'kernel_avg_us': round(kern_avg * 1e3, 3), 'kernel_min_us': round(kern_ms[0] * 1e3, 3)},
        'calc_diff': diff,
        'wall_s_timed': round(wall, 4),
    }
    if not args.no_cpu:
        out['cpu_baseline'] = cpu_baseline(a, sfa, b, sfb, m, n, k, args.cpu_seconds)
    print(json.dumps(out), flush=True)


if __name__ == '__main__':
    main()
