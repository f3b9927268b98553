"""GPU tests of the host path: the C++ extension serves the common calls, sticky error words report
invalid fp32 scale factors and unpadded m_indices without a synchronisation, and the split-K
workspace the library owns per stream survives graph capture (grown only outside a capture, never
freed while a captured graph may use it).

Results are checked against the CPU oracle (calc_diff < 1e-5, the reference's bar,
tests/test_fp8_gemm.py:21)."""
import pytest
import torch

import deep_gemm
from deep_gemm import _lib
from oracle import gemm as og, layout as ol
from helpers import gen, operand, calc_diff

pytestmark = pytest.mark.gpu
THRESH = 1e-5


R = dict(recipe_a=(1, 128), recipe_b=(128, 128))


def _dense(m, n, k, seed):
    g = gen(seed)
    a, sfa, a_deq = operand(m, k, 'e4m3', (1, 128), g, 'randn')
    b, sfb, b_deq = operand(n, k, 'e4m3', (128, 128), g, 'randn')
    return (a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()), og.gemm_nt(a_deq, b_deq)


def _clear_pending():
    _lib.load().dg_take_errors()


def test_extension_serves_the_dense_call(monkeypatch):
    """The fast path launches (no Python GemmArgs is built) and gives the oracle's result."""
    assert _lib.ext() is not None, 'deep_gemm_C.so must be built and load on the GPU box'
    from deep_gemm import gemm as g_mod
    built = []
    real = g_mod._lib.GemmArgs
    monkeypatch.setattr(g_mod._lib, 'GemmArgs', lambda *a, **kw: built.append(1) or real(*a, **kw))
    a, b, ref = _dense(128, 2112, 7168, seed=1)
    d = torch.empty(128, 2112, dtype=torch.bfloat16, device='cuda')
    deep_gemm.fp8_gemm_nt(a, b, d, **R)
    torch.cuda.synchronize()
    assert not built, 'the C++ host path should have served this call'
    assert calc_diff(d.cpu(), ref) < THRESH


def test_invalid_fp32_sf_is_reported_by_the_next_call():
    _clear_pending()
    (a, sfa), (b, sfb), _ = _dense(64, 256, 512, seed=2)
    bad = sfa.clone()
    bad[3, 1] = 1.5                      # mantissa bits: not a UE8M0 value
    d = torch.empty(64, 256, dtype=torch.bfloat16, device='cuda')
    deep_gemm.fp8_gemm_nt((a, bad), (b, sfb), d, **R)     # no host synchronisation here
    torch.cuda.synchronize()
    with pytest.raises(RuntimeError, match='Invalid float32 SF'):
        deep_gemm.fp8_gemm_nt((a, sfa), (b, sfb), d, **R)
    # reported once: the next valid call runs
    deep_gemm.fp8_gemm_nt((a, sfa), (b, sfb), d, **R)


def test_check_errors_raises_for_the_offending_call():
    """deep_gemm.check_errors() synchronises and raises for the call that set the word (here the
    last call of a sequence, which no later deep_gemm call would report), and clears it."""
    _clear_pending()
    (a, sfa), (b, sfb), ref = _dense(64, 256, 512, seed=3)
    d = torch.empty(64, 256, dtype=torch.bfloat16, device='cuda')
    deep_gemm.fp8_gemm_nt((a, sfa), (b, sfb), d, **R)
    deep_gemm.check_errors()                              # nothing reported for a valid call
    assert calc_diff(d.cpu(), ref) < THRESH
    bad = sfa.clone()
    bad[5, 2] = -1.0                                      # sign bit: not a UE8M0 value
    deep_gemm.fp8_gemm_nt((a, bad), (b, sfb), d, **R)     # no synchronisation, no error yet
    with pytest.raises(RuntimeError, match='Invalid float32 SF.*before check_errors'):
        deep_gemm.check_errors()
    deep_gemm.check_errors()                              # cleared
    deep_gemm.fp8_gemm_nt((a, sfa), (b, sfb), d, **R)     # and the next call does not re-report it
    deep_gemm.check_errors()


def test_check_errors_unpadded_m_indices():
    """An m_indices layout with a row of another group inside a block is reported by
    check_errors() right after the offending call (the last call: no later call would report it)."""
    _clear_pending()
    alignment, g_num, n, k = 128, 3, 256, 256
    total, ps = ol.psum_from_sizes([130, 60, 128], alignment)
    idx = ol.m_indices_from_psum(ps, alignment, total).clone()
    idx[200] = 2
    g = gen(5)
    a, sfa, _ = operand(total, k, 'e4m3', (1, 32), g)
    b, sfb, _ = operand(n, k, 'e4m3', (1, 32), g, batch=g_num)
    d = torch.empty(total, n, dtype=torch.bfloat16, device='cuda')
    old = deep_gemm.get_mk_alignment_for_contiguous_layout()
    deep_gemm.set_mk_alignment_for_contiguous_layout(alignment)
    try:
        deep_gemm.m_grouped_fp8_gemm_nt_contiguous((a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()), d, idx.cuda(),
                                                   use_psum_layout=False)
        with pytest.raises(RuntimeError, match='m_indices is not padded'):
            deep_gemm.check_errors()
        deep_gemm.check_errors()
    finally:
        deep_gemm.set_mk_alignment_for_contiguous_layout(old)


@pytest.mark.parametrize('case', ['mixed_block', 'group_after_padding', 'id_out_of_range'])
def test_unpadded_m_indices_are_reported(case):
    _clear_pending()
    alignment, g_num, n, k = 128, 3, 256, 256
    sizes = [130, 60, 128]
    total, ps = ol.psum_from_sizes(sizes, alignment)
    idx = ol.m_indices_from_psum(ps, alignment, total).clone()
    if case == 'mixed_block':
        idx[200] = 2                     # a row of group 2 inside group 1's block
    elif case == 'group_after_padding':
        idx[total - 1] = 2               # group 2's block: a group row after its padding rows
        idx[total - 2] = -1
    else:
        idx[0:alignment] = g_num         # an id past the last group
    g = gen(3)
    a, sfa, _ = operand(total, k, 'e4m3', (1, 32), g)
    b, sfb, _ = operand(n, k, 'e4m3', (1, 32), g, batch=g_num)
    d = torch.empty(total, n, dtype=torch.bfloat16, device='cuda')
    old = deep_gemm.get_mk_alignment_for_contiguous_layout()
    deep_gemm.set_mk_alignment_for_contiguous_layout(alignment)
    try:
        args = ((a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()), d, idx.cuda())
        deep_gemm.m_grouped_fp8_gemm_nt_contiguous(*args, use_psum_layout=False)
        torch.cuda.synchronize()
        with pytest.raises(RuntimeError, match='m_indices is not padded'):
            deep_gemm.m_grouped_fp8_gemm_nt_contiguous(*args, use_psum_layout=False)
        torch.cuda.synchronize()
        _clear_pending()
    finally:
        deep_gemm.set_mk_alignment_for_contiguous_layout(old)


def test_padded_m_indices_raise_nothing():
    _clear_pending()
    alignment, n, k = 128, 256, 256
    total, ps = ol.psum_from_sizes([130, 0, 60, 128], alignment)
    idx = ol.m_indices_from_psum(ps, alignment, total)
    g = gen(4)
    a, sfa, a_deq = operand(total, k, 'e4m3', (1, 32), g)
    b, sfb, b_deq = operand(n, k, 'e4m3', (1, 32), g, batch=4)
    d = torch.empty(total, n, dtype=torch.bfloat16, device='cuda')
    old = deep_gemm.get_mk_alignment_for_contiguous_layout()
    deep_gemm.set_mk_alignment_for_contiguous_layout(alignment)
    try:
        deep_gemm.m_grouped_fp8_gemm_nt_contiguous((a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()), d, idx.cuda(),
                                                   use_psum_layout=False)
        torch.cuda.synchronize()
        assert _lib.load().dg_take_errors() == 0
    finally:
        deep_gemm.set_mk_alignment_for_contiguous_layout(old)
    ref = og.m_grouped_contiguous(a_deq, b_deq, idx, False, alignment)
    valid = idx >= 0
    assert calc_diff(d.cpu()[valid], ref[valid]) < THRESH


def test_split_k_graph_survives_workspace_growth():
    """Capture a split-K GEMM, grow the stream's workspace with a larger eager split-K call, then
    replay: the graph still owns its (never freed) workspace and every replay matches."""
    s = torch.cuda.Stream()
    (a, sfa), (b, sfb), ref = _dense(64, 2112, 7168, seed=5)
    plan = deep_gemm.launch_plan(64, 2112, 7168)
    print('captured plan', plan, flush=True)
    assert plan['split_k'] > 1
    d = torch.empty(64, 2112, dtype=torch.bfloat16, device='cuda')
    with torch.cuda.stream(s):
        deep_gemm.fp8_gemm_nt((a, sfa), (b, sfb), d, **R)        # allocates the stream's workspace
    s.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        deep_gemm.fp8_gemm_nt((a, sfa), (b, sfb), d, **R)
    (a2, sfa2), (b2, sfb2), ref2 = _dense(128, 7168, 16384, seed=6)
    print('larger plan', deep_gemm.launch_plan(128, 7168, 16384), flush=True)
    for i in range(3):
        d.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert calc_diff(d.cpu(), ref) < THRESH, f'replay {i}'
        d2 = torch.empty(128, 7168, dtype=torch.bfloat16, device='cuda')
        with torch.cuda.stream(s):
            deep_gemm.fp8_gemm_nt((a2, sfa2), (b2, sfb2), d2, **R)   # grows the workspace (first time)
        s.synchronize()
        assert calc_diff(d2.cpu(), ref2) < THRESH


def test_split_k_capture_without_workspace_raises():
    s = torch.cuda.Stream()
    (a, sfa), (b, sfb), _ = _dense(64, 4096, 7168, seed=7)
    d = torch.empty(64, 4096, dtype=torch.bfloat16, device='cuda')
    # SF already in the kernels' layout, so the only capture-time work is the GEMM itself
    sfa_t = deep_gemm.transform_sf_into_required_layout(sfa, 64, 7168, (1, 128), is_sfa=True)
    sfb_t = deep_gemm.transform_sf_into_required_layout(sfb, 4096, 7168, (128, 128), is_sfa=False)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with pytest.raises(RuntimeError, match='before the capture'):
        with torch.cuda.graph(graph, stream=s):
            deep_gemm.fp8_gemm_nt((a, sfa_t), (b, sfb_t), d)
    torch.cuda.synchronize()
