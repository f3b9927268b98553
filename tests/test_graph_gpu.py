"""GEMM launches captured in a HIP graph (torch.cuda.CUDAGraph on the current stream): decode shapes on
the GEMV kernel (1x2112x7168) and the skinny-M kernel (with a cross-workgroup K split, whose arrival
counters the kernel itself resets: no memset node in the graph), the tile kernel and an M-grouped
masked launch.  Every
replay, with eager work between the replays, matches the eager launch bit for bit."""
import pytest
import torch

import deep_gemm
from helpers import gen, operand

pytestmark = pytest.mark.gpu


def _dense_case(m, n, k, seed):
    g = gen(seed)
    a, sfa, _ = operand(m, k, 'e4m3', (1, 128), g, 'randn')
    b, sfb, _ = operand(n, k, 'e4m3', (128, 128), g, 'randn')
    a, b = a.cuda(), b.cuda()
    sfa = deep_gemm.transform_sf_into_required_layout(sfa.cuda(), m, k, (1, 128), is_sfa=True)
    sfb = deep_gemm.transform_sf_into_required_layout(sfb.cuda(), n, k, (128, 128), is_sfa=False)
    return (a, sfa), (b, sfb)


@pytest.mark.parametrize('m,n,k', [(1, 2112, 7168), (1, 2112, 2048), (16, 7168, 2048), (128, 4096, 7168),
                                   (128, 2112, 7168), (4096, 2112, 1024)])
def test_graph_replay_dense(m, n, k):
    print(f'graph dense m={m} n={n} k={k}', flush=True)
    a, b = _dense_case(m, n, k, seed=m + n)
    d = torch.empty(m, n, dtype=torch.bfloat16, device='cuda')
    deep_gemm.fp8_gemm_nt(a, b, d)
    torch.cuda.synchronize()
    eager = d.clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):   # warm-up on the capture stream (plan memo, split-K workspace)
        deep_gemm.fp8_gemm_nt(a, b, d)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        deep_gemm.fp8_gemm_nt(a, b, d)
    for i in range(4):
        d.fill_(float(i + 1))                       # eager work between the replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(d.view(torch.int16), eager.view(torch.int16)), i


def test_graph_replay_masked():
    groups, max_m, n, k = 8, 16, 1024, 2048
    print(f'graph masked G={groups} max_m={max_m} n={n} k={k}', flush=True)
    g = gen(41)
    a, sfa, _ = operand(max_m, k, 'e4m3', (1, 32), g, batch=groups)
    b, sfb, _ = operand(n, k, 'e4m3', (1, 32), g, batch=groups)
    a, sfa, b, sfb = a.cuda(), sfa.cuda(), b.cuda(), sfb.cuda()
    sfa = deep_gemm.transform_sf_into_required_layout(sfa, max_m, k, (1, 32), num_groups=groups, is_sfa=True)
    sfb = deep_gemm.transform_sf_into_required_layout(sfb, n, k, (1, 32), num_groups=groups, is_sfa=False)
    masked = torch.tensor([16, 0, 3, 9, 16, 1, 7, 12], dtype=torch.int32, device='cuda')
    d = torch.zeros(groups, max_m, n, dtype=torch.bfloat16, device='cuda')
    deep_gemm.m_grouped_fp8_gemm_nt_masked((a, sfa), (b, sfb), d, masked, 8)
    torch.cuda.synchronize()
    eager = d.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        deep_gemm.m_grouped_fp8_gemm_nt_masked((a, sfa), (b, sfb), d, masked, 8)
    for i in range(3):
        d.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for gi in range(groups):
            mg = int(masked[gi])
            assert torch.equal(d[gi, :mg].view(torch.int16), eager[gi, :mg].view(torch.int16)), (i, gi)
