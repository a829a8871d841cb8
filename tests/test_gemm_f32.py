"""The fp32 GEMM behind the graph layer's matmul on float32 tensors
(agk_gemm_f32: cgadimpl/src/ops/linalg.cpp:12-20 and the VJP's products,
autodiff_vjp_ops.cpp:258-263).

Checked against a float64 product on the host.  Bar: the worst-case bound of
fp32 summation in any order, |C - C64| <= K * 2^-24 * (|A| |B|) element-wise
(plus one rounding of the stored result); every layout (A, B transposed or
not), odd sizes and edge tiles, leading dimensions wider than the rows, K == 0
(zeros, or C unchanged when accumulating), accumulation, bit-identical results
across calls, and replays of a captured HIP graph equal to eager calls.
"""
from __future__ import annotations

import numpy as np
import pytest

import cgadimpl_amd as agk
from gpu_util import to_dev, to_host

pytestmark = pytest.mark.gpu

OK, EINVAL = 0, 1  # agk_status
# below the CU count in 128-tiles: the 64 x 64 tile; from (2048, 2048, 40) on
# (256 and 289 128-tiles): the 128 x 128 tile, the second with edge tiles
SHAPES = [(1, 1, 1), (7, 5, 3), (64, 48, 33), (129, 257, 95), (300, 17, 1000), (1000, 520, 64),
          (256, 384, 513), (2048, 1024, 160), (2048, 2048, 40), (2100, 2060, 33)]


def _bound(a, b, K):
    return (K + 1) * 2.0 ** -24 * (np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64)) + 1e-30


@pytest.mark.parametrize("trans_b", [False, True])
@pytest.mark.parametrize("trans_a", [False, True])
@pytest.mark.parametrize("M,N,K", SHAPES, ids=lambda v: str(v))
def test_product_matches_fp64(cuda, M, N, K, trans_a, trans_b):
    g = np.random.default_rng(M * 7 + N * 3 + K)
    a = g.standard_normal((M, K)).astype(np.float32)
    b = g.standard_normal((K, N)).astype(np.float32)
    ad = to_dev(np.ascontiguousarray(a.T) if trans_a else a, cuda)
    bd = to_dev(np.ascontiguousarray(b.T) if trans_b else b, cuda)
    print(f"gemm_f32 {M}x{N}x{K} ta={trans_a} tb={trans_b}", flush=True)
    c = to_host(agk.gemm_f32(ad, bd, trans_a=trans_a, trans_b=trans_b))
    ref = a.astype(np.float64) @ b.astype(np.float64)
    assert c.shape == (M, N) and c.dtype == np.float32
    assert np.all(np.abs(c - ref) <= _bound(a, b, K))
    c2 = to_host(agk.gemm_f32(ad, bd, trans_a=trans_a, trans_b=trans_b))
    assert np.array_equal(c, c2)


def test_accumulate_and_empty_sum(cuda):
    import torch
    g = np.random.default_rng(5)
    a = g.standard_normal((33, 40)).astype(np.float32)
    b = g.standard_normal((40, 21)).astype(np.float32)
    c0 = g.standard_normal((33, 21)).astype(np.float32)
    c = to_host(agk.gemm_f32(to_dev(a, cuda), to_dev(b, cuda), c=to_dev(c0, cuda),
                             accumulate=True))
    ref = c0.astype(np.float64) + a.astype(np.float64) @ b.astype(np.float64)
    assert np.all(np.abs(c - ref) <= _bound(a, b, 40) + 2.0 ** -24 * np.abs(ref))
    # K == 0: zeros, or C unchanged when accumulating
    e_a = torch.empty(33, 0, device=cuda)
    e_b = torch.empty(0, 21, device=cuda)
    cz = to_dev(c0, cuda)
    assert np.array_equal(to_host(agk.gemm_f32(e_a, e_b, c=cz, accumulate=True)), c0)
    assert np.count_nonzero(to_host(agk.gemm_f32(e_a, e_b, c=cz))) == 0


def test_rejects_bad_arguments(cuda):
    import ctypes
    lib = agk.lib()
    # ldc < N, negative sizes, null operands with K > 0
    assert lib.agk_gemm_f32(None, 4, 0, None, 4, 0, None, 4, 4, 4, 4, 0, None) == EINVAL
    assert lib.agk_gemm_f32(None, 4, 0, None, 4, 0, None, 4, -1, 4, 4, 0, None) == EINVAL
    buf = to_dev(np.zeros((4, 4), np.float32), cuda)
    p = ctypes.c_void_p(buf.data_ptr())
    assert lib.agk_gemm_f32(p, 4, 0, p, 4, 0, p, 3, 4, 4, 4, 0, None) == EINVAL
    assert lib.agk_gemm_f32(p, 3, 0, p, 4, 0, p, 4, 4, 4, 4, 0, None) == EINVAL
    assert lib.agk_gemm_f32(None, 4, 0, None, 4, 0, None, 4, 0, 4, 4, 0, None) == OK


def test_leading_dimensions_wider_than_rows(cuda):
    """Operands and C inside wider buffers (ld > the used width), as views of
    larger matrices: the product of the views, C's other columns untouched."""
    import torch
    g = torch.Generator(device=cuda)
    g.manual_seed(11)
    M, N, K = 70, 90, 50
    abuf = torch.randn(M, K + 13, generator=g, device=cuda)
    bbuf = torch.randn(K, N + 7, generator=g, device=cuda)
    cbuf = torch.full((M, N + 5), 3.0, device=cuda)
    rc = agk.lib().agk_gemm_f32(abuf.data_ptr(), K + 13, 0, bbuf.data_ptr(), N + 7, 0,
                                cbuf.data_ptr(), N + 5, M, N, K, 0, None)
    torch.cuda.synchronize()
    assert rc == OK
    a, b = to_host(abuf)[:, :K], to_host(bbuf)[:, :N]
    c = to_host(cbuf)
    ref = a.astype(np.float64) @ b.astype(np.float64)
    assert np.all(np.abs(c[:, :N] - ref) <= _bound(a, b, K))
    assert np.all(c[:, N:] == 3.0)


def test_graph_capture_replays_match_eager(cuda):
    """agk_gemm_f32 is a plain kernel launch: captured once into a HIP graph,
    three replays on new operands (eager work and synchronisations between
    them) each equal the eager call bit for bit."""
    import torch
    M, N, K = 300, 260, 200
    a = torch.empty(M, K, device=cuda)
    b = torch.empty(N, K, device=cuda)  # given as B^T
    c = torch.empty(M, N, device=cuda)
    a.normal_()
    b.normal_()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        agk.gemm_f32(a, b, c=c, trans_b=True, stream=torch.cuda.current_stream())
    gen = torch.Generator(device=cuda)
    for k in range(3):
        gen.manual_seed(40 + k)
        a.copy_(torch.randn(M, K, generator=gen, device=cuda))
        b.copy_(torch.randn(N, K, generator=gen, device=cuda))
        graph.replay()
        torch.cuda.synchronize()
        got = c.clone()
        want = agk.gemm_f32(a, b, trans_b=True)
        torch.cuda.synchronize()
        assert torch.equal(got, want), k
    del graph
