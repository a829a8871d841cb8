"""bf16 GEMM on MFMA (agk_gemm_bf16) and the bf16 transpose, through the C ABI.

GPU: every operand layout (the direct-to-LDS kernel reads k-contiguous operands
with 16-byte LDS reads and k-strided ones with transposing reads; K not a
multiple of 64 and the k-scale take the register-staged kernel), the k- and
row-scales, fp32 and bf16 output, accumulation and ragged sizes, each against a
plain PyTorch fp32 product of the same bf16 operands; transposes bit-exact;
repeated calls bit-identical; the four layouts of one product bit-identical.
CPU: argument validation and the workspace rule.
"""
import pytest

import cgadimpl_amd as agk

FAKE = 0x1000  # never dereferenced: validation rejects before any HIP call


def test_gemm_argument_validation():
    lib = agk.lib()
    g = lib.agk_gemm_bf16

    def call(M=64, N=64, K=64, lda=64, ldb=64, ldc=64, ta=0, tb=1, dt=0, a=FAKE, b=FAKE, c=FAKE):
        return g(a, lda, ta, b, ldb, tb, c, ldc, dt, M, N, K, None, None, 0, None, 0, None)

    assert call(M=-1) == 1
    assert call(dt=7) == 2
    assert call(M=0) == 0 and call(N=0) == 0          # empty result: nothing to do
    assert call(a=None) == 1 and call(c=None) == 1
    assert call(M=60, lda=64) == 1                     # M not a multiple of 8
    assert call(K=36) == 1                             # K not a multiple of 8
    assert call(lda=60) == 1                           # lda < K
    assert call(ldc=32) == 1                           # ldc < N
    assert call(a=FAKE + 4) == 1                       # A not 16-byte aligned
    # K == 0: an empty sum; accumulating into C leaves it as it is (no launch),
    # C itself is still required and checked
    assert g(None, 0, 0, None, 64, 0, FAKE, 64, 0, 64, 64, 0, None, None, 1, None, 0, None) == 0
    assert g(None, 0, 0, None, 64, 0, None, 64, 0, 64, 64, 0, None, None, 1, None, 0, None) == 1
    assert g(None, 0, 0, None, 64, 0, FAKE, 32, 0, 64, 64, 0, None, None, 0, None, 0, None) == 1
    ws = lib.agk_gemm_bf16_workspace_bytes
    # the direct kernel stages either operand layout itself: no layout needs a workspace
    for ta in (0, 1):
        for tb in (0, 1):
            assert ws(8192, 11008, 4096, ta, tb) == 0
    assert ws(64, 64, 72, 1, 0) == 0                   # K % 64: staged kernel
    t = lib.agk_transpose_bf16
    assert t(FAKE, 64, FAKE, 64, 64, 60, None) == 1    # cols not a multiple of 8
    assert t(FAKE, 64, FAKE, 32, 64, 64, None) == 1    # ld_dst < rows
    assert t(None, 64, None, 64, 0, 64, None) == 0


def _ref(a, b, ta, tb, ks, rs):
    A = (a.t() if ta else a).float()
    B = (b.t() if tb else b).float()
    if ks is not None:
        A = (A * ks[None, :]).bfloat16().float()   # the stored product is bf16
    C = A @ B
    if rs is not None:
        C = C * rs[:, None]
    return C


# K / 64 = 1, 2, 3, 5, 7, 16 on the direct-to-LDS kernel (K a multiple of 64):
# odd and even tile counts of its peeled two-stage loop, with ragged M and N tiles.
CASES = [(256, 256, 64), (264, 520, 72), (8, 8, 8), (1000, 1032, 520), (512, 768, 1024),
         (136, 264, 192), (264, 520, 128), (520, 264, 320), (200, 136, 448)]


@pytest.mark.gpu
@pytest.mark.parametrize("M,N,K", CASES)
@pytest.mark.parametrize("ta,tb", [(0, 1), (0, 0), (1, 1), (1, 0)])
@pytest.mark.parametrize("ws", ["auto", None])
def test_gemm_against_torch(cuda, M, N, K, ta, tb, ws):
    import torch
    torch.manual_seed(M * 7 + N * 3 + K + ta * 2 + tb)
    a = torch.randn((K, M) if ta else (M, K), device=cuda).bfloat16()
    b = torch.randn((N, K) if tb else (K, N), device=cuda).bfloat16()
    for scaled in (False, True):
        ks = torch.rand(K, device=cuda) + 0.5 if scaled else None
        rs = torch.rand(M, device=cuda) + 0.5 if scaled else None
        r = _ref(a, b, ta, tb, ks, rs)
        for od, tol in ((torch.float32, 1e-5), (torch.bfloat16, 8e-3)):
            c = agk.gemm_bf16(a, b, trans_a=bool(ta), trans_b=bool(tb), out_dtype=od, kscale=ks,
                              rowscale=rs, workspace=ws)
            torch.cuda.synchronize()
            err = ((c.float() - r).abs().max() / r.abs().max()).item()
            assert err <= tol, (M, N, K, ta, tb, ws, scaled, od, err)
    # accumulate into an existing fp32 C, and bit-identical repeats
    base = torch.randn(M, N, device=cuda)
    c = agk.gemm_bf16(a, b, c=base.clone(), trans_a=bool(ta), trans_b=bool(tb), accumulate=True,
                      workspace=ws)
    c2 = agk.gemm_bf16(a, b, c=base.clone(), trans_a=bool(ta), trans_b=bool(tb), accumulate=True,
                       workspace=ws)
    torch.cuda.synchronize()
    r = _ref(a, b, ta, tb, None, None) + base
    assert ((c - r).abs().max() / r.abs().max()).item() <= 1e-5
    assert torch.equal(c, c2)


@pytest.mark.gpu
@pytest.mark.parametrize("rows,cols", [(8, 8), (128, 128), (136, 264), (4096, 11008), (1000, 8)])
def test_transpose_bit_exact(cuda, rows, cols):
    import torch
    x = torch.randn(rows, cols, device=cuda).bfloat16()
    y = agk.transpose_bf16(x)
    torch.cuda.synchronize()
    assert torch.equal(y, x.t().contiguous())


@pytest.mark.gpu
def test_gemm_c5_shapes(cuda):
    """The three products of the RMSNorm + linear layer at full size (8192 x 4096 x 11008),
    against torch fp32 on sampled rows."""
    import torch
    torch.manual_seed(5)
    M, K, N = 8192, 4096, 11008
    h = torch.randn(M, K, device=cuda).bfloat16()
    W = (torch.randn(K, N, device=cuda) * 0.02).bfloat16()
    dy = torch.randn(M, N, device=cuda).bfloat16()
    rows = torch.randint(0, M, (64,), device=cuda)
    y = agk.gemm_bf16(h, W)                                     # y = h W
    dh = agk.gemm_bf16(dy, W, trans_b=True)                     # dh = dy W^T
    dW = agk.gemm_bf16(h, dy, trans_a=True, out_dtype=torch.float32)   # dW = h^T dy
    torch.cuda.synchronize()
    ry = h[rows].float() @ W.float()
    rdh = dy[rows].float() @ W.float().t()
    assert ((y[rows].float() - ry).abs().max() / ry.abs().max()).item() <= 8e-3
    assert ((dh[rows].float() - rdh).abs().max() / rdh.abs().max()).item() <= 8e-3
    cols = torch.randint(0, K, (16,), device=cuda)
    rdW = h[:, cols].float().t() @ dy.float()
    assert ((dW[cols] - rdW).abs().max() / rdW.abs().max()).item() <= 1e-5


@pytest.mark.gpu
@pytest.mark.parametrize("M,N,K", [(264, 520, 128), (520, 264, 320), (1000, 1032, 512)])
@pytest.mark.parametrize("f32", [True, False])
def test_gemm_layouts_bit_identical(cuda, M, N, K, f32):
    """The same product with A and B in each storage layout: the k-strided operands are staged
    as they lie and read with transposing LDS reads, the k-contiguous ones with plain reads; the
    MFMAs see the same values in the same order, so all four results are bit-identical."""
    import torch
    torch.manual_seed(M + 3 * N + 7 * K)
    a = torch.randn(M, K, device=cuda).bfloat16()      # [M, K]
    b = torch.randn(N, K, device=cuda).bfloat16()      # [N, K]
    at, bt = a.t().contiguous(), b.t().contiguous()    # [K, M], [K, N]
    od = torch.float32 if f32 else torch.bfloat16
    outs = [agk.gemm_bf16(a, b, trans_b=True, out_dtype=od),          # both k-contiguous
            agk.gemm_bf16(at, b, trans_a=True, trans_b=True, out_dtype=od),
            agk.gemm_bf16(a, bt, out_dtype=od),
            agk.gemm_bf16(at, bt, trans_a=True, out_dtype=od)]          # both k-strided
    torch.cuda.synchronize()
    for c in outs[1:]:
        assert torch.equal(c, outs[0])
    r = a.float() @ b.float().t()
    assert ((outs[0].float() - r).abs().max() / r.abs().max()).item() <= (1e-5 if f32 else 8e-3)


@pytest.mark.gpu
@pytest.mark.parametrize("ta,tb", [(0, 1), (1, 0)])
def test_gemm_empty_reduction(cuda, ta, tb):
    """K == 0: the product is zero; with accumulation C is left as it was."""
    import torch
    M, N = 264, 136
    a = torch.empty((0, M) if ta else (M, 0), device=cuda, dtype=torch.bfloat16)
    b = torch.empty((N, 0) if tb else (0, N), device=cuda, dtype=torch.bfloat16)
    for od in (torch.float32, torch.bfloat16):
        c = agk.gemm_bf16(a, b, c=torch.full((M, N), 7.0, device=cuda).to(od),
                          trans_a=bool(ta), trans_b=bool(tb))
        base = torch.randn(M, N, device=cuda).to(od)
        c2 = agk.gemm_bf16(a, b, c=base.clone(), trans_a=bool(ta), trans_b=bool(tb),
                           accumulate=True)
        torch.cuda.synchronize()
        assert torch.count_nonzero(c).item() == 0
        assert torch.equal(c2, base)


@pytest.mark.gpu
@pytest.mark.parametrize("M,N,K", [(16, 8, 32), (264, 520, 128), (200, 136, 72), (1000, 1032, 512),
                                   (64, 64, 0)])
def test_linear_bias_epilogue(cuda, M, N, K):
    """agk_linear_bf16: y = bf16(bf16(x w^T) + b), the bias added in the GEMM's
    store.  Bit-identical to the plain product (same kernel, no bias) followed
    by a bf16 add of b; against a plain fp32 product + b within bf16 rounding.
    K = 0 gives b in every row."""
    import torch
    gen = torch.Generator(device=cuda)
    gen.manual_seed(M * 7 + N * 3 + K)
    x = torch.randn(M, K, generator=gen, device=cuda).bfloat16()
    w = (torch.randn(N, K, generator=gen, device=cuda) * 0.2).bfloat16()
    b = torch.randn(N, generator=gen, device=cuda).bfloat16()
    y = agk.linear_bf16(x, w, b)
    y0 = agk.linear_bf16(x, w, None)
    plain = agk.gemm_bf16(x, w, trans_b=True)
    torch.cuda.synchronize()
    assert torch.equal(y0, plain)
    assert torch.equal(y, (plain.float() + b.float()).bfloat16())
    r = x.float() @ w.float().t() + b.float()
    assert ((y.float() - r).abs().max() / r.abs().max()).item() <= 8e-3
