"""cgadimpl_amd -- MI355X (gfx950) RMSNorm layer path for cgadimpl's autodiff API.

The product is native: HIP kernels behind the C ABI in ``include/agk_rmsnorm.h``
and ``include/agk_rowops.h`` (``lib/libagk_rmsnorm.so``) and the C++ ``ag::`` layer above it.  This Python
module is plumbing for tests and benchmarks: it binds that C ABI with ctypes
and hands it torch device tensors (memory) and the current HIP stream.  There
is no Python or CPU fallback: if the library is missing, every call raises.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional, Tuple

__all__ = [
    "AgkError", "lib", "lib_path", "rmsnorm_fwd", "rmsnorm_bwd", "rmsnorm_bwd_workspace_bytes",
    "mul_rowbcast_fwd", "mul_rowbcast_bwd", "launch_plan", "gemm_bf16", "gemm_bf16_workspace_bytes",
    "transpose_bf16", "rmsnorm_linear_fwd", "rmsnorm_linear_bwd", "rmsnorm_jvp", "layernorm_fwd",
    "layernorm_bwd", "softmax_fwd", "softmax_bwd", "logsumexp_fwd", "logsumexp_bwd",
    "logsumexp_jvp", "logsumexp_fwd_keep", "logsumexp_bwd_from_value", "rms_mul_bwd", "sum_rows", "linear_bf16",
    "mul_bcast_shape", "mul_bcast_fwd", "mul_bcast_bwd",
    "mul_bcast_grad_dtype", "gemm_f32", "set_exchange_wait_limit", "set_team_backward",
    "AGK_F32", "AGK_BF16", "STATUS",
]

_PKG = os.path.dirname(os.path.abspath(__file__))
# AGK_LIB_DIR selects another build of the libraries (tests/run_sanitized.py
# points it at the host-sanitised build); the default is the in-tree build.
LIB_DIR = os.environ.get("AGK_LIB_DIR") or os.path.join(_PKG, "lib")

AGK_F32 = 0
AGK_BF16 = 1
AGK_ACCUM_DX = 1
AGK_ACCUM_DGAMMA = 2
AGK_ACCUM_ALL = 3
AGK_WIDE_MIN_COLS = 16385  # rows this wide and wider can take the split paths
STATUS = {0: "AGK_OK", 1: "AGK_EINVAL", 2: "AGK_EDTYPE", 3: "AGK_EWORKSPACE", 4: "AGK_EHIP"}

# Every symbol include/agk_rmsnorm.h and include/agk_rowops.h declare, with its
# ctypes signature.
_P = ctypes.c_void_p
_I64 = ctypes.c_int64
SIGNATURES = {
    "agk_rmsnorm_fwd": (ctypes.c_int, [_P, _P, _P, _P, _I64, _I64, ctypes.c_float, ctypes.c_int, _P]),
    "agk_rmsnorm_fwd_workspace_bytes": (ctypes.c_size_t, [_I64, _I64]),
    "agk_rmsnorm_fwd_ws": (ctypes.c_int, [_P, _P, _P, _P, _P, ctypes.c_size_t, _I64, _I64,
                                          ctypes.c_float, ctypes.c_int, _P]),
    "agk_rmsnorm_bwd_workspace_bytes": (ctypes.c_size_t, [_I64, _I64]),
    "agk_rmsnorm_bwd": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, ctypes.c_size_t, _I64, _I64,
                                       ctypes.c_int, ctypes.c_int, _P]),
    "agk_rmsnorm_bwd_noalloc": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _I64, _I64, ctypes.c_int,
                                               ctypes.c_int, _P]),
    "agk_mul_rowbcast_fwd": (ctypes.c_int, [_P, _P, _P, _I64, _I64, ctypes.c_int, _P]),
    "agk_mul_rowbcast_bwd_workspace_bytes": (ctypes.c_size_t, [_I64, _I64]),
    "agk_mul_rowbcast_bwd": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, ctypes.c_size_t, _I64, _I64,
                                            ctypes.c_int, ctypes.c_int, _P]),
    "agk_rms_mul_bwd": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, _P, ctypes.c_size_t, _I64,
                                       _I64, ctypes.c_int, ctypes.c_int, _P]),
    "agk_mul_bcast_shape": (ctypes.c_int, [_P, ctypes.c_int, _P, ctypes.c_int, _P, _P]),
    "agk_mul_bcast_fwd": (ctypes.c_int, [_P, _P, ctypes.c_int, _P, _P, ctypes.c_int, _P,
                                         ctypes.c_int, ctypes.c_int, _P]),
    "agk_mul_bcast_bwd": (ctypes.c_int, [_P, _P, _P, ctypes.c_int, _P, _P, ctypes.c_int, _P, _P,
                                         ctypes.c_int, ctypes.c_int, _P]),
    "agk_gemm_f32": (ctypes.c_int, [_P, _I64, ctypes.c_int, _P, _I64, ctypes.c_int, _P, _I64,
                                    _I64, _I64, _I64, ctypes.c_int, _P]),
    "agk_sum_rows_workspace_bytes": (ctypes.c_size_t, [_I64, _I64]),
    "agk_sum_rows": (ctypes.c_int, [_P, _P, _P, ctypes.c_size_t, _I64, _I64, ctypes.c_int,
                                    ctypes.c_int, _P]),
    "agk_linear_bf16": (ctypes.c_int, [_P, _I64, _P, _I64, _P, _P, _I64, _I64, _I64, _I64, _P]),
    "agk_gemm_bf16": (ctypes.c_int, [_P, _I64, ctypes.c_int, _P, _I64, ctypes.c_int, _P, _I64,
                                     ctypes.c_int, _I64, _I64, _I64, _P, _P, ctypes.c_int, _P,
                                     ctypes.c_size_t, _P]),
    "agk_gemm_bf16_workspace_bytes": (ctypes.c_size_t, [_I64, _I64, _I64, ctypes.c_int,
                                                        ctypes.c_int]),
    "agk_transpose_bf16": (ctypes.c_int, [_P, _I64, _P, _I64, _I64, _I64, _P]),
    "agk_rmsnorm_launch_plan": (ctypes.c_int, [_I64, _I64, ctypes.c_int, ctypes.c_int, _P]),
    "agk_set_exchange_wait_limit": (ctypes.c_int, [ctypes.c_int]),
    "agk_set_team_backward": (ctypes.c_int, [ctypes.c_int]),
    "agk_set_team_forward": (ctypes.c_int, [ctypes.c_int]),
    "agk_rmsnorm_jvp": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _I64, _I64, ctypes.c_int, _P]),
    "agk_layernorm_fwd": (ctypes.c_int, [_P, _P, _P, _P, _I64, _I64, ctypes.c_float, ctypes.c_int,
                                         _P]),
    "agk_layernorm_bwd": (ctypes.c_int, [_P, _P, _P, _P, _P, _I64, _I64, ctypes.c_int, ctypes.c_int,
                                         _P]),
    "agk_softmax_fwd": (ctypes.c_int, [_P, _P, _I64, _I64, ctypes.c_int, _P]),
    "agk_softmax_bwd": (ctypes.c_int, [_P, _P, _P, _I64, _I64, ctypes.c_int, ctypes.c_int, _P]),
    "agk_logsumexp_fwd": (ctypes.c_int, [_P, _P, _I64, _I64, ctypes.c_int, _P]),
    "agk_logsumexp_bwd": (ctypes.c_int, [_P, _P, _P, _I64, _I64, ctypes.c_int, ctypes.c_int, _P]),
    "agk_logsumexp_jvp": (ctypes.c_int, [_P, _P, _P, _I64, _I64, ctypes.c_int, _P]),
    "agk_logsumexp_fwd_keep": (ctypes.c_int, [_P, _P, _P, _I64, _I64, ctypes.c_int, _P]),
    "agk_logsumexp_bwd_from_value": (ctypes.c_int, [_P, _P, _P, _P, _I64, _I64, ctypes.c_int,
                                                    ctypes.c_int, _P]),
    "agk_rowops_workspace_bytes": (ctypes.c_size_t, [_I64, _I64]),
    "agk_softmax_fwd_ws": (ctypes.c_int, [_P, _P, _P, ctypes.c_size_t, _I64, _I64, ctypes.c_int,
                                          _P]),
    "agk_softmax_bwd_ws": (ctypes.c_int, [_P, _P, _P, _P, ctypes.c_size_t, _I64, _I64,
                                          ctypes.c_int, ctypes.c_int, _P]),
    "agk_logsumexp_bwd_ws": (ctypes.c_int, [_P, _P, _P, _P, ctypes.c_size_t, _I64, _I64,
                                            ctypes.c_int, ctypes.c_int, _P]),
    "agk_set_rowops_team": (ctypes.c_int, [ctypes.c_int]),
    "agk_rowops_team_plan": (ctypes.c_int, [ctypes.c_int, _I64, _I64, ctypes.c_int, ctypes.c_int,
                                            _P]),
    "agk_fill": (ctypes.c_int, [_P, _I64, ctypes.c_float, ctypes.c_int, _P]),
    "agk_status_str": (ctypes.c_char_p, [ctypes.c_int]),
    "agk_last_error": (ctypes.c_char_p, []),
    "agk_version": (ctypes.c_char_p, []),
}


class AgkError(RuntimeError):
    """A non-zero agk_status returned through the C ABI."""

    def __init__(self, status: int, where: str):
        self.status = status
        detail = _status_str(status)
        if status == 4:
            try:
                detail += "; HIP: " + lib().agk_last_error().decode()
            except Exception:  # noqa: BLE001 - only used while formatting an error
                pass
        super().__init__(f"{where}: {STATUS.get(status, status)} ({detail})")


_lib: Optional[ctypes.CDLL] = None


def lib_path() -> str:
    return os.path.join(LIB_DIR, "libagk_rmsnorm.so")


def lib() -> ctypes.CDLL:
    """Load libagk_rmsnorm.so (built by __graft_entry__.build()); raise if absent."""
    global _lib
    if _lib is None:
        path = lib_path()
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is missing: run __graft_entry__.build() first "
                               "(the RMSNorm path has no fallback)")
        # torch ships its own HIP runtime (SONAME libamdhip64.so.7) and links it
        # by the name libamdhip64.so.  Loading torch first makes this library's
        # libamdhip64.so.7 dependency resolve to that same runtime; loading this
        # library first would bring in /opt/rocm's copy, torch would then load
        # a second runtime beside it, and one of the two sees no device.
        import torch  # noqa: F401
        handle = ctypes.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def _status_str(status: int) -> str:
    try:
        return lib().agk_status_str(status).decode()
    except Exception:  # noqa: BLE001 - only used while formatting an error
        return "?"


def _check(status: int, where: str) -> None:
    if status != 0:
        raise AgkError(status, where)


# ---- torch plumbing ------------------------------------------------------------

_torch_mod = None
_dtype_codes: dict = {}


def _torch():
    global _torch_mod
    if _torch_mod is None:
        import torch
        _torch_mod = torch
    return _torch_mod


def _dtype_code(t) -> int:
    if not _dtype_codes:
        torch = _torch()
        _dtype_codes.update({torch.float32: AGK_F32, torch.bfloat16: AGK_BF16})
    code = _dtype_codes.get(t.dtype)
    if code is None:
        raise TypeError(f"unsupported storage dtype {t.dtype} (float32 or bfloat16)")
    return code


def _ptr(t) -> Optional[int]:
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("tensor must live on the GPU")
    if not t.is_contiguous():
        raise ValueError("tensor must be contiguous (row-major, normalised axis last)")
    return t.data_ptr()


def _stream(stream) -> int:
    torch = _torch()
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


def rmsnorm_bwd_workspace_bytes(rows: int, cols: int) -> int:
    return int(lib().agk_rmsnorm_bwd_workspace_bytes(rows, cols))


def rmsnorm_fwd_workspace_bytes(rows: int, cols: int) -> int:
    return int(lib().agk_rmsnorm_fwd_workspace_bytes(rows, cols))


def rmsnorm_fwd(x, gamma, eps: float, y=None, inv_rms=None, workspace=False, stream=None):
    """y = x * rsqrt(mean(x^2, -1) + eps) * gamma; returns (y, inv_rms[rows]).

    workspace: False (default) calls agk_rmsnorm_fwd; None allocates what
    agk_rmsnorm_fwd_ws uses for the shape (wide rows then take the team
    kernel, one read of x); a device tensor is passed to agk_rmsnorm_fwd_ws
    as given."""
    torch = _torch()
    cols = x.shape[-1] if x.dim() else 1
    rows = x.numel() // cols if cols else 0
    if y is None:
        y = torch.empty_like(x)
    if inv_rms is None:
        inv_rms = torch.empty(x.shape[:-1], dtype=torch.float32, device=x.device)
    if workspace is False:
        rc = lib().agk_rmsnorm_fwd(_ptr(x), _ptr(gamma), _ptr(y), _ptr(inv_rms), rows, cols,
                                   float(eps), _dtype_code(x), _stream(stream))
        _check(rc, "agk_rmsnorm_fwd")
        return y, inv_rms
    if workspace is None:
        need = rmsnorm_fwd_workspace_bytes(rows, cols)
        workspace = torch.empty(need, dtype=torch.uint8, device=x.device) if need else None
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    rc = lib().agk_rmsnorm_fwd_ws(_ptr(x), _ptr(gamma), _ptr(y), _ptr(inv_rms), _ptr(workspace),
                                  ws_bytes, rows, cols, float(eps), _dtype_code(x),
                                  _stream(stream))
    _check(rc, "agk_rmsnorm_fwd_ws")
    return y, inv_rms


def _accum_flags(accumulate) -> int:
    """True -> both outputs accumulate; False -> neither; an int is the bit set."""
    if isinstance(accumulate, bool):
        return AGK_ACCUM_ALL if accumulate else 0
    return int(accumulate)


def rmsnorm_bwd(x, gamma, inv_rms, dy, dx=None, dgamma=None, accumulate=False,
                want_dgamma: bool = True, want_dx: bool = True, workspace=None, stream=None):
    """VJP of the layer; returns (dx or None, dgamma or None).

    accumulate: bool (both outputs) or agk_accumulate bits."""
    torch = _torch()
    cols = x.shape[-1]
    rows = x.numel() // cols if cols else 0
    acc = _accum_flags(accumulate)
    if want_dx and dx is None:
        dx = torch.empty_like(x) if not acc & AGK_ACCUM_DX else torch.zeros_like(x)
    if want_dgamma and dgamma is None:
        dgamma = torch.empty(cols, dtype=torch.float32, device=x.device)
    # a workspace is required for dgamma, and lets dx alone take the split
    # path on wide rows
    if workspace is None and (dgamma is not None or cols >= AGK_WIDE_MIN_COLS):
        ws_bytes = rmsnorm_bwd_workspace_bytes(rows, cols)
        if ws_bytes:
            workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device)
    ws_have = workspace.numel() * workspace.element_size() if workspace is not None else 0
    rc = lib().agk_rmsnorm_bwd(_ptr(x), _ptr(gamma), _ptr(inv_rms), _ptr(dy), _ptr(dx),
                               _ptr(dgamma), _ptr(workspace), ws_have, rows, cols,
                               _dtype_code(x), acc, _stream(stream))
    _check(rc, "agk_rmsnorm_bwd")
    return dx, dgamma


def gemm_bf16_workspace_bytes(M: int, N: int, K: int, trans_a: bool, trans_b: bool) -> int:
    return int(lib().agk_gemm_bf16_workspace_bytes(M, N, K, int(trans_a), int(trans_b)))


def transpose_bf16(src, dst=None, stream=None):
    """dst = src.T for a 2-D bfloat16 device tensor (through agk_transpose_bf16)."""
    torch = _torch()
    rows, cols = src.shape
    if dst is None:
        dst = torch.empty(cols, rows, dtype=src.dtype, device=src.device)
    _check(lib().agk_transpose_bf16(_ptr(src), cols, _ptr(dst), rows, rows, cols, _stream(stream)),
           "agk_transpose_bf16")
    return dst


def gemm_bf16(a, b, c=None, trans_a: bool = False, trans_b: bool = False, out_dtype=None,
              kscale=None, rowscale=None, accumulate: bool = False, workspace="auto",
              stream=None):
    """C (+)= rowscale[:, None] * ((A * kscale[None, :]) @ B) on MFMA, bf16 in, fp32 accumulate.

    a is A [M, K] (or A^T [K, M] with trans_a); b is B [K, N] (or B^T [N, K]
    with trans_b); both bfloat16 and contiguous.  kscale: float32 [K] applied
    to A as it is staged (rounded to bf16); rowscale: float32 [M] applied to
    the result.  out_dtype: torch.float32 or torch.bfloat16 (default bf16).
    """
    torch = _torch()
    if a.dtype != torch.bfloat16 or b.dtype != torch.bfloat16:
        raise TypeError("gemm_bf16 takes bfloat16 operands")
    M, K = (a.shape[1], a.shape[0]) if trans_a else (a.shape[0], a.shape[1])
    N = b.shape[0] if trans_b else b.shape[1]
    if (b.shape[1] if trans_b else b.shape[0]) != K:
        raise ValueError("inner dimensions differ")
    if c is None:
        c = torch.empty(M, N, dtype=out_dtype or torch.bfloat16, device=a.device)
    if isinstance(workspace, str):  # "auto": allocate what the fast path needs
        need = gemm_bf16_workspace_bytes(M, N, K, trans_a, trans_b) if kscale is None else 0
        workspace = torch.empty(need, dtype=torch.uint8, device=a.device) if need else None
    ws_bytes = workspace.numel() if workspace is not None else 0
    rc = lib().agk_gemm_bf16(_ptr(a), a.shape[1], int(trans_a), _ptr(b), b.shape[1], int(trans_b),
                             _ptr(c), c.shape[1], _dtype_code(c), M, N, K, _ptr(kscale),
                             _ptr(rowscale), int(bool(accumulate)), _ptr(workspace), ws_bytes,
                             _stream(stream))
    _check(rc, "agk_gemm_bf16")
    return c


def gemm_f32(a, b, c=None, trans_a: bool = False, trans_b: bool = False, accumulate=False,
             stream=None):
    """C (+)= op(A) op(B) in fp32 (agk_gemm_f32: the fp32 MFMA kernel, deterministic).

    a: [M, K] (or [K, M] with trans_a), b: [K, N] (or [N, K] with trans_b),
    row-major contiguous float32; c [M, N] float32."""
    torch = _torch()
    M = a.shape[1] if trans_a else a.shape[0]
    K = a.shape[0] if trans_a else a.shape[1]
    N = b.shape[0] if trans_b else b.shape[1]
    if c is None:
        c = torch.empty(M, N, dtype=torch.float32, device=a.device)
    rc = lib().agk_gemm_f32(_ptr(a), a.shape[1], int(trans_a), _ptr(b), b.shape[1], int(trans_b),
                            _ptr(c), c.shape[1], M, N, K, int(bool(accumulate)), _stream(stream))
    _check(rc, "agk_gemm_f32")
    return c


def launch_plan(rows: int, cols: int, dtype: int, backward, fwd_workspace: bool = False) -> dict:
    """The launch shape agk_rmsnorm_{fwd,bwd} picks for these sizes (diagnostic;
    fwd_workspace: the forward of agk_rmsnorm_fwd_ws given a workspace).

    tpr == 0 with nv > 0 is the split path: nv segments and g chunks per
    row, rpb rows per backward tile, nblk dgamma partial rows (0: the tiles
    write dgamma directly).  g == 0 with tpr > 0 (backward, or the forward
    with a workspace) is the team kernel: a row over tpr / 256 workgroups of
    nv slots per lane, nblk teams (the backward's dgamma partial rows) taking
    the rows in turn."""
    out = (ctypes.c_int32 * 5)()
    mode = 1 if backward else (2 if fwd_workspace else 0)
    _check(lib().agk_rmsnorm_launch_plan(rows, cols, dtype, mode, out),
           "agk_rmsnorm_launch_plan")
    return {"tpr": out[0], "nv": out[1], "g": out[2], "rpb": out[3], "nblk": out[4]}


def set_exchange_wait_limit(polls: int) -> int:
    """Polls of the team kernel's wait before it recomputes a missing partial
    sum itself (testing knob; the results do not change).  Negative: read
    only.  Returns the previous value."""
    return int(lib().agk_set_exchange_wait_limit(int(polls)))


def set_team_backward(enabled: int) -> int:
    """1 (default): the wide RMSNorm backward may take the team kernel; 0: the
    split path instead (measurement and testing knob).  Negative: read only.
    Returns the previous value."""
    return int(lib().agk_set_team_backward(int(enabled)))


def set_team_forward(enabled: int) -> int:
    """1 (default): agk_rmsnorm_fwd_ws may take the team kernel for wide rows;
    0: the split path instead (measurement and testing knob).  Negative: read
    only.  Returns the previous value."""
    return int(lib().agk_set_team_forward(int(enabled)))


def mul_rowbcast_fwd(a, b, y=None, stream=None):
    torch = _torch()
    cols = a.shape[-1]
    rows = a.numel() // cols if cols else 0
    if y is None:
        y = torch.empty_like(a)
    rc = lib().agk_mul_rowbcast_fwd(_ptr(a), _ptr(b), _ptr(y), rows, cols, _dtype_code(a),
                                    _stream(stream))
    _check(rc, "agk_mul_rowbcast_fwd")
    return y


def mul_rowbcast_bwd(gy, a, b, da=None, db=None, accumulate=False, want_da: bool = True,
                     want_db: bool = True, stream=None) -> Tuple[object, object]:
    torch = _torch()
    cols = a.shape[-1]
    rows = a.numel() // cols if cols else 0
    acc = _accum_flags(accumulate)
    if want_da and da is None:
        da = torch.empty_like(a) if not acc & AGK_ACCUM_DX else torch.zeros_like(a)
    if want_db and db is None:
        db = torch.empty(cols, dtype=torch.float32, device=a.device)
    ws = None
    ws_bytes = int(lib().agk_mul_rowbcast_bwd_workspace_bytes(rows, cols)) if db is not None else 0
    if ws_bytes:
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=a.device)
    rc = lib().agk_mul_rowbcast_bwd(_ptr(gy), _ptr(a), _ptr(b), _ptr(da), _ptr(db), _ptr(ws),
                                    ws_bytes, rows, cols, _dtype_code(a), acc, _stream(stream))
    _check(rc, "agk_mul_rowbcast_bwd")
    return da, db


def rms_mul_bwd(x, gamma, inv_rms, gy, dx=None, dgamma=None, accumulate=False,
                want_dx: bool = True, want_dgamma: bool = True, dr=None, workspace=None,
                stream=None):
    """Both VJPs of y = rms(x) * gamma in one pass (agk_rms_mul_bwd).

    Returns (dr, dx, dgamma): dr = gy * gamma (the gradient of rms(x)), dx and
    dgamma as mul_rowbcast_bwd followed by rmsnorm_bwd(gamma=None) on dr give
    them, bit for bit.  inv_rms comes from rmsnorm_fwd(x, None, eps).  dr and
    the workspace (rmsnorm_bwd_workspace_bytes) are allocated when not given.
    """
    torch = _torch()
    cols = x.shape[-1]
    rows = x.numel() // cols if cols else 0
    acc = _accum_flags(accumulate)
    if dr is None:
        dr = torch.empty_like(x)
    if want_dx and dx is None:
        dx = torch.empty_like(x) if not acc & AGK_ACCUM_DX else torch.zeros_like(x)
    if want_dgamma and dgamma is None:
        dgamma = torch.empty(cols, dtype=torch.float32, device=x.device)
    if workspace is None and (dgamma is not None or cols >= AGK_WIDE_MIN_COLS):
        ws_bytes = rmsnorm_bwd_workspace_bytes(rows, cols)  # as rmsnorm_bwd
        if ws_bytes:
            workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device)
    ws_have = workspace.numel() * workspace.element_size() if workspace is not None else 0
    rc = lib().agk_rms_mul_bwd(_ptr(x), _ptr(gamma), _ptr(inv_rms), _ptr(gy), _ptr(dr), _ptr(dx),
                               _ptr(dgamma), _ptr(workspace), ws_have, rows, cols, _dtype_code(x),
                               acc, _stream(stream))
    _check(rc, "agk_rms_mul_bwd")
    return dr, dx, dgamma


def _shape_arg(shape):
    n = len(shape)
    return (ctypes.c_int64 * max(1, n))(*shape), n


def mul_bcast_shape(a_shape, b_shape) -> tuple:
    """The broadcast output shape of a * b (numpy rules; agk_mul_bcast_shape)."""
    ab, an = _shape_arg(tuple(a_shape))
    bb, bn = _shape_arg(tuple(b_shape))
    out = (ctypes.c_int64 * 8)()
    nd = ctypes.c_int(0)
    _check(lib().agk_mul_bcast_shape(ab, an, bb, bn, out, ctypes.byref(nd)), "agk_mul_bcast_shape")
    return tuple(out[i] for i in range(nd.value))


def mul_bcast_fwd(a, b, y=None, accumulate=False, stream=None):
    """y (+)= a * b under numpy broadcasting (agk_mul_bcast_fwd)."""
    torch = _torch()
    shape = mul_bcast_shape(a.shape, b.shape)
    if y is None:
        y = torch.empty(shape, dtype=a.dtype, device=a.device)
    ab, an = _shape_arg(tuple(a.shape))
    bb, bn = _shape_arg(tuple(b.shape))
    rc = lib().agk_mul_bcast_fwd(_ptr(a), ab, an, _ptr(b), bb, bn, _ptr(y), _dtype_code(a),
                                 int(bool(accumulate)), _stream(stream))
    _check(rc, "agk_mul_bcast_fwd")
    return y


def mul_bcast_grad_dtype(operand_shape, out_shape, dtype):
    """The dtype agk_mul_bcast_bwd writes an operand's gradient in: the storage
    dtype when the operand covers the output, fp32 when it was broadcast."""
    torch = _torch()
    n = len(out_shape)
    aligned = (1,) * (n - len(operand_shape)) + tuple(operand_shape)
    return dtype if aligned == tuple(out_shape) else torch.float32


def mul_bcast_bwd(gy, a, b, da=None, db=None, accumulate=False, want_da: bool = True,
                  want_db: bool = True, stream=None):
    """vjp_Mul with reduce_for_broadcast (agk_mul_bcast_bwd): da (+)= the sum of
    gy * b over a's broadcast axes, db likewise; gradients of broadcast operands
    in fp32, of full-shape operands in the storage dtype."""
    torch = _torch()
    out_shape = mul_bcast_shape(a.shape, b.shape)
    acc = _accum_flags(accumulate)
    if want_da and da is None:
        da = torch.empty(tuple(a.shape), dtype=mul_bcast_grad_dtype(a.shape, out_shape, a.dtype),
                         device=a.device)
    if want_db and db is None:
        db = torch.empty(tuple(b.shape), dtype=mul_bcast_grad_dtype(b.shape, out_shape, b.dtype),
                         device=b.device)
    ab, an = _shape_arg(tuple(a.shape))
    bb, bn = _shape_arg(tuple(b.shape))
    rc = lib().agk_mul_bcast_bwd(_ptr(gy), _ptr(a), ab, an, _ptr(b), bb, bn, _ptr(da), _ptr(db),
                                 _dtype_code(a), acc, _stream(stream))
    _check(rc, "agk_mul_bcast_bwd")
    return da, db


def sum_rows(x, out=None, accumulate=False, stream=None):
    """out[j] (+)= sum_i x[i, j] in fp32, deterministic (agk_sum_rows)."""
    torch = _torch()
    cols = x.shape[-1]
    rows = x.numel() // cols if cols else 0
    if out is None:
        out = torch.empty(cols, dtype=torch.float32, device=x.device)
    wsb = int(lib().agk_sum_rows_workspace_bytes(rows, cols))
    ws = torch.empty(wsb, dtype=torch.uint8, device=x.device) if wsb else None
    rc = lib().agk_sum_rows(_ptr(x), _ptr(out), _ptr(ws), wsb, rows, cols, _dtype_code(x),
                            int(bool(accumulate)), _stream(stream))
    _check(rc, "agk_sum_rows")
    return out


def linear_bf16(x, w, bias=None, y=None, stream=None):
    """y = x @ w^T + bias (agk_linear_bf16): x [M, K], w [N, K], bias [N], bf16."""
    torch = _torch()
    if x.dtype != torch.bfloat16 or w.dtype != torch.bfloat16:
        raise TypeError("linear_bf16 takes bfloat16 operands")
    if x.dim() != 2 or w.dim() != 2:
        raise ValueError("linear_bf16 takes a 2-D x [M, K] and w [N, K]")
    M, K = x.shape
    N = w.shape[0]
    if w.shape[1] != K:
        raise ValueError("x and w disagree on the input width")
    if bias is not None:
        if bias.dtype != torch.bfloat16:
            raise TypeError("the bias must be bfloat16 (it is added as bf16 values)")
        if bias.numel() != N or not bias.is_contiguous():
            raise ValueError(f"the bias must be a contiguous tensor of N = {N} values")
    if y is None:
        y = torch.empty(M, N, dtype=torch.bfloat16, device=x.device)
    elif y.dtype != torch.bfloat16 or tuple(y.shape) != (M, N):
        raise ValueError(f"y must be a bfloat16 [{M}, {N}] tensor")
    rc = lib().agk_linear_bf16(_ptr(x), x.shape[1], _ptr(w), w.shape[1], _ptr(bias), _ptr(y),
                               y.shape[1], M, N, K, _stream(stream))
    _check(rc, "agk_linear_bf16")
    return y


# ---- the RMSNorm + linear layer (configuration c5) --------------------------------

def rmsnorm_linear_fwd(x, gamma, W, eps: float, stream=None):
    """h = rms_norm(x) * gamma, y = h @ W.  bf16 x [M, K], gamma [K], W [K, N].

    W is read as it lies ([K, N], n contiguous): the GEMM stages it with its
    transposing LDS reads, the same product path bench.py times for c5.
    Returns (y, h, inv_rms).
    """
    h, inv = rmsnorm_fwd(x, gamma, eps, stream=stream)
    y = gemm_bf16(h, W, workspace=None, stream=stream)
    return y, h, inv


def rmsnorm_linear_bwd(x, gamma, inv_rms, h, W, dy, dw_dtype=None, stream=None):
    """VJP of the layer: dW = h^T @ dy, dh = dy @ W^T, then the RMSNorm VJP of dh.

    dW runs first so that dh is still in the caches when the RMSNorm VJP reads it.
    Returns (dx, dgamma, dW); dW is float32 unless dw_dtype says otherwise.
    """
    torch = _torch()
    dW = gemm_bf16(h, dy, trans_a=True, out_dtype=dw_dtype or torch.float32, stream=stream)
    dh = gemm_bf16(dy, W, trans_b=True, workspace=None, stream=stream)
    dx, dgamma = rmsnorm_bwd(x, gamma, inv_rms, dh, stream=stream)
    return dx, dgamma, dW


# ---- row ops sharing the row-reduce skeleton (include/agk_rowops.h) -------------

def _rows_cols(t):
    cols = t.shape[-1] if t.dim() else 1
    return (t.numel() // cols if cols else 0), cols


def _row_stat_like(x, dtype):
    torch = _torch()
    return torch.empty(x.shape[:-1] + (1,), dtype=dtype, device=x.device)


def _acc_dx(accumulate) -> int:
    return AGK_ACCUM_DX if accumulate else 0


def rmsnorm_jvp(x, gamma, inv_rms, tx, tgamma=None, ty=None, stream=None):
    """Tangent of y = rms_norm(x) * gamma along (tx, tgamma); inv_rms from rmsnorm_fwd."""
    torch = _torch()
    rows, cols = _rows_cols(x)
    if ty is None:
        ty = torch.empty_like(x)
    rc = lib().agk_rmsnorm_jvp(_ptr(x), _ptr(gamma), _ptr(inv_rms), _ptr(tx), _ptr(tgamma),
                               _ptr(ty), rows, cols, _dtype_code(x), _stream(stream))
    _check(rc, "agk_rmsnorm_jvp")
    return ty


def layernorm_fwd(x, eps: float = 1e-5, y=None, mean=None, rstd=None, stream=None):
    """y = (x - mean) / sqrt(var + eps) over the last axis; returns (y, mean, rstd)."""
    torch = _torch()
    rows, cols = _rows_cols(x)
    y = torch.empty_like(x) if y is None else y
    mean = _row_stat_like(x, torch.float32) if mean is None else mean
    rstd = _row_stat_like(x, torch.float32) if rstd is None else rstd
    rc = lib().agk_layernorm_fwd(_ptr(x), _ptr(y), _ptr(mean), _ptr(rstd), rows, cols,
                                 float(eps), _dtype_code(x), _stream(stream))
    _check(rc, "agk_layernorm_fwd")
    return y, mean, rstd


def layernorm_bwd(x, mean, rstd, dy, dx=None, accumulate: bool = False, stream=None):
    """dx (+)= VJP of LayerNorm for upstream dy (also the JVP for dy = a tangent)."""
    torch = _torch()
    rows, cols = _rows_cols(x)
    dx = (torch.zeros_like(x) if accumulate else torch.empty_like(x)) if dx is None else dx
    rc = lib().agk_layernorm_bwd(_ptr(x), _ptr(mean), _ptr(rstd), _ptr(dy), _ptr(dx), rows, cols,
                                 _dtype_code(x), _acc_dx(accumulate), _stream(stream))
    _check(rc, "agk_layernorm_bwd")
    return dx


def rowops_workspace_bytes(rows: int, cols: int) -> int:
    return int(lib().agk_rowops_workspace_bytes(rows, cols))


def _rowops_ws(workspace, rows, cols, device):
    """(pointer, bytes) for the *_ws row ops: None allocates what the shape
    uses (nothing when it uses none), False passes no workspace (the
    workspace-free kernels), a tensor is used as given."""
    if workspace is False:
        return None, 0
    if workspace is None:
        need = rowops_workspace_bytes(rows, cols)
        if not need:
            return None, 0
        workspace = _torch().empty(need, dtype=_torch().uint8, device=device)
    return workspace, workspace.numel() * workspace.element_size()


def softmax_fwd(z, y=None, workspace=None, stream=None):
    """y = softmax(z) over the last axis.  workspace: None (allocated as the
    shape needs: rows too wide for one workgroup then take the team kernel),
    False (the workspace-free entry point) or a device tensor."""
    torch = _torch()
    rows, cols = _rows_cols(z)
    y = torch.empty_like(z) if y is None else y
    ws, ws_bytes = _rowops_ws(workspace, rows, cols, z.device)
    if ws is None and workspace is False:
        rc = lib().agk_softmax_fwd(_ptr(z), _ptr(y), rows, cols, _dtype_code(z),
                                   _stream(stream))
    else:
        rc = lib().agk_softmax_fwd_ws(_ptr(z), _ptr(y), _ptr(ws), ws_bytes, rows, cols,
                                      _dtype_code(z), _stream(stream))
    _check(rc, "agk_softmax_fwd")
    return y


def softmax_bwd(y, dy, dz=None, accumulate: bool = False, workspace=None, stream=None):
    """dz (+)= y * (dy - sum(y * dy)) (also the JVP for dy = a tangent).
    workspace as for softmax_fwd."""
    torch = _torch()
    rows, cols = _rows_cols(y)
    dz = (torch.zeros_like(y) if accumulate else torch.empty_like(y)) if dz is None else dz
    ws, ws_bytes = _rowops_ws(workspace, rows, cols, y.device)
    if ws is None and workspace is False:
        rc = lib().agk_softmax_bwd(_ptr(y), _ptr(dy), _ptr(dz), rows, cols, _dtype_code(y),
                                   _acc_dx(accumulate), _stream(stream))
    else:
        rc = lib().agk_softmax_bwd_ws(_ptr(y), _ptr(dy), _ptr(dz), _ptr(ws), ws_bytes, rows,
                                      cols, _dtype_code(y), _acc_dx(accumulate),
                                      _stream(stream))
    _check(rc, "agk_softmax_bwd")
    return dz


ROWOPS_TEAM_OPS = {"softmax_fwd": 0, "softmax_bwd": 1, "logsumexp_bwd": 2}


def rowops_team_plan(op: str, rows: int, cols: int, dtype: int, aligned: bool = True) -> dict:
    """The team launch a *_ws row op ('softmax_fwd', 'softmax_bwd',
    'logsumexp_bwd') takes for these sizes (parts 0: none)."""
    out = (ctypes.c_int32 * 3)()
    _check(lib().agk_rowops_team_plan(ROWOPS_TEAM_OPS[op], rows, cols, dtype,
                                      int(bool(aligned)), out), "agk_rowops_team_plan")
    return {"parts": out[0], "slots_per_part": out[1], "teams": out[2]}


def set_rowops_team(mode: int) -> int:
    """When the *_ws row ops take the team kernel: 0 never, 1 (default) for
    rows too wide for one workgroup, 2 whenever the row fits it (testing and
    measurement knob).  Other values: read only.  Returns the previous mode."""
    return int(lib().agk_set_rowops_team(int(mode)))


def logsumexp_fwd(z, y=None, stream=None):
    """y[..., 0] = log(sum(exp(z), -1)); y has z's dtype and shape z.shape[:-1] + (1,)."""
    rows, cols = _rows_cols(z)
    y = _row_stat_like(z, z.dtype) if y is None else y
    rc = lib().agk_logsumexp_fwd(_ptr(z), _ptr(y), rows, cols, _dtype_code(z), _stream(stream))
    _check(rc, "agk_logsumexp_fwd")
    return y


def logsumexp_bwd(z, dy, dz=None, accumulate: bool = False, workspace=None, stream=None):
    """dz (+)= dy * softmax(z); dy has shape z.shape[:-1] + (1,) and z's dtype.
    workspace as for softmax_fwd."""
    torch = _torch()
    rows, cols = _rows_cols(z)
    dz = (torch.zeros_like(z) if accumulate else torch.empty_like(z)) if dz is None else dz
    ws, ws_bytes = _rowops_ws(workspace, rows, cols, z.device)
    if ws is None and workspace is False:
        rc = lib().agk_logsumexp_bwd(_ptr(z), _ptr(dy), _ptr(dz), rows, cols, _dtype_code(z),
                                     _acc_dx(accumulate), _stream(stream))
    else:
        rc = lib().agk_logsumexp_bwd_ws(_ptr(z), _ptr(dy), _ptr(dz), _ptr(ws), ws_bytes, rows,
                                        cols, _dtype_code(z), _acc_dx(accumulate),
                                        _stream(stream))
    _check(rc, "agk_logsumexp_bwd")
    return dz


def logsumexp_fwd_keep(z, y=None, lse=None, stream=None):
    """logsumexp_fwd that also returns lse, the same values in float32, for
    logsumexp_bwd_from_value; returns (y, lse)."""
    torch = _torch()
    rows, cols = _rows_cols(z)
    y = _row_stat_like(z, z.dtype) if y is None else y
    lse = _row_stat_like(z, torch.float32) if lse is None else lse
    rc = lib().agk_logsumexp_fwd_keep(_ptr(z), _ptr(y), _ptr(lse), rows, cols, _dtype_code(z),
                                      _stream(stream))
    _check(rc, "agk_logsumexp_fwd_keep")
    return y, lse


def logsumexp_bwd_from_value(z, lse, dy, dz=None, accumulate: bool = False, stream=None):
    """dz (+)= dy * exp(z - lse), lse the forward's float32 value (one pass over z)."""
    torch = _torch()
    rows, cols = _rows_cols(z)
    dz = (torch.zeros_like(z) if accumulate else torch.empty_like(z)) if dz is None else dz
    rc = lib().agk_logsumexp_bwd_from_value(_ptr(z), _ptr(lse), _ptr(dy), _ptr(dz), rows, cols,
                                            _dtype_code(z), _acc_dx(accumulate),
                                            _stream(stream))
    _check(rc, "agk_logsumexp_bwd_from_value")
    return dz


def logsumexp_jvp(z, tz, ty=None, stream=None):
    """ty[..., 0] = sum(softmax(z) * tz, -1)."""
    rows, cols = _rows_cols(z)
    ty = _row_stat_like(z, z.dtype) if ty is None else ty
    rc = lib().agk_logsumexp_jvp(_ptr(z), _ptr(tz), _ptr(ty), rows, cols, _dtype_code(z),
                                 _stream(stream))
    _check(rc, "agk_logsumexp_jvp")
    return ty
