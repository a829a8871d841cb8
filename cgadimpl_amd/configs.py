"""Benchmark configurations of the RMSNorm layer path and their seeded inputs.

Shapes, distributions and eps follow the configuration list the benchmark is
quoted on.  Inputs come from ``lib/libagk_synth.so``: std::mt19937_64(seed)
with Box-Muller normals, drawn in the order x, gamma, dy, outlier mask, so the
GPU path and the CPU checker see identical bytes.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass, field
from typing import Dict, Optional, Tuple

import numpy as np

from . import LIB_DIR


@dataclass(frozen=True)
class LayerConfig:
    name: str
    shape: Tuple[int, ...]
    dtype: str                      # storage: "f32" or "bf16"
    eps: float
    x_std: float = 1.0
    outlier_p: float = 0.0          # fraction of x entries scaled by outlier_scale
    outlier_scale: float = 1.0
    seed: int = 0
    note: str = ""

    @property
    def cols(self) -> int:
        return self.shape[-1]

    @property
    def rows(self) -> int:
        n = 1
        for d in self.shape[:-1]:
            n *= d
        return n

    @property
    def storage_bytes(self) -> int:
        return 4 if self.dtype == "f32" else 2

    def algorithmic_bytes(self) -> int:
        """fwd+bwd bytes: 5*R*D*s + 2*D*s_gamma + 2*R*4 + D*4.

        fwd reads x, writes y; bwd reads x and dy, writes dx (5 passes of R*D
        elements), gamma read once per pass, inv_rms written then read,
        fp32 dgamma written once.
        """
        r, d, s = self.rows, self.cols, self.storage_bytes
        return 5 * r * d * s + 2 * d * s + 2 * r * 4 + d * 4

    def fwd_bytes(self) -> int:
        r, d, s = self.rows, self.cols, self.storage_bytes
        return 2 * r * d * s + d * s + r * 4

    def bwd_bytes(self) -> int:
        """bwd kernel + dgamma finalize: read x, dy, gamma, inv_rms; write dx, dgamma."""
        r, d, s = self.rows, self.cols, self.storage_bytes
        return 3 * r * d * s + d * s + r * 4 + d * 4


CONFIGS: Dict[str, LayerConfig] = {
    "c1": LayerConfig("c1", (4, 128, 512), "f32", 1e-6,
                      note="plumbing and correctness case"),
    "c2": LayerConfig("c2", (32, 2048, 4096), "f32", 1e-6,
                      note="headline: 65,536 rows x 4096, memory-bound"),
    "c3": LayerConfig("c3", (16, 4096, 8192), "bf16", 1e-5, x_std=2.0, outlier_p=1e-3,
                      outlier_scale=100.0, note="bf16 storage, fp32 math, outlier channels"),
    "c4a": LayerConfig("c4a", (7, 1023, 5120), "f32", 1e-6, note="irregular rows"),
    "c4b": LayerConfig("c4b", (1048576, 128), "f32", 1e-6, note="per-head q/k-norm width"),
    "c4c": LayerConfig("c4c", (3, 17, 13824), "f32", 1e-6, note="few wide rows"),
}


_synth: Optional[ctypes.CDLL] = None


def synth_lib() -> ctypes.CDLL:
    global _synth
    if _synth is None:
        path = os.path.join(LIB_DIR, "libagk_synth.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is missing: run __graft_entry__.build() first")
        h = ctypes.CDLL(path)
        P, I64, D = ctypes.c_void_p, ctypes.c_int64, ctypes.c_double
        h.agk_synth_new.restype = P
        h.agk_synth_new.argtypes = [ctypes.c_uint64]
        h.agk_synth_free.argtypes = [P]
        h.agk_synth_normal_f32.argtypes = [P, P, I64, D, D]
        h.agk_synth_uniform_f32.argtypes = [P, P, I64, D, D]
        h.agk_synth_outliers_f32.restype = I64
        h.agk_synth_outliers_f32.argtypes = [P, P, I64, D, D]
        h.agk_synth_to_bf16.argtypes = [P, P, I64]
        h.agk_synth_raw_u64.argtypes = [P, P, I64]
        _synth = h
    return _synth


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def to_bf16_bits(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape, dtype=np.uint16)
    synth_lib().agk_synth_to_bf16(_ptr(a), _ptr(out), a.size)
    return out


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32)


def make_inputs(shape, dtype: str = "f32", seed: int = 0, x_std: float = 1.0,
                outlier_p: float = 0.0, outlier_scale: float = 1.0, with_gamma: bool = True,
                with_dy: bool = True):
    """Seeded (x, gamma, dy) as numpy arrays: float32, or uint16 bf16 bit patterns."""
    lib = synth_lib()
    shape = tuple(int(s) for s in shape)
    n = int(np.prod(shape)) if shape else 1
    cols = shape[-1]
    g = lib.agk_synth_new(seed)
    try:
        x = np.empty(n, dtype=np.float32)
        lib.agk_synth_normal_f32(g, _ptr(x), n, 0.0, x_std)
        gamma = None
        if with_gamma:
            gamma = np.empty(cols, dtype=np.float32)
            lib.agk_synth_uniform_f32(g, _ptr(gamma), cols, 0.5, 1.5)
        dy = None
        if with_dy:
            dy = np.empty(n, dtype=np.float32)
            lib.agk_synth_normal_f32(g, _ptr(dy), n, 0.0, 1.0)
        if outlier_p > 0.0:
            lib.agk_synth_outliers_f32(g, _ptr(x), n, outlier_p, outlier_scale)
    finally:
        lib.agk_synth_free(g)
    x = x.reshape(shape)
    if dy is not None:
        dy = dy.reshape(shape)
    if dtype == "bf16":
        x = to_bf16_bits(x)
        gamma = to_bf16_bits(gamma) if gamma is not None else None
        dy = to_bf16_bits(dy) if dy is not None else None
    return x, gamma, dy


def config_inputs(cfg: LayerConfig, shape: Optional[Tuple[int, ...]] = None):
    """Inputs for cfg (optionally at a reduced shape with the same distributions)."""
    return make_inputs(shape or cfg.shape, cfg.dtype, cfg.seed, cfg.x_std, cfg.outlier_p,
                       cfg.outlier_scale)
