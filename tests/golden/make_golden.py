"""Writes tests/golden/rmsnorm_golden.json and tests/golden/bf16_golden.json.

The reference (cgadimpl) holds no golden vectors for its RMSNorm path and
cannot be built here, so these fixtures come from an independent library
implementation: torch.nn.functional.rms_norm and torch autograd, evaluated in
float64 on the CPU.  Inputs are float32 values (stored exactly), so the fp32
oracle and the GPU path can be fed the same numbers.

Cases cover the reference's own test pattern (ag::rms on a [4,10] input with
loss sum(.), i.e. dy = 1, eps = 1e-5, cgadimpl/Tests/test_core_ops_gpu.cpp:262-267),
the layer with gamma, a rank-3 input, a large eps that makes the eps term
visible, special rows (zero, constant, one-hot, tiny) and outliers.

bf16_golden.json pins float32 -> bfloat16 round-to-nearest-even against
torch's conversion, including ties, subnormals, infinities and NaN.

Run:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import json
import os

import numpy as np
import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))


def _f32(a) -> np.ndarray:
    return np.asarray(a, dtype=np.float32)


def _case(name, x, gamma, dy, eps, note):
    x = _f32(x)
    dy = _f32(dy)
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    gt = None
    if gamma is not None:
        gamma = _f32(gamma)
        gt = torch.tensor(gamma, dtype=torch.float64, requires_grad=True)
    y = F.rms_norm(xt, (x.shape[-1],), weight=gt, eps=eps)
    y.backward(torch.tensor(dy, dtype=torch.float64))
    xd = xt.detach()
    inv = torch.rsqrt(xd.pow(2).mean(-1) + eps)
    out = {
        "name": name,
        "note": note,
        "shape": list(x.shape),
        "eps": eps,
        "x": x.ravel().astype(float).tolist(),
        "gamma": None if gamma is None else gamma.astype(float).tolist(),
        "dy": dy.ravel().astype(float).tolist(),
        "y": y.detach().numpy().ravel().tolist(),
        "inv_rms": inv.numpy().ravel().tolist(),
        "dx": xt.grad.numpy().ravel().tolist(),
        "dgamma": None if gt is None else gt.grad.numpy().tolist(),
    }
    return out


def rmsnorm_cases():
    rng = np.random.default_rng(20240607)
    cases = []
    x = rng.standard_normal((4, 10))
    cases.append(_case("ref_pattern_4x10", x, None, np.ones((4, 10)), 1e-5,
                       "ag::rms alone, loss sum(.), eps 1e-5 as in the reference test"))
    cases.append(_case("gamma_3x7", rng.standard_normal((3, 7)), rng.uniform(0.5, 1.5, 7),
                       rng.standard_normal((3, 7)), 1e-6, "layer with gamma, odd width"))
    cases.append(_case("rank3_2x3x5", rng.standard_normal((2, 3, 5)), rng.uniform(0.5, 1.5, 5),
                       rng.standard_normal((2, 3, 5)), 1e-6, "rank-3 input, last-axis norm"))
    cases.append(_case("large_eps_2x16", 0.3 * rng.standard_normal((2, 16)),
                       rng.uniform(0.5, 1.5, 16), rng.standard_normal((2, 16)), 0.5,
                       "eps comparable to mean(x^2): eps term dominates"))
    sp = np.zeros((5, 8))
    sp[1, :] = 2.0                              # constant row
    sp[2, 3] = 1.5                              # one-hot row
    sp[3, :] = 1e-3 * rng.standard_normal(8)    # tiny row, mean(x^2) << eps
    sp[4, :] = rng.standard_normal(8)
    cases.append(_case("special_rows_5x8", sp, rng.uniform(0.5, 1.5, 8),
                       rng.standard_normal((5, 8)), 1e-5,
                       "rows: zero, constant 2, one-hot, tiny, random"))
    cases.append(_case("wide_2x64", rng.standard_normal((2, 64)), rng.uniform(0.5, 1.5, 64),
                       rng.standard_normal((2, 64)), 1e-6, "vector-width multiple"))
    xo = 2.0 * rng.standard_normal((4, 32))
    xo[rng.random((4, 32)) < 0.05] *= 100.0
    cases.append(_case("outlier_4x32", xo, rng.uniform(0.5, 1.5, 32),
                       rng.standard_normal((4, 32)), 1e-5, "outlier entries x100"))
    cases.append(_case("negative_gamma_3x12", rng.standard_normal((3, 12)),
                       rng.uniform(-1.5, 1.5, 12), rng.standard_normal((3, 12)), 1e-6,
                       "gamma of both signs"))
    return cases


def bf16_cases():
    vals = [0.0, -0.0, 1.0, -1.0, 1.00390625, 1.0078125, 1.01171875,  # ties around 1
            1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -9, 3.14159265, -2.71828183, 65504.0,
            3.3895314e38, 1e-38, 1e-40, 1e-45, -1e-40, 1e30, -1e-30, 0.1, 0.2, 0.3,
            123456.789, 7.0e-3]
    rng = np.random.default_rng(7)
    vals += rng.standard_normal(40).astype(np.float32).tolist()
    bits = np.array(vals, dtype=np.float32).view(np.uint32)
    # exact ties: low 16 bits == 0x8000 with even and odd kept parts
    ties = np.array([0x3F808000, 0x3F818000, 0xBF808000, 0x40490000 | 0x8000, 0x00008000,
                     0x7F7F8000], dtype=np.uint32)
    specials = np.array([0x7F800000, 0xFF800000, 0x7FC00000, 0x7F800001, 0xFFC12345],
                        dtype=np.uint32)
    allbits = np.concatenate([bits, ties, specials])
    f = allbits.view(np.float32)
    tb = torch.tensor(f).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    nan_mask = np.isnan(f)
    return {
        "note": "float32 bits -> bfloat16 bits via torch (RNE); NaN entries only need to stay NaN",
        "f32_bits": [int(b) for b in allbits],
        "bf16_bits": [int(b) for b in tb],
        "is_nan": [bool(m) for m in nan_mask],
    }


def main():
    rms = {"generator": "torch.nn.functional.rms_norm + autograd, float64, torch "
                        + torch.__version__, "cases": rmsnorm_cases()}
    with open(os.path.join(HERE, "rmsnorm_golden.json"), "w") as fh:
        json.dump(rms, fh, indent=0)
    with open(os.path.join(HERE, "bf16_golden.json"), "w") as fh:
        json.dump(bf16_cases(), fh, indent=0)
    print("wrote golden fixtures")


if __name__ == "__main__":
    main()
