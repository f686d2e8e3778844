#!/usr/bin/env python3
"""Writes reference_vectors.npz: outputs of the reference's own CPU path on small seeded inputs.

The reference's plain-C++ path (fpga/src/gemvq_ref.h) is compiled, where it lies in the reference tree, into
oracle/_ref/libgemvq_ref.so by `make -C oracle ref`; this script runs it through that library's C wrappers and
stores inputs and outputs, so that the oracle can be checked against the reference on machines without the
reference tree. Regenerate with:  python tests/golden/make_golden.py   (needs the reference tree and oracle/_ref)
"""
from __future__ import annotations

import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "fpga-llama-gguf_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

import gemvq as gq  # noqa: E402
import oracle  # noqa: E402

F = np.float32
Q4_0, Q4_1, Q8_0, Q5_K, Q6_K = 2, 3, 8, 13, 14


def p(a):
    return a.ctypes.data


def finite_halves(rng, n, lo, hi):
    """fp16 bit patterns of uniform values in [lo, hi) (finite, normal)."""
    return rng.uniform(lo, hi, n).astype(np.float16).view(np.uint16)


def q4_1_matrix(rng, rows, cols):
    """Random Q4_1 blocks (fp16 d, fp16 m, 16 bytes of nibbles): every nibble pattern, finite scales."""
    nb = rows * cols // 32
    blk = np.zeros((nb, 20), np.uint8)
    blk[:, 0:2] = finite_halves(rng, nb, 0.001, 0.01).reshape(nb, 1).view(np.uint8)
    blk[:, 2:4] = finite_halves(rng, nb, -0.08, 0.0).reshape(nb, 1).view(np.uint8)
    blk[:, 4:] = rng.integers(0, 256, (nb, 16), dtype=np.uint8)
    return blk.ravel()


def main() -> int:
    oracle.build(ref=True)
    if not oracle.ref_available():
        print("the reference tree is not present: nothing to do", file=sys.stderr)
        return 1
    ref = oracle.ref()
    rng = np.random.default_rng(20260101)
    out: dict[str, np.ndarray] = {}

    # fp16 conversion of special values: ties to even, subnormals, overflow, signed zero
    specials = np.array([0.0, -0.0, 1.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, 5.96e-8, 2.98e-8, 2.99e-8, 8.9e-8,
                         6.1035156e-05, 6.1e-05, 1.00048828125, 1.000732421875, 1.0009765625, -3.0517578e-05,
                         np.inf, -np.inf], F)
    specials = np.concatenate([specials, rng.standard_normal(236).astype(F) * np.float32(1000)])
    out["f2h_in"] = specials
    out["f2h_out"] = np.array([ref.refshim_float_to_half(float(v)) for v in specials], np.uint16)
    nin = np.array([0.5, 1.5, 2.5, -2.5, 3.5, -3.5, 1e6 + 0.5, -4194303.5], F)
    out["nearest_in"] = nin
    out["nearest_out"] = np.array([ref.refshim_nearest_int(float(v)) for v in nin], np.int32)

    # Q8_K activation quantize: random blocks, an all-zero block, a first-maximum tie, exact halves
    xk = gq.normal(1, 1, 1024)
    xk[256:512] = 0.0
    xk[512:768] = rng.standard_normal(256).astype(F) * 0.1
    xk[512 + 3], xk[512 + 7] = 5.0, -5.0  # equal magnitudes: the first one sets the sign of the scale
    xk[768:1024] = (np.arange(256) % 9 - 4).astype(F) * np.float32(0.5)
    xk[768] = -127.0  # iscale = 1: q = nearest_int(x), exact halves round to even
    q = np.empty(1024, np.int8)
    d = np.empty(4, F)
    ref.refshim_quantize_q8_k(p(xk), 1024, p(q), p(d))
    out["q8k_x"], out["q8k_q"], out["q8k_d"] = xk, q, d

    # GEMV, all formats the reference path knows
    rows, cols = 16, 512
    x = gq.normal(1, 2, cols)
    out["gemv_x"] = x
    for t in (Q4_0, Q4_1, Q8_0, Q5_K, Q6_K):
        if t == Q4_1:
            w = q4_1_matrix(rng, rows, cols)
        else:
            w = gq.matrix(t, rows, cols, 1, 100 + t, std=0.02)
        y = np.empty(rows, F)
        mag = np.empty(rows, np.float64)
        ref.refshim_gemv(p(w), p(x), rows, cols, t, p(y), p(mag))
        out[f"gemv{t}_w"], out[f"gemv{t}_y"], out[f"gemv{t}_mag"] = w, y, mag

    # norms: rmsnorm with weight; rownorm flags 0 (RMS + weight), 1 (L2), 2 (RMS, no weight), 3 (L2, no weight)
    xn = gq.normal(1, 3, 4 * 256, std=2.0)
    wn = gq.uniform(1, 4, 256, 0.5, 1.5)
    y = np.empty(256, F)
    ref.refshim_rmsnorm(p(xn), p(wn), 256, 1e-6, p(y))
    out["norm_x"], out["norm_w"], out["rmsnorm_y"] = xn, wn, y
    for fl in range(4):
        y = np.empty(4 * 256, F)
        ref.refshim_rownorm(p(xn), p(wn), 256, 4, 1e-6, fl, p(y))
        out[f"rownorm{fl}_y"] = y

    # element-wise: SiLU-mul, unary SiLU / sigmoid / softplus (values across the softplus threshold)
    g = gq.normal(1, 5, 512, std=4.0)
    g[:8] = np.array([20.0, 19.99, 20.01, -87.5, 88.0, 0.0, -0.0, 1e-30], F)
    u = gq.normal(1, 6, 512)
    y = np.empty(512, F)
    ref.refshim_silu_mul(p(g), p(u), 512, p(y))
    out["ew_g"], out["ew_u"], out["silu_mul_y"] = g, u, y
    for kind in (1, 2, 3):
        y = np.empty(512, F)
        ref.refshim_unary(p(g), 512, kind, p(y))
        out[f"unary{kind}_y"] = y

    # CONV: window [state (3), x], kernel of 4, with and without SiLU
    ch = 256
    st = gq.normal(1, 7, 3 * ch)
    xc = gq.normal(1, 8, ch)
    wc = gq.normal(1, 9, 4 * ch, std=0.5)
    out["conv_state"], out["conv_x"], out["conv_w"] = st, xc, wc
    for silu in (0, 1):
        y = np.empty(ch, F)
        ns = np.empty(3 * ch, F)
        ref.refshim_conv(p(st), p(xc), p(wc), ch, silu, p(y), p(ns))
        out[f"conv{silu}_y"], out[f"conv{silu}_ns"] = y, ns

    # GDN step: 2 value heads, 1 key head (tiled), state N(0, 0.1^2), q/k L2-normalized inputs, log decay < 0
    hv, hk = 2, 1
    state = gq.normal(1, 10, hv * 128 * 128, std=0.1)
    qg = gq.normal(1, 11, hk * 128)
    kg = gq.normal(1, 12, hk * 128)
    qg /= np.float32(np.sqrt(np.sum(qg.astype(np.float64) ** 2)))
    kg /= np.float32(np.sqrt(np.sum(kg.astype(np.float64) ** 2)))
    vg = gq.normal(1, 13, hv * 128)
    gg = -np.abs(gq.normal(1, 14, hv))
    bg = gq.uniform(1, 15, hv, 0.0, 1.0)
    st2 = state.copy()
    y = np.empty(hv * 128, F)
    ym = np.empty(hv * 128, np.float64)
    ref.refshim_gdn(p(st2), p(qg), p(kg), p(vg), p(gg), p(bg), hv, hk, float(1 / np.sqrt(128)), p(y), p(ym), None)
    # the input state is regenerated from its seed (stream 10 of seed 1, N(0, 0.1^2)); its hash detects drift
    out["gdn_state_sha256"] = np.frombuffer(hashlib.sha256(state.tobytes()).digest(), np.uint8)
    out.update(gdn_q=qg, gdn_k=kg, gdn_v=vg, gdn_g=gg, gdn_beta=bg, gdn_y=y, gdn_ymag=ym,
               gdn_state_out=st2)

    path = os.path.join(HERE, "reference_vectors.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} bytes, {len(out)} arrays)")
    return 0


if __name__ == "__main__":
    sys.exit(main())
