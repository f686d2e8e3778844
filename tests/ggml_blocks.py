"""Independent numpy restatement of the GGUF block formats and activation quantizers, for pinning the oracle.

Written from the GGUF/ggml block layouts (the structs the reference's gemvq_ref.h:94-265 reads), not from the
oracle's C code: every decoder returns the exact integers and scales, so that block sums and row values can be
checked as exact integer / float64 arithmetic.
"""
from __future__ import annotations

import numpy as np

Q4_0, Q4_1, Q8_0, Q5_K, Q6_K = 2, 3, 8, 13, 14
BLOCK_BYTES = {Q4_0: 18, Q4_1: 20, Q8_0: 34, Q5_K: 176, Q6_K: 210}
BLOCK_ELEMS = {Q4_0: 32, Q4_1: 32, Q8_0: 32, Q5_K: 256, Q6_K: 256}


def half(bits) -> np.ndarray:
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float64)


def blocks(t: int, w: np.ndarray, rows: int, cols: int) -> np.ndarray:
    nb = cols // BLOCK_ELEMS[t]
    return np.asarray(w, np.uint8).reshape(rows, nb, BLOCK_BYTES[t])


def q4_0(w, rows, cols):
    """-> (ints [rows, cols] in -8..7, d [rows, nb] float64). Low nibble of byte j is element j, high is j + 16."""
    b = blocks(Q4_0, w, rows, cols)
    d = half(b[..., 0:2].copy().view(np.uint16)[..., 0])
    qs = b[..., 2:18].astype(np.int32)
    q = np.concatenate([(qs & 15) - 8, (qs >> 4) - 8], axis=-1)
    return q.reshape(rows, cols), d


def q4_1(w, rows, cols):
    """-> (ints [rows, cols] in 0..15, d [rows, nb], m [rows, nb] float64). Block: d, m (fp16), 16 bytes of nibbles;
    value = d * q + m."""
    b = blocks(Q4_1, w, rows, cols)
    d = half(b[..., 0:2].copy().view(np.uint16)[..., 0])
    m = half(b[..., 2:4].copy().view(np.uint16)[..., 0])
    qs = b[..., 4:20].astype(np.int32)
    q = np.concatenate([qs & 15, qs >> 4], axis=-1)
    return q.reshape(rows, cols), d, m


def q8_0(w, rows, cols):
    b = blocks(Q8_0, w, rows, cols)
    d = half(b[..., 0:2].copy().view(np.uint16)[..., 0])
    q = b[..., 2:34].copy().view(np.int8).astype(np.int32)
    return q.reshape(rows, cols), d


def _scale_min_k4(sc12: np.ndarray):
    """6-bit scales and mins of the 8 sub-blocks packed in 12 bytes."""
    s = sc12.astype(np.int32)
    sc = np.empty(s.shape[:-1] + (8,), np.int32)
    mn = np.empty_like(sc)
    for j in range(8):
        if j < 4:
            sc[..., j] = s[..., j] & 63
            mn[..., j] = s[..., j + 4] & 63
        else:
            sc[..., j] = (s[..., j + 4] & 0xF) | ((s[..., j - 4] >> 6) << 4)
            mn[..., j] = (s[..., j + 4] >> 4) | ((s[..., j] >> 6) << 4)
    return sc, mn


def q5_K(w, rows, cols):
    """-> (q [rows, cols] in 0..31, sc [rows, nb, 8], m [rows, nb, 8], d [rows, nb], dmin [rows, nb]).
    Block: d, dmin (fp16), scales[12], qh[32], qs[128]; value = d * sc * q - dmin * m."""
    b = blocks(Q5_K, w, rows, cols)
    d = half(b[..., 0:2].copy().view(np.uint16)[..., 0])
    dmin = half(b[..., 2:4].copy().view(np.uint16)[..., 0])
    sc, mn = _scale_min_k4(b[..., 4:16])
    qh = b[..., 16:48].astype(np.int32)
    qs = b[..., 48:176].astype(np.int32)
    nb = cols // 256
    q = np.empty((rows, nb, 256), np.int32)
    for j in range(4):  # 64 values per chunk: low nibbles then high nibbles of 32 bytes
        ql = qs[..., 32 * j:32 * j + 32]
        q[..., 64 * j:64 * j + 32] = (ql & 15) + ((qh >> (2 * j)) & 1) * 16
        q[..., 64 * j + 32:64 * j + 64] = (ql >> 4) + ((qh >> (2 * j + 1)) & 1) * 16
    return q.reshape(rows, cols), sc, mn, d, dmin


def q6_K(w, rows, cols):
    """-> (q [rows, cols] in -32..31, sc [rows, nb, 16] int8 scales, d [rows, nb]).
    Block: ql[128], qh[64], scales[16] (int8), d (fp16)."""
    b = blocks(Q6_K, w, rows, cols)
    ql = b[..., 0:128].astype(np.int32)
    qh = b[..., 128:192].astype(np.int32)
    sc = b[..., 192:208].copy().view(np.int8).astype(np.int32)
    d = half(b[..., 208:210].copy().view(np.uint16)[..., 0])
    nb = cols // 256
    q = np.empty((rows, nb, 256), np.int32)
    for n in range(2):  # halves of 128 values
        L = ql[..., 64 * n:64 * n + 64]
        H = qh[..., 32 * n:32 * n + 32]
        base = 128 * n
        q[..., base + 0:base + 32] = ((L[..., 0:32] & 15) | ((H & 3) << 4)) - 32
        q[..., base + 32:base + 64] = ((L[..., 32:64] & 15) | (((H >> 2) & 3) << 4)) - 32
        q[..., base + 64:base + 96] = ((L[..., 0:32] >> 4) | (((H >> 4) & 3) << 4)) - 32
        q[..., base + 96:base + 128] = ((L[..., 32:64] >> 4) | (((H >> 6) & 3) << 4)) - 32
    return q.reshape(rows, cols), sc, d


def dequantize(t: int, w, rows: int, cols: int) -> np.ndarray:
    """float64 weights (the products evaluated exactly in float64)."""
    if t in (Q4_0, Q8_0):
        q, d = (q4_0 if t == Q4_0 else q8_0)(w, rows, cols)
        return q.reshape(rows, -1, 32) * d[..., None]
    if t == Q4_1:
        q, d, m = q4_1(w, rows, cols)
        return (q.reshape(rows, -1, 32) * d[..., None] + m[..., None]).reshape(rows, cols)
    if t == Q5_K:
        q, sc, mn, d, dmin = q5_K(w, rows, cols)
        q = q.reshape(rows, -1, 8, 32)
        return (d[..., None, None] * sc[..., None] * q - dmin[..., None, None] * mn[..., None]).reshape(rows, cols)
    q, sc, d = q6_K(w, rows, cols)
    return (d[..., None, None] * sc[..., None] * q.reshape(rows, -1, 16, 16)).reshape(rows, cols)


# ---- activation quantizers, brute force ----
def roundf(x: np.ndarray) -> np.ndarray:
    """C roundf: half away from zero (np.round is half-even)."""
    return np.sign(x) * np.floor(np.abs(x) + 0.5)


def quantize_q8_0(x: np.ndarray):
    """Per 32: amax -> s = amax / 127 (FP32), d = fp16(s), q = roundf(x * (1 / s)) (all FP32 steps)."""
    x = np.asarray(x, np.float32).reshape(-1, 32)
    amax = np.max(np.abs(x), axis=1)
    s = (amax / np.float32(127)).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(s != 0, np.float32(1) / s, np.float32(0)).astype(np.float32)
    q = roundf((x * inv[:, None]).astype(np.float32)).astype(np.int32)
    with np.errstate(over="ignore"):  # scales beyond the fp16 range become infinity, as the conversion does
        d = s.astype(np.float16).view(np.uint16)
    return q.astype(np.int8).ravel(), d


def quantize_q8_1(x: np.ndarray):
    """Q8_0's quants and d, plus s = fp16(sum(q) * d) with the FP32 d (ggml quantize_row_q8_1_ref)."""
    q, dbits = quantize_q8_0(x)
    xr = np.asarray(x, np.float32).reshape(-1, 32)
    d = (np.max(np.abs(xr), axis=1) / np.float32(127)).astype(np.float32)
    sums = q.astype(np.int32).reshape(-1, 32).sum(axis=1).astype(np.float32)
    with np.errstate(over="ignore"):
        sbits = (sums * d).astype(np.float32).astype(np.float16).view(np.uint16)
    return q, dbits, sbits


def nearest_int(v: np.ndarray) -> np.ndarray:
    """Round half to even (the FP32 magic-number trick evaluates exactly this for |v| < 2^22)."""
    return np.rint(np.asarray(v, np.float64)).astype(np.int32)


def quantize_q8_K(x: np.ndarray):
    """Per 256: max = the value of largest magnitude (first one on ties); iscale = -127 / max (FP32);
    q = min(127, nearest_int(iscale * x)); d = 1 / iscale; bsums per 16."""
    x = np.asarray(x, np.float32).reshape(-1, 256)
    n = x.shape[0]
    q = np.zeros((n, 256), np.int32)
    d = np.zeros(n, np.float32)
    for b in range(n):
        i = int(np.argmax(np.abs(x[b])))  # argmax keeps the first index of the maximum
        mx = x[b, i]
        if np.abs(mx) == 0:
            continue
        iscale = np.float32(-127) / mx
        q[b] = np.minimum(127, nearest_int((iscale * x[b]).astype(np.float32)))
        d[b] = np.float32(1) / iscale
    bs = q.reshape(n, 16, 16).sum(axis=2)
    return q.astype(np.int8).ravel(), d, bs.astype(np.int16).ravel()


def block_sums(t: int, w, xq: np.ndarray, rows: int, cols: int, xbs: np.ndarray | None = None) -> np.ndarray:
    """Exact integer block sums in the oracle's debug layout: Q4_0/Q8_0 one per 32-block; K-quants (S, M) per
    super-block with S = sum over groups of scale * (q . q8) and M = sum over sub-blocks of min * bsum (Q6_K: 0)."""
    xq = np.asarray(xq, np.int64)
    if t == Q4_1:
        q = q4_1(w, rows, cols)[0]
        return (q.astype(np.int64) * xq[None, :]).reshape(rows, -1, 32).sum(axis=2).ravel()
    if t in (Q4_0, Q8_0):
        q, _ = (q4_0 if t == Q4_0 else q8_0)(w, rows, cols)
        return (q.astype(np.int64) * xq[None, :]).reshape(rows, -1, 32).sum(axis=2).ravel()
    nb = cols // 256
    if t == Q5_K:
        q, sc, mn, _, _ = q5_K(w, rows, cols)
        dots = (q.astype(np.int64) * xq[None, :]).reshape(rows, nb, 8, 32).sum(axis=3)
        S = (dots * sc).sum(axis=2)
        bsub = np.asarray(xbs, np.int64).reshape(nb, 8, 2).sum(axis=2)
        M = (mn * bsub[None]).sum(axis=2)
    else:
        q, sc, _ = q6_K(w, rows, cols)
        dots = (q.astype(np.int64) * xq[None, :]).reshape(rows, nb, 16, 16).sum(axis=3)
        S = (dots * sc).sum(axis=2)
        M = np.zeros_like(S)
    return np.stack([S, M], axis=-1).ravel()
