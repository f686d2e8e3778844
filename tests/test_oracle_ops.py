"""Pins the oracle's non-GEMV operators (CPU only): norms, element-wise ops, CONV, RoPE, the Gated DeltaNet step,
the attention core, the Q6_K row dequantize and argmax.

Each is checked against (a) the reference's own outputs on stored inputs (bit for bit for the oracle's restatement
of the reference path, within the reference's tolerances for the canonical path), (b) float64 numpy restatements
of the mathematics, and (c) closed forms chosen so that a dropped term, a wrong sign or a transposed operand fails.
"""
import numpy as np
import pytest

import ggml_blocks as B
from golden_data import golden

F = np.float32


def bits_equal(a, b) -> bool:
    return np.array_equal(np.asarray(a, F).view(np.uint32), np.asarray(b, F).view(np.uint32))


def p(a):
    return a.ctypes.data


def within_elementwise(got, ref):
    """gemvq_ref.h:399-402: |got - ref| <= 1e-6 + 2e-5 |ref|."""
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    return np.all(np.abs(got - ref) <= 1e-6 + 2e-5 * np.abs(ref))


# ---- reference vectors ----------------------------------------------------------------------------------------
def test_norms_reproduce_reference_vectors(orc):
    g = golden()
    o = orc.orc()
    y = np.empty(256, F)
    o.orc_ref_rmsnorm(p(g["norm_x"]), p(g["norm_w"]), 256, 1e-6, p(y))
    assert bits_equal(y, g["rmsnorm_y"])
    for fl in range(4):
        y = np.empty(1024, F)
        o.orc_ref_rownorm(p(g["norm_x"]), p(g["norm_w"]), 256, 4, 1e-6, fl, p(y))
        assert bits_equal(y, g[f"rownorm{fl}_y"]), fl
        # the canonical row norm (pairwise FP32 sum) within the reference's element-wise tolerance
        assert within_elementwise(orc.rownorm(g["norm_x"], g["norm_w"], 256, 4, 1e-6, fl), g[f"rownorm{fl}_y"])


def test_elementwise_reproduce_reference_vectors(orc):
    g = golden()
    o = orc.orc()
    for kind in (1, 2, 3):
        y = np.empty(512, F)
        o.orc_ref_unary(p(g["ew_g"]), 512, kind, p(y))
        assert bits_equal(y, g[f"unary{kind}_y"]), kind
        assert within_elementwise(orc.unary(g["ew_g"], kind), g[f"unary{kind}_y"]), kind
    assert within_elementwise(orc.silu_mul(g["ew_g"], g["ew_u"]), g["silu_mul_y"])
    for silu in (0, 1):
        y = np.empty(256, F)
        ns = np.empty(768, F)
        o.orc_ref_conv(p(g["conv_state"]), p(g["conv_x"]), p(g["conv_w"]), 256, silu, p(y), p(ns))
        assert bits_equal(y, g[f"conv{silu}_y"]) and bits_equal(ns, g[f"conv{silu}_ns"])
        yc, nsc = orc.conv(g["conv_state"], g["conv_x"], g["conv_w"], bool(silu))
        assert bits_equal(nsc, g[f"conv{silu}_ns"]) and within_elementwise(yc, g[f"conv{silu}_y"])


def test_gdn_reproduces_reference_vectors(orc, gq):
    import hashlib

    g = golden()
    hv, hk = 2, 1
    state = gq.normal(1, 10, hv * 128 * 128, std=0.1)
    assert hashlib.sha256(state.tobytes()).digest() == g["gdn_state_sha256"].tobytes(), "RNG drift"
    st = state.copy()
    y = np.empty(hv * 128, F)
    ym = np.empty(hv * 128, np.float64)
    orc.orc().orc_ref_gdn(p(st), p(g["gdn_q"]), p(g["gdn_k"]), p(g["gdn_v"]), p(g["gdn_g"]), p(g["gdn_beta"]), hv, hk,
                          float(1 / np.sqrt(128)), p(y), p(ym), None)
    assert bits_equal(y, g["gdn_y"]) and bits_equal(st, g["gdn_state_out"]) and np.array_equal(ym, g["gdn_ymag"])
    # the canonical step (pairwise dots, own exp) within the reference's GDN tolerance (ggml-xrt.cpp:1196)
    yc, stc = orc.gdn(state, g["gdn_q"], g["gdn_k"], g["gdn_v"], g["gdn_g"], g["gdn_beta"], hv, hk,
                      float(1 / np.sqrt(128)))
    assert np.all(np.abs(yc - g["gdn_y"]) <= 1e-6 + 4e-6 * g["gdn_ymag"])
    assert np.all(np.abs(stc - g["gdn_state_out"]) <= 1e-6 + 2e-5 * np.abs(g["gdn_state_out"]))


# ---- float64 restatements and closed forms --------------------------------------------------------------------
def test_rownorm_float64(orc, gq):
    x = gq.normal(2, 1, 5 * 320, std=3.0)
    w = gq.uniform(2, 2, 300, 0.5, 1.5)
    xd = x.reshape(5, 320)[:, :300].astype(np.float64)  # 5 rows of 300 every 320 floats
    for fl in range(4):
        y = orc.rownorm(x, w, 300, 5, 1e-6, fl, stride=320).reshape(5, 300)
        if fl & 1:
            s = 1 / np.maximum(np.sqrt((xd ** 2).sum(1)), 1e-6)
        else:
            s = 1 / np.sqrt((xd ** 2).mean(1) + 1e-6)
        want = xd * s[:, None] * (1.0 if fl & 2 else w.astype(np.float64))
        np.testing.assert_allclose(y, want, rtol=1e-6, atol=1e-7)


def test_conv_closed_forms(orc, gq):
    ch = 512
    st = gq.normal(2, 3, 3 * ch)
    x = gq.normal(2, 4, ch)
    e3 = np.tile(np.array([0, 0, 0, 1], F), ch)  # kernel e_3: the sum is x itself
    y, ns = orc.conv(st, x, e3, silu=True)
    o = orc.orc()
    assert bits_equal(y, [o.orc_silu(float(v)) for v in x])
    assert bits_equal(ns.reshape(ch, 3), np.stack([st.reshape(ch, 3)[:, 1], st.reshape(ch, 3)[:, 2], x], 1))
    w = gq.normal(2, 5, 4 * ch, std=0.5)
    y, _ = orc.conv(st, x, w, silu=False)
    win = np.concatenate([st.reshape(ch, 3), x[:, None]], 1).astype(np.float64)
    np.testing.assert_allclose(y, (win * w.reshape(ch, 4)).sum(1), rtol=1e-5, atol=1e-6)


def test_rope_float64(orc, gq):
    n_dims, ne0, rows, pos, base = 64, 256, 3, 517, 1e7
    cs = orc.rope_cache(pos, n_dims, base)
    theta = pos * base ** (-2.0 * np.arange(n_dims // 2) / n_dims)
    np.testing.assert_allclose(cs[0::2], np.cos(theta), atol=2e-5)
    np.testing.assert_allclose(cs[1::2], np.sin(theta), atol=2e-5)
    x = gq.normal(2, 6, rows * ne0)
    y = orc.rope(x, cs, n_dims, ne0, rows).reshape(rows, ne0)
    xr = x.reshape(rows, ne0).astype(np.float64)
    c, s, h = cs[0::2].astype(np.float64), cs[1::2].astype(np.float64), n_dims // 2
    want = xr.copy()
    want[:, :h] = xr[:, :h] * c - xr[:, h:n_dims] * s  # NEOX: pairs (i, i + n_dims / 2)
    want[:, h:n_dims] = xr[:, :h] * s + xr[:, h:n_dims] * c
    np.testing.assert_allclose(y, want, rtol=1e-6, atol=1e-6)
    assert bits_equal(y[:, n_dims:], x.reshape(rows, ne0)[:, n_dims:])


def gdn64(state, q, k, v, graw, braw, hv, hk, scale, flags=0, dt=None, a=None, z=None, w=None, eps=1e-6):
    """float64 statement of the fused step: value head h uses key head h % hk; row j of the head's state is the
    vector S_j: x = S_j e^g; delta = (v_j - x . k) beta; S_j' = x + k delta; y_j = (S_j' . q) scale."""
    S = state.reshape(hv, 128, 128).astype(np.float64).copy()
    q = q.reshape(hk, 128).astype(np.float64)
    k = k.reshape(hk, 128).astype(np.float64)
    if flags & 2:
        q = q / np.maximum(np.linalg.norm(q, axis=1, keepdims=True), eps)
        k = k / np.maximum(np.linalg.norm(k, axis=1, keepdims=True), eps)
    y = np.empty((hv, 128))
    for h in range(hv):
        g, beta = float(graw[h]), float(braw[h])
        if flags & 8:
            t = g + float(dt[h])
            g = (t if t > 20 else np.log1p(np.exp(t))) * float(a[h])
            beta = 1 / (1 + np.exp(-beta))
        X = S[h] * np.exp(g)
        delta = (v.reshape(hv, 128)[h] - X @ k[h % hk]) * beta
        S[h] = X + delta[:, None] * k[h % hk][None, :]
        y[h] = (S[h] @ q[h % hk]) * scale
        if flags & 4:
            zz = z.reshape(hv, 128)[h].astype(np.float64)
            y[h] = zz / (1 + np.exp(-zz)) * (y[h] / np.sqrt(np.mean(y[h] ** 2) + eps) * w)
    return y.ravel(), S.ravel()


@pytest.mark.parametrize("flags", [0, 2, 14])
def test_gdn_float64(orc, gq, flags):
    hv, hk = 4, 2
    state = gq.normal(2, 10, hv * 128 * 128, std=0.1)
    q, k, v = gq.normal(2, 11, hk * 128), gq.normal(2, 12, hk * 128), gq.normal(2, 13, hv * 128)
    if not flags & 2:
        q, k = q / np.float32(12), k / np.float32(12)
    graw, braw = gq.normal(2, 14, hv), gq.normal(2, 15, hv)
    if not flags & 8:
        graw, braw = -np.abs(graw), np.abs(braw) / np.float32(3)
    dt, a = gq.normal(2, 16, hv), -gq.uniform(2, 17, hv, 0.5, 1.5)
    z, w = gq.normal(2, 18, hv * 128), gq.uniform(2, 19, 128, 0.5, 1.5)
    y, st = orc.gdn(state, q, k, v, graw, braw, hv, hk, float(1 / np.sqrt(128)), flags, dt, a, z, w)
    y64, st64 = gdn64(state, q, k, v, graw, braw, hv, hk, 1 / np.sqrt(128), flags, dt, a, z, w.astype(np.float64))
    np.testing.assert_allclose(st, st64, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(y, y64, rtol=1e-4, atol=1e-5 * np.abs(y64).max())


def test_gdn_closed_forms(orc, gq):
    hv, hk, S = 2, 2, 128
    state = gq.normal(2, 20, hv * S * S, std=0.1)
    q, k, v = gq.normal(2, 21, hk * S), gq.normal(2, 22, hk * S), gq.normal(2, 23, hv * S)
    zero, one = np.zeros(hv, F), np.ones(hv, F)
    # decay 1, beta 0: the state is unchanged and y = S q scale
    y, st = orc.gdn(state, q, k, v, zero, zero, hv, hk, 0.125)
    assert bits_equal(st, state)
    want = np.einsum("hji,hi->hj", state.reshape(hv, S, S).astype(np.float64), q.reshape(hk, S).astype(np.float64))
    np.testing.assert_allclose(y, 0.125 * want.ravel(), rtol=1e-5, atol=1e-6)
    # decay 1, beta 1, k = e_i: component i of every row becomes v_j, the others are untouched
    i = 37
    ke = np.zeros(hk * S, F)
    ke[i] = ke[S + i] = 1.0
    _, st = orc.gdn(state, q, ke, v, zero, one, hv, hk, 0.125)
    st, s0 = st.reshape(hv, S, S), state.reshape(hv, S, S)
    mask = np.ones(S, bool)
    mask[i] = False
    assert bits_equal(st[:, :, mask], s0[:, :, mask])
    np.testing.assert_allclose(st[:, :, i], v.reshape(hv, S), rtol=0, atol=2e-7 * max(1.0, np.abs(v).max()))


@pytest.mark.parametrize("n_kv", [1, 64, 65, 130])
def test_attention_float64(orc, gq, n_kv):
    nh, nkv, hd = 8, 2, 128
    q = gq.normal(2, 30, nh * hd)
    kc = orc.f2h(gq.normal(2, 31, n_kv * nkv * hd)).reshape(n_kv, nkv, hd)
    vc = orc.f2h(gq.normal(2, 32, n_kv * nkv * hd)).reshape(n_kv, nkv, hd)
    out = orc.attn(q, kc, vc, nh, nkv, hd, n_kv, 1 / 16).reshape(nh, hd)
    q16 = q.astype(np.float16).astype(np.float64).reshape(nh, hd)  # the query is rounded to fp16 like the cache
    K = kc.view(np.float16).astype(np.float64)
    V = vc.view(np.float16).astype(np.float64)
    for h in range(nh):
        kh = h // (nh // nkv)  # GQA: consecutive q heads share a KV head
        s = K[:, kh, :] @ q16[h] / 16
        pr = np.exp(s - s.max())
        want = (pr[:, None] * V[:, kh, :]).sum(0) / pr.sum()
        np.testing.assert_allclose(out[h], want, rtol=2e-5, atol=2e-6)


def test_dequant_row_q6_K(orc, gq):
    w = gq.matrix(14, 1, 1024, 2, 40)
    q, sc, d = B.q6_K(w, 1, 1024)
    want = ((d[0].astype(F)[:, None] * sc[0].astype(F)).repeat(16, axis=1) * q[0].reshape(4, 256).astype(F))
    assert bits_equal(orc.dequant_row_q6_K(w, 1024), want.ravel())  # (d * sc) * q in FP32


def test_argmax_first_index(orc):
    x = np.array([1.0, 3.0, -2.0, 3.0, 3.0], F)
    assert orc.orc().orc_argmax(p(x), 5) == 1
    x = np.full(1000, -np.inf, F)
    x[999] = -1e30
    assert orc.orc().orc_argmax(p(x), 1000) == 999
