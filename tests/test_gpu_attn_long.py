"""Attention past 64 chunks of 64 positions (the combine then takes several rounds of 64 chunks): the Qwen3.5 shape
(16 q heads, 4 KV heads of 256, RoPE over 64 dims) with a cache of 8320 positions (130 chunks), the history written
by batched commands, then one-token commands at the end of the cache against the oracle bit for bit, and a batch
of 32 tokens against 32 one-token commands on a second cache."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def assert_bits(got, want, what=""):
    got, want = np.asarray(got, np.float32), np.asarray(want, np.float32)
    bad = np.nonzero(got.view(np.uint32) != want.view(np.uint32))[0]
    assert bad.size == 0, f"{what}: {bad.size}/{want.size} differ; first {bad[:4]}: got {got[bad[:4]]} want {want[bad[:4]]}"


def test_attention_8320_positions(gq, orc):
    nh, nkv, hd, nrot, n_ctx = 16, 4, 256, 64, 8320
    qrow, kvrow, arow = 2 * nh * hd, nkv * hd, nh * hd
    ctx = gq.Context(act_floats=1 << 22, weight_bytes=1 << 20, state_rows=0)
    try:
        O = dict(q=0, k=262144, v=294912, qn=327680, kn=327936, pos=328192, y=328704, y2=460800, cs=1 << 21)
        qn = gq.uniform(2, 71, hd, 0.5, 1.5)
        kn = gq.uniform(2, 72, hd, 0.5, 1.5)
        table = np.concatenate([orc.rope_cache(p, nrot, 1e7) for p in range(n_ctx)])
        ctx.write(O["qn"], qn)
        ctx.write(O["kn"], kn)
        ctx.write(O["cs"], table)
        kv_a, kv_b = ctx.kv_create(n_ctx, nkv, hd), ctx.kv_create(n_ctx, nkv, hd)

        def attn(kv, q, y, pos_slot, n_tok=1):
            return gq.attn(nh, nkv, q, kv, y, hd, nrot, pos_slot, O["k"] + (q - O["q"]) // qrow * kvrow,
                           O["v"] + (q - O["q"]) // qrow * kvrow, 1 / 16, 1e-6, O["qn"], O["kn"], O["cs"],
                           gate=q + hd, n_tok=n_tok)

        def tokens(first, n, seed):
            qg, k, v = gq.normal(6, seed, n * qrow), gq.normal(6, seed + 1, n * kvrow), gq.normal(6, seed + 2, n * kvrow)
            ctx.write(O["q"], qg)
            ctx.write(O["k"], k)
            ctx.write(O["v"], v)
            slots = np.zeros(16 * 32, np.int32)
            slots[0:16 * n:16] = np.arange(first, first + n)
            ctx.write(O["pos"], slots)
            return qg, k, v

        p_end = n_ctx - 32  # the batches write the history of both caches
        for b0 in range(0, p_end, 32):
            if b0 % 2048 == 0:
                print(f"[attn long] history at {b0}", flush=True)
            tokens(b0, 32, 1000 + b0)
            cmds = attn(kv_a, O["q"], O["y"], O["pos"], 32) + attn(kv_b, O["q"], O["y"], O["pos"], 32)
            assert ctx.run(cmds) == 0, ctx.error()
        # the last 32 positions: one-token commands on cache a, one batch on cache b
        qg, k, v = tokens(p_end, 32, 77)
        one = sum((attn(kv_a, O["q"] + t * qrow, O["y"] + t * arow, O["pos"] + 16 * t) for t in range(32)), [])
        print("[attn long] last 32 positions", flush=True)
        assert ctx.run(one) == 0, ctx.error()
        assert ctx.run(attn(kv_b, O["q"], O["y2"], O["pos"], 32)) == 0, ctx.error()
        y_one, y_batch = ctx.read(O["y"], 32 * arow), ctx.read(O["y2"], 32 * arow)
        assert_bits(y_batch, y_one, "batched vs one-token outputs")
        ka, va = ctx.kv_read(kv_a, 0, n_ctx, kvrow)
        kb, vb = ctx.kv_read(kv_b, 0, n_ctx, kvrow)
        assert np.array_equal(ka, kb) and np.array_equal(va, vb)
        ka, va = ka.reshape(n_ctx, nkv, hd), va.reshape(n_ctx, nkv, hd)
        for t in (0, 16, 31):  # positions 8288 (129 chunks), 8304, 8319 (130 chunks)
            pos = p_end + t
            cs = table[pos * nrot:(pos + 1) * nrot]
            kh = orc.rope(orc.rownorm(k[t * kvrow:(t + 1) * kvrow], kn, hd, nkv, 1e-6), cs, nrot, hd, nkv)
            assert np.array_equal(ka[pos], orc.f2h(kh).reshape(nkv, hd)), f"stored key at {pos}"
            q_t = qg[t * qrow:(t + 1) * qrow]
            qh = orc.rope(orc.rownorm(q_t, qn, hd, nh, 1e-6, 0, 2 * hd), cs, nrot, hd, nh)
            att = orc.attn(qh, ka, va, nh, nkv, hd, pos + 1, 1 / 16)
            want = orc.silu_mul(q_t.reshape(nh, 2 * hd)[:, hd:].ravel(), att, sigmoid=True)
            assert_bits(y_one[t * arow:(t + 1) * arow], want, f"oracle at position {pos}")
    finally:
        ctx.close()


def test_reference_attention_past_the_lds_scores(gq, orc):
    """The reference-arithmetic attention past 6144 positions, where a head's scores and probabilities leave LDS for
    its scratch row: a 6400-position cache whose history is written by batched canonical commands, then one-token
    commands in the reference arithmetic at its last positions against the reference decoder's attention (the
    reference's norms, double sums in order) on the cache as read back, bit for bit."""
    nh, nkv, hd, nrot, n_ctx = 16, 4, 256, 64, 6400
    qrow, kvrow, arow = 2 * nh * hd, nkv * hd, nh * hd
    ctx = gq.Context(act_floats=1 << 22, weight_bytes=1 << 20, state_rows=0)
    try:
        O = dict(q=0, k=262144, v=294912, qn=327680, kn=327936, pos=328192, y=328704, cs=1 << 21)
        qn = gq.uniform(3, 71, hd, 0.5, 1.5)
        kn = gq.uniform(3, 72, hd, 0.5, 1.5)
        table = np.concatenate([orc.rope_cache(p, nrot, 1e7) for p in range(n_ctx)])
        ctx.write(O["qn"], qn)
        ctx.write(O["kn"], kn)
        ctx.write(O["cs"], table)
        kv = ctx.kv_create(n_ctx, nkv, hd)

        def attn(n_tok=1):
            return gq.attn(nh, nkv, O["q"], kv, O["y"], hd, nrot, O["pos"], O["k"], O["v"], 1 / 16, 1e-6, O["qn"],
                           O["kn"], O["cs"], gate=O["q"] + hd, n_tok=n_tok)

        def tokens(first, n, seed):
            qg, k, v = gq.normal(7, seed, n * qrow), gq.normal(7, seed + 1, n * kvrow), gq.normal(7, seed + 2, n * kvrow)
            ctx.write(O["q"], qg)
            ctx.write(O["k"], k)
            ctx.write(O["v"], v)
            slots = np.zeros(16 * 32, np.int32)
            slots[0:16 * n:16] = np.arange(first, first + n)
            ctx.write(O["pos"], slots)
            return qg, k, v

        p_end = n_ctx - 32
        for b0 in range(0, p_end, 32):
            if b0 % 2048 == 0:
                print(f"[ref attn long] history at {b0}", flush=True)
            tokens(b0, 32, 2000 + b0)
            assert ctx.run(attn(32)) == 0, ctx.error()
        ctx.set_arith(gq.ARITH_REFERENCE)
        for pos in (p_end, p_end + 1, n_ctx - 1):
            print(f"[ref attn long] reference arithmetic at {pos}", flush=True)
            qg, k, v = tokens(pos, 1, 99 + pos)
            assert ctx.run(attn()) == 0, ctx.error()
            kc, vc = ctx.kv_read(kv, 0, pos + 1, kvrow)
            kc, vc = kc.reshape(pos + 1, nkv, hd), vc.reshape(pos + 1, nkv, hd)
            cs = table[pos * nrot:(pos + 1) * nrot]
            kh = orc.rope(orc.ref_rownorm(k, kn, hd, nkv, 1e-6), cs, nrot, hd, nkv)
            assert np.array_equal(kc[pos], orc.f2h(kh).reshape(nkv, hd)), f"stored key at {pos}"
            qh = orc.rope(orc.ref_rownorm(qg.reshape(nh, 2 * hd)[:, :hd].ravel(), qn, hd, nh, 1e-6), cs, nrot, hd, nh)
            att = orc.ref_attn_cr(qh, kc, vc, nh, nkv, hd, pos + 1, 1 / 16)
            gate = qg.reshape(nh, 2 * hd)[:, hd:].ravel()
            assert_bits(ctx.read(O["y"], arow), orc.ref_unary_cr(gate, 2) * att, f"reference attention at {pos}")
    finally:
        ctx.close()
