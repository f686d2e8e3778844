"""The ggml-facing backend on the GPU: one decode token of the Qwen3.5 hybrid as a ggml graph (the planner's
command list, cached and replayed as a hipGraph; token ids and positions copied in, logits copied back) against the
oracle decoder: greedy tokens identical and every step's logits bit for bit. Clearing the state and KV buffers
starts the sequence over with the same results."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def test_ggml_graph_greedy_matches_oracle(gq, orc):
    import ggml_ir as ir
    import qwen35
    import qwen35_ggml

    cfg = qwen35.tiny(n_layer=4, n_ctx=64)
    blob = qwen35.generate(cfg, seed=5)
    prompt = qwen35.prompt_ids(cfg, 6, seed=5)
    n_gen = 10
    om = orc.Model(qwen35.config_c(cfg), blob.table, blob.n, blob.data)
    want = om.generate(prompt, n_gen)
    lo = np.empty(cfg.n_vocab, np.float32)
    om2 = orc.Model(qwen35.config_c(cfg), blob.table, blob.n, blob.data)
    rows = sum(not cfg.is_attn(i) for i in range(cfg.n_layer)) * cfg.ssm_v_heads * 128
    with ir.Backend(act_floats=1 << 21, weight_bytes=blob.data.size + (1 << 20), state_rows=rows) as b:
        g = qwen35_ggml.Qwen35Graph(blob, b)
        try:
            for run in range(2):
                toks = [int(prompt[0])]
                for pos in range(len(prompt) - 1 + n_gen):
                    print(f"[ggml] run {run} position {pos}", flush=True)
                    logits = g.step(toks[pos], pos)
                    if run == 0:
                        om2.decode(int(want[pos]), pos, lo)
                        assert np.array_equal(logits.view(np.uint32), lo.view(np.uint32)), f"logits at position {pos}"
                    nxt = int(prompt[pos + 1]) if pos + 1 < len(prompt) else int(np.argmax(logits))
                    toks.append(nxt)
                assert np.array_equal(np.array(toks, np.int32), want), f"run {run}: {toks} vs {want}"
                # one plan, replayed for every later token
                assert b.stats()[0] == 1
                # a new sequence: the recurrent states and the KV caches back to zero
                assert b.L.gqg_buffer_clear(g.rs, 0) == 0, b.error()
                assert b.L.gqg_buffer_clear(g.kvb, 0) == 0, b.error()
        finally:
            g.close()


def test_state_buffer_io(gq):
    """set/get of a DeltaNet state and a conv window through the state buffer: whole rows round trip."""
    import ctypes as C

    import ggml_ir as ir

    with ir.Backend(act_floats=1 << 16, weight_bytes=1 << 20, state_rows=2 * 128) as b:
        buf = b.buffer(2 * 128 * 512 + 4096, ir.BUF_RS)
        base = b.L.gqg_buffer_base(buf)
        G = ir.Graph()
        s = G.at(ir.F32, [2 * 128 * 128], base, "cache_s_l0")
        r = G.at(ir.F32, [3 * 256], base + 2 * 128 * 512, "cache_r_l0")
        for t in (s, r):
            assert b.L.gqg_buffer_init_tensor(buf, C.byref(t)) == 0, b.error()
        sv = np.arange(2 * 128 * 128, dtype=np.float32)
        rv = -np.arange(3 * 256, dtype=np.float32)
        assert b.L.gqg_buffer_set(buf, C.byref(s), sv.ctypes.data, 0, sv.nbytes) == 0, b.error()
        assert b.L.gqg_buffer_set(buf, C.byref(r), rv.ctypes.data, 0, rv.nbytes) == 0, b.error()
        got_s = np.zeros_like(sv)
        got_r = np.zeros_like(rv)
        assert b.L.gqg_buffer_get(buf, C.byref(s), got_s.ctypes.data, 0, got_s.nbytes) == 0, b.error()
        assert b.L.gqg_buffer_get(buf, C.byref(r), got_r.ctypes.data, 0, got_r.nbytes) == 0, b.error()
        assert np.array_equal(got_s, sv) and np.array_equal(got_r, rv)
        part = np.zeros(128, np.float32)  # one row of the second head
        assert b.L.gqg_buffer_get(buf, C.byref(s), part.ctypes.data, 128 * 512, 512) == 0, b.error()
        assert np.array_equal(part, sv[128 * 128:128 * 128 + 128])
        assert b.L.gqg_buffer_get(buf, C.byref(s), part.ctypes.data, 4, 512) != 0  # not a whole row
        b.free_buffer(buf)


def test_ggml_graph_in_per_layer_splits_matches_oracle(gq, orc):
    """The token as one split per layer and a head split (the residual stream flagged as a split output at every
    boundary, copied back to the host by one split and in by the next, ggml-xrt.cpp:1399-1478): greedy tokens and
    every step's logits identical to the oracle decoder, each split's plan built once and replayed."""
    import ggml_ir as ir
    import qwen35
    import qwen35_ggml

    cfg = qwen35.tiny(n_layer=8, n_ctx=64)
    blob = qwen35.generate(cfg, seed=6)
    prompt = qwen35.prompt_ids(cfg, 5, seed=6)
    n_gen = 8
    om = orc.Model(qwen35.config_c(cfg), blob.table, blob.n, blob.data)
    want = om.generate(prompt, n_gen)
    lo = np.empty(cfg.n_vocab, np.float32)
    om2 = orc.Model(qwen35.config_c(cfg), blob.table, blob.n, blob.data)
    rows = sum(not cfg.is_attn(i) for i in range(cfg.n_layer)) * cfg.ssm_v_heads * 128
    with ir.Backend(act_floats=1 << 21, weight_bytes=blob.data.size + (1 << 20), state_rows=rows) as b:
        g = qwen35_ggml.Qwen35Graph(blob, b)
        try:
            splits = g.layer_splits()
            toks = [int(prompt[0])]
            for pos in range(len(prompt) - 1 + n_gen):
                print(f"[ggml splits] position {pos}", flush=True)
                logits = g.step_splits(toks[pos], pos)
                om2.decode(int(want[pos]), pos, lo)
                assert np.array_equal(logits.view(np.uint32), lo.view(np.uint32)), f"logits at position {pos}"
                toks.append(int(prompt[pos + 1]) if pos + 1 < len(prompt) else int(np.argmax(logits)))
            assert np.array_equal(np.array(toks, np.int32), want)
            assert b.stats()[0] == len(splits)
        finally:
            g.close()
