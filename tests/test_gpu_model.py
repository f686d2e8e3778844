"""Greedy decode of the synthetic Qwen3.5-shaped model on the GPU (one hipGraph per token, tokens fed back on the
device) against the oracle decoder: identical tokens, and logits and hidden state bit for bit."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def q35():
    import qwen35

    return qwen35


@pytest.mark.parametrize("wtype,n_layer,n_prompt,n_gen", [(2, 4, 8, 24), (8, 4, 5, 12), (2, 8, 70, 20)])
def test_tiny_model_greedy_matches_oracle(gq, orc, q35, wtype, n_layer, n_prompt, n_gen):
    cfg = q35.tiny(n_layer=n_layer, wtype=wtype)
    blob = q35.generate(cfg, seed=0)
    prompt = q35.prompt_ids(cfg, n_prompt)
    om = orc.Model(q35.config_c(cfg), blob.table, blob.n, blob.data)
    want = om.generate(prompt, n_gen)
    with q35.Model(blob) as m:
        got = m.generate(prompt, n_gen)
        assert np.array_equal(got, want), f"first mismatch at {np.nonzero(got != want)[0][:3]}: {got} vs {want}"
        # logits and hidden state of the last step, bit for bit
        lg = m.logits()
        hd = m.hidden()
    lo = np.empty(cfg.n_vocab, np.float32)
    om2 = orc.Model(q35.config_c(cfg), blob.table, blob.n, blob.data)
    toks = want
    for pos in range(n_prompt - 1 + n_gen):
        om2.decode(int(toks[pos]), pos, lo if pos == n_prompt - 2 + n_gen else None)
    assert np.array_equal(lg.view(np.uint32), lo.view(np.uint32))
    assert np.array_equal(hd.view(np.uint32), om2.hidden().view(np.uint32))


def test_graph_replay_is_deterministic(gq, q35):
    cfg = q35.tiny(n_layer=4)
    blob = q35.generate(cfg, seed=1)
    prompt = q35.prompt_ids(cfg, 6, seed=1)
    with q35.Model(blob) as m:
        a = m.generate(prompt, 30)
        b = m.generate(prompt, 30)
    assert np.array_equal(a, b)


def test_full_width_model_greedy_matches_oracle(gq, orc, q35):
    """The C5 widths (hidden 4096, FFN 12288, vocab 151936, 16/4 heads of 256, 32/16 DeltaNet heads) with 4 layers
    (3 DeltaNet + 1 attention): greedy tokens, logits and hidden state identical to the oracle decoder."""
    cfg = q35.Config(n_layer=4, n_ctx=64)
    blob = q35.generate(cfg, seed=0)
    prompt = q35.prompt_ids(cfg, 8)
    n_gen = 16
    om = orc.Model(q35.config_c(cfg), blob.table, blob.n, blob.data)
    want = om.generate(prompt, n_gen)
    with q35.Model(blob) as m:
        got = m.generate(prompt, n_gen)
        lg, hd = m.logits(), m.hidden()
    assert np.array_equal(got, want), f"first mismatch at {np.nonzero(got != want)[0][:3]}"
    lo = np.empty(cfg.n_vocab, np.float32)
    om2 = orc.Model(q35.config_c(cfg), blob.table, blob.n, blob.data)
    for pos in range(len(prompt) - 1 + n_gen):
        om2.decode(int(want[pos]), pos, lo if pos == len(prompt) - 2 + n_gen else None)
    assert np.array_equal(lg.view(np.uint32), lo.view(np.uint32))
    assert np.array_equal(hd.view(np.uint32), om2.hidden().view(np.uint32))


def test_model_from_gguf_file_matches_oracle(gq, orc, q35, tmp_path):
    """A model written to a GGUF file, with Q4_1 ffn_down in two layers (the type mix of real Qwen3.5 Q4_0 files),
    read back through the GGUF reader and decoded from the file's mapping: tokens and logits identical to the oracle
    decoder on the in-memory tensors."""
    import gguf

    cfg = q35.tiny(n_layer=8)
    types = {f"blk.{il}.ffn_down.weight": gq.Q4_1 for il in (1, 3)}
    blob = q35.generate(cfg, seed=4, types=types)
    path = str(tmp_path / "model.gguf")
    gguf.write_model(path, blob)
    fb = gguf.open_model(path, n_ctx=cfg.n_ctx)
    prompt = q35.prompt_ids(cfg, 6, seed=4)
    n_gen = 16
    om = orc.Model(q35.config_c(cfg), blob.table, blob.n, blob.data)
    want = om.generate(prompt, n_gen)
    try:
        with q35.Model(fb) as m:
            got = m.generate(prompt, n_gen)
            lg = m.logits()
    finally:
        fb.owner.close()
    assert np.array_equal(got, want), f"first mismatch at {np.nonzero(got != want)[0][:3]}"
    lo = np.empty(cfg.n_vocab, np.float32)
    om2 = orc.Model(q35.config_c(cfg), blob.table, blob.n, blob.data)
    for pos in range(len(prompt) - 1 + n_gen):
        om2.decode(int(want[pos]), pos, lo if pos == len(prompt) - 2 + n_gen else None)
    assert np.array_equal(lg.view(np.uint32), lo.view(np.uint32))


@pytest.fixture(scope="module")
def c5(q35):
    """The C5 model (32 layers: 24 DeltaNet + 8 attention, hidden 4096, FFN 12288, vocab 151936, Q4_0 layers, Q6_K
    embedding and head, seed 0), its 512-id prompt, and its GPU run: the prompt through the batched prefill (all but
    the last prompt token), then 128 greedy decode steps, so the context reaches 640."""
    cfg = q35.Config(n_ctx=640)
    blob = q35.generate(cfg, seed=0)
    prompt = q35.prompt_ids(cfg, 512)
    print("[c5] model generated; GPU prefill + 128 steps", flush=True)
    with q35.Model(blob) as m:
        m.reset(prompt)
        assert m.prefill(len(prompt) - 1)
        m.step(128)
        toks, logits = m.tokens(640), m.logits()
    return cfg, blob, prompt, toks, logits


@pytest.mark.timeout(900)
def test_c5_full_size_matches_oracle(orc, q35, c5):
    """C5 at its stated size: 128 greedy tokens identical to the oracle decoder's, and the last step's logits bit
    for bit (the oracle runs the prompt as chunked prefill too; its prefill equals its decode steps bit for bit)."""
    cfg, blob, prompt, toks, logits = c5
    om = orc.Model(q35.config_c(cfg), blob.table, blob.n, blob.data)
    lo = np.empty(cfg.n_vocab, np.float32)
    print("[c5] oracle prefill + 128 steps", flush=True)
    want = om.generate_fast(prompt, 128, lo)
    om.close()
    assert np.array_equal(toks, want), f"first mismatch at {np.nonzero(toks != want)[0][:3]}"
    assert np.array_equal(logits.view(np.uint32), lo.view(np.uint32))


@pytest.mark.timeout(1200)
def test_c5_reference_arithmetic_matches_cpu_path(gq, orc, q35, c5):
    """C5 in the reference arithmetic (gemvq_set_arith): the 512-id prompt through the prefill (its GEMMs token by
    token in this arithmetic), then 128 greedy steps: all 640 token ids and the last step's logits identical, bit for
    bit, to the reference-arithmetic decoder on the CPU (gemvq_ref.h's sequential FP32 rows, double norm sums,
    sequential DeltaNet dots, ggml's CPU attention, correctly rounded exp / log)."""
    cfg, blob, prompt, toks, _ = c5
    print("[c5] GPU reference arithmetic: prefill + 128 steps", flush=True)
    with q35.Model(blob) as m:
        m.set_arith(gq.ARITH_REFERENCE)
        m.reset(prompt)
        assert m.prefill(len(prompt) - 1)
        m.step(128)
        got, lg = m.tokens(640), m.logits()
    om = orc.Model(q35.config_c(cfg), blob.table, blob.n, blob.data, mode=orc.MODE_REFERENCE)
    lr = np.empty(cfg.n_vocab, np.float32)
    print("[c5] CPU reference arithmetic: prefill + 128 steps", flush=True)
    want = om.generate_fast(prompt, 128, lr)
    om.close()
    assert np.array_equal(got, want), f"first mismatch at {np.nonzero(got != want)[0][:3]}"
    assert np.array_equal(lg.view(np.uint32), lr.view(np.uint32))
    # how far the canonical arithmetic's greedy run stays with it (reported; FP32 roundings flip Q8_0 decisions)
    d = np.nonzero(toks != want)[0]
    print(f"[c5] canonical vs reference arithmetic: first differing position {int(d[0]) if d.size else None}", flush=True)


@pytest.mark.timeout(900)
@pytest.mark.parametrize("n_seq", [4, 8])
def test_c5_lockstep_sequences_match_single_decodes(gq, orc, q35, c5, n_seq):
    """Lockstep decode at C5's size (the 9B shape, 32 layers): n_seq sequences with prompts of different lengths, 12
    steps. Every sequence's token ids and last logits equal, bit for bit, a single-sequence decode of its own prompt
    on the GPU, and sequence 0's equal the oracle decoder's. 4 sequences run the layer projections as small-token
    GEMVs, 8 as MFMA batched GEMVs (the paths whose rates profiles/c5_sequences_decode.md reports)."""
    cfg, blob, _, _, _ = c5
    steps = 12
    rng = np.random.default_rng(40 + n_seq)
    lens = [int(v) for v in rng.integers(1, 17, n_seq)]  # some longer than the steps: prompt positions only
    lens[0] = 5
    prompts = [rng.integers(0, cfg.n_vocab, L).astype(np.int32) for L in lens]
    print(f"[c5 lockstep] {n_seq} sequences, prompts {lens}, {steps} steps", flush=True)
    with q35.BatchModel(blob, n_seq) as bm:
        bm.reset(prompts)
        bm.step(steps)
        got = [(bm.tokens(s, steps + 1), bm.logits(s)) for s in range(n_seq)]
    print("[c5 lockstep] single-sequence decodes", flush=True)
    with q35.Model(blob) as m:
        for s in range(n_seq):
            m.reset(prompts[s])
            m.step(steps)
            want = m.tokens(steps + 1)
            assert np.array_equal(got[s][0], want), f"sequence {s}: {got[s][0]} vs {want}"
            assert np.array_equal(got[s][1].view(np.uint32), m.logits().view(np.uint32)), f"sequence {s} logits"
    print("[c5 lockstep] oracle decode of sequence 0", flush=True)
    om = orc.Model(q35.config_c(cfg), blob.table, blob.n, blob.data)
    lo = np.empty(cfg.n_vocab, np.float32)
    n_gen = steps - len(prompts[0]) + 1  # positions 0 .. steps - 1 processed, as the GPU's steps
    want = om.generate_fast(prompts[0], n_gen, lo)
    om.close()
    assert np.array_equal(got[0][0], want), f"{got[0][0]} vs {want}"
    assert np.array_equal(got[0][1].view(np.uint32), lo.view(np.uint32))


def _decode_state(m, cfg, npos):
    """DeltaNet states, the attention layers' K/V up to npos, and the device's token ids up to npos + 1."""
    gdn_layers = sum(1 for il in range(cfg.n_layer) if (il + 1) % cfg.attn_interval != 0)
    st = m.ctx.state_read(0, gdn_layers * cfg.ssm_v_heads * 128)
    kvs = [m.ctx.kv_read(i, 0, npos, cfg.n_head_kv * cfg.head_dim)
           for i in range(cfg.n_layer - gdn_layers)]
    return st, kvs, m.tokens(npos + 1)


@pytest.mark.parametrize("q4_1", [False, True])
def test_batched_prefill_equals_decode_steps(gq, q35, q4_1):
    """The batched prefill (GEMM commands over chunks of up to 32 prompt tokens, the conv and DeltaNet step over the
    tokens in order, attention token by token) leaves the model where the decode steps do, bit for bit: DeltaNet
    states, KV cache, token ids; and the generation that follows has identical tokens, logits and hidden state. C5
    widths, 4 layers (3 DeltaNet + 1 attention); 44 prompt positions = chunks of 32 and 12; and a prefill split
    around decode steps. With q4_1, two layers' ffn_down are Q4_1 (the type mix of real Qwen3.5 Q4_0 files)."""
    cfg = q35.Config(n_layer=4, n_ctx=96)
    types = {f"blk.{il}.ffn_down.weight": gq.Q4_1 for il in (1, 3)} if q4_1 else None
    blob = q35.generate(cfg, seed=1, types=types)
    prompt = q35.prompt_ids(cfg, 45, seed=1)
    n_gen = 12
    with q35.Model(blob) as m:
        m.reset(prompt)
        m.step(len(prompt) - 1)
        s_steps = _decode_state(m, cfg, len(prompt) - 1)
        m.step(n_gen)
        t_steps, l_steps, h_steps = m.tokens(len(prompt) + n_gen), m.logits(), m.hidden()

        m.reset(prompt)
        print("[prefill] 44 positions", flush=True)
        assert m.prefill(len(prompt) - 1)
        s_pre = _decode_state(m, cfg, len(prompt) - 1)
        assert np.array_equal(s_pre[0].view(np.uint32), s_steps[0].view(np.uint32)), "DeltaNet states"
        for a, b in zip(s_pre[1], s_steps[1]):
            assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1]), "KV cache"
        assert np.array_equal(s_pre[2], s_steps[2]), "token ids"
        m.step(n_gen)
        assert np.array_equal(m.tokens(len(prompt) + n_gen), t_steps)
        assert np.array_equal(m.logits().view(np.uint32), l_steps.view(np.uint32))
        assert np.array_equal(m.hidden().view(np.uint32), h_steps.view(np.uint32))

        m.reset(prompt)  # prefill, steps, prefill again: positions read back from the device
        print("[prefill] split 7 + 3 steps + 34", flush=True)
        assert m.prefill(7)
        m.step(3)
        assert m.prefill(len(prompt) - 1 - 10)
        m.step(n_gen)
        assert np.array_equal(m.tokens(len(prompt) + n_gen), t_steps)
        assert np.array_equal(m.logits().view(np.uint32), l_steps.view(np.uint32))
        m.reset(prompt)
        with pytest.raises(gq.GemvqError):
            m.prefill(len(prompt))  # the last prompt token is a decode step (its logits pick the first new token)


def test_batched_prefill_declines_unbatchable_models(gq, q35):
    """Projections without a batched form (columns not a multiple of 512): prefill runs nothing and says so."""
    cfg = q35.tiny(n_layer=4)
    blob = q35.generate(cfg, seed=2)
    with q35.Model(blob) as m:
        m.reset(q35.prompt_ids(cfg, 10, seed=2))
        assert not m.prefill(5)
        m.step(9)
        assert m.tokens(10)[9] >= 0
