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


@pytest.mark.timeout(600)
def test_c5_greedy_128_steps_matches_oracle(gq, orc, q35):
    """The full C5 model (32 layers: 24 DeltaNet + 8 attention, hidden 4096, FFN 12288, vocab 151936, Q4_0 layers,
    Q6_K embedding and head, seed 0): 128 greedy tokens after an 8-token prompt, identical to the oracle decoder's,
    and the last step's logits bit for bit."""
    cfg = q35.Config(n_ctx=160)
    blob = q35.generate(cfg, seed=0)
    prompt = q35.prompt_ids(cfg, 8)
    n_gen = 128
    om = orc.Model(q35.config_c(cfg), blob.table, blob.n, blob.data)
    lo = np.empty(cfg.n_vocab, np.float32)
    toks = [int(t) for t in prompt]
    for pos in range(len(prompt) - 1 + n_gen):  # the oracle's greedy decode, keeping the last logits
        last = pos == len(prompt) - 2 + n_gen
        nxt = om.decode(toks[pos], pos, lo if last else None)
        if pos + 1 >= len(prompt):
            toks.append(nxt)
    om.close()
    want = np.array(toks, np.int32)
    with q35.Model(blob) as m:
        got = m.generate(prompt, n_gen)
        lg = m.logits()
    assert np.array_equal(got, want), f"first mismatch at {np.nonzero(got != want)[0][:3]}"
    assert np.array_equal(lg.view(np.uint32), lo.view(np.uint32))
