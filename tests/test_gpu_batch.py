"""Lockstep decode of several sequences (include/gemvq_qwen35.h gemvq_qwen35_batch_*): one step advances every
sequence by one position with each layer's weight rows read once for all of them (GEMM commands), CONV, the DeltaNet
step and attention in their sequences forms. Every sequence must equal a single-sequence decode of its own prompt
bit for bit: its token ids over the prompt and the generation, and its last logits. Prompts of different lengths
(sequences switch from prompt tokens to generated ones at different steps), a K-quant head (one GEMV per sequence)
and a Q8_0 head (one GEMM over all sequences), up to the largest batch; 2-4 sequences run their projections as
small-token GEMVs, 5 and more as MFMA batched GEMVs."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def q35():
    import qwen35

    return qwen35


def small(n_layer=4, n_ctx=48):
    import qwen35

    # widths that have batched GEMVs (multiples of 512), the structure of the 9B shape
    return qwen35.Config(n_layer=n_layer, n_embd=1024, n_ff=2048, n_vocab=2048, n_head=4, n_head_kv=1,
                         head_dim=128, n_rot=32, ssm_k_heads=2, ssm_v_heads=4, n_ctx=n_ctx)


@pytest.mark.parametrize("n_seq,head,steps", [(2, "q8_0", 14), (3, "q6_k", 12), (4, "q6_k", 20), (5, "q8_0", 16),
                                             (32, "q6_k", 6)])
def test_lockstep_sequences_equal_single_decodes(gq, q35, n_seq, head, steps):
    cfg = small()
    types = {"output.weight": gq.Q8_0} if head == "q8_0" else None
    blob = q35.generate(cfg, seed=11, types=types)
    rng = np.random.default_rng(12 + n_seq)
    lens = [int(v) for v in rng.integers(1, 14, n_seq)]
    lens[0] = 1
    prompts = [rng.integers(0, cfg.n_vocab, L).astype(np.int32) for L in lens]
    print(f"[batch] {n_seq} sequences, prompts {lens[:6]}..., {steps} steps, {head} head", flush=True)
    with q35.BatchModel(blob, n_seq) as bm:
        bm.reset(prompts)
        bm.step(steps)
        got = [(bm.tokens(s, steps + 1), bm.logits(s)) for s in range(n_seq)]
        bm.reset(prompts)  # a second run from a reset (the captured graph replayed) gives the same
        bm.step(steps)
        for s in range(n_seq):
            assert np.array_equal(bm.tokens(s, steps + 1), got[s][0])
    with q35.Model(blob) as m:
        for s in range(n_seq) if n_seq <= 8 else (0, 7, 19, 31):
            m.reset(prompts[s])
            m.step(steps)
            want = m.tokens(steps + 1)
            assert np.array_equal(got[s][0], want), f"sequence {s}: {got[s][0]} vs {want}"
            assert np.array_equal(got[s][1].view(np.uint32), m.logits().view(np.uint32)), f"sequence {s} logits"
            assert np.array_equal(want[:min(lens[s], steps + 1)], prompts[s][:min(lens[s], steps + 1)])


@pytest.mark.parametrize("n_seq,head", [(3, "q8_0"), (5, "q6_k")])
def test_lockstep_sequences_in_reference_arithmetic(gq, q35, n_seq, head):
    """The batch model in the reference arithmetic (its GEMMs as token GEMVs, the sequences forms of CONV, the
    DeltaNet step and attention token by token): every sequence's ids and last logits equal a single-sequence model's
    decode of its prompt in the reference arithmetic, bit for bit."""
    cfg = small()
    types = {"output.weight": gq.Q8_0} if head == "q8_0" else None
    blob = q35.generate(cfg, seed=21, types=types)
    rng = np.random.default_rng(30 + n_seq)
    lens = [int(v) for v in rng.integers(1, 10, n_seq)]
    prompts = [rng.integers(0, cfg.n_vocab, L).astype(np.int32) for L in lens]
    steps = 12
    print(f"[batch ref] {n_seq} sequences, prompts {lens}, {steps} steps, {head} head", flush=True)
    with q35.BatchModel(blob, n_seq) as bm:
        bm.reset(prompts)
        bm.step(steps)
        canonical = [bm.logits(s) for s in range(n_seq)]
        bm.set_arith(gq.ARITH_REFERENCE)
        bm.reset(prompts)
        bm.step(steps)
        got = [(bm.tokens(s, steps + 1), bm.logits(s)) for s in range(n_seq)]
    # the mode took effect: the two arithmetics' logits differ in their low bits
    assert any(not np.array_equal(c.view(np.uint32), g[1].view(np.uint32)) for c, g in zip(canonical, got))
    with q35.Model(blob) as m:
        m.set_arith(gq.ARITH_REFERENCE)
        for s in range(n_seq):
            m.reset(prompts[s])
            m.step(steps)
            assert np.array_equal(got[s][0], m.tokens(steps + 1)), f"sequence {s}"
            assert np.array_equal(got[s][1].view(np.uint32), m.logits().view(np.uint32)), f"sequence {s} logits"


def test_batch_model_rejects_single_sequence_calls(gq, q35):
    cfg = small(n_layer=4, n_ctx=32)
    blob = q35.generate(cfg, seed=13)
    with q35.BatchModel(blob, 2) as bm:
        lib = bm.lib
        assert lib.gemvq_qwen35_reset(bm.h, np.zeros(1, np.int32).ctypes.data, 1) == gq.EINVAL
        assert lib.gemvq_qwen35_prefill(bm.h, 1) == gq.EINVAL
        assert lib.gemvq_qwen35_batch_tokens(bm.h, 2, np.zeros(4, np.int32).ctypes.data, 4) == gq.EINVAL
        with pytest.raises(gq.GemvqError):
            bm.reset([np.zeros(0, np.int32), np.zeros(3, np.int32)])  # an empty prompt
