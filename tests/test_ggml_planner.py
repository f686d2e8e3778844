"""The ggml-facing planner (include/gemvq_ggml.h) on the CPU, in a dry backend (offsets only, no device):

- one decode token of the Qwen3.5 hybrid as a ggml graph compiles to the model builder's per-token command list
  (gemvq_qwen35_dry_commands): the same commands in the same order with the same opcodes, flags, shapes, constants,
  state rows and weight offsets; activation offsets may differ, but consistently (each planner buffer offset stands
  for one builder offset throughout the list). The builder's list ends in the device-side greedy pick (the head
  GEMV's ARGMAX epilog, ARGMAX, NEXT_TOKEN), which a ggml graph leaves to the sampler;
- the plan cache returns the same plan for the same split and builds a new one when the structure changes;
- supports_op and the failure of an unsupported split."""
import ctypes as C

import numpy as np
import pytest

import gemvq as gq
import ggml_ir as ir
import qwen35
import qwen35_ggml

# act offset words per opcode (command slot 0); GDN and ATTN have more slots
ACT_WORDS = {gq.OP_GEMV: (6, 7), gq.OP_RMSNORM: (2, 3, 4), gq.OP_ADD: (2, 3, 4), 8: (2, 3, 4, 5, 6), 13: (6, 7)}
WEIGHT_WORDS = {gq.OP_GEMV: (4, 5), 13: (4, 5)}
OP_GDN, OP_ATTN, OP_ARGMAX, OP_NEXT = 7, 12, 14, 15


def slots(words):
    """Commands as (opcode, [slot arrays])."""
    out, i = [], 0
    while i < len(words):
        op = int(words[i][0])
        n = 1
        if op == OP_GDN:
            n = 3 if int(words[i + 1][3]) & gq.GDN_GATES else 2
        elif op == OP_ATTN:
            n = 2
        out.append((op, [words[j] for j in range(i, i + n)]))
        i += n
    return out


def act_positions(op, n_slots):
    """(slot, word) positions holding act offsets."""
    if op == OP_GDN:
        return [(0, w) for w in (2, 3, 4, 5, 6, 7)] + [(1, 6), (1, 7)] + ([(2, 0), (2, 1)] if n_slots == 3 else [])
    if op == OP_ATTN:
        return [(0, 2), (0, 4), (0, 6)] + [(1, w) for w in (0, 1, 4, 5, 6, 7)]
    return [(0, w) for w in ACT_WORDS.get(op, ())]


def compare(planned, built):
    """Equal lists up to a consistent renaming of act offsets; returns the number of commands compared."""
    P, B = slots(planned), slots(built)
    assert [op for op, _ in P] == [op for op, _ in B], ([op for op, _ in P], [op for op, _ in B])
    ren = {}
    for ci, ((op, ps), (_, bs)) in enumerate(zip(P, B)):
        assert len(ps) == len(bs), (ci, op)
        act = set(act_positions(op, len(ps)))
        for s, (pw, bw) in enumerate(zip(ps, bs)):
            for w in range(8):
                a, b = int(pw[w]), int(bw[w])
                if (s, w) in act:
                    assert ren.setdefault(a, b) == b, f"command {ci} op {op} slot {s} word {w}: offset {a} -> {b}, " \
                                                     f"earlier -> {ren[a]}"
                elif op == OP_ATTN and (s, w) == (0, 3):
                    assert ren.setdefault(("kv", a), b) == b, f"command {ci}: KV buffer {a} -> {b}"
                else:
                    assert a == b, f"command {ci} op {op} slot {s} word {w}: planner {a:#x} builder {b:#x}"
    return len(P)


@pytest.fixture(scope="module")
def tiny_blob():
    cfg = qwen35.tiny(n_layer=4, n_embd=512, n_ff=1024, n_vocab=512, n_ctx=64)
    return qwen35.generate(cfg, seed=3)


def dry_backend(blob):
    cfg = blob.cfg
    rows = sum(not cfg.is_attn(i) for i in range(cfg.n_layer)) * cfg.ssm_v_heads * 128
    return ir.Backend(act_floats=1 << 21, weight_bytes=1 << 30, state_rows=rows, dry=True)


def builder_words(blob):
    L = qwen35._lib()
    gq._c_fn(L, "gemvq_qwen35_dry_commands", C.c_int, C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_size_t)
    cfg_c = qwen35.config_c(blob.cfg)
    n = L.gemvq_qwen35_dry_commands(C.byref(cfg_c), blob.table, blob.n, None, 0)
    assert n > 0
    w = np.zeros(n * 8, np.uint32)
    assert L.gemvq_qwen35_dry_commands(C.byref(cfg_c), blob.table, blob.n, w.ctypes.data, w.size) == n
    return w.reshape(n, 8)


def test_qwen35_graph_compiles_to_the_builders_list(tiny_blob):
    built = builder_words(tiny_blob)
    # the builder ends with the device-side greedy pick: drop ARGMAX and NEXT_TOKEN, and the head's ARGMAX flag
    assert built[-2][0] == OP_ARGMAX and built[-1][0] == OP_NEXT
    built = built[:-2].copy()
    assert built[-1][0] == gq.OP_GEMV and built[-1][1] & gq.GEMV_ARGMAX
    built[-1][1] &= ~np.uint32(gq.GEMV_ARGMAX)
    with dry_backend(tiny_blob) as b:
        g = qwen35_ggml.Qwen35Graph(tiny_blob, b)
        try:
            planned = g.words()
            n = compare(planned, built)
            cfg = tiny_blob.cfg
            # 1 + per layer (norm, projections, step or attention, output + add, norm, pair, down + add) + head
            assert n == len(slots(built))
            assert b.stats() == (1, 0)
            assert np.array_equal(g.words(), planned)  # the same split again: the cached plan
            assert b.stats() == (1, 1)
            assert cfg.n_layer == 4
        finally:
            g.close()


def placeholder_blob(cfg):
    """The tensor table of cfg over a 64-byte buffer: a dry backend plans from shapes and never reads weight bytes."""
    specs = qwen35.tensor_specs(cfg)
    table = (qwen35.TensorDesc * len(specs))()
    off = 0
    for i, (name, t, ne0, ne1, _) in enumerate(specs):
        nb = qwen35.tensor_bytes(t, ne0, ne1)
        table[i] = qwen35.TensorDesc(name.encode(), t, ne0, ne1, 0, off, nb)
        off += (nb + 255) // 256 * 256
    return qwen35.Blob(cfg, table, np.zeros(64, np.uint8), len(specs))


def test_qwen35_9b_graph_compiles_to_the_builders_list():
    """The 9B shape (32 layers, 24 DeltaNet + 8 attention, hidden 4096, FFN 12288, vocab 151936)."""
    blob = placeholder_blob(qwen35.QWEN35_9B)
    built = builder_words(blob)[:-2].copy()
    built[-1][1] &= ~np.uint32(gq.GEMV_ARGMAX)
    cfg = blob.cfg
    rows = 24 * cfg.ssm_v_heads * 128
    with ir.Backend(act_floats=1 << 23, weight_bytes=8 << 30, state_rows=rows, dry=True) as b:
        g = qwen35_ggml.Qwen35Graph(blob, b)
        try:
            assert compare(g.words(), built) == len(slots(built))
        finally:
            g.close()


def test_compare_catches_planted_differences(tiny_blob):
    """The comparison itself: a changed flag and an offset used for two different builder buffers both fail."""
    built = builder_words(tiny_blob)[:-2].copy()
    built[-1][1] &= ~np.uint32(gq.GEMV_ARGMAX)
    with dry_backend(tiny_blob) as b:
        g = qwen35_ggml.Qwen35Graph(tiny_blob, b)
        try:
            planned = g.words()
        finally:
            g.close()
    conv = [i for i in range(len(planned)) if planned[i][0] == gq.OP_GEMV and planned[i][1] & gq.GEMV_CONV][0]
    bad = planned.copy()
    bad[conv][1] &= ~np.uint32(gq.GEMV_CONV)
    with pytest.raises(AssertionError, match="word 1"):
        compare(bad, built)
    bad = planned.copy()
    gemvs = [i for i in range(len(planned)) if planned[i][0] == gq.OP_GEMV]
    bad[gemvs[1]][7] = bad[gemvs[0]][7]  # z written where qkv is
    with pytest.raises(AssertionError, match="offset"):
        compare(bad, built)


def test_plan_cache_keys_on_structure(tiny_blob):
    with dry_backend(tiny_blob) as b:
        g = qwen35_ggml.Qwen35Graph(tiny_blob, b)
        try:
            first = g.words()
            g.logits_t.flags &= ~ir.FLAG_OUTPUT  # a field the plan depends on
            g.words()
            assert b.stats() == (2, 0)
            g.logits_t.flags |= ir.FLAG_OUTPUT
            assert np.array_equal(g.words(), first)
            assert b.stats() == (2, 1)
        finally:
            g.close()


def test_supports_op_and_unsupported_split(tiny_blob):
    with dry_backend(tiny_blob) as b:
        G = ir.Graph()
        w = G.at(ir.Q4_0, [512, 64], tiny_blob.data.ctypes.data, "w", ir.BUF_WEIGHTS)
        x = G.new(ir.F32, [512], "x", ir.FLAG_INPUT)
        y = G.mul_mat(w, x, "y")
        sm = G.soft_max(y, "sm")
        assert b.supports(y)
        assert not b.supports(sm)
        sm.flags |= ir.FLAG_OUTPUT
        G.expand(sm)
        with pytest.raises(RuntimeError, match="not supported"):
            b.plan(G.cgraph())
        # the GEMV alone plans to one command reading x and writing y
        y.flags |= ir.FLAG_OUTPUT
        w2 = b.plan(G.cgraph([y]))
        assert w2.shape == (1, 8) and w2[0][0] == gq.OP_GEMV and w2[0][2] == 64 and w2[0][3] == 512


def test_registration_table():
    L = ir.lib()

    class Reg(C.Structure):
        _fields_ = [("name", C.c_char_p), ("get_description", C.c_void_p), ("get_memory", C.c_void_p),
                    ("device_type", C.c_int)]

    reg = C.cast(L.gqg_backend_get_reg(), C.POINTER(Reg)).contents
    assert reg.name == b"GEMVQ" and reg.device_type == 2 and reg.get_description and reg.get_memory


def test_buffer_outlives_its_backend():
    """A ggml context may free its backend before the buffers of its caches: the buffers are then detached, refuse
    every access, and are still freed by gqg_buffer_free (the memory is reserved, never touched)."""
    L = ir.lib()
    b = ir.Backend(act_floats=1 << 16, weight_bytes=1 << 20, state_rows=2 * 128, dry=True)
    buf = L.gqg_rs_buffer_alloc(b.h, 2 * 128 * 512)
    base = L.gqg_buffer_base(buf)
    G = ir.Graph()
    s = G.at(ir.F32, [2 * 128 * 128], base, "cache_s_l0")
    assert L.gqg_buffer_init_tensor(buf, C.byref(s)) == 0
    row = np.zeros(128, np.float32)
    assert L.gqg_buffer_get(buf, C.byref(s), row.ctypes.data, 0, 512) == 0  # dry: accepted, nothing moves
    b.close()
    assert L.gqg_buffer_get(buf, C.byref(s), row.ctypes.data, 0, 512) != 0
    assert L.gqg_buffer_set(buf, C.byref(s), row.ctypes.data, 0, 512) != 0
    assert L.gqg_buffer_clear(buf, 0) != 0
    assert L.gqg_buffer_init_tensor(buf, C.byref(s)) != 0
    L.gqg_buffer_free(buf)
    with ir.Backend(act_floats=1 << 16, weight_bytes=1 << 20, state_rows=128, dry=True):
        pass  # the process's one backend slot is free again


def test_per_layer_splits_copy_only_split_outputs(tiny_blob):
    """The token cut into one split per layer (and the head): every split compiles, each copies back exactly the
    tensors flagged as split outputs or graph outputs (the residual stream it hands on, the logits), and copies in
    the previous split's residual and the token's host inputs (the reference's readback filter and flush,
    ggml-xrt.cpp:1399-1478); the plans are reused for the next token."""
    cfg = tiny_blob.cfg
    with dry_backend(tiny_blob) as b:
        g = qwen35_ggml.Qwen35Graph(tiny_blob, b)
        try:
            splits = g.layer_splits()
            assert len(splits) == cfg.n_layer + 1
            names = {}
            for t in g.G.tensors:
                names[t.data] = t
            produced = []
            for k, sg in enumerate(splits):
                ins, outs = b.io(sg)
                flagged = [sg.nodes[i].contents for i in range(sg.n_nodes)]
                want_out = {t.data for t in flagged if t.flags & (ir.FLAG_SPLIT_OUTPUT | ir.FLAG_OUTPUT) and not t.view_src}
                assert set(outs) == want_out, (k, [names[o].name for o in outs])
                assert len(outs) == 1  # the residual it hands on, or the logits
                if k > 0:
                    assert produced[-1] in ins, k  # the previous split's residual comes back in
                produced.extend(outs)
            built = b.stats()[0]
            for sg in splits:  # the next token: every split's plan again
                b.plan(sg)
            assert b.stats()[0] == built
        finally:
            g.close()
