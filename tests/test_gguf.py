"""GGUF ingestion on the host (no GPU): the reader of include/gemvq_gguf.h against files written here byte by byte
from the published GGUF layout, the configuration a Qwen3.5 file implies, and the inverse of ggml's CPU_REPACK
Q4_0x8 layout (ggml-xrt.cpp:675-710) against blocks built from its definition and a hand-placed known answer."""
import struct

import numpy as np
import pytest

import gemvq as gq
import gguf
import qwen35 as qw


def _s(x: bytes) -> bytes:
    return struct.pack("<Q", len(x)) + x


@pytest.fixture(scope="module")
def tiny_file(tmp_path_factory):
    cfg = qw.tiny()
    blob = qw.generate(cfg, seed=5)
    path = str(tmp_path_factory.mktemp("gguf") / "tiny.gguf")
    gguf.write_model(path, blob)
    return cfg, blob, path


def test_round_trip_tensors_and_metadata(tiny_file):
    cfg, blob, path = tiny_file
    with gguf.GGUF(path) as g:
        assert g.version == 3 and len(g.tensors) == blob.n
        for d, t in zip(blob.table, g.tensors):
            assert t.name == d.name.decode() and t.type == d.type and t.nbytes == d.nbytes
            assert t.ne == ((d.ne0, 1, 1, 1) if d.ne1 == 1 else (d.ne0, d.ne1, 1, 1))
            assert t.offset % 32 == 0
            assert np.array_equal(g.tensor(t.name), blob.data[d.offset:d.offset + d.nbytes])
        assert g.get("general.architecture") == "qwen35"
        assert g.get("qwen35.block_count") == cfg.n_layer
        assert g.get("qwen35.rope.freq_base") == cfg.rope_base
        assert np.float32(g.get("qwen35.attention.layer_norm_rms_epsilon")) == np.float32(cfg.eps)
        assert g.get("no.such.key", "absent") == "absent"
        got = gguf.config_from(g, n_ctx=cfg.n_ctx)
    for f in qw.Config.__dataclass_fields__:
        a, b = getattr(got, f), getattr(cfg, f)
        assert (np.float32(a) == np.float32(b)) if f == "eps" else a == b, f


def test_open_model_points_into_the_file(tiny_file):
    cfg, blob, path = tiny_file
    m = gguf.open_model(path, n_ctx=cfg.n_ctx)
    assert m.n == blob.n and not m.data.flags.writeable
    for d, e in zip(blob.table, m.table):
        assert (d.name, d.type, d.ne0, d.ne1, d.nbytes) == (e.name, e.type, e.ne0, e.ne1, e.nbytes)
        assert np.array_equal(blob.data[d.offset:d.offset + d.nbytes], m.data[e.offset:e.offset + e.nbytes])
    m.owner.close()


def test_mixed_types_and_tied_head(tmp_path):
    """Q4_1 ffn_down in a Q4_0 model (as real Qwen3.5 Q4_0 files are) and a file without output.weight."""
    cfg = qw.tiny(n_layer=4)
    types = {f"blk.{il}.ffn_down.weight": gq.Q4_1 for il in (0, 3)}
    blob = qw.generate(cfg, seed=2, types=types)
    keep = [(d.name.decode(), d.type, (d.ne0,) if d.ne1 == 1 else (d.ne0, d.ne1),
             blob.data[d.offset:d.offset + d.nbytes]) for d in blob.table if d.name != b"output.weight"]
    path = str(tmp_path / "tied.gguf")
    gguf.write(path, gguf.config_kv(cfg), keep)
    m = gguf.open_model(path, n_ctx=cfg.n_ctx)
    tab = {d.name.decode(): d for d in m.table}
    assert tab["blk.0.ffn_down.weight"].type == gq.Q4_1 and tab["blk.1.ffn_down.weight"].type == gq.Q4_0
    assert tab["output.weight"].offset == tab["token_embd.weight"].offset
    assert m.cfg.wtype == gq.Q4_0 and m.cfg.etype == cfg.etype
    m.owner.close()


def _raw(kvs: bytes, n_kv: int, tensors: bytes = b"", n_t: int = 0, version: int = 3, magic: bytes = b"GGUF",
         tail: bytes = b"") -> bytes:
    return magic + struct.pack("<IQQ", version, n_t, n_kv) + kvs + tensors + tail


def test_every_metadata_value_type(tmp_path):
    """GGUF value types 0-12: scalars read back converted to double, strings as text, arrays skipped (including
    arrays of strings) without losing the keys after them."""
    k = lambda name, t, payload: _s(name.encode()) + struct.pack("<I", t) + payload
    kvs = [k("u8", 0, struct.pack("<B", 200)), k("i8", 1, struct.pack("<b", -7)), k("u16", 2, struct.pack("<H", 65535)),
           k("i16", 3, struct.pack("<h", -30000)), k("u32", 4, struct.pack("<I", 4000000000)),
           k("i32", 5, struct.pack("<i", -2000000000)), k("f32", 6, struct.pack("<f", 0.375)),
           k("bool", 7, b"\x01"), k("str", 8, _s(b"qwen35")),
           k("arr_i32", 9, struct.pack("<IQ", 5, 3) + struct.pack("<3i", 1, 2, 3)),
           k("arr_str", 9, struct.pack("<IQ", 8, 2) + _s(b"a") + _s(b"bcd")),
           k("u64", 10, struct.pack("<Q", 1 << 40)), k("i64", 11, struct.pack("<q", -(1 << 40))),
           k("f64", 12, struct.pack("<d", -2.5))]
    p = tmp_path / "kv.gguf"
    p.write_bytes(_raw(b"".join(kvs), len(kvs), tail=b"\0" * 32))
    with gguf.GGUF(str(p)) as g:
        assert len(g.tensors) == 0
        want = {"u8": 200, "i8": -7, "u16": 65535, "i16": -30000, "u32": 4000000000, "i32": -2000000000, "f32": 0.375,
                "bool": 1, "str": "qwen35", "u64": float(1 << 40), "i64": -float(1 << 40), "f64": -2.5}
        for key, v in want.items():
            assert g.get(key) == v, key
        assert g.get("arr_i32") is None and g.get("arr_str") is None


def _tensor_info(name: bytes, ne: tuple, t: int, off: int) -> bytes:
    return _s(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", d) for d in ne) + struct.pack("<IQ", t, off)


@pytest.mark.parametrize("case", ["magic", "version", "truncated", "outside", "misaligned", "ragged", "type", "dims"])
def test_reader_rejects_malformed_files(tmp_path, case):
    info = _tensor_info(b"w", (32, 2), 2, 0)
    body = _raw(b"", 0, info, 1)
    pad = b"\0" * ((-len(body)) % 32)
    good = body + pad + b"\1" * 36
    bad = {"magic": good.replace(b"GGUF", b"GGUX", 1),
           "version": _raw(b"", 0, info, 1, version=4) + pad + b"\1" * 36,
           "truncated": good[:len(body) - 5],
           "outside": body + pad + b"\1" * 35,
           "misaligned": _raw(b"", 0, _tensor_info(b"w", (32, 2), 2, 4), 1) + pad + b"\1" * 40,
           "ragged": _raw(b"", 0, _tensor_info(b"w", (48, 2), 2, 0), 1) + pad + b"\1" * 54,
           "type": _raw(b"", 0, _tensor_info(b"w", (32, 2), 99, 0), 1) + pad + b"\1" * 36,
           "dims": _raw(b"", 0, _tensor_info(b"w", (32, 1, 1, 1, 2), 2, 0), 1) + b"\1" * 64}[case]
    p = tmp_path / "ok.gguf"
    p.write_bytes(good)
    with gguf.GGUF(str(p)) as g:  # the well-formed file parses
        assert g.tensors[0].ne == (32, 2, 1, 1) and g.tensors[0].nbytes == 36
        assert np.all(g.tensor("w") == 1)
    p = tmp_path / f"{case}.gguf"
    p.write_bytes(bad)
    with pytest.raises(gguf.GGUFError):
        gguf.GGUF(str(p))


def _q4_0x8(rows: int, cols: int, q4: np.ndarray) -> np.ndarray:
    """block_q4_0x8 from GGUF Q4_0 rows, by the layout's definition: per group of 8 rows and column block, the 8
    fp16 scales, then chunk c (0..15) = quant bytes 8 (c // 8) .. + 7 of row c % 8, each byte XOR 0x88."""
    nb = cols // 32
    b = q4.reshape(rows // 8, 8, nb, 18)
    scales = b[..., :2].transpose(0, 2, 1, 3).reshape(rows // 8, nb, 16)
    quants = b[..., 2:].reshape(rows // 8, 8, nb, 2, 8).transpose(0, 2, 3, 1, 4).reshape(rows // 8, nb, 128)
    return np.concatenate([scales, quants ^ 0x88], axis=2).reshape(-1)


def test_unrepack_q4_0x8_known_answer():
    """One x8 block with every byte distinct: each output byte comes from the place the layout names."""
    x8 = np.arange(144, dtype=np.uint8)
    out = gguf.unrepack_q4_0x8(8, 32, x8).reshape(8, 18)
    for r in range(8):
        assert list(out[r, :2]) == [2 * r, 2 * r + 1]                       # scale of row r
        for j in range(16):
            c = 8 * (j // 8) + r                                            # chunk holding quant byte j of row r
            assert out[r, 2 + j] == (16 + 8 * c + j % 8) ^ 0x88, (r, j)
    # row 1, quant byte 11: chunk 9 (second half of row 1), byte 3 of the chunk
    assert out[1, 13] == (16 + 72 + 3) ^ 0x88


@pytest.mark.parametrize("rows,cols", [(8, 32), (16, 256), (64, 4096)])
def test_unrepack_q4_0x8_inverts_the_layout(rows, cols):
    rng = np.random.default_rng(rows + cols)
    q4 = rng.integers(0, 256, rows * cols // 32 * 18, dtype=np.uint8)
    x8 = _q4_0x8(rows, cols, q4)
    assert not np.array_equal(x8, q4)
    assert np.array_equal(gguf.unrepack_q4_0x8(rows, cols, x8), q4)


@pytest.mark.parametrize("rows,cols", [(4, 32), (12, 64), (8, 48), (0, 32)])
def test_unrepack_q4_0x8_rejects_bad_shapes(rows, cols):
    with pytest.raises(ValueError):
        gguf.unrepack_q4_0x8(rows, cols, np.zeros(max(rows, 1) * max(cols, 32) // 32 * 18, np.uint8))
