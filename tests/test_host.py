"""Host-side checks that need no GPU: the C-ABI libraries load and export every declared entry point, the weight
repack is a lossless permutation, command words follow the documented layout, the synthetic-data generators
(portable RNG, ggml's closed-form weight quantizers) reproduce their published definitions, and the model sizes
match the workload's byte counts."""
import ctypes as C
import os
import re
import struct

import numpy as np
import pytest

import ggml_blocks as B

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(ROOT, "include")


@pytest.fixture(scope="module")
def libs(gq):
    if not (os.path.exists(gq.HIP_LIB_PATH) and os.path.exists(gq.SYNTH_LIB_PATH)):
        import build  # the package's build script (hipcc cross-compiles for gfx950 without a GPU)

        build.build()
    return {"gemvq_hip.h": C.CDLL(gq.HIP_LIB_PATH), "gemvq_qwen35.h": C.CDLL(gq.HIP_LIB_PATH),
            "gemvq_gguf.h": C.CDLL(gq.HIP_LIB_PATH), "gemvq_ggml.h": C.CDLL(gq.HIP_LIB_PATH),
            "gemvq_synth.h": C.CDLL(gq.SYNTH_LIB_PATH)}


def declared_functions(header: str) -> list[str]:
    text = open(os.path.join(INCLUDE, header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    text = re.sub(r"#[^\n]*", "", text)
    return re.findall(r"\b((?:gemvq|gqs|gqg)_\w+)\s*\([^;{]*\)\s*;", text)


def test_every_declared_symbol_is_exported(libs):
    headers = sorted(f for f in os.listdir(INCLUDE) if f.endswith(".h"))
    assert set(headers) == set(libs), headers
    total = 0
    for h in headers:
        names = declared_functions(h)
        assert names, h
        missing = [n for n in names if not hasattr(libs[h], n)]
        assert not missing, (h, missing)
        total += len(names)
    assert total >= 40


@pytest.mark.parametrize("t", [B.Q4_0, B.Q4_1, B.Q8_0, B.Q5_K, B.Q6_K])
def test_repack_round_trip(gq, libs, t):
    rows, cols = 37, 2048
    rng = np.random.default_rng(t)
    gguf = rng.integers(0, 256, rows * gq.row_bytes(t, cols), dtype=np.uint8)
    packed = gq.repack(t, rows, cols, gguf)
    assert packed.size == gguf.size and not np.array_equal(packed, gguf)
    if t == B.Q6_K:  # high bits regrouped per 64-weight unit: the same bits, moved within and between bytes
        assert np.unpackbits(packed).sum() == np.unpackbits(gguf).sum()
        ns = cols // 256
        assert np.array_equal(packed[:rows * ns * 128], gguf.reshape(-1, 210)[:, :128].ravel())  # ql as it is
    else:
        assert np.array_equal(np.sort(packed), np.sort(gguf))  # the same bytes, reordered
    assert np.array_equal(gq.unpack(t, rows, cols, packed), gguf)


def test_repack_rejects_bad_shapes(gq, libs):
    lib = gq.hip_lib()
    buf = np.zeros(1 << 16, np.uint8)
    for t, rows, cols in [(1, 4, 256), (6, 4, 256), (2, 4, 48), (3, 4, 40), (13, 4, 128), (2, 0, 256), (8, 4, 32768)]:
        assert lib.gemvq_repack(t, rows, cols, buf.ctypes.data, buf.ctypes.data) == gq.EINVAL, (t, rows, cols)


def test_command_words(gq):
    """Word layouts documented in gemvq_hip.h (the reference's gemvqc16.h:26-98 layout)."""
    assert gq.gemv(2, 9728, 2560, (5 << 32) | 1234, 16, 32, gq.GEMV_ADD) == [1, 2 | 0x400, 9728, 2560, 1234, 5, 16, 32]
    eps = struct.unpack("<I", struct.pack("<f", 1e-6))[0]
    assert gq.rmsnorm(4096, 0, 16, 32, 1e-6, rows=2, flags=gq.NORM_DEFER, stride_words=3) == \
        [2, 4096, 0, 16, 32, eps, 2, 4 | (3 << 8)]
    g = gq.gdn(32, 16, 1, 2, 3, 4, 5, 6, 7, 8, 0.5, flags=gq.GDN_GATES | gq.GDN_L2_QK, w=9, z=10, dt=11, a=12)
    assert len(g) == 24 and g[:2] == [7, 32 | (16 << 16)] and g[8:10] == [7, 8] and g[16:18] == [11, 12]
    a = gq.attn(16, 4, 0, 1, 2, 256, 64, 3, 4, 5, 0.0625, 1e-6, 6, 7, 8, gate=256)
    assert len(a) == 16 and a[1] == 16 | (4 << 16) and a[5] == 256 | (64 << 16) and a[7] == 1 and a[15] == 256
    assert all(len(c) == 8 for c in (gq.add(16, 0, 16, 32), gq.fill(16, 0, 1.0), gq.next_token(0, 16, 32, 48, 5, 64)))
    m = gq.gemm(2, 64, 1024, (7 << 32) | 5, 16, 32, 4, 1024, 64, gq.GEMV_ADD, 48, 64, 80, 1e-6, gq.NORM_DEFER)
    assert m == [17, 2 | 0x400, 64, 1024, 5, 7, 16, 32, 4, 1024, 64, 48, 64, 80, eps, 4]
    # token counts: ATTN flags bits 23:16 (with the gate bit 0), GET_ROWS format word bits 23:16; one token is 0
    at = gq.attn(16, 4, 0, 1, 2, 256, 64, 3, 4, 5, 0.0625, 1e-6, 6, 7, 8, gate=256, n_tok=32)
    assert at[7] == 1 | (32 << 16) and at[:7] == a[:7] and at[8:] == a[8:]
    assert gq.get_rows(14, 151936, 4096, (1 << 32) | 2, 16, 32, n_tok=7) == [13, 14 | (7 << 16), 151936, 4096, 2, 1, 16, 32]
    assert gq.get_rows(14, 151936, 4096, 2, 16, 32)[1] == 14


# ---- synthetic data ---------------------------------------------------------------------------------------------
GAMMA = 0x9E3779B97F4A7C15
M64 = (1 << 64) - 1


def mix64(z: int) -> int:
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
    return z ^ (z >> 31)


def test_splitmix64(gq, libs):
    """SplitMix64 (Steele, Lea, Flood 2014): the published first outputs from state 0, then the counter form the
    generator uses, value i of a stream = the (i + 1)-th SplitMix64 output from the stream key."""
    outs, s = [], 0
    for _ in range(3):
        s = (s + GAMMA) & M64
        outs.append(mix64(s))
    assert outs == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]
    lib = gq.synth_lib()
    for seed, stream in [(0, 0), (1, 7), (12345, 1 << 40)]:
        key = mix64(mix64((seed + GAMMA) & M64) ^ ((stream * 0xD1B54A32D192ED03) & M64))
        for i in (0, 1, 2, 1000, 123456789):
            assert lib.gqs_u64(seed, stream, i) == mix64((key + (i + 1) * GAMMA) & M64)


def test_normal_and_uniform_moments(gq, libs):
    x = gq.normal(0, 3, 1 << 20, mean=0.5, std=2.0).astype(np.float64)
    assert abs(x.mean() - 0.5) < 0.01 and abs(x.std() - 2.0) < 0.01
    assert abs(np.abs(((x - 0.5) / 2) ** 3).mean() - np.sqrt(8 / np.pi)) < 0.02  # E|z|^3 of a standard normal
    u = gq.uniform(0, 4, 1 << 20, -1.0, 3.0).astype(np.float64)
    assert u.min() >= -1.0 and u.max() <= 3.0 and abs(u.mean() - 1.0) < 0.01
    assert np.array_equal(gq.normal(0, 3, 100, first=50), gq.normal(0, 3, 150)[50:])  # counter-based


def q4_0_ggml(x: np.ndarray) -> np.ndarray:
    """ggml quantize_row_q4_0_ref: max = value of largest magnitude (first), d = max / -8, id = 1 / d,
    q = min(15, (int8)(x * id + 8.5)) (truncation), low nibble j, high nibble j + 16."""
    x = x.astype(np.float32).reshape(-1, 32)
    out = np.zeros((x.shape[0], 18), np.uint8)
    for b, row in enumerate(x):
        mx = row[int(np.argmax(np.abs(row)))]
        d = np.float32(mx / np.float32(-8))
        idv = np.float32(1) / d if d != 0 else np.float32(0)
        q = np.minimum(15, np.trunc((row * idv + np.float32(8.5)).astype(np.float32))).astype(np.uint8)
        out[b, 0:2] = np.array([d], np.float16).view(np.uint8)
        out[b, 2:] = q[:16] | (q[16:] << 4)
    return out.ravel()


def q4_1_ggml(x: np.ndarray) -> np.ndarray:
    """ggml quantize_row_q4_1_ref: d = (max - min) / 15, m = min, q = min(15, (int8)((x - min) / d + 0.5))."""
    x = x.astype(np.float32).reshape(-1, 32)
    out = np.zeros((x.shape[0], 20), np.uint8)
    for b, row in enumerate(x):
        mn, mx = row.min(), row.max()
        d = np.float32((mx - mn) / np.float32(15))
        idv = np.float32(1) / d if d != 0 else np.float32(0)
        q = np.minimum(15, np.trunc(((row - mn) * idv).astype(np.float32) + np.float32(0.5))).astype(np.uint8)
        out[b, 0:2] = np.array([d], np.float16).view(np.uint8)
        out[b, 2:4] = np.array([mn], np.float16).view(np.uint8)
        out[b, 4:] = q[:16] | (q[16:] << 4)
    return out.ravel()


def test_weight_quantizers_closed_form(gq, libs):
    x = gq.normal(5, 1, 64 * 256, std=0.02)
    x[:32] = 0.0
    assert np.array_equal(gq.quantize(B.Q4_0, x, 64, 256), q4_0_ggml(x))
    assert np.array_equal(gq.quantize(B.Q4_1, x, 64, 256), q4_1_ggml(x))
    # Q8_0 weights use the activation quantizer's closed form
    q, d = B.quantize_q8_0(x)
    blk = np.concatenate([d.view(np.uint8).reshape(-1, 2), q.view(np.uint8).reshape(-1, 32)], axis=1).ravel()
    assert np.array_equal(gq.quantize(B.Q8_0, x, 64, 256), blk)


@pytest.mark.parametrize("t,tol", [(B.Q5_K, 0.06), (B.Q6_K, 0.03)])
def test_k_quant_weight_error(gq, libs, t, tol):
    """ggml's K-quant weight quantizers (iterative scale search; their exact bytes are not pinned here): the
    dequantized weights stay within a fraction of each super-block's range."""
    x = gq.normal(5, 2, 32 * 1024, std=0.02)
    w = gq.quantize(t, x, 32, 1024)
    err = np.abs(B.dequantize(t, w, 32, 1024).ravel() - x).reshape(-1, 256).max(axis=1)
    rng = np.abs(x).reshape(-1, 256).max(axis=1)
    assert np.all(err <= tol * rng)


def test_model_sizes(gq):
    import qwen35 as Q

    cfg = Q.QWEN35_9B
    assert Q.weight_bytes(cfg) == 4_402_163_712  # 24 GDN + 8 attention layers + Q6_K head
    by_layer: dict[int, int] = {}
    for name, t, ne0, ne1, _ in Q.tensor_specs(cfg):
        if name.startswith("blk.") and t != Q.F32:
            il = int(name.split(".")[1])
            by_layer[il] = by_layer.get(il, 0) + Q.tensor_bytes(t, ne0, ne1)
    assert by_layer[0] == 122_830_848 and by_layer[3] == 117_964_800  # a DeltaNet layer, an attention layer
    assert sum(by_layer.values()) + 151936 * gq.row_bytes(B.Q6_K, 4096) == 4_402_163_712


def test_activation_rounding_matches_roundf(tmp_path):
    """The GEMV activation quantizer rounds with an add and a truncation; exhaustively equal to roundf for every
    float of magnitude <= 128 (the quantizer's range)."""
    import shutil
    import subprocess

    if shutil.which("gcc") is None:
        pytest.skip("gcc is not available")
    exe = tmp_path / "round_check"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-fno-fast-math", os.path.join(os.path.dirname(__file__),
                    "round_check.c"), "-o", str(exe), "-lm"], check=True)
    n, bad = map(int, subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split())
    assert n == 2248146946 and bad == 0


def test_wait_timeout_setting_is_validated(gq, libs, monkeypatch):
    """The wait bound (ggml-xrt.cpp:69-78's GGML_XRT_WAIT_TIMEOUT_MS): a malformed GEMVQ_WAIT_TIMEOUT_MS fails the
    create before any device call, with the reason; the setter rejects 0 and a NULL context; NULL is not usable."""
    lib = gq.hip_lib()
    for bad in ("0", "abc", "12x", "-5", ""):
        monkeypatch.setenv("GEMVQ_WAIT_TIMEOUT_MS", bad)
        assert not lib.gemvq_ctx_create(0, 1024, 0, 0), bad
        assert b"GEMVQ_WAIT_TIMEOUT_MS" in lib.gemvq_last_error(None)
    assert lib.gemvq_set_wait_timeout(None, 5) == gq.EINVAL
    assert lib.gemvq_usable(None) == 0
