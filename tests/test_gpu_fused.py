"""The fused DeltaNet step + gated norm + ssm_out + residual sum that GDN_WITH_OUT asks for (one launch: the heads'
workgroups publish their quantized outputs, every workgroup forms its ssm_out rows from all of them) against the
oracle bit for bit: a whole DeltaNet layer at the 9B widths with a 2048-wide FFN, run twice in a row (the exchange
counters are clear again after each launch), with one and two layers per list, Q4_0 and Q8_0 ssm_out, the sum
written apart from its residual or over it (as the decoder does); without the flag, or with the sum partly over its
residual, or over the output gate the step reads, the same layer runs unfused with the same bits. A wait for the heads that runs out of polls latches the
context."""
import os
import subprocess
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

E, HK, HV, S, F = 4096, 16, 32, 128, 2048
CH = 2 * HK * S + HV * S
EPS = 1e-6


def assert_bits(got, want, what=""):
    got, want = np.asarray(got, np.float32), np.asarray(want, np.float32)
    bad = np.nonzero(got.view(np.uint32) != want.view(np.uint32))[0]
    assert bad.size == 0, f"{what}: {bad.size}/{want.size} differ; first {bad[:4]}: got {got[bad[:4]]} want {want[bad[:4]]}"


class Layer:
    """One DeltaNet layer's tensors (seeded by `seed`) and its place in the act buffer."""

    def __init__(self, gq, seed, wtype, base, e=E, hk=HK, hv=HV, f=F):
        self.wtype = wtype
        self.e, self.hk, self.hv, self.f, self.ch = e, hk, hv, f, 2 * hk * S + hv * S
        E, HK, HV, F, CH = e, hk, hv, f, self.ch  # noqa: N806 (this layer's widths)
        self.Wqkv, self.Wz = gq.matrix(2, CH, E, seed, 3), gq.matrix(2, HV * S, E, seed, 4)
        self.Wb, self.Wa = gq.matrix(2, HV, E, seed, 5), gq.matrix(2, HV, E, seed, 6)
        self.Wo = gq.matrix(wtype, E, HV * S, seed, 7)
        self.Wg, self.Wu, self.Wd = gq.matrix(2, F, E, seed, 8), gq.matrix(2, F, E, seed, 9), gq.matrix(2, E, F, seed, 10)
        self.nw, self.pw = gq.uniform(seed, 11, E, 0.5, 1.5), gq.uniform(seed, 12, E, 0.5, 1.5)
        self.cw, self.cst = gq.normal(seed, 13, 4 * CH, std=0.5), gq.normal(seed, 14, 3 * CH)
        self.dt, self.a = gq.normal(seed, 15, HV), -np.abs(gq.normal(seed, 16, HV))
        self.sw = gq.uniform(seed, 17, S, 0.5, 1.5)
        self.state = gq.normal(seed, 18, HV * S * S) * 0.1
        names = ["nw", "pw", "xn", "qkv", "cqkv", "z", "ba", "y", "cw", "cst", "dt", "a", "sw", "tmp", "ffn", "h2"]
        sizes = [E, E, E, CH, CH, HV * S, 64, HV * S, 4 * CH, 3 * CH, 64, 64, S, E, F, E]
        self.O = {}
        off = base
        for nm, sz in zip(names, sizes):
            self.O[nm] = off
            off += (sz + 15) // 16 * 16
        self.end = off

    def upload(self, ctx, row):
        E, HK, HV, F, CH = self.e, self.hk, self.hv, self.f, self.ch  # noqa: N806
        O = self.O
        self.w = [ctx.upload(t, r, c, w) for t, r, c, w in
                  ((2, CH, E, self.Wqkv), (2, HV * S, E, self.Wz), (2, HV, E, self.Wb), (2, HV, E, self.Wa),
                   (self.wtype, E, HV * S, self.Wo), (2, F, E, self.Wg), (2, F, E, self.Wu), (2, E, F, self.Wd))]
        for k_, v_ in dict(nw=self.nw, pw=self.pw, cw=self.cw, cst=self.cst, dt=self.dt, a=self.a, sw=self.sw).items():
            ctx.write(O[k_], v_)
        ctx.state_write(row, self.state)
        self.row = row

    def commands(self, gq, x, with_out=True):
        E, HK, HV, F, CH = self.e, self.hk, self.hv, self.f, self.ch  # noqa: N806
        O, w = self.O, self.w
        flags = gq.GDN_L2_QK | gq.GDN_GATED | gq.GDN_GATES | gq.GDN_Z_SILU | (gq.GDN_WITH_OUT if with_out else 0)
        return (gq.rmsnorm(E, x, O["nw"], O["xn"], EPS, flags=gq.NORM_DEFER) +
                gq.gemv(2, CH, E, w[0], O["xn"], O["qkv"], gq.GEMV_CONV) +
                gq.conv(CH, O["qkv"], O["cw"], O["cqkv"], O["cst"], O["cst"]) +
                gq.gemv(2, HV * S, E, w[1], O["xn"], O["z"], gq.GEMV_SILU) +
                gq.gemv(2, HV, E, w[2], O["xn"], O["ba"]) + gq.gemv(2, HV, E, w[3], O["xn"], O["ba"] + 32) +
                gq.gdn(HV, HK, O["cqkv"], O["cqkv"] + HK * S, O["cqkv"] + 2 * HK * S, O["ba"] + 32, O["ba"], O["y"],
                       self.row, self.row, 1 / np.sqrt(S), flags, EPS, EPS, O["sw"], O["z"], O["dt"], O["a"]) +
                gq.gemv(self.wtype, E, HV * S, w[4], O["y"], O["tmp"], gq.GEMV_ADD) + gq.add(E, O["tmp"], x, O["h2"]) +
                gq.rmsnorm(E, O["h2"], O["pw"], O["xn"], EPS, flags=gq.NORM_DEFER) +
                gq.gemv(2, F, E, w[5], O["xn"], O["ffn"], gq.GEMV_SWIGLU) + gq.gemv(2, F, E, w[6], O["xn"], O["ffn"]) +
                gq.gemv(2, E, F, w[7], O["ffn"], O["tmp"], gq.GEMV_ADD) + gq.add(E, O["tmp"], O["h2"], x))

    def oracle(self, orc, x, state, cst):
        """The layer in the oracle: (new x, new state, new conv state, gated y, ssm_out + residual)."""
        E, HK, HV, F, CH = self.e, self.hk, self.hv, self.f, self.ch  # noqa: N806
        flags = 2 | 4 | 8 | 32
        xn = orc.rownorm(x, self.nw, E, 1, EPS)
        yc, ns = orc.conv(cst, orc.fx_gemv(2, self.Wqkv, xn, CH, E), self.cw)
        z = orc.unary(orc.fx_gemv(2, self.Wz, xn, HV * S, E), 1)
        b, al = orc.fx_gemv(2, self.Wb, xn, HV, E), orc.fx_gemv(2, self.Wa, xn, HV, E)
        y, st = orc.gdn(state, yc[:HK * S], yc[HK * S:2 * HK * S], yc[2 * HK * S:], al, b, HV, HK, float(1 / np.sqrt(S)),
                        flags, self.dt, self.a, z, self.sw)
        h2 = orc.fx_gemv(self.wtype, self.Wo, y, E, HV * S) + x
        pn = orc.rownorm(h2, self.pw, E, 1, EPS)
        f = orc.silu_mul(orc.fx_gemv(2, self.Wg, pn, F, E), orc.fx_gemv(2, self.Wu, pn, F, E))
        return orc.fx_gemv(2, self.Wd, f, E, F) + h2, st, ns, y, h2


@pytest.mark.parametrize("wtype,n_layers", [(2, 1), (2, 2), (8, 1)])
def test_fused_deltanet_layers_match_oracle(gq, orc, wtype, n_layers):
    ctx = gq.Context(act_floats=1 << 19, weight_bytes=200 << 20, state_rows=2 * HV * 128)
    try:
        X = 0
        layers = []
        base = E
        for i in range(n_layers):
            L = Layer(gq, 20 + i, wtype, base)
            L.upload(ctx, i * HV * 128)
            layers.append(L)
            base = L.end
        cmds = sum((L.commands(gq, X) for L in layers), [])
        x = gq.normal(20, 1, E)
        ctx.write(X, x)
        states = [L.state for L in layers]
        csts = [L.cst for L in layers]
        for run in range(2):  # the exchange counters must be clear again after a launch
            print(f"[fused] {n_layers} layer(s), ssm_out type {wtype}, run {run}", flush=True)
            assert ctx.run(cmds) == 0, ctx.error()
            # per layer: the projection group, the fused step + ssm_out, the FFN pair, the down projection; an odd
            # number of fused launches ends with a fill of the first exchange counter slot
            assert ctx.launch_count() == 4 * n_layers + n_layers % 2
            for i, L in enumerate(layers):
                x, st, ns, y, h2 = L.oracle(orc, x, states[i], csts[i])
                states[i], csts[i] = st, ns
                assert_bits(ctx.state_read(L.row, HV * 128), st, f"run {run} layer {i} state")
                assert_bits(ctx.read(L.O["cst"], 3 * CH), ns, f"run {run} layer {i} conv state")
                assert_bits(ctx.read(L.O["y"], HV * S), y, f"run {run} layer {i} gated output")
                assert_bits(ctx.read(L.O["h2"], E), h2, f"run {run} layer {i} ssm_out + residual")
            assert_bits(ctx.read(X, E), x, f"run {run} layer output")
    finally:
        ctx.close()


@pytest.mark.parametrize("hv,hk,fused", [(12, 4, True), (8, 2, True), (6, 3, False)])
def test_fused_narrow_layers(gq, orc, hv, hk, fused):
    """Narrower layers (hidden 2048, FFN 1024): 12 and 8 value heads run the fused launch with fewer blocks per lane
    than its registers hold (the unused ones re-read a valid block and add nothing); 6 heads (not a multiple of 4)
    run unfused. Two runs in a row, bit for bit against the oracle; the launches' kernels show which form ran."""
    e, f = 2048, 1024
    ctx = gq.Context(act_floats=1 << 18, weight_bytes=64 << 20, state_rows=hv * 128)
    try:
        L = Layer(gq, 50 + hv, 2, e, e=e, hk=hk, hv=hv, f=f)
        L.upload(ctx, 0)
        cmds = L.commands(gq, 0)
        x = gq.normal(50, 1, e)
        ctx.write(0, x)
        state, cst = L.state, L.cst
        for run in range(2):
            print(f"[fused] narrow layer, {hv} value heads, run {run}", flush=True)
            assert ctx.run(cmds) == 0, ctx.error()
            x, state, cst, y, h2 = L.oracle(orc, x, state, cst)
            assert_bits(ctx.state_read(0, hv * 128), state, f"run {run} state")
            assert_bits(ctx.read(L.O["y"], hv * S), y, f"run {run} gated output")
            assert_bits(ctx.read(L.O["h2"], e), h2, f"run {run} ssm_out + residual")
            assert_bits(ctx.read(0, e), x, f"run {run} layer output")
        names = [st_["name"] for st_ in ctx.profile(np.array(cmds, np.uint32), 1)]
        assert any(nm.startswith("gdn_out_kernel") for nm in names) == fused, names
    finally:
        ctx.close()


@pytest.mark.parametrize("case", ["no_flag", "in_place", "over_z"])
def test_fused_and_unfused_forms(gq, orc, case):
    """Without GDN_WITH_OUT, or with ssm_out's residual sum written over the output gate z (which the step's gated
    norm reads), the unfused path runs; with the sum written over its own residual (the decoder's form) the fused
    launch runs. Either way the bits are the oracle's."""
    ctx = gq.Context(act_floats=1 << 19, weight_bytes=200 << 20, state_rows=HV * 128)
    try:
        L = Layer(gq, 30, 2, 2 * E)
        L.upload(ctx, 0)
        w = np.array(L.commands(gq, 0, with_out=case != "no_flag"), np.uint32).reshape(-1, 8)
        h2 = L.O["h2"]
        if case != "no_flag":
            h2 = 0 if case == "in_place" else L.O["z"]
            add = [i for i in range(len(w)) if w[i][0] == gq.OP_ADD][0]
            w[add][4] = h2  # the ssm_out sum over x, or over z
            w[add + 1][2] = h2  # the FFN norm reads it
            w[-1][3] = h2  # the down projection's residual is it
        x = gq.normal(30, 1, E)
        ctx.write(0, x)
        print(f"[fused] form {case}", flush=True)
        assert ctx.run(w.ravel().tolist()) == 0, ctx.error()
        xo, st, ns, y, h2v = L.oracle(orc, x, L.state, L.cst)
        assert_bits(ctx.read(0, E), xo, "layer output")
        assert_bits(ctx.state_read(0, HV * 128), st, "state")
        assert_bits(ctx.read(L.O["y"], HV * S), y, "gated output")
        if case == "no_flag":
            assert_bits(ctx.read(L.O["h2"], E), h2v, "ssm_out + residual")
        # which form ran: the launches' kernels (one more pass of the list; its results are not checked)
        names = [st_["name"] for st_ in ctx.profile(w.ravel(), 1)]
        assert any(nm.startswith("gdn_out_kernel") for nm in names) == (case == "in_place"), names
    finally:
        ctx.close()


_OUT_OF_POLLS = r"""
import sys
sys.path.insert(0, sys.argv[1])
sys.path.insert(0, sys.argv[2])
import numpy as np
import gemvq as gq
import test_gpu_fused as T
ctx = gq.Context(act_floats=1 << 19, weight_bytes=200 << 20, state_rows=T.HV * 128)
L = T.Layer(gq, 40, 2, T.E)
L.upload(ctx, 0)
ctx.write(0, gq.normal(40, 1, T.E))
try:
    ctx.run(L.commands(gq, 0))
    print("no error")
except gq.GemvqError as e:
    print("error:", e)
print("usable", ctx.usable())
ctx.close()
"""


def test_exchange_wait_out_of_polls_latches_the_context(tmp_path):
    """With the in-kernel wait bounded at 0 polls (GEMVQ_EXCHANGE_POLLS, read when a context is created) every
    workgroup of the fused launch gives up at once: the launch still ends normally, the fault word makes the run
    return GEMVQ_ETIMEDOUT and the context unusable. Run in a child process so the setting stays out of this one."""
    here = os.path.dirname(os.path.abspath(__file__))
    pkg = os.path.join(os.path.dirname(here), "fpga-llama-gguf_amd")
    env = dict(os.environ, GEMVQ_EXCHANGE_POLLS="0")
    print("[fused] exchange wait bounded at 0 polls (child process)", flush=True)
    r = subprocess.run([sys.executable, "-c", _OUT_OF_POLLS, pkg, here], env=env, capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "ran out of polls" in r.stdout and "usable False" in r.stdout, r.stdout
