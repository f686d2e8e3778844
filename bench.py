#!/usr/bin/env python3
"""Decode benchmark: batch-1 greedy decode of the synthetic Qwen3.5-9B-shaped Q4_0 model on one MI355X.

Workload: 32 layers (24 Gated DeltaNet + 8 gated attention, 3:1), hidden 4096, FFN 12288, vocab 151936, layer
matrices Q4_0 N(0, 0.02^2), embedding and head Q6_K, norms fp32 ones; prompt of 512 random ids (run as decode steps,
then again, after a reset, as a batched prefill; both rates are reported, neither is `value`), then `--warmup`
untimed and `--steps` timed greedy decode steps (one hipGraph replay each, tokens fed back on the device). value = timed tokens / wall time between two stream synchronizations.

roofline: the dominant kernel (largest share of a token's device time), its algorithmic bytes (GGUF weights +
fp32 vectors read and written once + state/KV traffic) over its measured duration, from device start/stop events
of every kernel of one token (gemvq_profile, the median over --profile-reps repetitions). cpu_baseline: the oracle decoder in the reference's CPU arithmetic
(gemvq_ref.h: int8 block dots, here in AVX2, each row summed sequentially in FP32, double sums of squares) on the
host, one thread per physical core, for up to 15 s (160 steps) of decode steps at the positions of the first timed GPU steps;
the JSON names the CPU model, sockets, cores and SIMD extensions.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "fpga-llama-gguf_amd"))

import numpy as np  # noqa: E402

import gemvq as gq  # noqa: E402
import qwen35 as Q  # noqa: E402

METRIC = "decode tokens/s (9B-shape Q4_0, batch 1); GEMV HBM GB/s vs 8 TB/s peak"
HBM_PEAK_GBPS = 8000.0


def measured_traffic(kernel: str) -> tuple[int | None, str | None]:
    """HBM bytes per launch of `kernel` from the committed rocprofv3 --pmc summary (FETCH_SIZE + WRITE_SIZE, each
    scaled by the same counter on a copy kernel of known size), if that kernel was measured."""
    path = os.path.join(ROOT, "profiles", "c5_decode_pmc.md")
    if not os.path.exists(path):
        return None, None
    for line in open(path):
        parts = line.split()
        if len(parts) == 3 and parts[0] == "traffic_bytes_per_launch" and parts[1] == kernel:
            return int(float(parts[2])), os.path.relpath(path, ROOT)
    return None, None


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def profile(ctx: gq.Context, cmds: np.ndarray, reps: int) -> list[dict]:
    return ctx.profile(np.ascontiguousarray(cmds.ravel(), np.uint32), reps)


def cpu_info() -> dict:
    """The host CPU as lscpu reports it: model, sockets, physical cores, logical CPUs and the SIMD extensions."""
    info, procs = {}, []
    try:
        with open("/proc/cpuinfo") as f:
            cur = {}
            for line in f:
                if not line.strip():
                    if cur:
                        procs.append(cur)
                    cur = {}
                    continue
                k, _, v = line.partition(":")
                cur[k.strip()] = v.strip()
            if cur:
                procs.append(cur)
    except OSError:
        pass
    if procs:
        flags = set(procs[0].get("flags", "").split())
        info["model"] = procs[0].get("model name", "")
        info["sockets"] = len({p.get("physical id", "0") for p in procs})
        info["physical_cores"] = len({(p.get("physical id", "0"), p.get("core id", str(i))) for i, p in enumerate(procs)})
        info["logical_cpus"] = len(procs)
        info["simd"] = [x for x in ("sse4_2", "avx2", "fma", "avx512f", "avx512bw", "avx512_vnni", "avx_vnni", "amx_int8")
                        if x in flags]
    info["allowed_cpus"] = len(os.sched_getaffinity(0))
    return info


def one_cpu_per_core(n: int) -> list[int]:
    """Up to n of this process's allowed logical CPUs, the first of each physical core (sibling threads skipped)."""
    seen, out = set(), []
    for c in sorted(os.sched_getaffinity(0)):
        try:
            base = f"/sys/devices/system/cpu/cpu{c}/topology/"
            core = (open(base + "physical_package_id").read().strip(), open(base + "core_id").read().strip())
        except OSError:
            core = ("?", str(c))
        if core in seen:
            continue
        seen.add(core)
        out.append(c)
        if len(out) == n:
            break
    return out


def simd_name(oracle) -> str:
    """The fast rows' SIMD level on this host (AVX-512 VNNI for Q4_0 / Q4_1 / Q8_0 block sums where the CPU has it)."""
    return ("AVX-512 VNNI (Q4_0 / Q4_1 / Q8_0 blocks, 16 at a time) and AVX2 (Q6_K)"
            if oracle.orc().orc_fast_simd() == oracle.SIMD_AVX512_VNNI else "AVX2")


def pin_openmp(cpus: list[int]) -> None:
    """One OpenMP thread per listed CPU, bound in order (the oracle's runtime reads these when it loads)."""
    os.environ["OMP_PLACES"] = ",".join(f"{{{c}}}" for c in cpus)
    os.environ["OMP_PROC_BIND"] = "close"


def cpu_baseline(blob, cfg, tokens, pos0: int, max_tokens: int, seconds: float, threads: int) -> dict:
    """The oracle decoder in the reference's CPU arithmetic on the host: decode steps at the positions (and with the
    token ids) of the first timed GPU steps, until `seconds` have passed or max_tokens steps ran."""
    cpus = one_cpu_per_core(threads)
    pin_openmp(cpus)
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle  # noqa: E402  (the CPU baseline leg only)

    old = os.sched_getaffinity(0)
    os.sched_setaffinity(0, cpus)
    try:
        om = oracle.Model(Q.config_c(cfg), blob.table, blob.n, blob.data, threads=len(cpus), mode=oracle.MODE_REFERENCE)
        om.decode(int(tokens[0]), pos0)  # first touch of the weights and the thread pool, untimed
        max_tokens = min(max_tokens, len(tokens) - 1)
        n, t0 = 0, time.perf_counter()
        while n < max_tokens and (n < 2 or time.perf_counter() - t0 < seconds):
            om.decode(int(tokens[n + 1]), pos0 + 1 + n)
            n += 1
        dt = time.perf_counter() - t0
        om.close()
    finally:
        os.sched_setaffinity(0, old)
    return {"value": round(n / dt, 4), "unit": "tokens/s", "cores": len(cpus), "kind": "port",
            "arithmetic": "the reference's CPU arithmetic (gemvq_ref.h: int8 block dot products, each row summed "
                          "sequentially in FP32, sums of squares in double; exp / log correctly rounded, as the "
                          "GPU's reference mode evaluates them); the int8 dots in " + simd_name(oracle),
            "cpu": cpu_info(),
            "sample": f"{n} decode steps of the same 9B-shape model at positions {pos0 + 1}..{pos0 + n} with the ids "
                      f"the GPU generated there, from an empty state (a step's work depends on its position, not on "
                      f"the state); rows split over {len(cpus)} threads, one per physical core (CPUs {cpus[0]}.."
                      f"{cpus[-1]}); {dt:.1f} s"}


def copy_probe(mib: int) -> int:
    """y = -x over mib MiB of float32: an element-wise kernel that reads and writes exactly mib MiB each."""
    import torch

    n = mib * (1 << 20) // 4
    x = torch.ones(n, dtype=torch.float32, device="cuda")
    y = torch.empty_like(x)
    for _ in range(5):
        torch.neg(x, out=y)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes_read": n * 4, "copy_probe_bytes_written": n * 4, "launches": 5}), flush=True)
    return 0


# ---------------------------------------------------------------------------------------------------------------
# C1-C4: the single-op configurations, each timed over rotated weight copies (>= 512 MB, twice the 256 MB
# memory-side cache) inside one graph, and as single launches; the oracle on the host on the same bytes.
def _cfg_units(threads: int = 1, seed: int = 0):
    """[(name, description, algorithmic bytes per unit, rotated copies, setup(ctx) -> builder(copy) -> commands,
    cpu(oracle) -> (function, args[, scale]))]."""
    units = []

    # C1: Q4_0 GEMV [9728 x 2560], x ~ N(0, 1) quantized to Q8_0 on the GPU
    R1, K1 = 9728, 2560
    w1 = gq.matrix(gq.Q4_0, R1, K1, seed, 1)
    x1 = gq.normal(seed, 2, K1)

    C1_COPIES = 40

    def c1(ctx):
        offs = [ctx.upload(gq.Q4_0, R1, K1, w1) for _ in range(C1_COPIES)]
        ctx.write(0, x1)
        ctx.write(16384, x1)  # consecutive copies read different (equal) x: each is its own launch, not a group
        return lambda i: gq.gemv(gq.Q4_0, R1, K1, offs[i], 16384 * (i & 1), 4096)
    units.append(("C1", "Q4_0 GEMV 9728x2560", w1.size + 4 * K1 + 4 * R1, C1_COPIES, c1,
                  lambda orc: (orc.fast_gemv, (1, gq.Q4_0, w1, x1, R1, K1, threads))))

    # C2: norm + SwiGLU gate/up (Q8_0 [9728 x 2560] x 2) + down (Q8_0 [2560 x 9728]) + residual
    E, F = 2560, 9728
    wg, wu = gq.matrix(gq.Q8_0, F, E, seed, 3), gq.matrix(gq.Q8_0, F, E, seed, 4)
    wd = gq.matrix(gq.Q8_0, E, F, seed, 5)
    x2, r2, nw2 = gq.normal(seed, 6, E), gq.normal(seed, 7, E), gq.uniform(seed, 8, E, 0.5, 1.5)
    C2_COPIES = 8

    def c2(ctx):
        offs = [(ctx.upload(gq.Q8_0, F, E, wg), ctx.upload(gq.Q8_0, F, E, wu), ctx.upload(gq.Q8_0, E, F, wd))
                for _ in range(C2_COPIES)]
        ctx.write(0, x2)
        ctx.write(4096, r2)
        ctx.write(8192, nw2)
        X, XN, ACT, T, Y = 0, 12288, 16384, 32768, 36864
        return lambda i: (gq.rmsnorm(E, X, 8192, XN, 1e-6, flags=gq.NORM_DEFER) +
                          gq.gemv(gq.Q8_0, F, E, offs[i][0], XN, ACT, gq.GEMV_SWIGLU) +
                          gq.gemv(gq.Q8_0, F, E, offs[i][1], XN, ACT) +
                          gq.gemv(gq.Q8_0, E, F, offs[i][2], ACT, T, gq.GEMV_ADD) + gq.add(E, T, 4096, Y))

    def c2_cpu(orc):
        def run():
            xn = orc.rownorm(x2, nw2, E, 1, 1e-6)
            act = orc.silu_mul(orc.fast_gemv(1, gq.Q8_0, wg, xn, F, E, threads),
                               orc.fast_gemv(1, gq.Q8_0, wu, xn, F, E, threads))
            return orc.fast_gemv(1, gq.Q8_0, wd, act, E, F, threads) + r2
        return run, ()

    units.append(("C2", "RMSNorm + Q8_0 SwiGLU gate/up 2x9728x2560 + down 2560x9728 + residual",
                  wg.size + wu.size + wd.size + 4 * 4 * E, C2_COPIES, c2, c2_cpu))

    # C3: Q6_K head [151936 x 4096] and Q5_K [12288 x 4096], x quantized to Q8_K
    V, D3 = 151936, 4096
    wh = gq.matrix(gq.Q6_K, V, D3, seed, 9)
    w5 = gq.matrix(gq.Q5_K, 12288, D3, seed, 10)
    x3 = gq.normal(seed, 11, D3)

    def c3h(ctx):
        offs = [ctx.upload(gq.Q6_K, V, D3, wh) for _ in range(2)]
        ctx.write(0, x3)
        ctx.write(4096, x3)
        return lambda i: gq.gemv(gq.Q6_K, V, D3, offs[i], 4096 * (i & 1), 8192)

    def c35(ctx):
        offs = [ctx.upload(gq.Q5_K, 12288, D3, w5) for _ in range(16)]
        ctx.write(0, x3)
        ctx.write(4096, x3)
        return lambda i: gq.gemv(gq.Q5_K, 12288, D3, offs[i], 4096 * (i & 1), 8192)

    sl = 16384  # the CPU times a row slice of the head and scales it
    units.append(("C3 head", "Q6_K GEMV 151936x4096", wh.size + 4 * D3 + 4 * V, 2, c3h,
                  lambda orc: (orc.fast_gemv, (1, gq.Q6_K, wh[:sl * gq.row_bytes(gq.Q6_K, D3)], x3, sl, D3, threads),
                               V / sl)))
    units.append(("C3 Q5_K", "Q5_K GEMV 12288x4096", w5.size + 4 * D3 + 4 * 12288, 16, c35,
                  lambda orc: (orc.fast_gemv, (1, gq.Q5_K, w5, x3, 12288, D3, threads))))

    # C4: conv over 8192 channels (3x8192 cache, 4x8192 kernel), the GDN step (32 value / 16 key heads, L2 q/k,
    # gates, gated norm) and ssm_out Q4_0 [4096 x 4096] + residual
    Hk, Hv, S = 16, 32, 128
    ch = 2 * Hk * S + Hv * S
    wo = gq.matrix(gq.Q4_0, 4096, Hv * S, seed, 12)
    qkv, cw, cst = gq.normal(seed, 13, ch), gq.normal(seed, 14, 4 * ch, std=0.5), gq.normal(seed, 15, 3 * ch)
    z, ba = gq.normal(seed, 16, Hv * S), gq.normal(seed, 17, 2 * Hv)
    dt, av, sw = gq.normal(seed, 18, Hv), -np.abs(gq.normal(seed, 19, Hv)), gq.uniform(seed, 20, S, 0.5, 1.5)
    state = gq.normal(seed, 21, Hv * S * S) * 0.1
    C4_COPIES = 48
    O = dict(qkv=0, cqkv=8192, z=16384, ba=20480, y=20544, dt=24640, a=24704, sw=24768, x=24896, out=28992,
             res=33088, cw=37184, cst=69952)

    def c4(ctx):
        offs = [ctx.upload(gq.Q4_0, 4096, Hv * S, wo) for _ in range(C4_COPIES)]
        for k_, v_ in dict(qkv=qkv, cw=cw, z=z, ba=ba, dt=dt, a=av, sw=sw, x=gq.normal(seed, 22, 4096)).items():
            ctx.write(O[k_], v_)
        for i in range(C4_COPIES):
            ctx.write(O["cst"] + 3 * ch * i, cst)
            ctx.state_write(i * Hv * S, state)
        flags = gq.GDN_L2_QK | gq.GDN_GATED | gq.GDN_GATES

        def cmds(i):
            st = O["cst"] + 3 * ch * i
            return (gq.conv(ch, O["qkv"], O["cw"], O["cqkv"], st, st) +
                    gq.gdn(Hv, Hk, O["cqkv"], O["cqkv"] + Hk * S, O["cqkv"] + 2 * Hk * S, O["ba"] + Hv, O["ba"],
                           O["y"], i * Hv * S, i * Hv * S, 1 / np.sqrt(S), flags, 1e-6, 1e-6, O["sw"], O["z"], O["dt"],
                           O["a"]) +
                    gq.gemv(gq.Q4_0, 4096, Hv * S, offs[i], O["y"], O["out"], gq.GEMV_ADD) +
                    gq.add(4096, O["out"], O["x"], O["res"]))
        return cmds

    def c4_cpu(orc):
        def run():
            yc, _ = orc.conv(cst, qkv, cw)
            y, _ = orc.gdn(state, yc[:Hk * S], yc[Hk * S:2 * Hk * S], yc[2 * Hk * S:], ba[Hv:], ba[:Hv], Hv, Hk,
                           float(1 / np.sqrt(S)), gq.GDN_L2_QK | gq.GDN_GATED | gq.GDN_GATES, dt, av, z, sw)
            return orc.fast_gemv(1, gq.Q4_0, wo, y, 4096, Hv * S, threads)
        return run, ()

    units.append(("C4", "conv 8192 ch + GDN step (32 heads) + gated norm + ssm_out Q4_0 4096x4096 + residual",
                  wo.size + 2 * Hv * S * S * 4 + 2 * 3 * ch * 4 + 4 * ch * 4 + 4 * 4096 * 3, C4_COPIES, c4, c4_cpu))
    return units


CPU_REPS = 15  # cold-cache calls per unit on the CPU; the median is reported
CPU_FLUSH_BYTES = 1 << 30  # read between calls, larger than any host's last-level cache


def configs(args) -> int:
    cpus = one_cpu_per_core(args.threads)
    pin_openmp(cpus)
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle  # noqa: E402  (the CPU baseline only)

    # evicting reads by the oracle's own thread team on the same cores (each core complex has its own last-level
    # cache): one multithreaded GEMV over a matrix larger than the host's caches
    fl_rows = CPU_FLUSH_BYTES // gq.row_bytes(gq.Q4_0, 4096)
    fl_w = np.full(fl_rows * gq.row_bytes(gq.Q4_0, 4096), 0x11, np.uint8)  # blocks of d = fp16 0x1111, quants 1
    fl_x = gq.normal(1, 98, 4096)
    for name, desc, nbytes, copies, setup, cpu in _cfg_units(len(cpus)):
        ctx = gq.Context(act_floats=1 << 21, weight_bytes=1_100_000_000, state_rows=48 * 32 * 128)
        build = setup(ctx)
        cmds = sum((build(i) for i in range(copies)), [])
        g = ctx.graph(cmds)
        launches = ctx.launch_count()  # of the graph's list
        ctx.replay(g, 2)
        ctx.sync()
        t_graph = ctx.graph_time_us(g, 5) / copies
        stats = profile(ctx, np.array(build(0), np.uint32), args.profile_reps)
        assert launches == copies * len(stats), (name, launches, copies, len(stats))  # no launch spans two copies
        t_single = sum(s["us"] for s in stats)
        ctx.close()
        spec = cpu(oracle)
        fn, fargs = spec[0], spec[1]
        scale = spec[2] if len(spec) > 2 else 1.0
        old = os.sched_getaffinity(0)
        os.sched_setaffinity(0, cpus)
        try:
            fn(*fargs)
            times = []
            for _ in range(CPU_REPS):
                oracle.fast_gemv(1, gq.Q4_0, fl_w, fl_x, fl_rows, 4096, len(cpus))  # untimed: evicts the unit's bytes
                t0 = time.perf_counter()
                fn(*fargs)
                times.append(time.perf_counter() - t0)
            t_cpu = float(np.median(times)) * scale
        finally:
            os.sched_setaffinity(0, old)
        line = {"config": name, "what": desc, "algorithmic_bytes": nbytes, "copies_rotated": copies,
                "graph_us_per_unit": round(t_graph, 3), "graph_launches_per_unit": launches / copies,
                "graph_GBps": round(nbytes / t_graph / 1e3, 1),
                "graph_frac_of_8TBps": round(nbytes / t_graph / 1e3 / HBM_PEAK_GBPS, 4),
                "single_launch_device_us": round(t_single, 3), "launches_per_unit": len(stats),
                "cpu_oracle_s": round(t_cpu, 4), "cpu_GBps": round(nbytes / t_cpu / 1e9, 2),
                "cpu_kind": f"port (the oracle in the reference's CPU arithmetic: GEMV rows summed sequentially in "
                            f"FP32, int8 dots in {simd_name(oracle)}; rows split over {len(cpus)} threads, one per "
                            f"physical core, CPUs {cpus[0]}..{cpus[-1]}; median of {CPU_REPS} calls, each after reading "
                            f"{CPU_FLUSH_BYTES >> 20} MiB (a GEMV on the same threads) to evict the unit's bytes "
                            f"from the caches)",
                "cpu_cores": len(cpus)}
        print(json.dumps(line), flush=True)
    return 0


# ---------------------------------------------------------------------------------------------------------------
# The batched GEMV (GEMM command) on the C5 layer shapes: M tokens per weight read, over rotated weight copies
# (>= 512 MB) in one graph, against M single-token GEMVs of the same rows.
def sequences(args) -> int:
    """Lockstep decode of n sequences of the C5 model (gemvq_qwen35_batch_*): aggregate tokens/s over all of them.
    Each sequence starts from its own 16-id prompt (consumed by the same steps); timed: --steps steps after the
    prompts, every step one token per sequence. One JSON line per sequence count."""
    counts = [int(v) for v in args.sequences.split(",")]
    cfg = Q.Config(n_layer=args.layers, n_ctx=16 + args.warmup + args.steps + 8)
    t = time.perf_counter()
    blob = Q.generate(cfg, seed=0, threads=args.threads)
    log(f"generated the synthetic model ({blob.data.size / 1e9:.2f} GB) in {time.perf_counter() - t:.1f} s")
    wbytes = Q.weight_bytes(cfg)
    for n in counts:
        prompts = [Q.prompt_ids(cfg, 16, seed=100 + s) for s in range(n)]
        with Q.BatchModel(blob, n) as bm:
            bm.reset(prompts)
            bm.step(15 + args.warmup)  # the prompts, then the untimed steps (captures the graph)
            bm.sync()
            t0 = time.perf_counter()
            bm.step(args.steps)
            bm.sync()
            dt = time.perf_counter() - t0
            launches = bm.ctx.launch_count()
        tok_s = n * args.steps / dt
        print(json.dumps({"sequences_decode": n, "tokens_per_s": round(tok_s, 1), "steps": args.steps,
                          "ms_per_step": round(dt * 1e3 / args.steps, 4), "launches_per_step": launches,
                          "weight_GBps_per_step": round(wbytes / (dt / args.steps) / 1e9, 1),
                          "workload": "C5 model (32 layers, Q4_0 layers, Q6_K head: one GEMV per sequence), "
                                      "16-id prompts then timed lockstep steps", "data": "synthetic"}), flush=True)
        log(f"{n} sequences: {tok_s:.1f} tokens/s aggregate ({dt * 1e3 / args.steps:.3f} ms per step)")
    return 0


def batched(args) -> int:
    shapes = [("FFN gate/up pair 2x12288x4096 (+ norm)", 12288, 4096, True),
              ("FFN down 4096x12288 (+ residual)", 4096, 12288, False),
              ("DeltaNet q/k/v 8192x4096", 8192, 4096, False)]
    for name, R, K, pair in shapes:
        w = gq.matrix(gq.Q4_0, R, K, 0, 90 + R % 7, std=0.02)
        mats = 2 if pair else 1
        per = w.size * mats
        copies = max(2, int(np.ceil(520e6 / per)))
        ctx = gq.Context(act_floats=1 << 22, weight_bytes=per * copies + (1 << 20))
        offs = [[ctx.upload(gq.Q4_0, R, K, w) for _ in range(mats)] for _ in range(copies)]
        # 32 rows of up to 12288 floats each; consecutive copies read X and X2 (equal rows) in turn, so no GEMV
        # group or reused quantization spans two copies
        X, X2, NW, Y, YG, RES = 0, 1 << 19, 15 << 16, 1 << 20, 3 << 19, 1 << 21
        xs = gq.normal(0, 91, 32 * K)
        ctx.write(X, xs)
        ctx.write(X2, xs)
        ctx.write(NW, gq.uniform(0, 92, K, 0.5, 1.5))
        ctx.write(RES, gq.normal(0, 93, 32 * R))
        norm = dict(norm_w=NW, eps=1e-6, norm_flags=gq.NORM_DEFER) if pair else {}

        def unit(o, m, x):
            if pair:
                return (gq.gemm(gq.Q4_0, R, K, o[0], x, YG, m, K, R, gq.GEMV_SWIGLU, **norm) +
                        gq.gemm(gq.Q4_0, R, K, o[1], x, Y, m, K, R, **norm))
            if K == 12288:
                return gq.gemm(gq.Q4_0, R, K, o[0], x, Y, m, K, R, gq.GEMV_ADD, RES, R)
            return gq.gemm(gq.Q4_0, R, K, o[0], x, Y, m, K, R)

        def single(o, x):
            if pair:
                return (gq.rmsnorm(K, x, NW, YG, 1e-6, flags=gq.NORM_DEFER) + gq.gemv(gq.Q4_0, R, K, o[0], YG, Y, gq.GEMV_SWIGLU) +
                        gq.gemv(gq.Q4_0, R, K, o[1], YG, Y))
            if K == 12288:
                return gq.gemv(gq.Q4_0, R, K, o[0], x, Y, gq.GEMV_ADD) + gq.add(R, Y, RES, Y)
            return gq.gemv(gq.Q4_0, R, K, o[0], x, Y)

        g1 = ctx.graph(sum((single(o, (X, X2)[i & 1]) for i, o in enumerate(offs)), []))
        l1 = ctx.launch_count() / copies
        ctx.replay(g1, 2)
        t1 = ctx.graph_time_us(g1, 5) / copies
        for m in (1, 2, 4, 8, 16, 32):
            g = ctx.graph(sum((unit(o, m, (X, X2)[i & 1]) for i, o in enumerate(offs)), []))
            lm = ctx.launch_count() / copies
            ctx.replay(g, 2)
            t = ctx.graph_time_us(g, 5) / copies
            ops = 2.0 * R * K * m * mats
            print(json.dumps({"batched": name, "tokens": m, "us_per_copy": round(t, 3), "launches_per_copy": lm,
                              "weight_GBps": round(per / t / 1e3, 1), "token_rows_per_us": round(m / t, 3),
                              "int8_TOPs": round(ops / t / 1e6, 2), "vs_single_token": round(m * t1 / t, 2),
                              "single_token_us": round(t1, 3), "single_token_launches": l1,
                              "copies_rotated": copies}), flush=True)
        ctx.close()
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128, help="timed decode steps (tokens)")
    ap.add_argument("--warmup", type=int, default=0, help="untimed decode steps after the prompt")
    ap.add_argument("--prompt", type=int, default=512, help="prompt length (outside the timed steps)")
    ap.add_argument("--cpu-tokens", type=int, default=160, help="most decode steps timed for the CPU baseline (0: skip)")
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="time the CPU baseline samples for")
    ap.add_argument("--threads", type=int, default=min(16, os.cpu_count() or 1))
    ap.add_argument("--profile-reps", type=int, default=9,
                    help="repetitions of the per-kernel pass (each launch's median duration is reported)")
    ap.add_argument("--ref-steps", type=int, default=32,
                    help="decode steps timed in the reference arithmetic after the profile (0: skip)")
    ap.add_argument("--layers", type=int, default=32, help="(testing) fewer layers; the reported line is then invalid")
    ap.add_argument("--reference", action="store_true",
                    help="(profiling) run the prompt, the timed steps and the per-kernel pass in the reference "
                         "arithmetic (gemvq_set_arith); the line then reports that mode's rate, not the headline one")
    ap.add_argument("--direct", action="store_true",
                    help="plain stream launches instead of graph replays (for tracing tools); slower per step")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy kernel of MIB MiB 5 times (calibrates the HBM byte counters "
                         "of rocprofv3 --pmc) and exit")
    ap.add_argument("--configs", action="store_true",
                    help="only time the single-op configurations C1-C4 (one JSON line each) and exit")
    ap.add_argument("--batched", action="store_true",
                    help="only time the batched GEMV on the C5 layer shapes at 1..32 tokens and exit")
    ap.add_argument("--sequences", default="", metavar="N[,N...]",
                    help="only time lockstep decode of N sequences of the C5 model (aggregate tokens/s) and exit")
    args = ap.parse_args()
    if args.sequences:
        return sequences(args)
    if args.batched:
        return batched(args)
    if args.copy_probe:
        return copy_probe(args.copy_probe)
    if args.configs:
        return configs(args)
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              f"(the multi-GPU sharding is a design note, not code)", file=sys.stderr)
        return 2

    slack = args.profile_reps + args.ref_steps + 20
    cfg = Q.Config(n_layer=args.layers, n_ctx=args.prompt + args.warmup + args.steps + slack)
    t = time.perf_counter()
    blob = Q.generate(cfg, seed=0, threads=args.threads)
    log(f"generated the synthetic model ({blob.data.size / 1e9:.2f} GB) in {time.perf_counter() - t:.1f} s")
    prompt = Q.prompt_ids(cfg, args.prompt + 1)
    wbytes = Q.weight_bytes(cfg)

    t = time.perf_counter()
    m = Q.Model(blob)
    if args.reference:
        m.set_arith(gq.ARITH_REFERENCE)
    log(f"uploaded and captured the per-token graph in {time.perf_counter() - t:.1f} s "
        f"({len(m.commands())} commands, weight bytes per token {wbytes})")
    m.reset(prompt[:args.prompt])
    step = m.step_direct if args.direct else m.step
    t = time.perf_counter()
    step(args.prompt - 1)
    m.sync()
    t_steps = time.perf_counter() - t
    prefill = None
    if not args.direct and args.prompt > 1:  # the same prompt positions again, batched (bit-identical state)
        m.reset(prompt[:args.prompt])
        warm = m.prefill(min(32, args.prompt - 1))  # captures the full-chunk graph (once per model), untimed
        m.reset(prompt[:args.prompt])
        t = time.perf_counter()
        if warm and m.prefill(args.prompt - 1):
            m.sync()
            t_pre = time.perf_counter() - t
            prefill = {"positions": args.prompt - 1, "batched_tokens_per_s": round((args.prompt - 1) / t_pre, 1),
                       "decode_step_tokens_per_s": round((args.prompt - 1) / t_steps, 1),
                       "method": "chunks of 32 tokens: GEMM projections, conv and DeltaNet over the tokens in order, "
                                 "attention over the chunk's tokens in one launch pair; full chunks replay one "
                                 "captured graph (captured by an untimed first prefill); wall time of the whole "
                                 "prefill call"}
            log(f"prompt: {args.prompt - 1} positions batched in {t_pre:.3f} s ({prefill['batched_tokens_per_s']} tok/s) "
                f"vs {t_steps:.3f} s as decode steps")
        else:
            m.reset(prompt[:args.prompt])
            step(args.prompt - 1)
    t = time.perf_counter()
    step(args.warmup)
    m.sync()
    log(f"prompt ({args.prompt}) + warmup ({args.warmup}) steps in {t_steps + time.perf_counter() - t:.2f} s")
    try:
        import torch

        if torch.cuda.is_available():
            torch.cuda.synchronize()
    except Exception:
        pass

    t0 = time.perf_counter()
    step(args.steps)
    m.sync()
    t1 = time.perf_counter()
    dt = t1 - t0
    tok_s = args.steps / dt
    n_all = args.prompt + args.warmup + args.steps
    toks = m.tokens(n_all)
    gen = toks[args.prompt:]
    log(f"{args.steps} timed steps in {dt * 1e3:.2f} ms: {tok_s:.1f} tok/s, {wbytes * tok_s / 1e9:.1f} GB/s of weights; "
        f"generated ids {gen[:8].tolist()} ... ({len(set(gen.tolist()))} distinct)")

    # per-kernel device times of one token at the final position
    stats = profile(m.ctx, m.commands(), args.profile_reps)
    agg: dict[str, dict] = {}
    for s in stats:
        a = agg.setdefault(s["name"], {"us": 0.0, "bytes": 0, "n": 0})
        a["us"] += s["us"]
        a["bytes"] += s["bytes"]
        a["n"] += 1
    tot_us = sum(a["us"] for a in agg.values())
    for name, a in sorted(agg.items(), key=lambda kv: -kv[1]["us"]):
        log(f"  {name:28s} {a['n']:4d} launches {a['us']:9.1f} us ({100 * a['us'] / tot_us:5.1f} %) "
            f"{a['bytes'] / a['us'] / 1e3:8.1f} GB/s")
    dom_name, dom = max(agg.items(), key=lambda kv: kv[1]["us"])
    achieved = dom["bytes"] / dom["us"] / 1e3  # GB/s
    traffic, traffic_src = measured_traffic(dom_name)
    ref = None
    if args.ref_steps > 0 and not args.direct and not args.reference:
        # the same model continuing in the reference arithmetic (gemvq_set_arith): bit-identical to the reference's
        # CPU path, not the timed workload
        m.set_arith(gq.ARITH_REFERENCE)
        m.step(2)  # captures the graph
        m.sync()
        t = time.perf_counter()
        m.step(args.ref_steps)
        m.sync()
        t_ref = time.perf_counter() - t
        ref = {"tokens_per_s": round(args.ref_steps / t_ref, 1), "steps": args.ref_steps,
               "vs_canonical": round(args.ref_steps / t_ref / tok_s, 3),
               "what": "the same decode in the reference arithmetic (the reference CPU path's sequential FP32 rows, "
                       "double norm sums, in-order DeltaNet dots, double-sum attention, correctly rounded exp / "
                       "log; its tokens equal the CPU reference decoder's bit for bit), graph replays after the "
                       "profile pass"}
        log(f"reference arithmetic: {ref['tokens_per_s']} tok/s ({ref['vs_canonical']} of the canonical rate)")
    m.close()

    cpu = None
    if args.cpu_tokens > 0:
        t = time.perf_counter()
        cpu = cpu_baseline(blob, cfg, toks[args.prompt + args.warmup - 1:], args.prompt + args.warmup - 1,
                           args.cpu_tokens, args.cpu_seconds, args.threads)
        log(f"cpu baseline {cpu['value']} tok/s in {time.perf_counter() - t:.1f} s")

    line = {
        "metric": METRIC,
        "value": round(tok_s, 3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dt * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "launch": "direct" if args.direct else "graph",
        "data": "synthetic",
        "config": {
            "workload": (f"C5: greedy decode of the random-init Qwen3.5-9B-shaped hybrid ({cfg.n_layer} layers, 3:1 "
                         f"Gated DeltaNet:attention, hidden 4096, FFN 12288, vocab 151936, Q4_0 layers, Q6_K "
                         f"embedding/head), prompt {args.prompt} random ids then {args.steps} timed tokens, "
                         f"context to {n_all}"),
            "weight_bytes_per_token": wbytes,
            "weight_GBps": round(wbytes * tok_s / 1e9, 2),
            "weight_roofline_frac": round(wbytes * tok_s / 1e9 / HBM_PEAK_GBPS, 4),
            "token_device_us": round(tot_us, 1),
            "launches_per_token": len(stats),
            "prompt_prefill": prefill,
            "reference_arithmetic": ref,
            "arithmetic": "reference (gemvq_set_arith)" if args.reference else "canonical",
        },
        "roofline": {
            "bound": "hbm",
            "kernel": dom_name,
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": traffic,
            "traffic_source": traffic_src,
            "launches": dom["n"],
            "bytes_per_launch": dom["bytes"] // dom["n"],
            "us_per_launch": round(dom["us"] / dom["n"], 3),
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
