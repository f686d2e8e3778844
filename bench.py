#!/usr/bin/env python3
"""Decode benchmark: batch-1 greedy decode of the synthetic Qwen3.5-9B-shaped Q4_0 model on one MI355X.

Workload: 32 layers (24 Gated DeltaNet + 8 gated attention, 3:1), hidden 4096, FFN 12288, vocab 151936, layer
matrices Q4_0 N(0, 0.02^2), embedding and head Q6_K, norms fp32 ones; prompt of 512 random ids run token by token
(untimed), then `--warmup` untimed and `--steps` timed greedy decode steps (one hipGraph replay each, tokens fed
back on the device). value = timed tokens / wall time between two stream synchronizations.

roofline: the dominant kernel (largest share of a token's device time), its algorithmic bytes (GGUF weights +
fp32 vectors read and written once + state/KV traffic) over its measured duration, from device start/stop events
of every kernel of one token (gemvq_profile). cpu_baseline: the oracle decoder (a C restatement of the reference's
CPU arithmetic, multithreaded over rows) on the host cores for a bounded sample of decode steps at the same shape.
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


class LaunchStat(C.Structure):
    _fields_ = [("name", C.c_char * 40), ("first_cmd", C.c_int32), ("n_cmds", C.c_int32), ("bytes", C.c_uint64),
                ("us", C.c_double)]


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
    lib = gq.hip_lib()
    lib.gemvq_profile.restype = C.c_int
    lib.gemvq_profile.argtypes = [C.c_void_p, C.POINTER(C.c_uint32), C.c_uint, C.c_int, C.c_void_p, C.c_int]
    w = np.ascontiguousarray(cmds.ravel(), np.uint32)
    out = (LaunchStat * 4096)()
    n = lib.gemvq_profile(ctx.h, w.ctypes.data_as(C.POINTER(C.c_uint32)), w.size // 8, reps, out, 4096)
    if n < 0:
        raise gq.GemvqError(f"profile: {n}: {ctx.error()}")
    return [dict(name=out[i].name.decode(), first=out[i].first_cmd, bytes=int(out[i].bytes), us=out[i].us)
            for i in range(n)]


def cpu_baseline(blob, cfg, prompt, n_tokens: int, threads: int) -> dict:
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle  # noqa: E402  (the CPU baseline leg only)

    om = oracle.Model(Q.config_c(cfg), blob.table, blob.n, blob.data, threads=threads)
    om.decode(int(prompt[0]), 0)  # first touch of the weights, untimed
    t0 = time.perf_counter()
    for pos in range(1, 1 + n_tokens):
        om.decode(int(prompt[pos]), pos)
    dt = time.perf_counter() - t0
    om.close()
    return {"value": round(n_tokens / dt, 4), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"{n_tokens} decode steps (positions 1..{n_tokens}) of the same 9B-shape model with the oracle "
                      f"decoder (C restatement of the reference CPU arithmetic, rows split over {threads} threads, "
                      f"{dt:.1f} s)"}


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


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128, help="timed decode steps (tokens)")
    ap.add_argument("--warmup", type=int, default=0, help="untimed decode steps after the prompt")
    ap.add_argument("--prompt", type=int, default=512, help="prompt length (run token by token, untimed)")
    ap.add_argument("--cpu-tokens", type=int, default=6, help="decode steps timed for the CPU baseline (0: skip)")
    ap.add_argument("--threads", type=int, default=min(16, os.cpu_count() or 1))
    ap.add_argument("--profile-reps", type=int, default=3)
    ap.add_argument("--layers", type=int, default=32, help="(testing) fewer layers; the reported line is then invalid")
    ap.add_argument("--direct", action="store_true",
                    help="plain stream launches instead of graph replays (for tracing tools); slower per step")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy kernel of MIB MiB 5 times (calibrates the HBM byte counters "
                         "of rocprofv3 --pmc) and exit")
    args = ap.parse_args()
    if args.copy_probe:
        return copy_probe(args.copy_probe)
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              f"(the multi-GPU sharding is a design note, not code)", file=sys.stderr)
        return 2

    slack = args.profile_reps + 16
    cfg = Q.Config(n_layer=args.layers, n_ctx=args.prompt + args.warmup + args.steps + slack)
    t = time.perf_counter()
    blob = Q.generate(cfg, seed=0, threads=args.threads)
    log(f"generated the synthetic model ({blob.data.size / 1e9:.2f} GB) in {time.perf_counter() - t:.1f} s")
    prompt = Q.prompt_ids(cfg, args.prompt + 1)
    wbytes = Q.weight_bytes(cfg)

    t = time.perf_counter()
    m = Q.Model(blob)
    log(f"uploaded and captured the per-token graph in {time.perf_counter() - t:.1f} s "
        f"({len(m.commands())} commands, weight bytes per token {wbytes})")
    m.reset(prompt[:args.prompt])
    step = m.step_direct if args.direct else m.step
    t = time.perf_counter()
    step(args.prompt - 1)
    step(args.warmup)
    m.sync()
    log(f"prompt ({args.prompt}) + warmup ({args.warmup}) steps in {time.perf_counter() - t:.2f} s")
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
    m.close()

    cpu = None
    if args.cpu_tokens > 0:
        t = time.perf_counter()
        cpu = cpu_baseline(blob, cfg, prompt, args.cpu_tokens, args.threads)
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
