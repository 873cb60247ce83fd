#!/usr/bin/env python3
"""Headline benchmark: int8 decode tok/s and achieved HBM GB/s on the
Gemma-3-1B shape (BASELINE.json metric; config 5).

Workload (one GPU): Gemma-3-1B architecture, int8 per-channel weights from the
seeded synthetic generator (seed 2), a 512-token random prompt, then greedy
decode to context 4096.  A "step" is one decode token for every stream.  The
prompt and W warm-up steps are untimed; exactly K steps are timed between
device synchronisations (default: every remaining step up to ctx 4096).

Extra fields of the JSON line:
  roofline      the dominant kernel.  Low-latency executor (the default where
                it supports the model and batch): the step kernel, one
                cooperative launch per run of up to 256 tokens that does the
                whole step (every layer's GEMVs and attention, the lm-head,
                the argmax), so achieved = algorithmic bytes of the timed
                steps / their device time (HIP events on the decoder
                stream).  Phase-kernel executors: the GEMV family, from
                per-launch events in one profiled step at the end context.
  hbm           whole-step algorithmic bytes (weights + scales + KV read at
                the mean context of the timed steps) / measured step time
  batch64       the metric's second batch size (config 5 at b = 64): the same
                workload for 64 streams, the whole decode to ctx 4096 timed
                (projections on the MFMA GEMM path); its roofline is the whole
                step's algorithmic bytes (weights + every stream's KV at the
                mean context) / its device time
  cpu_baseline  the CPU oracle (oracle/, a C restatement of the reference's
                decode arithmetic) on a bounded sample of the same workload,
                timed on this host's cores
Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--batch B] [--batch2 B2]
"""
import argparse
import importlib.util
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
HBM_PEAK_GBPS = 8000.0
# HBM bytes per step of the low-latency step kernel at the default workload
# (b = 1, prompt 512, decode to ctx 4096): rocprofv3 --pmc FETCH_SIZE and
# WRITE_SIZE per dispatch over the timed region, each scaled by what the same
# counter reads for a 1 GiB device copy (bench.py --copy-probe); commands and
# numbers in profiles/ll_traffic_gemma3_1b_b1.md.  Measured offline (counters
# need their own profiler run); null for any other workload.
LL_TRAFFIC_BYTES_PER_STEP = 1345337816


def load_xe():
    spec = importlib.util.spec_from_file_location(
        "xdna_engine", os.path.join(ROOT, "xdna-engine_amd", "xdna_engine.py"))
    mod = importlib.util.module_from_spec(spec)
    sys.modules["xdna_engine"] = mod
    spec.loader.exec_module(mod)
    return mod


def cpu_baseline(cfg, prompt_len, budget_s, seed):
    """Oracle decode on the host: feed a short prompt, then time greedy steps
    until ~budget_s of CPU work (bounded sample of the same workload)."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as O
    oc = O.ModelConfig()
    for name, _ in O.ModelConfig._fields_:
        setattr(oc, name, getattr(cfg, name))
    oc.max_ctx = 2048
    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or (os.cpu_count() or 1)
    O.lib().xo_set_threads(threads)
    om = O.OracleModel(oc, seed, 1)
    rng = np.random.default_rng(seed)
    toks = rng.integers(0, cfg.vocab, prompt_len).astype(np.int32)
    for p in range(prompt_len):
        logits = om.step(toks[p:p + 1], np.array([p], np.int32))
    tok = om.argmax(logits[0])
    n, pos = 0, prompt_len
    t0 = time.perf_counter()
    while True:
        logits = om.step(np.array([tok], np.int32), np.array([pos], np.int32))
        tok = om.argmax(logits[0])
        n += 1
        pos += 1
        el = time.perf_counter() - t0
        if el >= budget_s or pos >= oc.max_ctx - 1:
            break
    om.close()
    return {"value": n / el, "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": "oracle Gemma-3-1B int8 decode (C restatement), %d-token prompt then %d "
                      "greedy steps at ctx <= %d, %.1f s, OpenMP %d threads"
                      % (prompt_len, n, pos, el, threads)}


def run_batch(xe, dev, cfg, args, B, steps, warmup, profile):
    """Prompt feed, W untimed steps, then K timed greedy steps (default: to the
    end of the context) for B streams; returns the measurement as a dict."""
    dec = xe.Decoder(dev, cfg, max_batch=B)
    t = time.perf_counter()
    dec.init_synthetic(args.seed)
    print("[bench] b=%d: weights initialised in %.1f s (%.1f MB)" % (B, time.perf_counter() - t,
          dec.weight_bytes() / 1e6), file=sys.stderr, flush=True)
    rng = np.random.default_rng(args.seed)
    prompt = rng.integers(0, cfg.vocab, (B, args.prompt)).astype(np.int32)
    dec.feed(prompt)
    room = args.ctx - args.prompt - (1 if profile else 0)  # one profiled step at the end
    W = min(warmup, room)
    K = steps if steps > 0 else room - W
    if W + K > room:
        sys.exit("bench.py: warmup + steps exceed the context (%d)" % room)
    dec.decode(W, want_tokens=False)
    dev.synchronize()
    t0 = time.perf_counter()
    _, dev_us = dec.decode(K, want_tokens=False)
    dev.synchronize()
    t1 = time.perf_counter()
    step_s = (t1 - t0) / K
    tok_s = B * K / (t1 - t0)
    executor = dec.executor(B)
    prof = dec.profile_step() if profile else []
    by_label = {}
    for l, u, b in prof:
        e = by_label.setdefault(l, [0, 0.0, 0.0])
        e[0] += 1
        e[1] += u
        e[2] += b
    # whole-step algorithmic bytes at the mean context of the timed region
    mean_ctx = args.prompt + W + K / 2.0
    kv_bytes = B * cfg.n_layers * mean_ctx * cfg.n_kv_heads * cfg.head_dim * 2 * 2
    step_bytes = dec.weight_bytes() + kv_bytes
    hbm_gbps = step_bytes / step_s / 1e9
    if executor == "ll" or not profile:
        # the timed launches: bytes and device time summed over them
        r_bytes, r_us = step_bytes * K, dev_us
        r_kernel = ("ll_step_kernel (whole decode step per token; %d launches of <= 256 "
                    "steps in the timed region)" % ((K + 255) // 256) if executor == "ll" else
                    "whole decode step (%s executor: every kernel of the step)" % executor)
    else:
        r_bytes = sum(b for l, u, b in prof if l.startswith("gemv"))
        r_us = sum(u for l, u, b in prof if l.startswith("gemv"))
        r_kernel = "gemv (decode GEMV family, one profiled step)"
    r_gbps = r_bytes / r_us / 1e3
    res = {
        "value": round(tok_s, 2), "unit": "tok/s", "steps": K, "warmup": W,
        "ms_per_step": round(step_s * 1e3, 4),
        "config": {"workload": "gemma3-1b int8 greedy decode, batch %d, prompt %d, decode to "
                               "ctx %d" % (B, args.prompt, args.ctx),
                   "layers": cfg.n_layers, "hidden": cfg.d_model, "heads": "4q/1kv x 256",
                   "ffn": cfg.ffn, "vocab": cfg.vocab, "batch": B, "prompt": args.prompt,
                   "ctx": args.ctx, "seed": args.seed, "executor": executor},
        "device_us_per_step": round(dev_us / max(K, 1), 3),
        "hbm": {"achieved": round(hbm_gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                "frac": round(hbm_gbps / HBM_PEAK_GBPS, 4),
                "bytes_per_step": int(step_bytes)},
        "roofline": {"bound": "hbm", "kernel": r_kernel,
                     "achieved": round(r_gbps, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(r_gbps / HBM_PEAK_GBPS, 4),
                     "traffic": (LL_TRAFFIC_BYTES_PER_STEP if executor == "ll" and B == 1 and
                                 args.prompt == 512 and args.ctx == 4096 and args.steps == 0 else None),
                     "traffic_unit": "bytes per step",
                     "bytes": int(r_bytes), "us": round(r_us, 2)},
    }
    if profile:
        res["phases"] = {l: {"launches": v[0], "us": round(v[1], 2),
                             "gbps": round(v[2] / v[1] / 1e3, 1) if v[1] > 0 else None}
                         for l, v in by_label.items()}
    dec.close()
    print("[bench] b=%d: %.1f tok/s, %.3f ms/step (%s)" % (B, tok_s, step_s * 1e3, executor),
          file=sys.stderr, flush=True)
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=0, help="timed steps (0: decode to --ctx)")
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--batch2", type=int, default=64,
                    help="second batch size measured in the same run (0: none)")
    ap.add_argument("--prompt", type=int, default=512)
    ap.add_argument("--ctx", type=int, default=4096)
    ap.add_argument("--seed", type=int, default=2)
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only copy MIB MiB device to device (torch), three times: the plain "
                         "copy kernel that scales rocprofv3's FETCH_SIZE / WRITE_SIZE counters")
    args = ap.parse_args()
    if args.copy_probe > 0:
        import torch
        n = args.copy_probe * (1 << 20) // 4
        x = torch.ones(n, dtype=torch.float32, device="cuda:0")
        y = torch.empty_like(x)
        for _ in range(3):
            y.copy_(x)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes": n * 4, "copies": 3}), flush=True)
        return
    if args.gpus != 1:
        print("bench.py: this build runs on one GPU only (every GPU box here has one); "
              "--gpus %d is not supported" % args.gpus, file=sys.stderr)
        sys.exit(2)

    xe = load_xe()
    cfg = xe.GEMMA3_1B.replace(max_ctx=args.ctx)
    dev = xe.Device(0)
    B = args.batch
    head = run_batch(xe, dev, cfg, args, B, args.steps, args.warmup, profile=True)
    out = {
        "metric": "int8 decode tok/s, Gemma3-1B-shape b=%d" % B,
        "value": head["value"],
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": head["steps"],
        "warmup": head["warmup"],
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 weights, fp32 accumulate, bf16 KV",
        "data": "synthetic (seeded random-init weights N(0,0.02) quantised int8 per channel; "
                "uniform random prompt ids)",
        "config": head["config"],
        "device_us_per_step": head["device_us_per_step"],
        "hbm": head["hbm"],
        "roofline": head["roofline"],
        "phases": head["phases"],
    }
    if args.batch2 > 0 and args.batch2 != B:
        # the metric's second batch size: the whole decode to ctx, timed the same way
        out["batch%d" % args.batch2] = run_batch(xe, dev, cfg, args, args.batch2, 0, args.warmup,
                                                 profile=False)
    dev.close()
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(cfg, 4, args.cpu_seconds, args.seed)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
