#!/usr/bin/env python3
"""Writes workloads_7b.json: the oracle's answers for the benchmark
workloads at Qwen2.5-7B width (the model and inputs of workloads.py).

    python tests/golden/make_workload_fixtures.py [--threads N] [--only NAME]

The oracle is the CPU checker (oracle/), run token by token the way the
reference's generate loop runs (INTEGER_LLM/runtime/src/generate.rs:28-50);
batches are independent sequences, each on its own cache.  What is written
is answers, not inputs: hashes of logits and KV caches, greedy tokens,
log-softmax sums.  About 25 minutes on 8 cores (the 28-layer prompt included).
"""
from __future__ import annotations

import argparse
import json
import sys
import time
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(HERE))

import workloads as W  # noqa: E402
from myelith_amd.luts import LutSet  # noqa: E402
from oracle.binding import OracleModel, logsoftmax_at  # noqa: E402

OUT = HERE / "workloads_7b.json"


def log(msg: str) -> None:
    print(f"[fixtures {time.strftime('%H:%M:%S')}] {msg}", flush=True)


def run_prompt(om, toks) -> np.ndarray:
    om.reset()
    logits = None
    n = len(toks)
    for p, t in enumerate(toks):
        logits = om.forward_token(int(t), p, want_logits=p == n - 1)
    return logits


def decode_b1(om, spec) -> dict:
    cfg = W.DECODE_B1
    prompt = W.uniform_tokens(cfg["prompt_seed"], cfg["ctx"], spec["vocab"])
    logits = run_prompt(om, prompt)
    dig = W.Digest()
    tok = int(np.argmax(logits))
    tokens, lh = [tok], [W.h64(logits)]
    for i in range(cfg["steps"]):
        dig.step(logits, tok)
        logits = om.forward_token(tok, cfg["ctx"] + i)
        tok = int(np.argmax(logits))
        tokens.append(tok)
        lh.append(W.h64(logits))
    dig.step(logits, tok)
    n_pos = cfg["ctx"] + cfg["steps"]
    kv_greedy = W.kv_hash(om.read_kv, spec["layers"], spec["kv_heads"], n_pos)
    forced_tokens = W.uniform_tokens(cfg["forced_seed"], cfg["forced"], spec["vocab"])
    forced_h = []
    for i, t in enumerate(forced_tokens):
        forced_h.append(W.h64(om.forward_token(int(t), n_pos + i)))
    return {"tokens": tokens, "logits_h64": lh, "digest": dig.hexdigest(), "kv_sha256": kv_greedy,
            "forced_logits_h64": forced_h,
            "forced_kv_sha256": W.kv_hash(om.read_kv, spec["layers"], spec["kv_heads"], n_pos + cfg["forced"])}


def batch_decode(om, spec, cfg) -> dict:
    prompts = W.batch_prompts(cfg, spec["vocab"])
    first, tokens, last_h, step_h, kv = [], [], [], [], []
    for s in range(cfg["B"]):
        logits = run_prompt(om, prompts[s])
        tok = int(np.argmax(logits))
        first.append(tok)
        seq_toks, seq_h = [], []
        for i in range(cfg["steps"]):
            logits = om.forward_token(tok, cfg["ctx"][s] + i)
            tok = int(np.argmax(logits))
            seq_toks.append(tok)
            seq_h.append(W.h64(logits))
        tokens.append(seq_toks)
        step_h.append(seq_h)
        last_h.append(W.h64(logits))
        kv.append(W.kv_hash(om.read_kv, spec["layers"], spec["kv_heads"], cfg["ctx"][s] + cfg["steps"]))
        log(f"  B={cfg['B']} sequence {s} (context {cfg['ctx'][s]}) done")
    return {"first": first, "tokens": tokens, "last_logits_h64": last_h, "step_logits_h64": step_h, "kv_sha256": kv}


def teacher_forced(om, spec) -> dict:
    cfg = W.TEACHER_4x1024
    toks = W.teacher_tokens(cfg, spec["vocab"])
    lut = np.asarray(LutSet.for_head_dim(spec["head_dim"]).exp, np.int16)
    rows, argmax, sums, kv = [], [], [], []
    for b in range(cfg["B"]):
        om.reset()
        total = 0
        for p in range(cfg["T"]):
            logits = om.forward_token(int(toks[b, p]), p)
            rows.append(W.h64(logits))
            argmax.append(int(np.argmax(logits)))
            if p + 1 < cfg["T"]:
                total += logsoftmax_at(logits, lut, int(toks[b, p + 1]))
        sums.append(int(total))
        kv.append(W.kv_hash(om.read_kv, spec["layers"], spec["kv_heads"], cfg["T"]))
        log(f"  teacher-forced sequence {b} done")
    return {"row_logits_h64": rows, "argmax": argmax, "logsoftmax_sum_q16": sums, "kv_sha256": kv}


def full_depth(threads: int) -> dict:
    """The 28-layer model: a prompt then greedy steps, token by token on the
    oracle (its own model object: the other workloads use the two-layer cut)."""
    cfg, spec = W.FULL_DEPTH, W.spec_full()
    t0 = time.time()
    om = OracleModel(spec, LutSet.for_head_dim(spec["head_dim"]), threads=threads)
    log(f"28-layer oracle model built in {time.time() - t0:.1f} s")
    prompt = W.uniform_tokens(cfg["prompt_seed"], cfg["ctx"], spec["vocab"])
    logits = run_prompt(om, prompt)
    out = {"prompt_logits_h64": W.h64(logits),
           "prompt_kv_sha256": W.kv_hash(om.read_kv, spec["layers"], spec["kv_heads"], cfg["ctx"])}
    tok = int(np.argmax(logits))
    tokens, lh = [tok], []
    for i in range(cfg["steps"]):
        logits = om.forward_token(tok, cfg["ctx"] + i)
        tok = int(np.argmax(logits))
        tokens.append(tok)
        lh.append(W.h64(logits))
    out.update(tokens=tokens, step_logits_h64=lh,
               kv_sha256=W.kv_hash(om.read_kv, spec["layers"], spec["kv_heads"], cfg["ctx"] + cfg["steps"]))
    om.close()
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--threads", type=int, default=8)
    ap.add_argument("--only", choices=("decode_b1", "batch_8", "batch_32", "teacher_4x1024", "full_depth"))
    args = ap.parse_args()
    spec = W.spec()
    data = json.loads(OUT.read_text()) if OUT.exists() else {}
    data["spec"] = spec
    data["spec_full"] = W.spec_full()
    data["workloads"] = {"decode_b1": W.DECODE_B1, "batch_8": W.BATCH_8, "batch_32": W.BATCH_32,
                         "teacher_4x1024": W.TEACHER_4x1024, "full_depth": W.FULL_DEPTH}
    if args.only == "full_depth":
        t0 = time.time()
        data.setdefault("answers", {})["full_depth"] = full_depth(args.threads)
        log(f"full_depth: {time.time() - t0:.0f} s")
        OUT.write_text(json.dumps(data, indent=1) + "\n")
        return 0
    t0 = time.time()
    om = OracleModel(spec, LutSet.for_head_dim(spec["head_dim"]), threads=args.threads)
    log(f"oracle model built in {time.time() - t0:.1f} s")
    jobs = {"decode_b1": lambda: decode_b1(om, spec),
            "batch_8": lambda: batch_decode(om, spec, W.BATCH_8),
            "batch_32": lambda: batch_decode(om, spec, W.BATCH_32),
            "teacher_4x1024": lambda: teacher_forced(om, spec)}
    for name, fn in jobs.items():
        if args.only and name != args.only:
            continue
        t0 = time.time()
        data.setdefault("answers", {})[name] = fn()
        log(f"{name}: {time.time() - t0:.0f} s")
        OUT.write_text(json.dumps(data, indent=1) + "\n")
    om.close()
    if not args.only:
        t0 = time.time()
        data.setdefault("answers", {})["full_depth"] = full_depth(args.threads)
        log(f"full_depth: {time.time() - t0:.0f} s")
        OUT.write_text(json.dumps(data, indent=1) + "\n")
    return 0


if __name__ == "__main__":
    sys.exit(main())
