"""GPU parity at the benchmark workloads' real sizes, Qwen2.5-7B width.

The device runs the same calls the benchmark times, on the two-layer cut of
the benchmark model (tests/golden/workloads.py), and is compared with the
oracle's answers written by tests/golden/make_workload_fixtures.py
(workloads_7b.json): the oracle needs minutes of CPU for these sizes, so it
runs once where the fixtures are made, not on every GPU run.

  - batch 1: a 2048-token prompt through the prompt row path, 24 greedy steps
    from the captured step graph at positions 2048-2071 (RoPE LUT rows wrap at
    2048, GQA group 7): every step's logits, the tokens, the generate.rs
    digest and the whole KV cache; then 24 steps at positions 2072-2095 on
    SplitMix64-drawn tokens (every step a different embedding row): every
    step's logits and the KV cache again;
  - lock-step greedy decode of 8 sequences over 2048-token contexts and of 32
    sequences over contexts of 600-2048 positions, contexts prefilled through
    the batched forward in the benchmark's chunks: first tokens, every step's
    tokens, the last step's logits, every sequence's KV cache; then the same
    decode again one step per call, every step's logits of every sequence;
  - 4 x 1024 teacher-forced Zipf(1.1) rows in one batch (256 x 256 tiles at
    K = 18944, the byte-plane int16 head at V = 152064, four 256-position
    attention ranges): every row's logits and argmax, the four integer
    log-softmax sums, the KV caches;
  - the whole 28-layer benchmark model: a 1024-token prompt through the
    prompt row path (last row's logits, the KV cache of all 28 layers, so
    every layer's row kernels are pinned by the oracle's own cache), then 8
    greedy steps from the captured step graph (every step's logits, the
    tokens, the KV cache).
"""
from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np
import pytest

from conftest import case

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLDEN))
import workloads as W  # noqa: E402


@pytest.fixture(scope="module")
def answers():
    data = json.loads((GOLDEN / "workloads_7b.json").read_text())
    assert data["spec"] == W.spec(), "workloads_7b.json was written for another model; rerun its generator"
    assert data["spec_full"] == W.spec_full(), "workloads_7b.json was written for another model; rerun its generator"
    return data["answers"]


@pytest.fixture(scope="module")
def model(backend):
    from myelith_amd.luts import LutSet
    from myelith_amd.model import IntegerModel
    spec = W.spec()
    m = IntegerModel(backend, spec, LutSet.for_head_dim(spec["head_dim"]))
    yield m
    m.close()


def test_decode_b1_2048_context(model, answers):
    cfg, want = W.DECODE_B1, answers["decode_b1"]
    spec = W.spec()
    case(f"7B width decode b1: prompt {cfg['ctx']} rows, {cfg['steps']} graph steps")
    prompt = W.uniform_tokens(cfg["prompt_seed"], cfg["ctx"], spec["vocab"])
    model.reset()
    logits = model.prefill(prompt, 0)
    assert W.h64(logits) == want["logits_h64"][0], "last prompt row's logits"
    first = int(np.argmax(logits))
    assert first == want["tokens"][0]
    toks, steps = model.decode_greedy(first, cfg["ctx"], cfg["steps"], want_logits=True)
    for i in range(cfg["steps"]):
        assert W.h64(steps[i]) == want["logits_h64"][i + 1], f"logits at position {cfg['ctx'] + i}"
    assert [first] + [int(t) for t in toks] == want["tokens"]
    dig = W.Digest()
    for lg, t in zip([logits] + list(steps), want["tokens"]):
        dig.step(lg, t)
    assert dig.hexdigest() == want["digest"]
    n_pos = cfg["ctx"] + cfg["steps"]
    assert W.kv_hash(model.read_kv, spec["layers"], spec["kv_heads"], n_pos) == want["kv_sha256"]
    case(f"7B width decode b1: {cfg['forced']} steps on drawn tokens at positions {n_pos}-")
    forced = W.uniform_tokens(cfg["forced_seed"], cfg["forced"], spec["vocab"])
    for i, t in enumerate(forced):
        lg = model.forward_token(int(t), n_pos + i)
        assert W.h64(lg) == want["forced_logits_h64"][i], f"logits at position {n_pos + i} (token {int(t)})"
    assert (W.kv_hash(model.read_kv, spec["layers"], spec["kv_heads"], n_pos + cfg["forced"])
            == want["forced_kv_sha256"])


@pytest.mark.parametrize("name", ["batch_8", "batch_32"])
def test_batch_decode_long_contexts(model, answers, name):
    cfg = W.BATCH_8 if name == "batch_8" else W.BATCH_32
    want = answers[name]
    spec = W.spec()
    B, ctx = cfg["B"], cfg["ctx"]
    case(f"7B width lock-step decode B={B}, contexts {min(ctx)}-{max(ctx)}, {cfg['steps']} steps")
    prompts = W.batch_prompts(cfg, spec["vocab"])
    model.batch_begin(B)
    first = [None] * B
    for seq, pos in W.prefill_chunks(ctx, B):
        toks = np.array([prompts[s][p] for s, p in zip(seq, pos)], np.uint32)
        _, am = model.forward_batch(seq, pos, toks, want_logits=False)
        for i, (s, p) in enumerate(zip(seq, pos)):
            if p == ctx[s] - 1:
                first[s] = int(am[i])
    assert first == want["first"], "argmax of each context's last row"
    out = model.batch_decode_greedy(np.arange(B), np.array(ctx), np.array(first), cfg["steps"])
    for s in range(B):
        assert [int(t) for t in out[:, s]] == want["tokens"][s], f"greedy tokens of sequence {s}"
    last = model.batch_logits_dev(B).cpu().numpy()
    for s in range(B):
        assert W.h64(last[s]) == want["last_logits_h64"][s], f"last step's logits of sequence {s}"
    for s in range(B):
        got = W.kv_hash(lambda l, h, n: model.batch_read_kv(s, l, h, n), spec["layers"], spec["kv_heads"],
                        ctx[s] + cfg["steps"])
        assert got == want["kv_sha256"][s], f"KV cache of sequence {s}"
    # every step's logits: the same decode once more, one step per call (the
    # steps rewrite the same cache rows with the same values)
    case(f"7B width lock-step decode B={B}: every step's logits")
    tok = np.array(first)
    for i in range(cfg["steps"]):
        step = model.batch_decode_greedy(np.arange(B), np.array(ctx) + i, tok, 1)
        lg = model.batch_logits_dev(B).cpu().numpy()
        for s in range(B):
            assert W.h64(lg[s]) == want["step_logits_h64"][s][i], f"logits of sequence {s} at step {i}"
        tok = step[0]


def test_teacher_forced_4x1024(model, backend, answers):
    import torch
    cfg, want = W.TEACHER_4x1024, answers["teacher_4x1024"]
    spec = W.spec()
    B, T = cfg["B"], cfg["T"]
    case(f"7B width teacher-forced {B} x {T} rows")
    toks = W.teacher_tokens(cfg, spec["vocab"])
    seq = np.repeat(np.arange(B), T).astype(np.uint32)
    pos = np.tile(np.arange(T), B).astype(np.uint32)
    tgt = np.concatenate([np.append(toks[b, 1:].astype(np.int64), -1) for b in range(B)])
    model.batch_begin(B)
    _, am = model.forward_batch(seq, pos, toks.ravel(), want_logits=False)
    lut = torch.from_numpy(np.ascontiguousarray(model.luts.exp, dtype=np.int16)).cuda()
    lp = backend.logsoftmax_dev(model.batch_logits_dev(B * T), lut, torch.from_numpy(tgt).cuda())
    sums = [int(v) for v in lp.view(B, T).sum(dim=1).cpu().tolist()]
    assert [int(a) for a in am] == want["argmax"]
    logits = model.batch_logits_dev(B * T)
    bad = []
    for r0 in range(0, B * T, 256):
        blk = logits[r0:r0 + 256].cpu().numpy()
        bad += [r0 + i for i in range(blk.shape[0]) if W.h64(blk[i]) != want["row_logits_h64"][r0 + i]]
    assert not bad, f"{len(bad)} rows' logits differ, first (seq, pos) = {divmod(bad[0], T)}"
    assert sums == want["logsoftmax_sum_q16"]
    for b in range(B):
        got = W.kv_hash(lambda l, h, n: model.batch_read_kv(b, l, h, n), spec["layers"], spec["kv_heads"], T)
        assert got == want["kv_sha256"][b], f"KV cache of sequence {b}"


def test_full_depth_prompt_and_decode(backend, answers):
    """The 28-layer benchmark model: the prompt's KV cache at every layer and
    the last row's logits, then graph decode steps, against the oracle's own
    token-by-token run (no device state handed to the oracle)."""
    from myelith_amd.luts import LutSet
    from myelith_amd.model import IntegerModel
    cfg, want = W.FULL_DEPTH, answers["full_depth"]
    spec = W.spec_full()
    case(f"7B 28 layers: prompt {cfg['ctx']} rows, {cfg['steps']} graph steps")
    m = IntegerModel(backend, spec, LutSet.for_head_dim(spec["head_dim"]))
    try:
        prompt = W.uniform_tokens(cfg["prompt_seed"], cfg["ctx"], spec["vocab"])
        logits = m.prefill(prompt, 0)
        assert W.h64(logits) == want["prompt_logits_h64"], "last prompt row's logits"
        assert W.kv_hash(m.read_kv, spec["layers"], spec["kv_heads"], cfg["ctx"]) == want["prompt_kv_sha256"]
        first = int(np.argmax(logits))
        toks, steps = m.decode_greedy(first, cfg["ctx"], cfg["steps"], want_logits=True)
        for i in range(cfg["steps"]):
            assert W.h64(steps[i]) == want["step_logits_h64"][i], f"logits at position {cfg['ctx'] + i}"
        assert [first] + [int(t) for t in toks] == want["tokens"]
        assert (W.kv_hash(m.read_kv, spec["layers"], spec["kv_heads"], cfg["ctx"] + cfg["steps"])
                == want["kv_sha256"])
    finally:
        m.close()
