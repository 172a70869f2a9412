"""The benchmark workloads at Qwen2.5-7B width, shared by the fixture writer
(make_workload_fixtures.py, which runs the oracle) and the GPU test that
checks the device against the written answers (test_gpu_workloads.py).

The model is the Qwen2.5-7B architecture (hidden 3584, 28 query / 4 KV
heads, head_dim 128, intermediate 18944, vocab 152064, int16 LM head, q/k/v
biases) cut to two layers.  Which kernels and tiles run depends on the
widths, the number of rows and the positions, never on the depth, so two
layers exercise every kernel of the 28-layer model at its real shape; and
since every tensor is seeded by (model seed, layer, role), these two layers
are the first two layers of the 28-layer benchmark model of the same seed.

FULL_DEPTH is the whole 28-layer model of the same seed (the benchmark
model): a prompt through the row path and greedy steps, so every layer's K/V
rows are pinned independently of the device's own cache.

Token ids come from the SplitMix64 stream (the reference PRNG,
INTEGER_LLM/kernels/src/prng.rs:7-14), so the workload does not depend on
numpy's generators.
"""
from __future__ import annotations

import hashlib

import numpy as np

MASK64 = (1 << 64) - 1
GAMMA = 0x9E3779B97F4A7C15

ARCH_7B = dict(vocab=152064, hidden=3584, layers=2, heads=28, kv_heads=4, head_dim=128, inter=18944,
               lm_head_int16=1, attention_bias=1)
SEED = 7
MAX_POS = 2104

# batch 1: a 2048-token prompt through the prompt row path, then greedy steps
# at positions 2048-2071 (RoPE LUT rows wrap at 2048), then `forced` steps at
# positions 2072-2095 whose tokens come from the SplitMix64 stream of
# forced_seed (a synthetic model's greedy chain tends to settle on one token;
# drawn tokens make every step read a different embedding row).
DECODE_B1 = dict(prompt_seed=101, ctx=2048, steps=24, forced=24, forced_seed=102)
# lock-step greedy decode of B sequences after their contexts were prefilled
# through the batched forward in chunks of 4096 // B positions per sequence.
BATCH_8 = dict(B=8, ctx=[2048] * 8, steps=8, prompt_seed=200)
BATCH_32 = dict(B=32, ctx=[2048 if s % 9 == 0 else 600 + 7 * s for s in range(32)], steps=8, prompt_seed=300)
# teacher-forced rows: 4 sequences x 1024 Zipf(1.1) token ids in one batch.
TEACHER_4x1024 = dict(B=4, T=1024, zipf_s=1.1, token_seed=400)

# the whole 28-layer benchmark model (same seed): a 1024-token prompt through
# the prompt row path (every layer's K/V rows written by the row kernels),
# then greedy steps from the captured step graph.
FULL_DEPTH = dict(layers=28, max_pos=1040, prompt_seed=500, ctx=1024, steps=8)


def spec() -> dict:
    s = dict(ARCH_7B)
    s.update(seed=SEED, max_pos=MAX_POS)
    return s


def spec_full() -> dict:
    s = dict(ARCH_7B)
    s.update(seed=SEED, layers=FULL_DEPTH["layers"], max_pos=FULL_DEPTH["max_pos"])
    return s


def mix64(z: int) -> int:
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & MASK64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & MASK64
    return z ^ (z >> 31)


def stream(seed: int, n: int) -> np.ndarray:
    """The first n outputs of the SplitMix64 stream starting at `seed`."""
    return np.array([mix64((seed + (i + 1) * GAMMA) & MASK64) for i in range(n)], dtype=np.uint64)


def uniform_tokens(seed: int, n: int, vocab: int) -> np.ndarray:
    return (stream(seed, n) % np.uint64(vocab)).astype(np.uint32)


def zipf_tokens(seed: int, n: int, vocab: int, s: float) -> np.ndarray:
    """Zipf(s) over [0, vocab) by inverse CDF of 53-bit uniforms."""
    u = (stream(seed, n) >> np.uint64(11)).astype(np.float64) / float(1 << 53)
    w = 1.0 / np.arange(1, vocab + 1, dtype=np.float64) ** s
    cdf = np.cumsum(w)
    cdf /= cdf[-1]
    return np.minimum(np.searchsorted(cdf, u), vocab - 1).astype(np.uint32)


def batch_prompts(cfg: dict, vocab: int) -> list[np.ndarray]:
    return [uniform_tokens(cfg["prompt_seed"] + s, cfg["ctx"][s], vocab) for s in range(cfg["B"])]


def teacher_tokens(cfg: dict, vocab: int) -> np.ndarray:
    return zipf_tokens(cfg["token_seed"], cfg["B"] * cfg["T"], vocab, cfg["zipf_s"]).reshape(cfg["B"], cfg["T"])


def prefill_chunks(ctx: list[int], B: int):
    """The (seq, pos) rows of each forward_batch call that prefills the
    contexts: 4096 // B positions of every unfinished sequence per call."""
    chunk = max(1, 4096 // B)
    for p0 in range(0, max(ctx), chunk):
        seq, pos = [], []
        for s in range(B):
            for p in range(p0, min(p0 + chunk, ctx[s])):
                seq.append(s)
                pos.append(p)
        if seq:
            yield np.array(seq, np.uint32), np.array(pos, np.uint32)


def h64(a: np.ndarray) -> str:
    """First 16 hex digits of the SHA-256 of an array's little-endian bytes."""
    return hashlib.sha256(np.ascontiguousarray(a).astype(a.dtype.newbyteorder("<")).tobytes()).hexdigest()[:16]


def kv_hash(read_kv, layers: int, kv_heads: int, n_pos: int) -> str:
    """SHA-256 over K then V of every (layer, KV head), positions [0, n_pos)."""
    h = hashlib.sha256()
    for layer in range(layers):
        for kvh in range(kv_heads):
            k, v = read_kv(layer, kvh, n_pos)
            h.update(np.ascontiguousarray(k, "<i2").tobytes())
            h.update(np.ascontiguousarray(v, "<i2").tobytes())
    return h.hexdigest()


class Digest:
    """generate.rs:98-137: per decode step, all logits as i32 LE, then the
    chosen token as u32 LE."""

    def __init__(self):
        self.h = hashlib.sha256()

    def step(self, logits, token: int) -> None:
        self.h.update(np.ascontiguousarray(logits, "<i4").tobytes())
        self.h.update(np.uint32(token).astype("<u4").tobytes())

    def hexdigest(self) -> str:
        return self.h.hexdigest()
