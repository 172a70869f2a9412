"""GPU parity of the batched forward (many sequences, each with its own KV
cache) and of the integer log-softmax, against the oracle.

The reference has no batching (generate.rs:28-32 loops forward_token), so a
batch row (seq, pos, token) must equal forward_token(token, pos) run on that
sequence alone, bit for bit: logits, argmax, KV cache and greedy tokens.
Batches above 8 rows take the int8 matrix-core products, batches of up to 8
the streaming GEMVs; both are exercised.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import case
from test_gpu_model import build, tiny

pytestmark = pytest.mark.gpu


def oracle_rows(om, seqs_tokens):
    """Per sequence, forward_token over its tokens from position 0: logits [T x V]."""
    out = []
    for toks in seqs_tokens:
        om.reset()
        out.append(np.stack([om.forward_token(int(t), p) for p, t in enumerate(toks)]))
    return out


def compare_batch_kv(gm, om, spec, seq, toks):
    om.reset()
    for p, t in enumerate(toks):
        om.forward_token(int(t), p)
    for l in range(spec["layers"]):
        for h in range(spec["kv_heads"]):
            gk, gv = gm.batch_read_kv(seq, l, h, len(toks))
            ok, ov = om.read_kv(l, h, len(toks))
            assert np.array_equal(gk, ok), ("K", seq, l, h)
            assert np.array_equal(gv, ov), ("V", seq, l, h)


@pytest.mark.parametrize("hd,lm16,bias,kvh", [(64, 0, 1, 2), (128, 1, 1, 2), (128, 0, 0, 4)])
def test_batch_rows_interleaved(backend, hd, lm16, bias, kvh):
    """Three sequences of different lengths, rows interleaved and unsorted, in
    a 34-row batch (matrix cores) then a 4-row continuation (GEMV)."""
    spec = tiny(hd, lm16, bias, kvh)
    case(f"batch rows {spec}")
    gm, om = build(backend, spec)
    r = np.random.default_rng(hd * 7 + kvh)
    lens1 = [10, 5, 19]
    toks = [r.integers(0, spec["vocab"], 30) for _ in lens1]
    rows = [(s, p) for s, n in enumerate(lens1) for p in range(n)]
    order = r.permutation(len(rows))
    rows = [rows[i] for i in order]
    gm.batch_begin(3)
    seq = [s for s, _ in rows]
    pos = [p for _, p in rows]
    tk = [int(toks[s][p]) for s, p in rows]
    logits, am = gm.forward_batch(seq, pos, tk)
    ref = oracle_rows(om, [toks[s][:30] for s in range(3)])
    for i, (s, p) in enumerate(rows):
        assert np.array_equal(logits[i], ref[s][p]), ("row", s, p)
        assert am[i] == int(np.argmax(ref[s][p]))
    # continuation: seq 0 positions 10..12, seq 2 position 19 (4 rows -> GEMV path)
    rows2 = [(0, 10), (2, 19), (0, 11), (0, 12)]
    logits2, _ = gm.forward_batch([s for s, _ in rows2], [p for _, p in rows2], [int(toks[s][p]) for s, p in rows2])
    for i, (s, p) in enumerate(rows2):
        assert np.array_equal(logits2[i], ref[s][p]), ("continuation", s, p)
    compare_batch_kv(gm, om, spec, 0, toks[0][:13])
    compare_batch_kv(gm, om, spec, 2, toks[2][:20])
    # the invalid cases the boundary rejects
    with pytest.raises(ValueError):
        gm.forward_batch([1, 1], [7, 9], [1, 2])  # gap and beyond the cached length
    with pytest.raises(ValueError):
        gm.forward_batch([3], [0], [1])  # no such sequence


@pytest.mark.parametrize("hd,lm16", [(128, 1), (64, 0)])
def test_batch_many_rows(backend, hd, lm16):
    """340 rows in one batch (the large-M products, byte-plane int16 head):
    a 300-position sequence (two 256-position attention ranges, tiles of many
    rows) and a 40-position one, rows shuffled; every row's logits, the argmax
    and both KV caches equal the oracle's."""
    spec = tiny(hd, lm16, 1, 2)
    case(f"batch many rows {spec}")
    gm, om = build(backend, spec)
    r = np.random.default_rng(hd + 3 * lm16)
    lens = [300, 40]
    toks = [r.integers(0, spec["vocab"], n) for n in lens]
    rows = [(s, p) for s, n in enumerate(lens) for p in range(n)]
    rows = [rows[i] for i in r.permutation(len(rows))]
    gm.batch_begin(2)
    logits, am = gm.forward_batch([s for s, _ in rows], [p for _, p in rows], [int(toks[s][p]) for s, p in rows])
    ref = oracle_rows(om, toks)
    for i, (s, p) in enumerate(rows):
        assert np.array_equal(logits[i], ref[s][p]), ("row", s, p)
        assert am[i] == int(np.argmax(ref[s][p]))
    compare_batch_kv(gm, om, spec, 0, toks[0])
    compare_batch_kv(gm, om, spec, 1, toks[1])


@pytest.mark.parametrize("hd", [128, 64])
def test_batch_many_sequences(backend, hd):
    """300 sequences: their 4-token prompts in one batch of 1200 rows, then
    one row per sequence twice (decode batches).  With this many tiles the
    attention blocks loop over their ranges and finish the output in place,
    and the one-row tiles take the narrow P.V variant; every row's logits
    equal the oracle's."""
    spec = tiny(hd, 0, 1, 2)
    case(f"batch many sequences hd={hd}")
    gm, om = build(backend, spec)
    r = np.random.default_rng(hd + 11)
    S, P = 300, 4
    toks = [r.integers(0, spec["vocab"], P + 2) for _ in range(S)]
    ref = oracle_rows(om, toks)
    gm.batch_begin(S)
    rows = [(s, p) for s in range(S) for p in range(P)]
    logits, _ = gm.forward_batch([s for s, _ in rows], [p for _, p in rows], [int(toks[s][p]) for s, p in rows])
    for i, (s, p) in enumerate(rows):
        assert np.array_equal(logits[i], ref[s][p]), ("prompt row", s, p)
    for p in (P, P + 1):
        logits, am = gm.forward_batch(list(range(S)), [p] * S, [int(toks[s][p]) for s in range(S)])
        for s in range(S):
            assert np.array_equal(logits[s], ref[s][p]), ("decode row", s, p)
            assert am[s] == int(np.argmax(ref[s][p]))


def test_batch_many_tiles_loop_ranges(backend):
    """32 sequences x 300 rows (320 attention tiles of 32 rows): the blocks
    loop over two 256-position ranges each and finish the attention output in
    place; every row's logits equal the oracle's."""
    spec = tiny(128, 1, 1, 2)
    case("batch 32 x 300 rows")
    gm, om = build(backend, spec)
    r = np.random.default_rng(5)
    S, T = 32, 300
    toks = [r.integers(0, spec["vocab"], T) for _ in range(S)]
    ref = oracle_rows(om, toks)
    gm.batch_begin(S)
    rows = [(s, p) for s in range(S) for p in range(T)]
    rows = [rows[i] for i in r.permutation(len(rows))]
    logits, _ = gm.forward_batch([s for s, _ in rows], [p for _, p in rows], [int(toks[s][p]) for s, p in rows])
    for i, (s, p) in enumerate(rows):
        assert np.array_equal(logits[i], ref[s][p]), ("row", s, p)


def test_batch_decode_greedy_lock_step(backend):
    """Four sequences prefilled to different lengths, then 12 lock-step greedy
    steps on the device: each sequence's tokens equal its own greedy run."""
    spec = tiny(128, 1, 1, 2)
    case("batch greedy decode")
    gm, om = build(backend, spec)
    r = np.random.default_rng(3)
    prompts = [r.integers(0, spec["vocab"], n) for n in (3, 9, 1, 6)]
    gm.batch_begin(4)
    rows = [(s, p) for s, pr in enumerate(prompts) for p in range(len(pr))]
    _, am = gm.forward_batch([s for s, _ in rows], [p for _, p in rows], [int(prompts[s][p]) for s, p in rows])
    last = {s: i for i, (s, p) in enumerate(rows)}  # the last row of each sequence
    first = [int(am[last[s]]) for s in range(4)]
    steps = 12
    toks = gm.batch_decode_greedy(range(4), [len(p) for p in prompts], first, steps)
    for s, pr in enumerate(prompts):
        om.reset()
        logits = None
        for p, t in enumerate(pr):
            logits = om.forward_token(int(t), p)
        nxt = int(np.argmax(logits))
        assert nxt == first[s]
        exp = []
        pos = len(pr)
        for _ in range(steps):
            logits = om.forward_token(nxt, pos)
            nxt = int(np.argmax(logits))
            exp.append(nxt)
            pos += 1
        assert [int(t) for t in toks[:, s]] == exp, s


@pytest.mark.parametrize("hd,heads,bias", [(64, 8, 1), (128, 14, 0), (64, 16, 1)])
def test_batch_decode_rows_grouped_heads(backend, hd, heads, bias):
    """Decode batches (one row per sequence) take the per-row attention
    kernels when 4, 7 or 8 query heads share a KV head: sequences of 1, 63,
    64, 257 and 300 positions (chunk and range edges), one decode row each,
    then lock-step greedy steps; logits, tokens and KV cache equal each
    sequence's own forward_token run."""
    spec = dict(seed=5, vocab=1000, hidden=heads * hd, layers=2, heads=heads, kv_heads=2, head_dim=hd, inter=320,
                max_pos=640, lm_head_int16=0, attention_bias=bias)
    case(f"batch decode rows {spec}")
    gm, om = build(backend, spec)
    r = np.random.default_rng(hd + heads)
    lens = [1, 63, 64, 257, 300]
    toks = [r.integers(0, spec["vocab"], n + 1) for n in lens]
    S = len(lens)
    gm.batch_begin(S)
    rows = [(s, p) for s, n in enumerate(lens) for p in range(n)]
    gm.forward_batch([s for s, _ in rows], [p for _, p in rows], [int(toks[s][p]) for s, p in rows],
                     want_logits=False)
    logits, am = gm.forward_batch(list(range(S)), lens, [int(toks[s][n]) for s, n in enumerate(lens)])
    first = []
    for s, n in enumerate(lens):
        om.reset()
        for p in range(n + 1):
            ref = om.forward_token(int(toks[s][p]), p)
        assert np.array_equal(logits[s], ref), ("decode row", s, n)
        first.append(int(np.argmax(ref)))
    assert [int(a) for a in am] == first
    steps = 5
    out = gm.batch_decode_greedy(range(S), [n + 1 for n in lens], first, steps)
    for s, n in enumerate(lens):
        om.reset()
        for p in range(n + 1):
            logits_o = om.forward_token(int(toks[s][p]), p)
        nxt, exp = int(np.argmax(logits_o)), []
        for i in range(steps):
            logits_o = om.forward_token(nxt, n + 1 + i)
            nxt = int(np.argmax(logits_o))
            exp.append(nxt)
        assert [int(t) for t in out[:, s]] == exp, s
        compare_batch_kv(gm, om, spec, s, list(toks[s][:n + 1]) + [first[s]] + exp[:-1])


def test_batch_decode_rows_past_4096_positions(backend):
    """Decode rows over contexts past 4096 positions (4100 and 4350, beside a
    300-position one): the per-row score kernel over 68 position chunks, the
    P.V kernel over 17 ranges and the output kernel's second batch of range
    partials.  The contexts go in as batches of 2048 rows; the decode rows'
    logits, the argmax and three lock-step greedy steps equal each sequence's
    own forward_token run."""
    spec = dict(seed=12, vocab=1000, hidden=8 * 64, layers=1, heads=8, kv_heads=2, head_dim=64, inter=320,
                max_pos=4400, lm_head_int16=0, attention_bias=1)
    case(f"batch decode rows past 4096 {spec}")
    gm, om = build(backend, spec)
    r = np.random.default_rng(4101)
    lens = [4100, 4350, 300]
    toks = [r.integers(0, spec["vocab"], n + 1) for n in lens]
    S = len(lens)
    gm.batch_begin(S)
    rows = [(s, p) for s, n in enumerate(lens) for p in range(n)]
    for i in range(0, len(rows), 2048):
        chunk = rows[i:i + 2048]
        gm.forward_batch([s for s, _ in chunk], [p for _, p in chunk], [int(toks[s][p]) for s, p in chunk],
                         want_logits=False)
    logits, am = gm.forward_batch(list(range(S)), lens, [int(toks[s][n]) for s, n in enumerate(lens)])
    steps = 3
    first, expected = [], []
    for s, n in enumerate(lens):
        om.reset()
        for p in range(n + 1):
            ref = om.forward_token(int(toks[s][p]), p)
        assert np.array_equal(logits[s], ref), ("decode row", s, n)
        nxt = int(np.argmax(ref))
        first.append(nxt)
        exp = []
        for i in range(steps):
            nxt = int(np.argmax(om.forward_token(nxt, n + 1 + i)))
            exp.append(nxt)
        expected.append(exp)
    assert [int(a) for a in am] == first
    out = gm.batch_decode_greedy(range(S), [n + 1 for n in lens], first, steps)
    for s in range(S):
        assert [int(t) for t in out[:, s]] == expected[s], s


@pytest.mark.parametrize("rows", [2, 5, 9, 16, 17, 32])
@pytest.mark.parametrize("shape", ["k7", "k64_down2"])
def test_batch_fragment_products(backend, monkeypatch, shape, rows):
    """Decode batches through the fragment-major gate/up and down products
    (MYL_BATCH_FRAG=1 takes them at every size they support): 2 and 5 rows
    (one 16-row plane tile), 9 and 16 (two), 17 and 32 (four), so the least
    and the most rows of each tile count; a hidden size of 7 K tiles
    (one of the eight waves carries K) and one of 64 tiles (eight per wave)
    whose down product runs in two K slices.  The decode row's logits and
    argmax and two greedy steps equal the tiled products' (MYL_BATCH_FRAG=0)
    bit for bit, and the decode row's logits equal the oracle's for the
    first, a middle and the last sequence."""
    if shape == "k7":
        spec = dict(seed=9, vocab=1000, hidden=7 * 64, layers=2, heads=7, kv_heads=1, head_dim=64, inter=320,
                    max_pos=64, lm_head_int16=0, attention_bias=1)
    else:
        spec = dict(seed=10, vocab=1000, hidden=32 * 128, layers=1, heads=32, kv_heads=4, head_dim=128, inter=4160,
                    max_pos=64, lm_head_int16=1, attention_bias=0)
    case(f"fragment products, {rows} rows, {spec}")
    gm, om = build(backend, spec)
    r = np.random.default_rng(rows * 3 + len(shape))
    lens = [int(n) for n in r.integers(1, 4, rows)]
    toks = [r.integers(0, spec["vocab"], n + 1) for n in lens]
    runs = {}
    for mode in ("0", "1"):
        monkeypatch.setenv("MYL_BATCH_FRAG", mode)
        gm.batch_begin(rows)
        pre = [(s, p) for s, n in enumerate(lens) for p in range(n)]
        gm.forward_batch([s for s, _ in pre], [p for _, p in pre], [int(toks[s][p]) for s, p in pre],
                         want_logits=False)
        logits, am = gm.forward_batch(list(range(rows)), lens, [int(toks[s][n]) for s, n in enumerate(lens)])
        out = gm.batch_decode_greedy(range(rows), [n + 1 for n in lens], [int(a) for a in am], 2)
        runs[mode] = (np.array(logits), np.array(am), np.array(out))
    for a, b, what in zip(runs["0"], runs["1"], ("logits", "argmax", "greedy tokens")):
        assert np.array_equal(a, b), what
    for s in sorted({0, rows // 2, rows - 1}):
        om.reset()
        for p in range(lens[s] + 1):
            ref = om.forward_token(int(toks[s][p]), p)
        assert np.array_equal(runs["1"][0][s], ref), ("decode row", s)


@pytest.mark.parametrize("variant", ["zero", "long_tail"])
def test_batch_decode_rows_exp_table_variants(backend, variant):
    """Decode batches with an all-zero exp table (every head sum is 0: the
    uniform split, softmax.rs:42-48, inside the P.V kernel) and with one whose
    nonzero entries run past the 4096 the P.V kernel copies into LDS (the
    probabilities then come from their own kernel): logits and greedy tokens
    equal each sequence's own forward_token run."""
    from myelith_amd.luts import LutSet
    from myelith_amd.model import IntegerModel
    from oracle.binding import OracleModel
    spec = dict(seed=6, vocab=1000, hidden=7 * 64, layers=2, heads=7, kv_heads=1, head_dim=64, inter=320,
                max_pos=640, lm_head_int16=0, attention_bias=1)
    case(f"batch decode rows, exp table {variant} {spec}")
    base = LutSet.for_head_dim(64)
    exp = np.asarray(base.exp, dtype=np.int16).copy()
    if variant == "zero":
        exp[:] = 0
    else:
        exp[2600:6000] = np.maximum(exp[2600:6000], 1)
    luts = LutSet.from_tables(64, base.rsqrt, base.silu, exp, base.cos, base.sin)
    gm, om = IntegerModel(backend, spec, luts), OracleModel(spec, luts, threads=16)
    r = np.random.default_rng(len(variant))
    lens = [1, 64, 257, 300]
    toks = [r.integers(0, spec["vocab"], n + 1) for n in lens]
    S = len(lens)
    gm.batch_begin(S)
    rows = [(s, p) for s, n in enumerate(lens) for p in range(n)]
    gm.forward_batch([s for s, _ in rows], [p for _, p in rows], [int(toks[s][p]) for s, p in rows],
                     want_logits=False)
    logits, am = gm.forward_batch(list(range(S)), lens, [int(toks[s][n]) for s, n in enumerate(lens)])
    first = []
    for s, n in enumerate(lens):
        om.reset()
        for p in range(n + 1):
            ref = om.forward_token(int(toks[s][p]), p)
        assert np.array_equal(logits[s], ref), ("decode row", s, n)
        first.append(int(np.argmax(ref)))
    steps = 3
    out = gm.batch_decode_greedy(range(S), [n + 1 for n in lens], first, steps)
    for s, n in enumerate(lens):
        om.reset()
        for p in range(n + 1):
            logits_o = om.forward_token(int(toks[s][p]), p)
        nxt, exp_t = int(np.argmax(logits_o)), []
        for i in range(steps):
            logits_o = om.forward_token(nxt, n + 1 + i)
            nxt = int(np.argmax(logits_o))
            exp_t.append(nxt)
        assert [int(t) for t in out[:, s]] == exp_t, s


def test_logsoftmax_dev(backend, oracle):
    import torch
    from myelith_amd.luts import exp_lut
    lut = exp_lut()
    r = np.random.default_rng(17)
    for M, n in ((1, 1), (3, 7), (5, 1000), (4, 152064)):
        case(f"logsoftmax M={M} n={n}")
        z = r.integers(-30000, 30000, (M, n)).astype(np.int32)
        z[:, 0] = z[:, -1]
        t = r.integers(0, n, M).astype(np.int64)
        t[0] = -1
        got = backend.logsoftmax_dev(torch.from_numpy(z).cuda(), lut, t).cpu().numpy()
        exp = np.array([oracle.logsoftmax_at(z[i], lut, int(t[i])) for i in range(M)], np.int64)
        assert np.array_equal(got, exp)


def test_qwen7b_teacher_forced_rows(backend):
    """Qwen2.5-7B architecture at full size (int16 LM head on the matrix
    cores): two sequences x 20 teacher-forced positions in one 40-row batch;
    every row's logits and the per-sequence integer log-softmax sums equal the
    oracle's."""
    import torch
    from myelith_amd.model import QWEN25_7B, make_spec
    from oracle.binding import logsoftmax_at
    spec = make_spec(QWEN25_7B, seed=7, max_pos=64)
    case("qwen2.5-7b teacher-forced 2 x 20")
    gm, om = build(backend, spec)
    r = np.random.default_rng(44)
    T = 20
    toks = [r.integers(0, spec["vocab"], T) for _ in range(2)]
    gm.batch_begin(2)
    seq = [s for s in range(2) for _ in range(T)]
    pos = [p for _ in range(2) for p in range(T)]
    logits, _ = gm.forward_batch(seq, pos, [int(toks[s][p]) for s, p in zip(seq, pos)])
    ref = oracle_rows(om, toks)
    for i, (s, p) in enumerate(zip(seq, pos)):
        assert np.array_equal(logits[i], ref[s][p]), ("row", s, p)
    lut = gm.luts.exp
    targets = np.array([int(toks[s][p + 1]) if p + 1 < T else -1 for s, p in zip(seq, pos)], np.int64)
    lp = backend.logsoftmax_dev(gm.batch_logits_dev(len(seq)), lut, targets).cpu().numpy()
    for s in range(2):
        exp = sum(logsoftmax_at(ref[s][p], lut, int(toks[s][p + 1])) for p in range(T - 1))
        assert int(lp[s * T:(s + 1) * T].sum()) == exp
    torch.cuda.synchronize()
