"""GPU parity of the device-resident model against the oracle's IntegerModel.

Compared bit for bit: every step's logits, the KV cache (kv_cache.rs), the
pipeline-stage API (embed_token / run_layers / head_logits, model.rs:323-399),
the greedy token stream and the generate.rs:98-137 logits digest.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import case

pytestmark = pytest.mark.gpu


def tiny(hd=64, lm16=0, bias=1, kv_heads=2, layers=2, max_pos=640, seed=11):
    heads = 4 if kv_heads <= 2 else 8
    return dict(seed=seed, vocab=1000, hidden=heads * hd, layers=layers, heads=heads, kv_heads=kv_heads, head_dim=hd,
                inter=320, max_pos=max_pos, lm_head_int16=lm16, attention_bias=bias)


def build(backend, spec, threads=16):
    from myelith_amd.luts import LutSet
    from myelith_amd.model import IntegerModel
    from oracle.binding import OracleModel
    luts = LutSet.for_head_dim(spec["head_dim"])
    return IntegerModel(backend, spec, luts), OracleModel(spec, luts, threads=threads)


def compare_kv(gm, om, spec, n_pos):
    for l in range(spec["layers"]):
        for h in range(spec["kv_heads"]):
            gk, gv = gm.read_kv(l, h, n_pos)
            ok, ov = om.read_kv(l, h, n_pos)
            assert np.array_equal(gk, ok), ("K", l, h)
            assert np.array_equal(gv, ov), ("V", l, h)


@pytest.mark.parametrize("hd,lm16,bias,kvh", [(64, 0, 1, 2), (64, 1, 0, 1), (128, 1, 1, 2), (128, 0, 1, 4)])
def test_tiny_forward_parity(backend, hd, lm16, bias, kvh):
    spec = tiny(hd, lm16, bias, kvh)
    case(f"tiny forward {spec}")
    gm, om = build(backend, spec)
    r = np.random.default_rng(hd + lm16 + bias)
    toks = r.integers(0, spec["vocab"], 300)
    for pos, t in enumerate(toks):  # 300 positions: two attention chunks
        g = gm.forward_token(int(t), pos)
        o = om.forward_token(int(t), pos)
        assert np.array_equal(g, o), f"logits differ at pos {pos}"
        assert gm.last_argmax == int(np.argmax(o))
    compare_kv(gm, om, spec, len(toks))


@pytest.mark.parametrize("heads,kvh", [(6, 3), (16, 16)])
def test_decode_kv_heads_not_dividing_eight(backend, heads, kvh):
    """KV-head counts that do not divide the 8 XCDs take the attention's
    three-dimensional launch shape (and 16 KV heads with one query head
    each): 200 positions, logits and KV cache equal the oracle's."""
    spec = dict(seed=9, vocab=1000, hidden=heads * 64, layers=2, heads=heads, kv_heads=kvh, head_dim=64, inter=320,
                max_pos=256, lm_head_int16=0, attention_bias=1)
    case(f"decode kv heads {spec}")
    gm, om = build(backend, spec)
    toks = np.random.default_rng(heads + kvh).integers(0, spec["vocab"], 200)
    for pos, t in enumerate(toks):
        assert np.array_equal(gm.forward_token(int(t), pos), om.forward_token(int(t), pos)), pos
    compare_kv(gm, om, spec, len(toks))


def test_device_weights_match_the_synthetic_definition(backend):
    spec = tiny(64, 1, 1, 2)
    case("device-generated weights")
    gm, om = build(backend, spec)
    H, hd = spec["hidden"], spec["head_dim"]
    nq, nkv = spec["heads"] * hd, spec["kv_heads"] * hd
    w = gm.read_tensor("wqkv", 1, (nq + 2 * nkv) * H).reshape(-1, H)
    wq = om.tensor("wq", 1).reshape(nq, H)
    half = hd // 2
    for o in range(nq):  # pair order: rows 2i, 2i+1 of a head are (j, j + hd/2)
        head, j = divmod(o, hd)
        d = head * hd + (2 * j if j < half else 2 * (j - half) + 1)
        assert np.array_equal(w[d], wq[o])
    assert np.array_equal(gm.read_tensor("emb", 0, spec["vocab"] * H), om.tensor("emb"))
    assert np.array_equal(gm.read_tensor("lm16", 0, spec["vocab"] * H * 2, np.int16), om.tensor("lm16", 0, np.int16))
    wgu = gm.read_tensor("wgu", 0, 2 * spec["inter"] * H).reshape(-1, H)
    assert np.array_equal(wgu[0::2], om.tensor("wg", 0).reshape(-1, H))
    assert np.array_equal(wgu[1::2], om.tensor("wu", 0).reshape(-1, H))


def test_stage_api_parity(backend):
    spec = tiny(128, 1, 1, 2, layers=3)
    case("embed_token / run_layers / head_logits")
    gm, om = build(backend, spec)
    for pos, t in enumerate((5, 999, 0, 123)):
        he = gm.embed_token(t)
        assert np.array_equal(he, om.embed_token(t))
        h1 = gm.run_layers(he, pos, 0, 2)
        assert np.array_equal(h1, om.run_layers(he, pos, 0, 2))
        h2 = gm.run_layers(h1, pos, 2, 3)
        assert np.array_equal(h2, om.run_layers(h1, pos, 2, 3))
        assert np.array_equal(gm.head_logits(h2), om.head_logits(h2))


def test_rope_row_wraps_past_2048(backend):
    """Positions >= 2048 reuse LUT row pos % 2048 (model.rs:469-471)."""
    spec = tiny(64, 0, 1, 2, layers=1, max_pos=2200)
    case("rope wrap 2200 positions")
    gm, om = build(backend, spec)
    r = np.random.default_rng(3)
    toks = r.integers(0, spec["vocab"], 2200)
    for pos, t in enumerate(toks):
        g = gm.forward_token(int(t), pos, want_logits=pos >= 2040)
        o = om.forward_token(int(t), pos, want_logits=pos >= 2040)
        if pos >= 2040:
            assert np.array_equal(g, o), pos
    compare_kv(gm, om, spec, 2200)


def test_decode_greedy_digest(backend):
    from myelith_amd.model import dekodieren_mit_digest
    spec = tiny(128, 1, 1, 2)
    case("greedy decode + digest")
    gm, om = build(backend, spec)
    prompt = [17, 3, 999, 42, 7]
    toks_o, dig_o = dekodieren_mit_digest(om, prompt, 40)
    toks_g, dig_g = dekodieren_mit_digest(gm, prompt, 40)
    assert toks_g == toks_o and dig_g == dig_o
    # the on-device greedy chain gives the same tokens and logits
    gm.reset()
    logits = None
    for pos, t in enumerate(prompt):
        logits = gm.forward_token(t, pos)
    first = int(np.argmax(logits))
    dev_toks, dev_logits = gm.decode_greedy(first, len(prompt), 39, want_logits=True)
    assert [first] + [int(t) for t in dev_toks] == toks_o[:40]
    om.reset()
    for pos, t in enumerate(prompt):
        om.forward_token(t, pos)
    for i, t in enumerate([first] + list(dev_toks[:-1])):
        assert np.array_equal(dev_logits[i], om.forward_token(int(t), len(prompt) + i))


def test_sampled_digest(backend):
    """dekodieren_mit_digest with greedy false (generate.rs:98-137): each
    token drawn by sample_integer_cdf (sampling.rs:27-46) from the step's
    logits with the SplitMix64 state carried across steps; tokens and digest
    equal the oracle's for two seeds."""
    from myelith_amd.model import dekodieren_mit_digest
    spec = tiny(64, 0, 1, 2)
    case("sampled decode + digest")
    gm, om = build(backend, spec)
    prompt = [5, 77, 901, 3]
    for seed in (0, 0xDEADBEEF12345678):
        toks_g, dig_g = dekodieren_mit_digest(gm, prompt, 24, seed=seed, greedy=False)
        toks_o, dig_o = dekodieren_mit_digest(om, prompt, 24, seed=seed, greedy=False)
        assert toks_g == toks_o and dig_g == dig_o, seed
    assert dekodieren_mit_digest(gm, prompt, 24, seed=1, greedy=False)[0] != \
        dekodieren_mit_digest(gm, prompt, 24, greedy=True)[0]


def test_qwen05b_config1_prompt256_decode128(backend):
    """Qwen2.5-0.5B architecture: 256-token seeded prompt + 128 greedy steps:
    identical digest, tokens and KV cache."""
    from myelith_amd.model import QWEN25_05B, dekodieren_mit_digest, make_spec
    spec = make_spec(QWEN25_05B, seed=2025, max_pos=512)
    case("qwen2.5-0.5b shape, 256 + 128")
    gm, om = build(backend, spec)
    r = np.random.default_rng(256)
    prompt = [int(t) for t in r.integers(0, spec["vocab"], 256)]
    toks_g, dig_g = dekodieren_mit_digest(gm, prompt, 128)
    toks_o, dig_o = dekodieren_mit_digest(om, prompt, 128)
    assert toks_g == toks_o
    assert dig_g == dig_o
    compare_kv(gm, om, spec, 256 + 128)


def test_qwen7b_fullsize_decode(backend):
    """Qwen2.5-7B architecture at full size (int16 LM head): a 6-token prompt
    and 4 greedy steps, identical digest."""
    from myelith_amd.model import QWEN25_7B, dekodieren_mit_digest, make_spec
    spec = make_spec(QWEN25_7B, seed=7, max_pos=64)
    case("qwen2.5-7b shape, 6 + 4")
    gm, om = build(backend, spec)
    prompt = [1, 151000, 77, 4242, 9, 152063]
    toks_g, dig_g = dekodieren_mit_digest(gm, prompt, 4)
    toks_o, dig_o = dekodieren_mit_digest(om, prompt, 4)
    assert toks_g == toks_o and dig_g == dig_o


@pytest.mark.parametrize("hd,lm16,kvh", [(128, 1, 2), (64, 0, 1)])
def test_prefill_rows_match_the_token_loop(backend, hd, lm16, kvh):
    """Prompts of 16 tokens and more run as one batch of rows over the
    model's own KV cache: the last logits, every cached K/V entry and the
    greedy continuation equal the reference's token-by-token prompt loop
    (generate.rs:28-32), also when a second prompt continues the cache."""
    spec = tiny(hd, lm16, 1, kvh, layers=2, max_pos=640)
    case(f"prefill rows hd={hd} lm16={lm16} kvh={kvh}")
    gm, om = build(backend, spec)
    r = np.random.default_rng(hd * 7 + lm16)
    p1 = [int(t) for t in r.integers(0, spec["vocab"], 300)]
    p2 = [int(t) for t in r.integers(0, spec["vocab"], 40)]
    g = gm.prefill(p1, 0)
    o = None
    for pos, t in enumerate(p1):
        o = om.forward_token(t, pos)
    assert np.array_equal(g, o)
    compare_kv(gm, om, spec, 300)
    g = gm.prefill(p2, 300)
    for i, t in enumerate(p2):
        o = om.forward_token(t, 300 + i)
    assert np.array_equal(g, o)
    compare_kv(gm, om, spec, 340)
    first = int(np.argmax(o))
    toks, _ = gm.decode_greedy(first, 340, 12)
    want = []
    t = first
    for i in range(12):
        o = om.forward_token(t, 340 + i)
        t = int(np.argmax(o))
        want.append(t)
    assert [int(x) for x in toks] == want
    # a short prompt (token loop) after the row path, re-running positions
    g = gm.prefill(p2[:5], 338)
    for i, t in enumerate(p2[:5]):
        o = om.forward_token(t, 338 + i)
    assert np.array_equal(g, o)


@pytest.mark.gpu
def test_backend_close_closes_its_models():
    """A model still referenced when its backend closes (as a failed test's
    frames keep it) is closed first, so its later finalisation does nothing."""
    from myelith_amd.backend import RocmBackend
    from myelith_amd.model import IntegerModel
    case("backend close order")
    b = RocmBackend(0)
    m = IntegerModel(b, tiny())
    b.close()
    assert m._h is None
    m.close()
    del m


def test_decode_with_a_long_exp_table_tail(backend):
    """An exp table whose nonzero entries run past what the decode P.V kernel
    copies into LDS (4096) is read in place; logits still match the oracle."""
    from myelith_amd.luts import LutSet
    from myelith_amd.model import IntegerModel
    from oracle.binding import OracleModel
    spec = tiny(128, 0, 1, 2)
    case(f"long exp tail {spec}")
    base = LutSet.for_head_dim(128)
    exp = np.asarray(base.exp, dtype=np.int16).copy()
    exp[2600:6000] = np.maximum(exp[2600:6000], 1)
    luts = LutSet.from_tables(128, base.rsqrt, base.silu, exp, base.cos, base.sin)
    gm, om = IntegerModel(backend, spec, luts), OracleModel(spec, luts, threads=16)
    r = np.random.default_rng(5)
    for pos, t in enumerate(r.integers(0, spec["vocab"], 160)):
        assert np.array_equal(gm.forward_token(int(t), pos), om.forward_token(int(t), pos)), pos


@pytest.mark.parametrize("hd,variant", [(64, "negative"), (128, "negative"), (128, "zero")])
def test_decode_attention_exp_table_variants(backend, hd, variant):
    """Exp tables unlike the calibrated one: negative entries (probabilities
    outside [0, 2^14], negative and wrapping sums) and an all-zero table
    (every head sum is 0: softmax.rs:37-44 splits one / L uniformly)."""
    from myelith_amd.luts import LutSet
    from myelith_amd.model import IntegerModel
    from oracle.binding import OracleModel
    spec = tiny(hd, 0, 1, 2)
    case(f"exp table {variant} {spec}")
    base = LutSet.for_head_dim(hd)
    exp = np.asarray(base.exp, dtype=np.int16).copy()
    if variant == "negative":
        exp[1:600:3] = -exp[1:600:3]
    else:
        exp[:] = 0
    luts = LutSet.from_tables(hd, base.rsqrt, base.silu, exp, base.cos, base.sin)
    gm, om = IntegerModel(backend, spec, luts), OracleModel(spec, luts, threads=16)
    r = np.random.default_rng(hd + len(variant))
    for pos, t in enumerate(r.integers(0, spec["vocab"], 200)):
        assert np.array_equal(gm.forward_token(int(t), pos), om.forward_token(int(t), pos)), pos
    compare_kv(gm, om, spec, 200)


@pytest.mark.parametrize("hd,kvh,variant", [(64, 2, "calibrated"), (128, 1, "calibrated"), (64, 1, "zero"),
                                             (128, 2, "zero")])
def test_decode_attention_short_cache(backend, hd, kvh, variant):
    """A cache of at most 512 (head_dim 64) or 256 (head_dim 128) positions
    takes the one-kernel attention (a block per query head): every position
    up to the full cache, through the token loop and the captured step graph,
    with the calibrated table and an all-zero one (the uniform split); logits
    and KV cache equal the oracle's."""
    from myelith_amd.luts import LutSet
    from myelith_amd.model import IntegerModel
    from oracle.binding import OracleModel
    max_pos = 512 if hd == 64 else 256
    spec = tiny(hd, 0, 1, kvh, max_pos=max_pos)
    case(f"short cache {variant} {spec}")
    base = LutSet.for_head_dim(hd)
    exp = np.asarray(base.exp, dtype=np.int16).copy()
    if variant == "zero":
        exp[:] = 0
    luts = LutSet.from_tables(hd, base.rsqrt, base.silu, exp, base.cos, base.sin)
    gm, om = IntegerModel(backend, spec, luts), OracleModel(spec, luts, threads=16)
    r = np.random.default_rng(hd + kvh + len(variant))
    n_loop = max_pos - 40
    for pos, t in enumerate(r.integers(0, spec["vocab"], n_loop)):
        assert np.array_equal(gm.forward_token(int(t), pos), om.forward_token(int(t), pos)), pos
    t = int(r.integers(0, spec["vocab"]))
    toks, logits = gm.decode_greedy(t, n_loop, 40, want_logits=True)
    for i in range(40):
        ref = om.forward_token(t, n_loop + i)
        assert np.array_equal(logits[i], ref), n_loop + i
        t = int(np.argmax(ref))
        assert int(toks[i]) == t, n_loop + i
    compare_kv(gm, om, spec, max_pos)


def test_decode_rsqrt_table_unlike_its_closed_form(backend):
    """An rsqrt table that differs from round(2^8 / sqrt(x / 2^8)) at every
    odd index: the norm factor must come from the table (the closed form is
    used only when every entry matches), for both decode and prompt rows."""
    from myelith_amd.luts import LutSet
    from myelith_amd.model import IntegerModel
    from oracle.binding import OracleModel
    spec = tiny(64, 0, 1, 2)
    case(f"rsqrt table unlike its closed form {spec}")
    base = LutSet.for_head_dim(64)
    rsqrt = np.asarray(base.rsqrt, dtype=np.int16).copy()
    rsqrt[1::2] += 3
    luts = LutSet.from_tables(64, rsqrt, base.silu, base.exp, base.cos, base.sin)
    gm, om = IntegerModel(backend, spec, luts), OracleModel(spec, luts, threads=16)
    r = np.random.default_rng(5)
    prompt = [int(t) for t in r.integers(0, spec["vocab"], 24)]
    g = gm.prefill(prompt, 0)
    for pos, t in enumerate(prompt):
        o = om.forward_token(t, pos)
    assert np.array_equal(g, o)
    for i, t in enumerate(r.integers(0, spec["vocab"], 40)):
        pos = len(prompt) + i
        assert np.array_equal(gm.forward_token(int(t), pos), om.forward_token(int(t), pos)), pos
    compare_kv(gm, om, spec, len(prompt) + 40)


def test_decode_past_4096_positions(backend):
    """Decode attention over more than 4096 cached positions with four KV
    heads (the P.V kernel's scores no longer fit its registers and are read
    in place): a 4130-token prompt, then decode steps past 4096."""
    spec = tiny(128, 0, 1, 4, layers=1, max_pos=4300)
    case(f"decode past 4096 positions {spec}")
    gm, om = build(backend, spec)
    r = np.random.default_rng(23)
    p = [int(t) for t in r.integers(0, spec["vocab"], 4130)]
    gm.prefill(p, 0)
    # the prompt's rows are checked elsewhere; the oracle continues from the
    # device's cache
    for l in range(spec["layers"]):
        for h in range(spec["kv_heads"]):
            om.write_kv(l, h, *gm.read_kv(l, h, 4130))
    om.set_cached(4130)
    for i, t in enumerate(r.integers(0, spec["vocab"], 6)):
        pos = 4130 + i
        assert np.array_equal(gm.forward_token(int(t), pos), om.forward_token(int(t), pos)), pos
    compare_kv(gm, om, spec, 4136)


def test_long_prompt_rows_match_the_oracle(backend):
    """A 4200-token prompt runs as three chunks of rows (2048, 2048, 104):
    the softmax kernel's register path (a wave per (row, head), rows up to
    1024 positions), its re-reading path for longer rows, and the four-wave
    path for few rows past 4096 positions.  Layer 1's K/V at every position
    depend on layer 0's attention for that row."""
    spec = tiny(64, 0, 1, 2, layers=2, max_pos=4300)
    case(f"long prompt rows {spec}")
    gm, om = build(backend, spec)
    r = np.random.default_rng(17)
    p = [int(t) for t in r.integers(0, spec["vocab"], 4200)]
    g = gm.prefill(p, 0)
    o = None
    for pos, t in enumerate(p):
        o = om.forward_token(t, pos)
    assert np.array_equal(g, o)
    compare_kv(gm, om, spec, 4200)


def test_repeated_gate_up_leaves_the_decode_unchanged(backend):
    """The measurement hook that launches each layer's gate/up GEMV twice per
    step (captured graph and eager launches) gives the oracle's tokens and
    logits."""
    spec = tiny(128, 1, 1, 2, layers=3)
    case("gate/up repeated twice")
    gm, om = build(backend, spec)
    prompt = [17, 3, 999, 42, 7]
    for pos, t in enumerate(prompt):
        o = om.forward_token(t, pos)
    gm.set_kernel_repeat("gate_up", 2)
    g = gm.prefill(prompt, 0)
    assert np.array_equal(g, o)
    first = int(np.argmax(o))
    toks, logits = gm.decode_greedy(first, len(prompt), 10, want_logits=True)
    t = first
    for i in range(10):
        ref = om.forward_token(t, len(prompt) + i)
        assert np.array_equal(logits[i], ref), i
        t = int(np.argmax(ref))
        assert int(toks[i]) == t, i
    gm.set_kernel_repeat("gate_up", 1)
    with pytest.raises(ValueError):
        gm.set_kernel_repeat("down", 2)
    with pytest.raises(ValueError):  # more repeats than the model's 3 layers
        gm.set_kernel_repeat("gate_up", 4)
