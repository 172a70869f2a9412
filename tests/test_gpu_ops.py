"""GPU parity of every op of the path against the CPU oracle (bit-exact).

Each test names its case before touching the GPU.  Inputs are seeded; sizes
go from the reference's own edge cases (length 1, odd lengths, extremes,
all-masked softmax, ties in argmax) up to the 7B shapes of the W8A16 sweep.
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

from conftest import case

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"


def rng(seed):
    return np.random.default_rng(seed)


def gauss16(r, n, sigma=2000):
    return np.clip(np.rint(r.normal(0, sigma, n)), -32767, 32767).astype(np.int16)


# ---- conformance vectors through the backend (golden_runner.rs:117-131) ------------

def test_conformance_vectors_on_gpu(backend):
    vecs = json.loads((GOLDEN / "op_vectors.json").read_text())
    case("conformance linear_w8a16_identity")
    v = vecs["linear_w8a16_identity"]
    m = v["metadata"]
    W = np.array(m["W"], np.int8)
    y = backend.linear_w8a16(v["inputs"]["x"]["data"], W.ravel(), W.shape[1], W.shape[0],
                             [m["weight_frac"]] * W.shape[0], m["act_frac"], m["out_frac"])
    assert list(y) == v["outputs"]["y"]["data"]
    case("conformance rmsnorm_basic")
    v = vecs["rmsnorm_basic"]
    m = v["metadata"]
    x = v["inputs"]["x"]["data"]
    y = backend.rmsnorm(x, [0] * len(x), v["inputs"]["gamma"]["data"], [m["gamma_shift"]] * len(x), m["rsqrt_lut"],
                        m["lut_input_shift"], m["lut_output_frac"], m["inv_n_q20"], m["out_frac"])
    assert list(y) == v["outputs"]["y"]["data"]
    case("conformance softmax_basic")
    v = vecs["softmax_basic"]
    m = v["metadata"]
    y = backend.softmax(v["inputs"]["logits"]["data"], m["exp_lut"], m["lut_shift"], m["frac_bits"])
    assert list(y) == v["outputs"]["probs"]["data"]


# ---- linear ------------------------------------------------------------------------------

@pytest.mark.parametrize("N,K", [(1, 1), (3, 5), (37, 53), (64, 16), (65, 896), (129, 4864), (300, 3584),
                                 (130, 18944), (7, 131)])
def test_linear_w8a16_trait(backend, oracle, N, K):
    case(f"linear_w8a16 trait N={N} K={K}")
    r = rng(N * 1000 + K)
    x = gauss16(r, K)
    W = r.integers(-128, 128, (N, K)).astype(np.int8)
    ws = r.integers(0, 16, N).astype(np.uint8)
    for act, out in ((10, 8), (4, 12), (0, 0)):
        ref = oracle.linear_w8a16(x, W.ravel(), K, ws, act, out)
        got = backend.linear_w8a16(x, W.ravel(), K, N, ws, act, out)
        assert np.array_equal(ref, got), (N, K, act, out)
    of = r.integers(2, 14, N).astype(np.uint8)
    assert np.array_equal(oracle.linear_w8a16_pc(x, W.ravel(), K, ws, 9, of),
                          backend.linear_w8a16_pc(x, W.ravel(), K, ws, 9, of))


def test_linear_extremes(backend, oracle):
    case("linear extremes")
    for K in (896, 3584, 18944):
        x = np.full(K, -32768, np.int16)
        W = np.full((3, K), -128, np.int8)
        W[1] = 127
        W[2, ::2] = -128
        W[2, 1::2] = 127
        ws = np.array([0, 7, 20], np.uint8)
        for act, out in ((0, 0), (5, 30), (20, 0)):
            assert np.array_equal(oracle.linear_w8a16(x, W.ravel(), K, ws, act, out),
                                  backend.linear_w8a16(x, W.ravel(), K, 3, ws, act, out))
        import torch
        xd = torch.from_numpy(np.stack([x, -x - 1])).cuda()
        Wd = torch.from_numpy(W).cuda()
        got = backend.dot_i8_i16_dev(xd, Wd).cpu().numpy()
        exp = np.stack([W.astype(np.int64) @ x.astype(np.int64), W.astype(np.int64) @ (-x.astype(np.int64) - 1)])
        assert np.array_equal(got, exp)


def test_linear_rejects_what_the_reference_panics_on(backend):
    case("linear invalid")
    with pytest.raises(ValueError):
        backend.linear_w8a16([1, 2], [1, 2, 3], 2, 2, [0, 0], 0, 0)  # W too short (linear.rs:51-58)


SWEEP = [(3584, 3584), (18944, 3584), (3584, 18944), (152064, 3584)]


def exact_sums(x, W, chunk=16384):
    """x [M x K] int16 times W [N x K] int8 as exact i64 sums: every product
    and partial sum is an integer below 2^53, so float64 arithmetic is exact
    in any summation order."""
    xf = x.astype(np.float64)
    out = np.empty((x.shape[0], W.shape[0]), np.int64)
    for n0 in range(0, W.shape[0], chunk):
        out[:, n0:n0 + chunk] = (xf @ W[n0:n0 + chunk].astype(np.float64).T).astype(np.int64)
    return out


@pytest.mark.parametrize("N,K", SWEEP)
@pytest.mark.parametrize("M", [1, 8, 64, 512])
def test_w8a16_sweep_shapes_dev(backend, oracle, M, N, K):
    """The W8A16 sweep cells (M x N x K) at their full size, so each takes
    the tile it runs in the benchmark (e.g. M = 8 x N = 152064 the K-split
    32-row plane tiles of 128 weight rows): shift requant and multiplier
    requant against the oracle's requant of the exact sums, and a row
    subset against the oracle's own linear_w8a16."""
    import torch
    case(f"sweep M={M} N={N} K={K}")
    r = rng(M * 7 + N * 3 + K)
    x = gauss16(r, M * K).reshape(M, K)
    W = r.integers(-127, 128, (N, K)).astype(np.int8)
    ws = r.integers(8, 14, N).astype(np.uint8)
    mult = r.integers(1 << 29, (1 << 30) + 1, N).astype(np.int32)
    sh = r.integers(20, 41, N).astype(np.uint8)
    oracle.lib().or_set_threads(16)
    xd, Wd = torch.from_numpy(x).cuda(), torch.from_numpy(W).cuda()
    got_s = backend.linear_w8a16_dev(xd, Wd, torch.from_numpy(ws).cuda(), 11, 10).cpu().numpy()
    got_m = backend.linear_w8a16_mult_dev(xd, Wd, torch.from_numpy(mult).cuda(), torch.from_numpy(sh).cuda())
    got_m = got_m.cpu().numpy()
    # multiplier = 2^k with shift = k + reference shift reproduces the reference rescale
    k = 29
    m2 = np.full(N, 1 << k, np.int32)
    s2 = (ws.astype(np.int32) + 11 - 10 + k).astype(np.uint8)
    got_2 = backend.linear_w8a16_mult_dev(xd, Wd, torch.from_numpy(m2).cuda(), torch.from_numpy(s2).cuda())
    got_2 = got_2.cpu().numpy()
    acc = exact_sums(x, W)
    want_s = oracle.requant_shift(acc, ws, 11, 10)
    assert np.array_equal(got_s, want_s)
    assert np.array_equal(got_m, oracle.requant_mult(acc, mult, sh))
    assert np.array_equal(got_2, want_s)
    rows = np.unique(np.concatenate([np.arange(min(N, 64)), r.integers(0, N, 192)]))
    assert np.array_equal(got_s[:, rows], oracle.linear_batch(x, W[rows], ws[rows], 11, 10))


# ---- matrix-core path (M > 8): every tile shape, with and without K splits ----------

MM_CASES = [(9, 37, 48), (33, 100, 208), (64, 130, 3584), (130, 257, 1040), (300, 64, 18944), (17, 5, 16)]


@pytest.mark.parametrize("tile", [0, 1, 2, 3])
@pytest.mark.parametrize("ksplit", [1, 3])
def test_mfma_tiles_and_splits(backend, oracle, monkeypatch, tile, ksplit):
    """Odd M/N/K (partial tiles, K tails of 16 bytes) through each forced tile
    shape and K split, against the oracle; shift and multiplier requant."""
    import torch
    monkeypatch.setenv("MYL_MM_TILE", str(tile))
    monkeypatch.setenv("MYL_MM_KSPLIT", str(ksplit))
    oracle.lib().or_set_threads(16)
    for M, N, K in MM_CASES:
        case(f"mfma tile={tile} ksplit={ksplit} M={M} N={N} K={K}")
        r = rng(M * 31 + N * 7 + K + tile)
        x = gauss16(r, M * K).reshape(M, K)
        x[0, :4] = (-32768, 32767, -1, 0)
        W = r.integers(-128, 128, (N, K)).astype(np.int8)
        ws = r.integers(8, 14, N).astype(np.uint8)
        xd, Wd = torch.from_numpy(x).cuda(), torch.from_numpy(W).cuda()
        got = backend.linear_w8a16_dev(xd, Wd, torch.from_numpy(ws).cuda(), 11, 10).cpu().numpy()
        assert np.array_equal(got, oracle.linear_batch(x, W, ws, 11, 10)), (M, N, K)
        mult = r.integers(1 << 29, (1 << 30) + 1, N).astype(np.int32)
        sh = r.integers(20, 41, N).astype(np.uint8)
        got = backend.linear_w8a16_mult_dev(xd, Wd, torch.from_numpy(mult).cuda(), torch.from_numpy(sh).cuda())
        assert np.array_equal(got.cpu().numpy(), oracle.linear_mult(x, W, mult, sh)), (M, N, K)
        raw = backend.dot_i8_i16_dev(xd, Wd).cpu().numpy()
        assert np.array_equal(raw, x.astype(np.int64) @ W.astype(np.int64).T), (M, N, K)


def test_mfma_extremes(backend):
    """All-extreme operands: every partial sum at its bound (K = 18944)."""
    import torch
    case("mfma extremes")
    K = 18944
    x = np.full((16, K), -32768, np.int16)
    x[1] = 32767
    x[2, ::2] = -32768
    x[2, 1::2] = 32767
    x[3] = -1
    W = np.full((40, K), -128, np.int8)
    W[1] = 127
    W[2, ::2] = -128
    W[2, 1::2] = 127
    got = backend.dot_i8_i16_dev(torch.from_numpy(x).cuda(), torch.from_numpy(W).cuda()).cpu().numpy()
    assert np.array_equal(got, x.astype(np.int64) @ W.astype(np.int64).T)


@pytest.mark.parametrize("M,N,K", [(300, 30000, 192), (1030, 8000, 128), (4096, 4608, 3584), (2049, 37888, 64)])
def test_mfma_large_m_byte_plane_product(backend, oracle, M, N, K):
    """M >= 256: activations split into interleaved byte-plane rows, the pipelined
    int8 product over 2M rows (odd M and N, the smallest K, the 7B q/k/v
    shape).  Exact sums against float64; the requant on sampled rows against
    the oracle."""
    import torch
    case(f"mfma2 M={M} N={N} K={K}")
    g = torch.Generator(device="cuda")
    g.manual_seed(M * 3 + N + K)
    x = torch.randint(-32768, 32768, (M, K), dtype=torch.int16, device="cuda", generator=g)
    x[0, :2] = torch.tensor([-32768, 32767], dtype=torch.int16)
    W = torch.randint(-128, 128, (N, K), dtype=torch.int8, device="cuda", generator=g)
    raw = backend.dot_i8_i16_dev(x, W)
    assert torch.equal(raw, (x.double() @ W.double().T).to(torch.int64))
    del raw
    ws = torch.randint(8, 14, (N,), dtype=torch.uint8, device="cuda", generator=g)
    y = backend.linear_w8a16_dev(x, W, ws, 11, 10).cpu().numpy()
    rows = sorted({0, 1, M // 2, M - 1})
    xs = x[rows].cpu().numpy()
    oracle.lib().or_set_threads(16)
    exp = oracle.linear_batch(xs, W.cpu().numpy(), ws.cpu().numpy(), 11, 10)
    assert np.array_equal(y[rows], exp)


@pytest.mark.parametrize("M", [64, 512])
@pytest.mark.parametrize("N,K", SWEEP)
def test_mfma_full_size_exact_sums(backend, M, N, K):
    """Full sweep sizes: the exact i64 sums equal a float64 matmul on the GPU
    (every partial sum is an integer below 2^53, so float64 is exact), and
    the shift-requant output equals the requant of those sums."""
    import torch
    case(f"mfma full size M={M} N={N} K={K}")
    g = torch.Generator(device="cuda")
    g.manual_seed(M + N + K)
    x = torch.randint(-32768, 32768, (M, K), dtype=torch.int16, device="cuda", generator=g)
    W = torch.randint(-127, 128, (N, K), dtype=torch.int8, device="cuda", generator=g)
    raw = backend.dot_i8_i16_dev(x, W)
    ref = (x.double() @ W.double().T).to(torch.int64)
    assert torch.equal(raw, ref)
    del ref
    # the requant epilogue on the same sums: rows 0..255 against the oracle's rescale
    from oracle import binding as ob
    ws = torch.randint(8, 14, (N,), dtype=torch.uint8, device="cuda", generator=g)
    y = backend.linear_w8a16_dev(x, W, ws, 11, 10)
    r = raw[:, :256].cpu().numpy()
    wsn = ws[:256].cpu().numpy()
    exp = np.vectorize(lambda a, s: max(-32768, min(32767, ob.rescale_i64(int(a), int(s) + 11, 10))))(r, wsn[None, :])
    assert np.array_equal(y[:, :256].cpu().numpy(), exp.astype(np.int16))


@pytest.mark.parametrize("bits", [8, 16])
def test_logits_dev(backend, oracle, bits):
    import torch
    case(f"logits w{bits}")
    r = rng(bits)
    V, H, M = 5000, 896, 3
    x = gauss16(r, M * H).reshape(M, H)
    if bits == 8:
        W = r.integers(-127, 128, (V, H)).astype(np.int8)
    else:
        W = r.integers(-32767, 32768, (V, H)).astype(np.int16)
    sh = r.integers(5, 20, V).astype(np.uint8)
    got = backend.logits_dev(torch.from_numpy(x).cuda(), torch.from_numpy(W).cuda(), torch.from_numpy(sh).cuda(),
                             9, 6).cpu().numpy()
    acc = x.astype(np.int64) @ W.astype(np.int64).T
    for m in range(M):
        for rr in range(0, V, 97):
            y = oracle.rescale_i64(int(acc[m, rr]), (int(sh[rr]) + 9) & 0xFF, 6)
            assert got[m, rr] == max(-2**31, min(2**31 - 1, y))


# ---- rmsnorm / softmax / attention / rope / mlp / bias / argmax ---------------------------

@pytest.mark.parametrize("n", [1, 2, 5, 896, 3584])
def test_rmsnorm(backend, oracle, luts64, n):
    case(f"rmsnorm n={n}")
    r = rng(n)
    lut = luts64.rsqrt
    for trial in range(6):
        x = gauss16(r, n, sigma=[50, 2000, 12000, 30000, 1, 200][trial])
        xs = r.integers(0, [1, 4, 12, 21, 3, 9][trial], n).astype(np.uint8)
        g = r.integers(-127, 128, n).astype(np.int8)
        gs = r.integers(4, 9, n).astype(np.uint8)
        inv = oracle.inv_n_q20(n)
        for of in (6, 10, 0):
            ref = oracle.rmsnorm_i16(x, xs, g, gs, lut, 8, 8, inv, of)
            got = backend.rmsnorm(x, xs, g, gs, lut, 8, 8, inv, of)
            assert np.array_equal(ref, got), (n, trial, of)
    z = np.zeros(n, np.int16)
    assert np.array_equal(backend.rmsnorm(z, np.zeros(n, np.uint8), np.ones(n, np.int8), np.ones(n, np.uint8), lut, 8,
                                          8, oracle.inv_n_q20(n), 6), z)
    with pytest.raises(ValueError):
        backend.rmsnorm([1], [0], [1], [0], lut, 7, 8, 1 << 20, 6)


@pytest.mark.parametrize("n", [896, 3584, 4096, 8192, 904])
def test_rmsnorm_many_rows(backend, oracle, luts64, n):
    """256 rows and more take the vectorized row kernel (8-element chunks,
    64-bit sums at the largest shift, 128-bit for the others); each row must
    match the oracle, with per-channel shift spreads up to 20 bits, rows of
    extreme values and an all-zero row."""
    import torch
    case(f"rmsnorm rows M=300 n={n}")
    r = rng(n + 17)
    M = 300
    x = np.stack([gauss16(r, n, sigma=[40, 3000, 30000][m % 3]) for m in range(M)])
    x[7] = 0
    x[11] = -32768
    x[12] = 32767
    g = r.integers(-127, 128, n).astype(np.int8)
    gs = r.integers(4, 9, n).astype(np.uint8)
    inv = oracle.inv_n_q20(n)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    for xs in (np.full(n, 9, np.uint8), r.integers(0, 21, n).astype(np.uint8)):
        for of in (10, 3):
            got = backend.rmsnorm_dev(T(x), T(xs), T(g), T(gs), T(luts64.rsqrt), 8, 8, inv, of).cpu().numpy()
            for m in range(M):
                ref = oracle.rmsnorm_i16(x[m], xs, g, gs, luts64.rsqrt, 8, 8, inv, of)
                assert np.array_equal(got[m], ref), (n, m, of)


@pytest.mark.parametrize("n", [1, 4, 33, 2304, 152064])
def test_softmax(backend, oracle, n):
    case(f"softmax n={n}")
    from myelith_amd.luts import exp_lut
    lut = exp_lut()
    r = rng(n)
    for spread in (10, 3000, 300000, 2**31 - 1):
        z = r.integers(-spread, spread, n, endpoint=True).astype(np.int64)
        z = np.clip(z, -2**31, 2**31 - 1).astype(np.int32)
        if n > 3:
            z[::3] = np.iinfo(np.int32).min  # masked positions (attention.rs:69)
        for shift, frac in ((6, 14), (4, 8), (0, 2)):
            assert np.array_equal(oracle.softmax_int(z, lut, shift, frac), backend.softmax(z, lut, shift, frac))
    # all-zero LUT -> uniform fallback with remainder (softmax.rs:42-48)
    zl = np.zeros(5, np.int16)
    z = r.integers(-100, 100, n).astype(np.int32)
    assert np.array_equal(oracle.softmax_int(z, zl, 6, 14), backend.softmax(z, zl, 6, 14))
    # negative and odd LUT entries exercise the signed division branch
    odd = r.integers(-500, 500, 64).astype(np.int16)
    assert np.array_equal(oracle.softmax_int(z, odd, 2, 10), backend.softmax(z, odd, 2, 10))


@pytest.mark.parametrize("q_len,kv_len,hd", [(1, 1, 64), (1, 300, 128), (3, 17, 64), (2, 2304, 128), (4, 9, 6)])
def test_attention_trait(backend, oracle, q_len, kv_len, hd):
    case(f"attention q={q_len} kv={kv_len} hd={hd}")
    from myelith_amd.luts import exp_lut
    lut = exp_lut()
    r = rng(q_len * kv_len + hd)
    q = gauss16(r, q_len * hd, 3000).reshape(q_len, hd)
    k = gauss16(r, kv_len * hd, 3000).reshape(kv_len, hd)
    v = gauss16(r, kv_len * hd, 8000).reshape(kv_len, hd)
    mask = (r.random((q_len, kv_len)) < 0.8).astype(np.uint8)
    for mult, shift in ((2896, 18), (4096, 25), (1 << 15, 40)):
        for mk in (None, mask):
            ref = oracle.attention_int(q, k, v, mult, shift, lut, 6, 14, mask=mk)
            got = backend.attention(q, k, v, mk, mult, shift, lut, 6, 14)
            assert np.array_equal(ref, got)


def test_rope(backend, oracle, luts128):
    case("rope")
    r = rng(11)
    n, hd = 7, 128
    q = gauss16(r, n * hd, 12000).reshape(n, hd)
    k = gauss16(r, n * hd, 12000).reshape(n, hd)
    pos = np.array([0, 1, 2047, 2048, 2303, 4095, 123456], np.uint64)  # wraps past 2048 rows (model.rs:470-471)
    qo, ko = oracle.apply_rope_i16(q, k, luts128.cos, luts128.sin, pos, 8)
    gq, gk = backend.rope(q, k, luts128.cos, luts128.sin, pos, 8)
    assert np.array_equal(qo, gq) and np.array_equal(ko, gk)


@pytest.mark.parametrize("H,I", [(16, 24), (896, 4864)])
def test_mlp_trait(backend, oracle, H, I):
    case(f"mlp H={H} I={I}")
    from myelith_amd.luts import silu_lut
    silu = silu_lut()
    r = rng(H + I)
    x = gauss16(r, H, 3000)
    Wg, Wu = r.integers(-127, 128, (I, H)).astype(np.int8), r.integers(-127, 128, (I, H)).astype(np.int8)
    Wd = r.integers(-127, 128, (H, I)).astype(np.int8)
    gs, us, ds = [r.integers(8, 14, n).astype(np.uint8) for n in (I, I, H)]
    of = r.integers(7, 11, H).astype(np.uint8)
    args = (x, Wg, Wu, Wd, gs, us, ds, silu, 10, 11, 10, 12, 6, 8192, 8, of)
    ref = oracle.mlp_int(x, Wg, Wu, Wd, H, I, gs, us, ds, silu, 10, 11, 10, 12, 6, 8192, 8, of)
    got = backend.mlp(*args)
    assert np.array_equal(ref, got)


def test_bias(backend, oracle):
    case("add_bias_i16")
    r = rng(5)
    n = 1000
    out = gauss16(r, n, 20000)
    b = gauss16(r, n, 20000)
    bs = r.integers(0, 20, n).astype(np.uint8)
    for of in (0, 8, 15):
        assert np.array_equal(oracle.add_bias_i16(out, b, bs, of), backend.add_bias_i16(out, b, bs, of))


def test_argmax(backend, oracle):
    case("argmax")
    r = rng(6)
    for n in (1, 2, 151936, 152064):
        v = r.integers(-1000, 1000, n).astype(np.int32)
        assert backend.argmax_int(v) == oracle.argmax_int(v)
        v[:] = 7
        assert backend.argmax_int(v) == 0
        if n > 10:
            v[n - 1] = 9
            v[5] = 9
            assert backend.argmax_int(v) == 5
    with pytest.raises(ValueError):
        backend.argmax_int([])


def test_sample_integer_cdf(backend, oracle):
    """sample_integer_cdf (sampling.rs:27-46) on the GPU against the oracle:
    ragged lengths around the 4096-position scan tiles, both vocab sizes,
    logits spanning the i32 range (wrapped weights, non-monotone running sums,
    totals <= 0), constant rows, the first and last tokens, many states."""
    case("sample_integer_cdf")
    r = rng(9)
    lo, hi = -2**31, 2**31 - 1
    rows = []
    for n in (1, 2, 3, 4095, 4096, 4097, 12293, 151936, 152064):
        rows.append(r.integers(-100000, 100000, n).astype(np.int32))
    rows.append(np.full(4099, 5, np.int32))
    rows.append(r.integers(lo, hi, 5000, endpoint=True).astype(np.int32))        # wrapped weights
    rows.append(np.array([lo, -2, -2, -1, -2], np.int32))                         # non-monotone sums
    rows.append(np.array([lo, hi - 1], np.int32))                                 # total 0
    rows.append(np.array([lo, hi], np.int32))                                     # a zero weight
    z = np.full(9000, -10, np.int32)
    z[-1] = 2**30                                                                  # nearly all weight last
    rows.append(z)
    for v in rows:
        for state in (0, 1, 42, 2**64 - 1, int(r.integers(0, 2**63)) * 2 + 1):
            assert backend.sample_integer_cdf(v, state) == oracle.sample_integer_cdf(v, state), (len(v), state)
    assert backend.sample_integer_cdf(np.zeros(0, np.int32), 3) == (0, 3)


def test_sample_dev_rows(backend, oracle):
    """Rows of the device sampler (myl_sample_dev) with their own states."""
    import torch
    case("sample_dev")
    r = rng(10)
    M, n = 37, 152064
    z = r.integers(-300000, 300000, (M, n)).astype(np.int32)
    states = np.array([int(x) for x in r.integers(0, 2**62, M)], dtype=np.uint64)
    zt = torch.from_numpy(z).cuda()
    st = torch.from_numpy(states.view(np.int64)).cuda()
    tok, ns = backend.sample_dev(zt, st)
    tok, ns = tok.cpu().numpy(), ns.cpu().numpy().view(np.uint64)
    for m in range(M):
        assert (int(tok[m]), int(ns[m])) == oracle.sample_integer_cdf(z[m], int(states[m])), m


def test_device_forms_batch_rows(backend, oracle, luts64):
    import torch
    case("rmsnorm/softmax/argmax dev batch")
    r = rng(9)
    M, n = 5, 896
    x = gauss16(r, M * n).reshape(M, n)
    xs = r.integers(7, 11, n).astype(np.uint8)
    g = r.integers(-127, 128, n).astype(np.int8)
    gs = r.integers(6, 8, n).astype(np.uint8)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    got = backend.rmsnorm_dev(T(x), T(xs), T(g), T(gs), T(luts64.rsqrt), 8, 8, oracle.inv_n_q20(n), 10).cpu().numpy()
    for m in range(M):
        assert np.array_equal(got[m], oracle.rmsnorm_i16(x[m], xs, g, gs, luts64.rsqrt, 8, 8, oracle.inv_n_q20(n), 10))
    z = r.integers(-10**6, 10**6, (M, 700)).astype(np.int32)
    got = backend.softmax_dev(T(z), T(luts64.exp), 6, 14).cpu().numpy()
    for m in range(M):
        assert np.array_equal(got[m], oracle.softmax_int(z[m], luts64.exp, 6, 14))
    got = backend.argmax_dev(T(z)).cpu().numpy()
    assert list(got) == [oracle.argmax_int(z[m]) for m in range(M)]
