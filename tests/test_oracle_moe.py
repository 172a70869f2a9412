"""Pins the oracle's MoE layer (build-defined: the reference is dense) before
the GPU layer is compared against it.  Each step is checked against an
independent restatement built from pinned primitives:
  - top-k: a stable numpy sort by (-logit, expert index);
  - gates: the pinned softmax_int over the selected logits;
  - dispatch: numpy bincount / cumsum / stable per-expert token lists;
  - combine: numpy int64 of sum_k g_k y_k + 2^14 s, then the pinned RNE shift;
  - load: the router bias makes top-4 load follow Zipf(1.0) to within 0.05 L1.
"""
from __future__ import annotations

import numpy as np
import pytest


@pytest.fixture(scope="module")
def moe():
    from myelith_amd.luts import LutSet
    from myelith_amd.moe import moe_spec, router_bias
    from oracle.binding import OracleMoe
    spec = moe_spec(5)
    m = OracleMoe(spec, router_bias(spec["n_experts"]), LutSet.for_head_dim(64), threads=8)
    yield m
    m.close()


def test_route_topk_gates_dispatch(moe, oracle):
    from myelith_amd.luts import exp_lut
    T, K, E = 512, moe.spec["top_k"], moe.spec["n_experts"]
    x = moe.synth_input(T)
    r = moe.route(x)
    lut = exp_lut()
    for t in range(0, T, 7):
        z = moe.router_logits(x[t])
        order = sorted(range(E), key=lambda e: (-int(z[e]), e))[:K]
        assert list(r["ids"][t]) == order, t
        assert np.array_equal(r["gates"][t], oracle.softmax_int(z[order], lut, 0, 14)), t
        assert abs(int(r["gates"][t].sum()) - 16384) <= K
    assert np.array_equal(r["counts"], np.bincount(r["ids"].ravel(), minlength=E))
    assert np.array_equal(r["offsets"], np.concatenate([[0], np.cumsum(r["counts"])]))
    for e in range(E):
        lst = r["list_tok"][r["offsets"][e]:r["offsets"][e + 1]]
        assert np.array_equal(lst, np.nonzero((r["ids"] == e).any(axis=1))[0]), e


def test_load_follows_zipf(moe):
    x = moe.synth_input(4096)
    r = moe.route(x)
    load = r["counts"] / r["counts"].sum()
    target = 1.0 / np.arange(1, len(load) + 1)
    target /= target.sum()
    assert np.abs(load - target).sum() < 0.05


def test_combine_is_one_weighted_sum_and_one_rounding(moe, oracle):
    x = moe.synth_input(8)
    r = moe.route(x)
    E = moe.spec["n_experts"]
    for t in range(8):
        ys = [moe.expert(x[t], int(e)).astype(np.int64) for e in r["ids"][t]]
        s = moe.expert(x[t], E).astype(np.int64)
        acc = s * 16384 + sum(int(g) * y for g, y in zip(r["gates"][t], ys))
        exp = np.array([max(-32768, min(32767, oracle.rshift_round_i64(int(a), 14))) for a in acc], np.int16)
        assert np.array_equal(moe.token(x[t], r["ids"][t], r["gates"][t]), exp), t


def test_oracle_rejects_routes_beyond_its_scratch():
    """The oracle's per-token route scratch holds 256 expert logits and 16
    selections (or_moe_route), the bounds the device layer checks too: a
    spec past either is refused at creation instead of overrunning it."""
    from myelith_amd.luts import LutSet
    from oracle.binding import OracleMoe
    luts = LutSet.for_head_dim(64)
    base = dict(seed=3, hidden=64, n_experts=8, inter=64, top_k=2, shared_inter=64)
    m = OracleMoe(base, np.zeros(8, np.int32), luts)  # within bounds: accepted
    m.close()
    for bad in (dict(n_experts=257), dict(n_experts=32, top_k=17)):
        spec = {**base, **bad}
        with pytest.raises(ValueError, match="creation failed"):
            OracleMoe(spec, np.zeros(spec["n_experts"], np.int32), luts)
