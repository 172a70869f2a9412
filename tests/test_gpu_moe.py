"""GPU parity of the integer MoE layer (route, dispatch, grouped experts,
combine) against the oracle, bit for bit.  The reference has no MoE; the
definition is the build's (include/myl_hip.h section 4), pinned in
tests/test_oracle_moe.py."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import case

pytestmark = pytest.mark.gpu


def build(backend, spec, bias=None):
    from myelith_amd.luts import LutSet
    from myelith_amd.moe import MoeLayer, router_bias
    from oracle.binding import OracleMoe
    luts = LutSet.for_head_dim(64)
    b = router_bias(spec["n_experts"]) if bias is None else np.asarray(bias, np.int32)
    return MoeLayer(backend, spec, luts, b), OracleMoe(spec, b, luts, threads=16)


def compare_route(g, o):
    for k in ("ids", "gates", "counts", "offsets", "list_tok"):
        assert np.array_equal(g[k], o[k]), k


@pytest.mark.parametrize("T,widths", [(1, (256, 128, 256)), (37, (256, 128, 256)), (300, (256, 128, 256)),
                                      (300, (240, 144, 272))])
def test_small_moe_all_tokens(backend, T, widths):
    """8 experts, top-2, two of them unreachable (no tokens): every token's output.
    Widths (hidden, inter, shared) that are multiples of 128 take the byte-plane
    expert products (and, past 64 tokens, the shared expert's fused SiLU);
    240 / 144 / 272 (not multiples of 64) take the int16-row products."""
    from myelith_amd.moe import moe_spec
    H, I, S = widths
    spec = moe_spec(9, hidden=H, n_experts=8, inter=I, top_k=2, shared_inter=S)
    bias = np.array([0, -100, -200, -10**7, -150, -10**7, -50, -300], np.int32)
    case(f"small moe T={T} widths={widths}")
    gm, om = build(backend, spec, bias)
    x = gm.synth_input(T)
    xh = x.cpu().numpy()
    assert np.array_equal(xh, om.synth_input(T))
    y = gm.forward(x).cpu().numpy()
    ro = om.route(xh)
    compare_route(gm.route(T), ro)
    assert ro["counts"][3] == 0 and ro["counts"][5] == 0
    for t in range(T):
        assert np.array_equal(y[t], om.token(xh[t], ro["ids"][t], ro["gates"][t])), t


def test_qwen15_moe_4096_tokens(backend):
    """The Qwen1.5-MoE-A2.7B-shaped layer on 4096 tokens: the whole route
    (ids, gates, counts, offsets, dispatch order) and the output of every
    one of the 4096 tokens equal the oracle's (about ten seconds of the
    oracle on the host's cores)."""
    from myelith_amd.moe import moe_spec
    spec = moe_spec(5)
    case("qwen1.5-moe 4096 tokens")
    gm, om = build(backend, spec)
    T = 4096
    x = gm.synth_input(T)
    y = gm.forward(x).cpu().numpy()
    xh = x.cpu().numpy()
    ro = om.route(xh)
    compare_route(gm.route(T), ro)
    bad = [t for t in range(T) if not np.array_equal(y[t], om.token(xh[t], ro["ids"][t], ro["gates"][t]))]
    assert not bad, f"{len(bad)} of {T} token outputs differ, first {bad[:8]}"
    # a second call with fewer tokens reuses the buffers
    y2 = gm.forward(x[:100]).cpu().numpy()
    r2 = om.route(xh[:100])
    compare_route(gm.route(100), r2)
    for t in range(5):
        assert np.array_equal(y2[t], om.token(xh[t], r2["ids"][t], r2["gates"][t])), t
