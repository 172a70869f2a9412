"""The allocation-free W8A16 product (myl_linear_w8a16_dev_noalloc) against
myl_linear_w8a16_dev on the same operands, bit for bit, through the C ABI:
two calls in a row with the second smaller (the shared scratch keeps the
first call's contents), K-split products that use the scratch accumulator,
one-row products, and the size limit."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import case

pytestmark = pytest.mark.gpu


def operands(seed, M, N, K):
    import torch
    r = np.random.default_rng(seed)
    x = np.clip(np.rint(r.normal(0, 2000, (M, K))), -32767, 32767).astype(np.int16)
    x[0, :3] = (-32768, 32767, 0)
    W = r.integers(-128, 128, (N, K)).astype(np.int8)
    ws = r.integers(8, 14, N).astype(np.uint8)
    of = r.integers(7, 11, N).astype(np.uint8)
    return [torch.from_numpy(a).cuda() for a in (x, W, ws, of)]


def test_noalloc_matches_linear_dev_on_two_calls(backend):
    import torch
    # (M, N, K): 16 x 4096 x 3584 splits K through the scratch accumulator;
    # the second call is smaller and also splits; then one row (no scratch)
    shapes = [(16, 4096, 3584), (4, 1000, 1024), (1, 3584, 3584)]
    for pc in (False, True):
        ops = [operands(7 + i, *s) for i, s in enumerate(shapes)]
        outs = []
        for (M, N, K), (x, W, ws, of) in zip(shapes, ops):
            case(f"noalloc M={M} N={N} K={K} per-channel={pc}")
            outs.append(torch.empty((M, N), dtype=torch.int16, device="cuda"))
            backend.linear_w8a16_dev_noalloc(x, W, ws, 11, 10, of if pc else None, out=outs[-1])
        for (M, N, K), (x, W, ws, of), got in zip(shapes, ops, outs):
            want = backend.linear_w8a16_dev(x, W, ws, 11, 10, of if pc else None)
            assert torch.equal(got, want), (M, N, K, pc)


def test_noalloc_rejects_planes_beyond_the_scratch(backend):
    import torch
    from myelith_amd._lib import lib
    case("noalloc size limit")
    limit = lib().myl_noalloc_scratch_bytes()
    assert limit >= 4 << 20
    M, K, N = 128, 32768, 16          # 2 * M * K = 8 MiB of planes
    x = torch.zeros((M, K), dtype=torch.int16, device="cuda")
    W = torch.zeros((N, K), dtype=torch.int8, device="cuda")
    ws = torch.zeros(N, dtype=torch.uint8, device="cuda")
    out = torch.empty((M, N), dtype=torch.int16, device="cuda")
    with pytest.raises(ValueError, match="scratch"):
        backend.linear_w8a16_dev_noalloc(x, W, ws, 0, 0, out=out)
