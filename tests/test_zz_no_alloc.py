"""The allocation-free W8A16 product (myl_linear_w8a16_dev_noalloc) against
myl_linear_w8a16_dev on the same operands, bit for bit, through the C ABI:
two calls in a row with the second smaller (the shared scratch keeps the
first call's contents), K-split products that use the scratch accumulator,
one-row products, and the size limit.  The property the entry point exists
for is checked directly: on a fresh context (no buffers of its own yet) the
device's free memory is the same before and after a call, and the call
captured into a HIP graph (where an allocation or a host synchronisation
would fail the capture) replays to the same result."""
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


def test_noalloc_allocates_nothing_on_a_fresh_context(backend):
    import torch
    from myelith_amd.backend import RocmBackend
    M, N, K = 16, 4096, 3584  # K split through the scratch accumulator
    x, W, ws, of = operands(21, M, N, K)
    case(f"noalloc fresh context M={M} N={N} K={K}")
    ref = torch.empty((M, N), dtype=torch.int16, device="cuda")
    backend.linear_w8a16_dev_noalloc(x, W, ws, 11, 10, of, out=ref)  # code objects loaded, scratch looked up
    torch.cuda.synchronize()
    fresh = RocmBackend(0)
    try:
        got = torch.empty_like(ref)
        word = torch.zeros(1, dtype=torch.int32, device="cuda")
        # a first launch on the context's own stream (the runtime sets up a
        # stream's queue on first use), one that allocates nothing
        fresh.read_probe_dev(x, word)
        torch.cuda.synchronize()
        fresh.synchronize()
        free0, _ = torch.cuda.mem_get_info()
        fresh.linear_w8a16_dev_noalloc(x, W, ws, 11, 10, of, out=got)
        fresh.synchronize()
        free1, _ = torch.cuda.mem_get_info()
        assert free1 == free0, f"device free memory changed by {free0 - free1} bytes"
        assert torch.equal(got, ref)
    finally:
        fresh.close()


def test_noalloc_replays_from_a_captured_graph(backend):
    import torch
    M, N, K = 16, 4096, 3584
    x, W, ws, of = operands(33, M, N, K)
    want = backend.linear_w8a16_dev(x, W, ws, 11, 10, of)
    out = torch.empty((M, N), dtype=torch.int16, device="cuda")
    case(f"noalloc graph capture M={M} N={N} K={K}")
    prev = torch.cuda.current_stream()
    cap = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    try:
        torch.cuda.set_stream(cap)
        backend.use_torch_stream()
        with torch.cuda.graph(g, stream=cap):
            backend.linear_w8a16_dev_noalloc(x, W, ws, 11, 10, of, out=out)
    finally:
        torch.cuda.set_stream(prev)
        backend.use_torch_stream()
    # eager work of the program between replays (another product that uses
    # the same scratch), a synchronisation, then the replay, every time
    x2, W2, ws2, _ = operands(34, 8, 1000, 1024)
    for r in range(3):
        out.zero_()
        other = torch.empty((8, 1000), dtype=torch.int16, device="cuda")
        backend.linear_w8a16_dev_noalloc(x2, W2, ws2, 11, 10, out=other)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {r}"
    del g
