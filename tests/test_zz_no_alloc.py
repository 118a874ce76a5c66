"""gh_attention_decode_noalloc (the allocation-free variant of
gh_attention_decode) against gh_attention_decode through the C ABI, on the
GPU: two calls in a row, the second smaller than the first, each equal to
the allocating entry point's output; a call whose chunk states exceed the
static scratch is GH_ERR_RANGE."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

import gemma_hip as gh
from gemma_hip import lib
from conftest import rel_err

pytestmark = pytest.mark.gpu


def _call(fn, ctx, q, k, v, nq, nkv, hd, pb, pe, ns, o):
    return fn(ctx.h, q.ptr, k.ptr, v.ptr, nq, nkv, hd, pb, pe, ns, o.ptr)


def test_noalloc_attention_matches_allocating_entry_point(ctx):
    rng = np.random.default_rng(17)
    cases = [  # (nq, nkv, hd, cache positions, p_begin, p_end, n_splits) -- second call smaller
        (4, 1, 256, 8192, 0, 8192, 0),
        (8, 4, 256, 1200, 1200 - 1024, 1200, 0),
    ]
    for nq, nkv, hd, L, pb, pe, ns in cases:
        print(f"noalloc attention: nq {nq} nkv {nkv} hd {hd} range [{pb}, {pe})", flush=True)
        q = gh.DeviceBuffer.from_numpy(ctx, rng.normal(size=nq * hd).astype(np.float32))
        k = gh.DeviceBuffer.from_numpy(ctx, rng.normal(size=L * nkv * hd).astype(np.float32))
        v = gh.DeviceBuffer.from_numpy(ctx, rng.normal(size=L * nkv * hd).astype(np.float32))
        o1, o2 = gh.DeviceBuffer(ctx, 4 * nq * hd), gh.DeviceBuffer(ctx, 4 * nq * hd)
        try:
            gh._lib.check(_call(lib().gh_attention_decode, ctx, q, k, v, nq, nkv, hd, pb, pe, ns, o1))
            gh._lib.check(_call(lib().gh_attention_decode_noalloc, ctx, q, k, v, nq, nkv, hd, pb, pe, ns, o2))
            want, got = o1.numpy(), o2.numpy()
            assert np.all(np.isfinite(got))
            assert rel_err(got, want) < 1e-6
            np.testing.assert_array_equal(got, want)
        finally:
            for b in (q, k, v, o1, o2):
                b.free()


def test_noalloc_attention_rejects_more_than_its_scratch(ctx):
    """8 kv heads x 256 splits x group 8 x 258 floats > 2^20: refused on the
    host before any launch."""
    nq, nkv, hd, L = 64, 8, 256, 8192
    q = gh.DeviceBuffer(ctx, 4 * nq * hd)
    kv = gh.DeviceBuffer(ctx, 4 * L * nkv * hd)
    o = gh.DeviceBuffer(ctx, 4 * nq * hd)
    try:
        rc = lib().gh_attention_decode_noalloc(ctx.h, q.ptr, kv.ptr, kv.ptr, nq, nkv, hd, 0, L, 256, o.ptr)
        assert rc == -5, rc  # GH_ERR_RANGE
        assert b"static" in lib().gh_last_error()
    finally:
        for b in (q, kv, o):
            b.free()
