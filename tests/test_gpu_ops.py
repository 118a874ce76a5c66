"""Op-level parity on the MI355X through the C ABI (marked gpu).

Bars: Q4_0 dequant bit-exact (incl. fp16 subnormal scales, both modes);
matvec within the fp32 accumulation bound of an fp64 dot product; norms,
RoPE, GELU, attention within the stated relative tolerances of the oracle;
argmax exact (first maximum).
"""
from __future__ import annotations

import numpy as np
import pytest

import gemma_hip as gh
import pyoracle as orc
from conftest import rel_err
from numpy_ref import q4_0_dequant_np

pytestmark = pytest.mark.gpu


def _random_q4(rows, cols, seed, subnormal_frac=0.0):
    rng = np.random.default_rng(seed)
    nb = rows * cols // 32
    b = rng.integers(0, 256, size=(nb, 18), dtype=np.uint8)
    sc = np.abs(rng.normal(0, 0.01, nb)).astype(np.float16)
    if subnormal_frac:
        m = rng.random(nb) < subnormal_frac
        sub = rng.integers(1, 1024, size=nb).astype(np.uint16) | (rng.integers(0, 2, nb).astype(np.uint16) << 15)
        sc = np.where(m, sub.view(np.float16), sc)
    b[:, :2] = sc.view(np.uint8).reshape(nb, 2)
    return b.reshape(-1)


@pytest.mark.parametrize("ieee", [False, True])
def test_q4_0_dequant_bit_exact(ctx, ieee):
    rows, cols = 300, 1152  # ragged last tile
    raw = _random_q4(rows, cols, 1, subnormal_frac=0.05)
    t = gh.Q4Tensor(ctx, raw, rows, cols, ieee_scales=ieee)
    got = t.dequant()
    want = orc.q4_0_dequant(raw, ftz=not ieee).reshape(rows, cols)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_q4_0_dequant_all_scale_patterns(ctx):
    """Every fp16 bit pattern as a block scale, FTZ mode: bit-exact."""
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    rows = 65536 // 36 + 1
    h = np.resize(h, rows * 36)
    b = np.empty((h.size, 18), np.uint8)
    b[:, :2] = h.astype("<u2").view(np.uint8).reshape(-1, 2)
    b[:, 2:] = np.random.default_rng(3).integers(0, 256, size=(h.size, 16), dtype=np.uint8)
    raw = b.reshape(-1)
    got = gh.Q4Tensor(ctx, raw, rows, 1152).dequant()
    want = orc.q4_0_dequant(raw).reshape(rows, 1152)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


@pytest.mark.parametrize("mfma", [0, 1])
@pytest.mark.parametrize("rl", [2, 1])
@pytest.mark.parametrize("rows,cols", [(6912, 1152), (1152, 6912), (262144, 1152), (1536, 1152),
                                       (1152, 1024), (4, 64), (130, 96), (200, 480)])
def test_q4_0_matvec_shapes(ctx, rows, cols, rl, mfma, monkeypatch):
    """Both workgroup shapes, 128 rows (2 per lane) and 64 rows (1 per lane),
    and both dot-product paths: VALU (mfma 0) and the int8 matrix cores
    (mfma 1, whose input limbs round x to 2^-27 of its block maximum, far
    inside the bound).  480 columns: 15 blocks, a partial last quad."""
    monkeypatch.setenv("GH_Q4_RL", str(rl))
    monkeypatch.setenv("GH_Q4_MFMA", str(mfma))
    monkeypatch.setenv("GH_Q4_RG16", "0")  # the row-group kernel has its own test
    raw = _random_q4(rows, cols, rows + cols, subnormal_frac=0.005)
    x = np.random.default_rng(rows).normal(size=cols).astype(np.float32)
    t = gh.Q4Tensor(ctx, raw, rows, cols)
    y = t.matvec(x)
    y64, ay = orc.q4_0_matvec_f64(raw, x, rows, cols)
    # fp32 accumulation bound of any summation order: |err| <= n*eps*sum|w x|
    bound = 2 * cols * np.finfo(np.float32).eps * ay
    assert np.all(np.abs(y - y64) <= bound + 1e-30)
    assert rel_err(y, orc.q4_0_matvec(raw, x, rows, cols)) < 1e-5


@pytest.mark.parametrize("rows,cols", [(6912, 1152), (1152, 6912), (1536, 1152)])
def test_q4_0_matvec_input_ordering_is_bit_identical(ctx, rows, cols, monkeypatch):
    """GH_Q4_ORDER_IN=0 drops the barrier between the input and weight loads;
    the arithmetic is the same, so the outputs are bit-identical."""
    raw = _random_q4(rows, cols, rows + 2 * cols)
    x = np.random.default_rng(5).normal(size=cols).astype(np.float32)
    ys = []
    for oi in ("0", "1"):
        monkeypatch.setenv("GH_Q4_ORDER_IN", oi)
        ys.append(gh.Q4Tensor(ctx, raw, rows, cols).matvec(x))
    assert np.array_equal(ys[0].view(np.uint32), ys[1].view(np.uint32))


@pytest.mark.parametrize("rg", ["default", "16", "8", "4"])
@pytest.mark.parametrize("rows,cols", [(1536, 1152), (1152, 1024), (1000, 2560), (130, 96), (4, 64), (200, 480),
                                       (1152, 6912), (40, 8192)])
def test_q4_0_matvec_row_groups(ctx, rows, cols, rg, monkeypatch):
    """The row-group kernel (k_mq_rows: one workgroup per 16, 8 or 4 rows over
    all columns, the waves splitting the quads): the default routes split
    plans of up to 5120 columns to it.  Ragged row counts (1000, 130, 200, 4)
    leave part of the last group unstored; 8192 columns fill the input
    registers; 480 columns end on a partial quad.  Against the f64 oracle's
    bound, the f32 oracle, and the split-K path (GH_Q4_RG16=0) within f32
    summation-order differences; with the soft-cap epilogue too."""
    if rg != "default":
        monkeypatch.setenv("GH_Q4_RG16", rg)
    raw = _random_q4(rows, cols, rows * 3 + cols, subnormal_frac=0.005)
    x = np.random.default_rng(cols + 1).normal(size=cols).astype(np.float32)
    t = gh.Q4Tensor(ctx, raw, rows, cols)
    y = t.matvec(x)
    y64, ay = orc.q4_0_matvec_f64(raw, x, rows, cols)
    bound = 2 * cols * np.finfo(np.float32).eps * ay
    assert np.all(np.abs(y - y64) <= bound + 1e-30)
    assert rel_err(y, orc.q4_0_matvec(raw, x, rows, cols)) < 1e-5
    monkeypatch.setenv("GH_Q4_RG16", "0")
    y_split = gh.Q4Tensor(ctx, raw, rows, cols).matvec(x)
    assert np.all(np.abs(y - y_split) <= 2 * bound + 1e-30)
    # soft-capped: cap * tanh(y / cap) of the same sums (runLinearQ4's arm)
    cap = float(np.median(np.abs(y64))) + 1e-3
    yc = t.matvec(x, softcap=True, cap=cap)
    assert np.allclose(yc, cap * np.tanh(y.astype(np.float64) / cap), rtol=4e-6, atol=1e-7 * cap)


@pytest.mark.parametrize("mfma", [0, 1])
@pytest.mark.parametrize("rl", [2, 1])
@pytest.mark.parametrize("rows,cols", [(256, 4096), (192, 2592)])
def test_q4_0_matvec_single_split_many_batches(ctx, rows, cols, rl, mfma, monkeypatch):
    """One column split (GH_Q4_MAXS=1): every work item walks all 128 / 81
    column blocks in several register batches, the last one partial."""
    monkeypatch.setenv("GH_Q4_RL", str(rl))
    monkeypatch.setenv("GH_Q4_MFMA", str(mfma))
    monkeypatch.setenv("GH_Q4_MAXS", "1")
    raw = _random_q4(rows, cols, rows * 7 + cols, subnormal_frac=0.005)
    x = np.random.default_rng(cols).normal(size=cols).astype(np.float32)
    y = gh.Q4Tensor(ctx, raw, rows, cols).matvec(x)
    y64, ay = orc.q4_0_matvec_f64(raw, x, rows, cols)
    bound = 2 * cols * np.finfo(np.float32).eps * ay
    assert np.all(np.abs(y - y64) <= bound + 1e-30)


@pytest.mark.parametrize("mfma", [0, 1])
def test_q4_0_matvec_nan_input_propagates(ctx, mfma, monkeypatch):
    """A NaN in x reaches every output row on both dot-product paths (the
    finish kernel's NaN check relies on it)."""
    monkeypatch.setenv("GH_Q4_MFMA", str(mfma))
    rows, cols = 256, 512
    raw = _random_q4(rows, cols, 4)
    x = np.random.default_rng(4).normal(size=cols).astype(np.float32)
    x[37] = np.nan
    y = gh.Q4Tensor(ctx, raw, rows, cols).matvec(x)
    assert np.all(np.isnan(y))


def test_runLinearQ4_reference_api(ctx):
    """runLinearQ4 (src/Gemma/Layers/LinearQ4.hs:41-48) on the 4x64 case of
    test/Gemma/Layers/DequantQ4GGUFSpec.hs: raw bytes as uint32 words."""
    rows, cols = 4, 64
    raw = _random_q4(rows, cols, 9)
    words = np.concatenate([raw, np.zeros((-raw.size) % 4, np.uint8)]).view(np.uint32)
    x = np.random.default_rng(9).normal(size=cols).astype(np.float32)
    y = gh.runLinearQ4(ctx, words, x, rows, cols, False, 30.0)
    W = q4_0_dequant_np(raw, rows, cols)
    np.testing.assert_allclose(y, W @ x, rtol=1e-5, atol=1e-6)
    ys = gh.runLinearQ4(ctx, words, 50 * x, rows, cols, True, 30.0)
    np.testing.assert_allclose(ys, orc.softcap(W @ (50 * x), 30.0), rtol=1e-5, atol=1e-5)


def test_linear_q4_rejects_bad_shapes(ctx):
    with pytest.raises(gh.GemmaHipError) as e:
        gh.runLinearQ4(ctx, np.zeros(9, np.uint32), np.zeros(48, np.float32), 1, 48)
    assert e.value.name == "GH_ERR_INVALID"


@pytest.mark.parametrize("n", [4, 128, 1152, 2560])
def test_rmsnorm(ctx, n):
    rng = np.random.default_rng(n)
    x = rng.normal(0, 2, n).astype(np.float32)
    w = rng.normal(0, 0.02, n).astype(np.float32)
    assert rel_err(gh.rmsnorm(ctx, x, w), orc.rmsnorm_tree(x, w)) < 1e-6
    assert rel_err(gh.rmsnorm(ctx, x, w + 1, zero_centered=False), orc.rmsnorm_tree(x, w + 1, zc=False)) < 1e-6


@pytest.mark.parametrize("hd,nh", [(256, 4), (256, 8), (32, 4), (128, 2)])
def test_qk_norm_and_rope(ctx, hd, nh):
    rng = np.random.default_rng(hd + nh)
    x = rng.normal(0, 3, nh * hd).astype(np.float32)
    w = rng.normal(0, 0.02, hd).astype(np.float32)
    assert rel_err(gh.qk_norm(ctx, x, w, nh, hd), orc.qk_norm(x, w, nh, hd)) < 1e-6
    for pos, theta in ((0, 1e4), (1, 1e4), (383, 1e6), (4351, 1e4)):
        got = gh.rope(ctx, x, nh, hd, theta, pos)
        want = orc.rope(x, nh, hd, theta, pos)
        assert rel_err(got, want) < 2e-6, (pos, theta)


def test_gelu_mul_and_argmax(ctx):
    rng = np.random.default_rng(5)
    g = rng.normal(0, 3, 6912).astype(np.float32)
    u = rng.normal(0, 1, 6912).astype(np.float32)
    assert rel_err(gh.gelu_mul(ctx, g, u), orc.geglu(g, u)) < 1e-6
    v = rng.normal(size=262144).astype(np.float32)
    assert gh.argmax(ctx, v) == int(np.argmax(v))
    v[[17, 100000, 262143]] = 50.0  # ties -> first index
    assert gh.argmax(ctx, v) == 17
    assert gh.argmax(ctx, -np.abs(v)) == int(np.argmax(-np.abs(v)))


@pytest.mark.parametrize("nq,nkv,hd,L", [(4, 1, 256, 8192), (4, 1, 256, 32768), (8, 4, 256, 4352),
                                         (8, 1, 256, 2050), (2, 2, 256, 3001), (4, 1, 32, 300), (4, 2, 128, 1000)])
def test_attention_decode_global_and_local(ctx, nq, nkv, hd, L):
    """Config C4 shapes: global layer over all L, local layer over the last 512.
    Chunks of 64 positions or more (head_dim 256) run the wave-streaming
    kernel, shorter ones the 32-position sub-chunk kernel; groups 1, 2, 4, 8
    and ragged lengths are covered."""
    rng = np.random.default_rng(L)
    q = rng.normal(size=nq * hd).astype(np.float32)
    K = rng.normal(size=(L, nkv, hd)).astype(np.float32)
    V = rng.normal(size=(L, nkv, hd)).astype(np.float32)
    for lo in (0, max(0, L - 512)):
        got = gh.attention_decode(ctx, q, K, V, nq, nkv, hd, lo, L)
        want = orc.attention(q, K, V, nq, nkv, hd, lo, L)
        assert rel_err(got, want) < 1e-5, lo
    # split count does not change the result beyond rounding
    a = gh.attention_decode(ctx, q, K, V, nq, nkv, hd, 0, L, n_splits=1)
    b = gh.attention_decode(ctx, q, K, V, nq, nkv, hd, 0, L, n_splits=min(L, 64))
    assert rel_err(a, b) < 1e-5


def test_capture_replay_matches_eager_calls(ctx):
    """gh_capture_begin / gh_capture_replay: op calls captured into a graph
    and replayed give the eager results; an op that would need new scratch
    during capture is refused."""
    rows, cols = 1152, 6912
    raw = _random_q4(rows, cols, 5)
    t = gh.Q4Tensor(ctx, raw, rows, cols)
    xv = np.random.default_rng(5).normal(size=cols).astype(np.float32)
    want = t.matvec(xv)
    x = gh.DeviceBuffer.from_numpy(ctx, xv)
    y = gh.DeviceBuffer(ctx, 4 * rows)
    ctx.capture_begin()
    gh._lib.check(gh.lib().gh_q4_0_matvec(t.h, x.ptr, y.ptr, 0, 0.0))
    assert ctx.capture_replay(3) > 0.0
    np.testing.assert_array_equal(y.numpy(), want)
    for b in (x, y):
        b.free()
    t.close()
    # a fresh context has no op scratch yet: attention may not allocate it during capture
    c2 = gh.Context(0)
    q = gh.DeviceBuffer.from_numpy(c2, np.ones(8 * 256, np.float32))
    kv = gh.DeviceBuffer.from_numpy(c2, np.ones(300 * 256 * 4, np.float32))
    o = gh.DeviceBuffer(c2, 4 * 8 * 256)
    c2.capture_begin()
    with pytest.raises(gh.GemmaHipError) as e:
        gh._lib.check(gh.lib().gh_attention_decode(c2.h, q.ptr, kv.ptr, kv.ptr, 8, 4, 256, 0, 300, 3, o.ptr))
    assert e.value.name == "GH_ERR_STATE"
    c2.capture_replay(1)
    for b in (q, kv, o):
        b.free()
    c2.close()


def test_sample_logits_matches_oracle(ctx):
    """Device Philox + two-level inversion against the oracle: equal logits
    give floor(u n) exactly (pins the device uniform); random logits give
    the oracle's draw except where u * total sits within 1e-4 of a boundary
    (float vs double running sums); temperature 0 is the argmax."""
    n = 1000
    for c in range(20):
        u = orc.philox_uniform(11, c)
        assert gh.sample_logits(ctx, np.zeros(n, np.float32), 0.9, 11, c) == int(np.floor(u * n))
    rng = np.random.default_rng(2)
    for n, T in ((262144, 1.0), (5000, 0.3), (130, 2.0)):
        logits = (3 * rng.normal(size=n)).astype(np.float32)
        for c in range(10):
            got = gh.sample_logits(ctx, logits, T, 99, c)
            want, margin = orc.sample(logits, T, orc.philox_uniform(99, c))
            assert got == want or margin < 1e-4, (n, T, c, got, want, margin)
        assert gh.sample_logits(ctx, logits, 0.0, 99, 0) == int(np.argmax(logits))


def test_sample_logits_top_k_matches_oracle(ctx):
    """Top-k draw (tile selection, wave sorting networks, rank-order
    inversion) against the oracle: equal logits give rank floor(u k) = that
    index exactly; k = 1 is the first maximum with the tied maxima in
    different tiles; random, heavily tied (values on a 0.5 grid, so the
    k-th value is shared across tiles), clustered (the top 64 in one block)
    and increasing logits, and more blocks than one staging pass holds
    (n = 300000), give the oracle's index except
    where u * total sits within 1e-4 of a boundary -- a tie broken the other
    way moves the index but not the boundary, so the margin never excuses
    it; k past n is n; out-of-range k is refused."""
    for k in (1, 5, 64):
        for c in range(8):
            u = orc.philox_uniform(11, c)
            got = gh.sample_logits(ctx, np.zeros(1000, np.float32), 0.9, 11, c, top_k=k)
            assert got == int(np.floor(u * k)), (k, c, got)
    rng = np.random.default_rng(4)
    l = rng.normal(size=262144).astype(np.float32)
    for i in (70000, 3, 250000):
        l[i] = 9.0
    for c in range(6):
        assert gh.sample_logits(ctx, l, 1.7, 5, c, top_k=1) == 3
    cases = [(262144, 1.0, 64, 3.0), (262144, 0.5, 17, 3.0), (5000, 2.0, 2, 3.0), (130, 1.0, 40, 3.0),
             (40, 1.0, 64, 3.0), (300000, 1.0, 50, 3.0), (262144, 1.0, 64, "ties"), (262144, 0.7, 33, "ties"),
             (262144, 4.0, 64, "cluster"), (262144, 30.0, 64, "ramp")]
    for n, T, k, scale in cases:
        if scale == "ties":  # a 0.5 grid: hundreds of exact ties at every top value
            logits = (np.round(2 * rng.normal(size=n) * 1.5) / 2).astype(np.float32)
        elif scale == "cluster":  # the 64 largest in one 64-row block, the next ones scattered
            logits = rng.normal(size=n).astype(np.float32)
            logits[131072:131136] = 8.0 + rng.normal(size=64).astype(np.float32)
        elif scale == "ramp":  # increasing with the index: every tile beats the ones before it
            logits = np.linspace(-20.0, 20.0, n, dtype=np.float32)
        else:
            logits = (scale * rng.normal(size=n)).astype(np.float32)
        for c in range(12):
            got = gh.sample_logits(ctx, logits, T, 21, c, top_k=k)
            want, margin = orc.sample_top_k(logits, T, k, orc.philox_uniform(21, c))
            assert got == want or margin < 1e-4, (n, T, k, scale, c, got, want, margin)
    assert gh.sample_logits(ctx, l, 0.0, 5, 0, top_k=8) == 3
    for bad in (-1, 65):
        with pytest.raises(gh.GemmaHipError):
            gh.sample_logits(ctx, l, 1.0, 5, 0, top_k=bad)


def test_exchange_probe(ctx):
    """gh_time_exchange: a positive, finite time per all-to-all exchange for
    small and chip-wide groups; group sizes past the CUs or 256 are refused."""
    for n in (8, 64):
        us = gh.time_exchange(ctx, n, 500)
        assert 0.0 < us < 1e3, (n, us)
    for bad in (0, 257):
        with pytest.raises(gh.GemmaHipError):
            gh.time_exchange(ctx, bad, 10)

