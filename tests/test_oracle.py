"""Pin the C oracle (CPU): the reference's golden vectors, closed forms,
exhaustive fp16 decoding, and an independent float64 numpy model.

A mistake planted in the oracle (dropped (1 + w), transposed head mapping,
wrong nibble order, interleaved instead of split-half RoPE, ...) fails at
least one of these checks; see test_planted_mistakes_are_caught.
"""
from __future__ import annotations

import numpy as np
import pytest

import pyoracle as orc
from conftest import load_ref_golden, rel_err
from numpy_ref import NumpyGemma, attention as np_attention, gelu_tanh as np_gelu
from numpy_ref import q4_0_dequant_np, rms_norm as np_rms, rope as np_rope


# ---------------------------------------------------------------- Q4_0
def _blocks_with_scales(scales_u16: np.ndarray, code_byte: int) -> np.ndarray:
    n = scales_u16.size
    b = np.empty((n, 18), np.uint8)
    b[:, :2] = scales_u16.astype("<u2").view(np.uint8).reshape(n, 2)
    b[:, 2:] = code_byte
    return b.reshape(-1)


def test_f16_scale_decoding_exhaustive():
    """All 65536 fp16 patterns: FTZ (src/Gemma/GGUF.hs:797-820) and IEEE modes."""
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    raw = _blocks_with_scales(h, 0x99)  # every code 9 -> value (9-8)*d = d
    ref = h.view(np.float16).astype(np.float32)
    sub = ((h & 0x7C00) == 0) & ((h & 0x3FF) != 0)
    ref_ftz = ref.copy()
    ref_ftz[sub] = np.copysign(np.float32(0), ref[sub])
    for ftz, want in ((True, ref_ftz), (False, ref)):
        got = orc.q4_0_dequant(raw, ftz=ftz)[::32]
        nan = np.isnan(want)
        assert np.array_equal(np.isnan(got), nan)
        assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    # FTZ keeps the sign: -subnormal -> -0.0
    assert np.signbit(orc.q4_0_dequant(_blocks_with_scales(np.array([0x8001], np.uint16), 0x99), True)[0])


def test_q4_0_nibble_layout_roundtrip():
    """Pack with llama.cpp's quantize_row_q4_0 layout (byte j = q[j] | q[j+16]<<4)
    then dequantise: must give (q - 8) * d exactly."""
    rng = np.random.default_rng(0)
    nb = 64
    q = rng.integers(0, 16, size=(nb, 32))
    d = rng.uniform(0.001, 0.05, size=nb).astype(np.float16)
    b = np.empty((nb, 18), np.uint8)
    b[:, :2] = d.view(np.uint8).reshape(nb, 2)
    b[:, 2:] = (q[:, :16] | (q[:, 16:] << 4)).astype(np.uint8)
    got = orc.q4_0_dequant(b.reshape(-1)).reshape(nb, 32)
    want = ((q - 8) * d.astype(np.float32)[:, None]).astype(np.float32)
    assert np.array_equal(got, want)
    # and the independent numpy dequant agrees bit for bit
    assert np.array_equal(q4_0_dequant_np(b.reshape(-1), 1, nb * 32).reshape(nb, 32).astype(np.float32), got)


def test_q4_0_matvec_against_fp64():
    rng = np.random.default_rng(1)
    rows, cols = 96, 256
    raw = rng.integers(0, 256, size=rows * cols // 32 * 18, dtype=np.uint8).reshape(-1, 18)
    raw[:, :2] = (np.abs(rng.normal(0, 0.01, raw.shape[0])).astype(np.float16)).view(np.uint8).reshape(-1, 2)
    raw = raw.reshape(-1)
    x = rng.normal(size=cols).astype(np.float32)
    W = q4_0_dequant_np(raw, rows, cols)
    y64 = W @ x.astype(np.float64)
    bound = cols * np.finfo(np.float32).eps * (np.abs(W) @ np.abs(x.astype(np.float64)))
    y = orc.q4_0_matvec(raw, x, rows, cols)
    assert np.all(np.abs(y - y64) <= bound + 1e-30)


def test_linear_golden():
    """test/golden-values/linear_* (test/GemmaSpec.hs:209-221): 2x3 -> [14, 32]."""
    w = load_ref_golden("linear_weight").reshape(2, 3)
    x = load_ref_golden("linear_input")
    np.testing.assert_allclose(orc.f32_matvec(w, x), load_ref_golden("linear_output"), atol=1e-5)
    np.testing.assert_array_equal(orc.f32_matvec(w, x), [14.0, 32.0])


# ---------------------------------------------------------------- norms
def test_rmsnorm_golden_and_closed_form():
    x = load_ref_golden("rmsnorm_input")
    w = load_ref_golden("rmsnorm_weight")
    want = load_ref_golden("rmsnorm_output")
    # standard mode with w = 1 == zero-centred mode with w = 0
    for f in (orc.rmsnorm_tree, orc.rmsnorm_seq):
        np.testing.assert_allclose(f(x, w, zc=False), want, atol=1e-5)
        np.testing.assert_allclose(f(x, w - 1.0, zc=True), want, atol=1e-5)
    # test/GemmaSpec.hs:176-190 closed form
    np.testing.assert_allclose(orc.rmsnorm_tree([1, 2, 3, 4], [1, 1, 1, 1], zc=False),
                               [0.3651, 0.7303, 1.0954, 1.4606], atol=1e-3)


@pytest.mark.parametrize("n", [128, 1152, 2560, 6912])
def test_rmsnorm_random_vs_fp64(n):
    rng = np.random.default_rng(n)
    x = rng.normal(0, 3, n).astype(np.float32)
    w = rng.normal(0, 0.02, n).astype(np.float32)
    want = np_rms(x.astype(np.float64), w.astype(np.float64), 1e-6)
    assert rel_err(orc.rmsnorm_tree(x, w), want) < 2e-6
    assert rel_err(orc.rmsnorm_seq(x, w), want) < 2e-6


def test_qk_norm_per_head():
    rng = np.random.default_rng(2)
    nh, hd = 4, 256
    x = rng.normal(0, 5, nh * hd).astype(np.float32)
    w = rng.normal(0, 0.02, hd).astype(np.float32)
    want = np_rms(x.reshape(nh, hd).astype(np.float64), w.astype(np.float64), 1e-6).reshape(-1)
    assert rel_err(orc.qk_norm(x, w, nh, hd), want) < 2e-6


# ---------------------------------------------------------------- RoPE
def test_rope_position_zero_is_identity():
    x = load_ref_golden("rope_input_pos0")
    np.testing.assert_array_equal(orc.rope(x, 1, 4, 10000.0, 0), load_ref_golden("rope_output_pos0"))


def test_rope_split_half_matches_rotate_half():
    rng = np.random.default_rng(3)
    for hd, theta in ((32, 1e4), (256, 1e4), (256, 1e6)):
        x = rng.normal(size=(4, hd)).astype(np.float32)
        for pos in (1, 7, 383, 4351):
            want = np_rope(x.astype(np.float64), pos, theta)
            got = orc.rope(x.reshape(-1), 4, hd, theta, pos).reshape(4, hd)
            # the angle pos*f is rounded to f32 (as in the reference): |da| <~ pos * 2^-24
            tol = max(2e-5, 8.0 * pos * 2.0 ** -24)
            assert rel_err(got, want) < tol, (hd, theta, pos)


def test_rope_relative_position_and_norm():
    rng = np.random.default_rng(4)
    hd = 256
    q = rng.normal(size=hd).astype(np.float32)
    k = rng.normal(size=hd).astype(np.float32)
    d1 = np.dot(orc.rope(q, 1, hd, 1e4, 10), orc.rope(k, 1, hd, 1e4, 3))
    d2 = np.dot(orc.rope(q, 1, hd, 1e4, 107), orc.rope(k, 1, hd, 1e4, 100))
    assert abs(d1 - d2) < 1e-3 * np.linalg.norm(q) * np.linalg.norm(k)
    y = orc.rope(q, 1, hd, 1e4, 55)
    a, b = y[: hd // 2], y[hd // 2:]
    np.testing.assert_allclose(a * a + b * b, q[: hd // 2] ** 2 + q[hd // 2:] ** 2, rtol=1e-5)


def test_reference_rope_fixture_is_interleaved_not_split_half():
    """rope_output_pos1 is interleaved RoPE (quirk Q10): the split-half hot-path
    shader must NOT reproduce it, while the interleaved formula does."""
    x = load_ref_golden("rope_input_pos0").astype(np.float64)
    want = load_ref_golden("rope_output_pos1")
    inv = 1.0 / 10000 ** (np.arange(0, 4, 2) / 4)
    y = x.copy()
    for i in range(2):
        a, b = x[2 * i], x[2 * i + 1]
        y[2 * i] = a * np.cos(inv[i]) - b * np.sin(inv[i])
        y[2 * i + 1] = a * np.sin(inv[i]) + b * np.cos(inv[i])
    np.testing.assert_allclose(y, want, atol=1e-5)
    assert np.max(np.abs(orc.rope(x, 1, 4, 10000.0, 1) - want)) > 1e-2


# ---------------------------------------------------------------- attention
def test_attention_golden():
    """test/golden-values/attention_* (test/GemmaSpec.hs:293-330): two query rows
    over two cached positions, head_dim 2 == two q heads sharing one kv head."""
    q = load_ref_golden("attention_q")
    k = load_ref_golden("attention_k").reshape(2, 1, 2)
    v = load_ref_golden("attention_v").reshape(2, 1, 2)
    got = orc.attention(q, k, v, 2, 1, 2, 0, 2)
    np.testing.assert_allclose(got, load_ref_golden("attention_output"), atol=1e-4)


def test_gqa_golden_via_single_position():
    """With one cached position softmax is 1, so o_h = V[kv(h)]: the GQA head
    map h -> h // (nq/nkv) must reproduce test/golden-values/gqa_*_expanded."""
    for kind in ("k", "v"):
        inp = load_ref_golden(f"gqa_{kind}_input")
        exp = load_ref_golden(f"gqa_{kind}_expanded")
        hd = 8
        nkv, nq = inp.size // hd, exp.size // hd
        cache = inp.reshape(1, nkv, hd)
        q = np.ones(nq * hd, np.float32)
        got = orc.attention(q, cache, cache, nq, nkv, hd, 0, 1)
        np.testing.assert_array_equal(got, exp)


@pytest.mark.parametrize("nq,nkv,hd,L", [(4, 1, 256, 37), (8, 4, 256, 100), (4, 1, 32, 17)])
def test_attention_vs_fp64(nq, nkv, hd, L):
    rng = np.random.default_rng(L)
    q = rng.normal(size=(nq, hd)).astype(np.float32)
    K = rng.normal(size=(L, nkv, hd)).astype(np.float32)
    V = rng.normal(size=(L, nkv, hd)).astype(np.float32)
    for lo, hi in ((0, L), (L // 3, L), (0, 1)):
        want = np_attention(q.astype(np.float64), K[lo:hi].astype(np.float64), V[lo:hi].astype(np.float64),
                            nq, nkv)
        got = orc.attention(q.reshape(-1), K, V, nq, nkv, hd, lo, hi).reshape(nq, hd)
        assert rel_err(got, want) < 1e-5


# ---------------------------------------------------------------- GELU / argmax
def test_gelu_closed_form_and_golden():
    xs = np.array([0.0, 1.0, -1.0, 2.0, 5.0, 11.0, 17.0, -3.0, 0.3, -12.0], np.float32)
    got = np.array([orc.gelu_tanh(float(v)) for v in xs])
    np.testing.assert_allclose(got, np_gelu(xs.astype(np.float64)), rtol=2e-6, atol=1e-7)
    # the golden fixture is erf-GELU; the reference's own tolerance is 2e-4
    gi, go = load_ref_golden("gelu_input"), load_ref_golden("gelu_output")
    np.testing.assert_allclose([orc.gelu_tanh(float(v)) for v in gi], go, atol=2e-4)
    g = np.array([0.5, -2.0, 3.0], np.float32)
    u = np.array([2.0, 1.0, -1.0], np.float32)
    np.testing.assert_allclose(orc.geglu(g, u), np_gelu(g.astype(np.float64)) * u, rtol=2e-6)


def test_argmax_first_maximum():
    v = np.array([1.0, 5.0, -2.0, 5.0, 3.0], np.float32)
    assert orc.argmax(v) == int(np.argmax(v)) == 1
    rng = np.random.default_rng(5)
    w = rng.normal(size=262144).astype(np.float32)
    assert orc.argmax(w) == int(np.argmax(w))


def test_philox_known_answer_vectors():
    """Random123's published philox4x32-10 known-answer vectors."""
    kat = [((0, 0, 0, 0), (0, 0), (0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8)),
           ((0xffffffff,) * 4, (0xffffffff,) * 2, (0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd)),
           ((0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344), (0xa4093822, 0x299f31d0),
            (0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1))]
    for ctr, key, want in kat:
        assert tuple(int(v) for v in orc.philox4x32_10(ctr, key)) == want
    u = [orc.philox_uniform(7, c) for c in range(2000)]
    assert all(0.0 <= x < 1.0 for x in u)
    assert abs(np.mean(u) - 0.5) < 0.02 and abs(np.var(u) - 1 / 12) < 0.01


def test_sampler_closed_forms_and_frequencies():
    """Equal logits: index floor(u n); one dominant logit: always it; small
    vocabulary: empirical frequencies match softmax(l / T)."""
    n = 37
    for u in (0.0, 0.2, 0.5, 0.999):
        assert orc.sample(np.zeros(n, np.float32), 0.7, u)[0] == int(np.floor(u * n))
    l = np.full(50, -40.0, np.float32)
    l[13] = 40.0
    assert all(orc.sample(l, 1.0, u)[0] == 13 for u in (1e-6, 0.5, 0.9999))
    rng = np.random.default_rng(1)
    logits = rng.normal(size=8).astype(np.float32)
    T = 0.8
    p = np.exp(logits / T - np.max(logits / T))
    p /= p.sum()
    draws = [orc.sample(logits, T, orc.philox_uniform(3, c))[0] for c in range(20000)]
    freq = np.bincount(draws, minlength=8) / len(draws)
    assert np.max(np.abs(freq - p)) < 0.015


def test_top_k_sampler_closed_forms_and_frequencies():
    """Top-k draw: k = 1 is the first maximum for every u; equal logits rank
    by index, so the pick is floor(u k); k = n over logits that decrease with
    the index walks the same order as the full sampler (same pick for every
    u); a permutation of the logits picks the same value; frequencies
    match softmax over the k largest (numpy argsort, an independent
    ranking)."""
    rng = np.random.default_rng(5)
    l = rng.normal(size=300).astype(np.float32)
    l[[17, 90, 250]] = l.max() + 1.0  # tied maximum: the first one wins
    us = [orc.philox_uniform(11, c) for c in range(200)]
    assert all(orc.sample_top_k(l, 0.9, 1, u)[0] == 17 for u in us)
    for k in (1, 5, 64):
        for u in (0.0, 0.3, 0.77, 0.999):
            assert orc.sample_top_k(np.zeros(100, np.float32), 1.3, k, u)[0] == int(np.floor(u * k))
    dec = np.sort(rng.normal(size=40).astype(np.float32))[::-1].copy()
    for u in us:
        a, ma = orc.sample_top_k(dec, 0.7, 40, u)
        b, mb = orc.sample(dec, 0.7, u)
        assert a == b or min(ma, mb) < 1e-9
    lp = l[rng.permutation(len(l))]
    for k in (3, 40):
        for u in us[:50]:  # the ranked values, hence the walk, do not depend on the order
            assert l[orc.sample_top_k(l, 1.1, k, u)[0]] == lp[orc.sample_top_k(lp, 1.1, k, u)[0]]
    logits = rng.normal(size=30).astype(np.float32) * 2
    T, k = 0.8, 6
    top = np.argsort(-logits, kind="stable")[:k]
    p = np.exp((logits[top] - logits[top[0]]) / T)
    p /= p.sum()
    draws = [orc.sample_top_k(logits, T, k, orc.philox_uniform(4, c))[0] for c in range(20000)]
    freq = np.array([np.mean(np.asarray(draws) == t) for t in top])
    assert set(draws) <= set(top.tolist())
    assert np.max(np.abs(freq - p)) < 0.015


def _softcap_violations(f, cap: float) -> list[str]:
    """Properties that fix a soft cap sigma * tanh(y / sigma) without
    restating it (the body of runMatmulQ4_0DSL, which
    src/Gemma/Layers/LinearQ4.hs:37-48 names, is absent from the reference):
      odd               f(-y) = -f(y)
      bounded           |f(y)| < cap and |f(y)| <= |y|
      unit slope at 0   f(y) = y - y^3 / (3 cap^2) + O(y^5)  (slope and cubic term)
      saturates         f(y) -> +-cap as y -> +-inf, monotone in between
      known point       f(cap * atanh(1/2)) = cap / 2
    Returns the names of the violated properties."""
    bad = []
    y = np.linspace(-8 * cap, 8 * cap, 4097).astype(np.float32)
    fy = np.asarray(f(y.copy(), cap), np.float64)
    fneg = np.asarray(f((-y).copy(), cap), np.float64)
    if np.max(np.abs(fy + fneg)) > 1e-6 * cap:
        bad.append("odd")
    if np.any(np.abs(fy) > cap * (1 + 1e-6)) or np.any(np.abs(fy) > np.abs(y) * (1 + 1e-6) + 1e-30):
        bad.append("bounded")
    small = np.array([1e-3, 1e-2, 3e-2, 0.1], np.float64) * cap
    fs = np.asarray(f(small.astype(np.float32), cap), np.float64)
    ys = small.astype(np.float32).astype(np.float64)
    taylor = ys - ys ** 3 / (3 * cap * cap)
    # 5th-order remainder 2 y^5 / (15 cap^4) plus f32 rounding
    if np.any(np.abs(fs - taylor) > 2 * ys ** 5 / (15 * cap ** 4) + 4e-7 * ys):
        bad.append("taylor")
    big = np.asarray(f(np.array([50 * cap, -50 * cap, 1e30], np.float32), cap), np.float64)
    if abs(big[0] - cap) > 1e-6 * cap or abs(big[1] + cap) > 1e-6 * cap or abs(big[2] - cap) > 1e-6 * cap:
        bad.append("saturates")
    if np.any(np.diff(fy) < -1e-6 * cap):
        bad.append("monotone")
    p = np.asarray(f(np.array([cap * np.arctanh(0.5)], np.float32), cap), np.float64)[0]
    if abs(p - cap / 2) > 2e-6 * cap:
        bad.append("atanh_half")
    return bad


def test_softcap_pinned_by_invariants():
    """orc_softcap (the runLinearQ4 soft-cap arm) satisfies every property,
    at the reference's default sigma 30 (src/Gemma/Layers/LinearQ4.hs:38)
    and other caps."""
    for cap in (30.0, 1.0, 7.5):
        assert _softcap_violations(orc.softcap, cap) == [], cap


def test_softcap_invariants_catch_planted_forms():
    """Plausible wrong soft caps each violate at least one property: a
    missing 1/cap inside tanh, a missing cap outside, a halved output, a
    rational cap, a hard clip and the identity."""
    planted = {
        "cap*tanh(y)": lambda y, c: c * np.tanh(y.astype(np.float64)),
        "tanh(y/cap)": lambda y, c: np.tanh(y.astype(np.float64) / c),
        "cap/2*tanh(y/cap)": lambda y, c: c / 2 * np.tanh(y.astype(np.float64) / c),
        "y/(1+|y|/cap)": lambda y, c: y.astype(np.float64) / (1 + np.abs(y.astype(np.float64)) / c),
        "clip": lambda y, c: np.clip(y.astype(np.float64), -c, c),
        "identity": lambda y, c: y.astype(np.float64),
        "cap*tanh(y/(2cap))": lambda y, c: c * np.tanh(y.astype(np.float64) / (2 * c)),
    }
    for name, f in planted.items():
        assert _softcap_violations(f, 30.0), name


# ---------------------------------------------------------------- whole model
def _tiny_cfg(**kw):
    c = orc.OrcConfig()
    base = dict(vocab=1024, hidden=128, n_layers=2, n_heads=4, n_kv_heads=1, head_dim=32, ffn=512,
                max_seq=64, sliding_window=0, global_every=0, rope_theta_local=1e4,
                rope_theta_global=1e4, rms_eps=1e-6, mode=orc.MODE_GEMMA3,
                flags=orc.QK_NORM | orc.POST_ATTN_NORM | orc.POST_FFN_NORM | orc.ZERO_CENTERED)
    base.update(kw)
    for k, v in base.items():
        setattr(c, k, v)
    return c


def _random_model(cfg, q4, seed, untied=False):
    rng = np.random.default_rng(seed)
    H, hd, F = cfg.hidden, cfg.head_dim, cfg.ffn
    shapes = {"token_embd.weight": (cfg.vocab, H), "output_norm.weight": (H,)}
    if untied:
        shapes["output.weight"] = (cfg.vocab, H)
    for l in range(cfg.n_layers):
        p = f"blk.{l}."
        shapes.update({p + "attn_norm.weight": (H,), p + "attn_q.weight": (cfg.n_heads * hd, H),
                       p + "attn_k.weight": (cfg.n_kv_heads * hd, H), p + "attn_v.weight": (cfg.n_kv_heads * hd, H),
                       p + "attn_q_norm.weight": (hd,), p + "attn_k_norm.weight": (hd,),
                       p + "attn_output.weight": (H, cfg.n_heads * hd), p + "post_attention_norm.weight": (H,),
                       p + "ffn_norm.weight": (H,), p + "ffn_gate.weight": (F, H), p + "ffn_up.weight": (F, H),
                       p + "ffn_down.weight": (H, F), p + "post_ffw_norm.weight": (H,)})
    om = orc.OracleModel(cfg)
    dense = {}
    for name, shp in shapes.items():
        if len(shp) == 1:
            a = rng.normal(0, 0.02, shp).astype(np.float32)
            om.set_tensor(name, a, orc.F32)
            dense[name] = a.astype(np.float64)
        elif q4:
            nbk = shp[0] * shp[1] // 32
            raw = rng.integers(0, 256, size=(nbk, 18), dtype=np.uint8)
            raw[:, :2] = np.abs(rng.normal(0, 0.01, nbk)).astype(np.float16).view(np.uint8).reshape(nbk, 2)
            raw = raw.reshape(-1)
            om.set_tensor(name, raw, orc.Q4_0)
            dense[name] = q4_0_dequant_np(raw, *shp)
        else:
            a = rng.normal(0, 0.02, shp).astype(np.float32)
            om.set_tensor(name, a, orc.F32)
            dense[name] = a.astype(np.float64)
    return om, dense


@pytest.mark.parametrize("q4,extra,untied", [
    (False, {}, False),
    (True, {"hidden": 256, "ffn": 512, "head_dim": 32, "n_heads": 8, "n_kv_heads": 2,
            "sliding_window": 5, "global_every": 2, "rope_theta_global": 1e6, "n_layers": 4}, False),
    (True, {}, True),
    (False, {}, True),
])
def test_oracle_model_matches_numpy_fp64(q4, extra, untied):
    """The whole step against an fp64 numpy restatement; `untied` gives the
    model an output.weight LM head (src/Gemma/Model.hs:412-414)."""
    cfg = _tiny_cfg(**extra)
    om, dense = _random_model(cfg, q4, seed=11, untied=untied)
    ref = NumpyGemma(cfg, dense)
    rng = np.random.default_rng(12)
    toks = rng.integers(0, cfg.vocab, size=12)
    for pos, tok in enumerate(toks):
        lg, layers, best = om.step(int(tok), pos, want_layers=True)
        rlg, rlayers = ref.step(int(tok), pos)
        for l in range(cfg.n_layers):
            assert rel_err(layers[l], rlayers[l]) < 1e-5, (pos, l)
        assert rel_err(lg, rlg) < 1e-5
        top2 = np.sort(rlg)[-2:]
        if top2[1] - top2[0] > 1e-4 * np.max(np.abs(rlg)):
            assert best == int(np.argmax(rlg))


def test_oracle_ref_mode_prefix_window():
    """Quirk Q3 (ref mode): every layer attends to the first min(len, W)
    positions; gemma3 mode uses the last W on local layers."""
    cfg_g = _tiny_cfg(sliding_window=3, global_every=0)
    cfg_r = _tiny_cfg(sliding_window=3, global_every=0, mode=orc.MODE_REF)
    om_g, dense = _random_model(cfg_g, False, seed=21)
    om_r, _ = _random_model(cfg_r, False, seed=21)
    toks = [5, 9, 100, 7, 3, 55]
    outs = []
    for om in (om_g, om_r):
        lg = None
        for pos, t in enumerate(toks):
            lg, _, _ = om.step(t, pos)
        outs.append(lg)
    # gemma3 mode with global_every=0 means all layers global -> full causal
    ref = NumpyGemma(cfg_g, dense)
    for pos, t in enumerate(toks):
        rlg, _ = ref.step(t, pos)
    assert rel_err(outs[0], rlg) < 1e-5
    # ref mode truncates to the first 3 positions at pos >= 3 -> differs
    assert rel_err(outs[1], rlg) > 1e-3


def test_untied_head_is_not_the_embedding():
    """With an output.weight, logits computed on the tied embedding (the
    mistake of ignoring lm_head.weight) are far from the oracle's, and the
    oracle's equal the fp64 restatement's on output.weight."""
    cfg = _tiny_cfg()
    om, dense = _random_model(cfg, True, seed=31, untied=True)
    ref = NumpyGemma(cfg, dense)
    tied = {k: v for k, v in dense.items() if k != "output.weight"}
    ref_tied = NumpyGemma(cfg, tied)
    for pos, tok in enumerate([3, 700, 41]):
        lg, _, _ = om.step(tok, pos)
        rlg, _ = ref.step(tok, pos)
        tlg, _ = ref_tied.step(tok, pos)
        assert rel_err(lg, rlg) < 1e-5
        assert rel_err(lg, tlg) > 0.5


def test_planted_mistakes_are_caught():
    """Each plausible mistake, planted in a copy of an oracle function, fails
    the corresponding check above."""
    x = load_ref_golden("rmsnorm_input")
    w = load_ref_golden("rmsnorm_weight") - 1.0
    want = load_ref_golden("rmsnorm_output")
    # dropped (1 + w): zero-centred weight used as a plain scale
    assert np.max(np.abs(orc.rmsnorm_tree(x, w, zc=False) - want)) > 0.1
    # wrong GQA head mapping (h % nkv instead of h // (nq/nkv))
    inp, exp = load_ref_golden("gqa_k_input"), load_ref_golden("gqa_k_expanded")
    nkv, nq, hd = 2, 4, 8
    bad = np.concatenate([inp.reshape(nkv, hd)[h % nkv] for h in range(nq)])
    assert not np.array_equal(bad, exp)
    # swapped nibble halves in Q4_0 unpacking
    b = np.zeros(18, np.uint8)
    b[:2] = np.array([1.0], np.float16).view(np.uint8)
    b[2] = 0x1F  # element 0 = 15, element 16 = 1
    got = orc.q4_0_dequant(b)
    assert got[0] == 7.0 and got[16] == -7.0


@pytest.mark.parametrize("q4,mode,untied", [(False, 0, False), (True, 0, False), (True, 1, False), (True, 0, True)])
def test_torch_cpu_restatement_agrees_with_the_c_oracle(q4, mode, untied):
    """oracle/torch_ref.py (bench.py's PyTorch-CPU baseline) against the C
    oracle on the tiny model: logits within 1e-5 relative and the same
    argmax at every step of a 24-token run (window 5 binds in both modes)."""
    import torch_ref
    import gemma_hip as gh
    cfg = gh.preset("tiny")
    cfg.sliding_window, cfg.global_every, cfg.max_seq, cfg.mode = 5, 2, 32, mode
    cfg.rope_theta_global = 1e6
    om = orc.OracleModel(cfg)
    tens = list(gh.synth_tensors(cfg, 11, q4, untied=untied))
    for name, dtype, arr in tens:
        om.set_tensor(name, arr, dtype)
    tm = torch_ref.TorchModel(cfg, tens)
    toks = gh.synth_tokens(3, "t", 24, cfg.vocab)
    for pos, t in enumerate(toks):
        ol, _, ob = om.step(int(t), pos)
        tl, tb = tm.step(int(t), pos)
        tl = tl.numpy()
        assert np.max(np.abs(tl - ol)) / np.max(np.abs(ol)) < 1e-5, pos
        s = np.sort(ol)
        if s[-1] - s[-2] > 1e-4 * np.max(np.abs(ol)):
            assert tb == ob, pos
