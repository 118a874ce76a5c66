"""Batched prompt prefill on the MI355X against the oracle (marked gpu).

The reference has no prefill: its prompt loop feeds one token per call
(app/Main.hs:426-436).  So the prefill's bar is the oracle stepping the same
tokens one at a time:
- the hidden state after every layer and the logits of the last prompt
  token are within 1e-4 relative (max |a-b| / max |b|), as for a decode step;
- the next token is identical;
- the greedy ids generated after the prefill are identical to the committed
  fixtures.
The decode steps after a prefill read the K/V rows it appended, so they
check the cache contents too.
"""
from __future__ import annotations

import numpy as np
import pytest

import gemma_hip as gh
import pyoracle as orc
from conftest import GOLDEN, rel_err

pytestmark = pytest.mark.gpu

ACT_TOL = 1e-4


def _gpu_model(ctx, cfg, seed, q4):
    m = gh.GemmaModel(ctx, cfg)
    m.synth(seed, q4)
    return m


def _oracle_model(cfg, seed, q4):
    om = orc.OracleModel(cfg)
    for name, dtype, arr in gh.synth_tensors(cfg, seed, q4):
        om.set_tensor(name, arr, dtype)
    return om


def _mini4b(mode, window=5, layers=4):
    cfg = gh.preset("gemma3-4b")
    cfg.vocab, cfg.hidden, cfg.n_layers, cfg.ffn = 2048, 512, layers, 1024
    cfg.sliding_window, cfg.global_every, cfg.max_seq, cfg.mode = window, 2, 128, mode
    return cfg


@pytest.mark.parametrize("name", ["tiny", "gemma3-1b"])
def test_prefill_matches_oracle_fixture(ctx, name):
    """Prefill of the fixture prompt: every layer of the last prompt token
    and its top-8 logits against the oracle's dump at that step; then the
    generated ids against the fixture's greedy ids."""
    fx = np.load(GOLDEN / f"{name}.npz")
    cfg = gh.preset("tiny" if name == "tiny" else "gemma3-1b")
    m = _gpu_model(ctx, cfg, int(fx["seed"]), bool(fx["q4"]))
    prompt, ids = fx["prompt"], fx["ids"]
    last = len(prompt) - 1
    dump = [int(p) for p in fx["dump_steps"]]
    assert last in dump
    i = dump.index(last)
    kv = gh.KVCache(m, 1024)
    logits, layers, nxt = gh.prefill(m, kv, prompt, want_logits=True, want_layers=True)
    assert len(kv) == len(prompt)
    for l in range(cfg.n_layers):
        err = rel_err(layers[l], fx["layers"][i][l])
        assert err < ACT_TOL, (l, err)
    assert rel_err(logits[fx["top_idx"][i]], fx["top_val"][i]) < ACT_TOL
    assert rel_err(logits[fx["topk_idx"][0]], fx["topk_val"][0]) < ACT_TOL
    assert nxt == ids[0]
    got = gh.generate(m, gh.KVCache(m, 1024), prompt, len(ids), prefill=True)
    np.testing.assert_array_equal(got, ids)


@pytest.mark.parametrize("mode", [gh.MODE_GEMMA3, gh.MODE_REF])
def test_prefill_gqa_window_then_decode_live_oracle(ctx, mode):
    """4B-shaped Q4_0 miniature (8 q heads / 4 kv heads, head_dim 256,
    window 5 that binds, global every 2nd layer): a 19-token prefill, then
    6 decode steps that attend over the prefilled K/V; every layer and the
    logits against the oracle stepping the same tokens."""
    cfg = _mini4b(mode)
    m = _gpu_model(ctx, cfg, 99, True)
    om = _oracle_model(cfg, 99, True)
    toks = gh.synth_tokens(8, "t", 25, cfg.vocab)
    n_pf = 19
    for pos in range(n_pf - 1):
        om.step(int(toks[pos]), pos)
    olog, olay, obest = om.step(int(toks[n_pf - 1]), n_pf - 1, want_layers=True)
    kv = gh.KVCache(m, 64)
    logits, layers, nxt = gh.prefill(m, kv, toks[:n_pf], want_layers=True)
    for l in range(cfg.n_layers):
        assert rel_err(layers[l], olay[l]) < ACT_TOL, l
    assert rel_err(logits, olog) < ACT_TOL
    assert nxt == obest
    for pos in range(n_pf, len(toks)):
        logits, _, layers, _ = gh.runGemmaInferenceCachedWithLayer0(m, int(toks[pos]), kv)
        olog, olay, _ = om.step(int(toks[pos]), pos, want_layers=True)
        for l in range(cfg.n_layers):
            assert rel_err(layers[l], olay[l]) < ACT_TOL, (pos, l)
        assert rel_err(logits, olog) < ACT_TOL, pos


def test_prefill_gqa_long_window_chunks_live_oracle(ctx):
    """GQA miniature (4 kv heads, group 2) with a 300-token prefill: the
    attention of each token is split over several chunks (one per 128
    positions), global layers attend to all 300 positions and local layers
    to a 160-token window; the last token's layers and logits against the
    oracle stepping the same tokens."""
    cfg = _mini4b(gh.MODE_GEMMA3, window=160, layers=2)
    cfg.max_seq = 320
    m = _gpu_model(ctx, cfg, 17, True)
    om = _oracle_model(cfg, 17, True)
    toks = gh.synth_tokens(9, "long", 300, cfg.vocab)
    for pos in range(len(toks) - 1):
        om.step(int(toks[pos]), pos)
    olog, olay, obest = om.step(int(toks[-1]), len(toks) - 1, want_layers=True)
    kv = gh.KVCache(m, 320)
    logits, layers, nxt = gh.prefill(m, kv, toks, want_layers=True)
    for l in range(cfg.n_layers):
        assert rel_err(layers[l], olay[l]) < ACT_TOL, l
    assert rel_err(logits, olog) < ACT_TOL
    assert nxt == obest


def test_prefill_passes_chunks_and_ragged_sizes(ctx):
    """f32 tiny model, 600 tokens: one prefill call (two passes of 512 + 88
    rows), the same tokens as prefills of 1, 63, 65, 7 and 464 tokens, and
    the decode step token by token all reach the same last-token logits and
    next token; the caches then continue identically."""
    cfg = gh.preset("tiny")
    m = _gpu_model(ctx, cfg, 7, False)
    toks = gh.synth_tokens(11, "long", 600, cfg.vocab)
    kv_a = gh.KVCache(m, 640)
    la, _, na = gh.prefill(m, kv_a, toks)
    kv_b = gh.KVCache(m, 640)
    at = 0
    for k in (1, 63, 65, 7, 464):
        lb, _, nb = gh.prefill(m, kv_b, toks[at:at + k])
        at += k
    assert at == 600 and len(kv_a) == len(kv_b) == 600
    kv_c = gh.KVCache(m, 640)
    for t in toks:
        lc, _, nc = gh.runGemmaInferenceCached(m, int(t), kv_c)
    assert rel_err(la, lc) < ACT_TOL and rel_err(lb, lc) < ACT_TOL
    assert na == nb == nc
    ga = gh.generate(m, kv_a, [na], 6)
    gb = gh.generate(m, kv_b, [nb], 6)
    gc = gh.generate(m, kv_c, [nc], 6)
    np.testing.assert_array_equal(ga, gc)
    np.testing.assert_array_equal(gb, gc)


@pytest.mark.parametrize("nq,nkv", [(4, 4), (8, 1)])
def test_prefill_matrix_core_attention_groups_ragged_windows(ctx, nq, nkv):
    """head_dim 256 with GQA groups 1 and 8 (the 2 and 4 of the other tests
    aside): 150 tokens prefilled as pieces of 70, 1 and 79 (so later pieces
    start past position 0 and their key chunks cover earlier pieces), a
    40-token window on the local layer; the last token's logits and next
    token against the decode step fed token by token, then both caches
    continue identically."""
    cfg = _mini4b(gh.MODE_GEMMA3, window=40, layers=2)
    cfg.n_heads, cfg.n_kv_heads, cfg.max_seq = nq, nkv, 160
    m = _gpu_model(ctx, cfg, 23, True)
    toks = gh.synth_tokens(12, "fa", 150, cfg.vocab)
    kv_a = gh.KVCache(m, 160)
    at = 0
    for k in (70, 1, 79):
        la, _, na = gh.prefill(m, kv_a, toks[at:at + k])
        at += k
    kv_b = gh.KVCache(m, 160)
    for t in toks:
        lb, _, nb = gh.runGemmaInferenceCached(m, int(t), kv_b)
    assert rel_err(la, lb) < ACT_TOL and na == nb
    np.testing.assert_array_equal(gh.generate(m, kv_a, [na], 5), gh.generate(m, kv_b, [nb], 5))


def test_prefill_single_token_equals_step(ctx):
    """A prefill of one token is the decode step of that token."""
    cfg = _mini4b(gh.MODE_GEMMA3, layers=2)
    m = _gpu_model(ctx, cfg, 5, True)
    toks = gh.synth_tokens(2, "one", 3, cfg.vocab)
    kv_a, kv_b = gh.KVCache(m, 16), gh.KVCache(m, 16)
    for t in toks:
        la, _, na = gh.prefill(m, kv_a, [int(t)])
        lb, _, nb = gh.runGemmaInferenceCached(m, int(t), kv_b)
        assert rel_err(la, lb) < ACT_TOL
        assert na == nb


def test_prefill_sampling_matches_step_sampling(ctx):
    """With temperature sampling set, the prefill's next token is the draw
    the decode step makes at the same position (Philox counter = position)."""
    cfg = gh.preset("tiny")
    m = _gpu_model(ctx, cfg, 3, False)
    toks = gh.synth_tokens(4, "s", 20, cfg.vocab)
    for seed in (1, 2, 3):
        kv_a, kv_b = gh.KVCache(m, 32), gh.KVCache(m, 32)
        kv_a.set_sampling(0.8, seed)
        kv_b.set_sampling(0.8, seed)
        _, _, na = gh.prefill(m, kv_a, toks, want_logits=False)
        for t in toks:
            _, _, nb = gh.runGemmaInferenceCached(m, int(t), kv_b, want_logits=False)
        assert na == nb, seed


def test_prefill_errors_leave_cache_unchanged(ctx):
    cfg = gh.preset("tiny")
    m = _gpu_model(ctx, cfg, 1, False)
    kv = gh.KVCache(m, 8)
    gh.prefill(m, kv, [1, 2, 3])
    with pytest.raises(gh.GemmaHipError) as e:
        gh.prefill(m, kv, list(range(1, 7)))  # 3 + 6 > 8
    assert e.value.name == "GH_ERR_RANGE"
    with pytest.raises(gh.GemmaHipError) as e:
        gh.prefill(m, kv, [1, cfg.vocab])
    assert e.value.name == "GH_ERR_INVALID"
    with pytest.raises(gh.GemmaHipError) as e:
        gh.prefill(m, kv, np.zeros(0, np.int32))
    assert e.value.name == "GH_ERR_INVALID"
    with pytest.raises(gh.GemmaHipError) as e:
        gh.generate(m, kv, [1, 2, 3], 4, prefill=True)  # 3 + 3 + 3 > 8
    assert e.value.name == "GH_ERR_RANGE"
    assert len(kv) == 3
