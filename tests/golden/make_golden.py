"""Write the committed oracle fixtures for the full-model parity tests.

  python tests/golden/make_golden.py [--config NAME] [--threads N]

For a config it regenerates the seeded synthetic weights (gh_synth_*; the
same bytes a GPU box regenerates), runs the C oracle and stores the results
in tests/golden/<config>.npz.  The oracle is the checker here; nothing in the
product reads these files.

From position 0 (tiny, gemma3-1b, gemma3-1b-centered, gemma3-1b-untied) the
run is
  - a seeded prompt fed one token per step, then greedy decoding, with the
    generated ids and top-1/top-2 logit margins,
  - a teacher-forced phase after it (seeded input tokens, not the argmax)
    with the argmax and margin of every step: a random tied-embedding model
    falls into a repeated-token fixed point under greedy decoding (the
    current token's own embedding row wins), so this phase is what compares
    varied argmaxes,
  - the top-8 logits (indices in order, values) of every step from the last
    prompt token on,
  - the hidden state after every layer and the top-8 logits at a few steps.
gemma3-1b uses the BASELINE C3 weights (Q4_0 codes uniform in [0, 15]).
With them every row of every projection carries a common -0.5 * d offset
per block, and the final state, hence the argmax, hardly depends on the
input: all of its compared argmaxes are one token.  gemma3-1b-centered is
the same shape with zero-mean codes (gemma_hip.center_q4_0), whose forced
argmaxes vary; the script asserts that they do.

gemma3-1b-untied adds an untied output.weight LM head (src/Gemma/Model.hs
:412-414, 988) to gemma3-1b-centered; the tied model's fixed point is gone
and the script asserts that the 64 greedy ids vary.

gemma3-4b (C5) starts from a 4096-position KV cache filled by gh_synth_kv
(the bytes KVCache.synth uploads), with centred codes, and records 32 greedy
steps at positions 4096.. and then 32 teacher-forced steps, with the layer
states at four of them.
"""
from __future__ import annotations

import argparse
import sys
import time
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parents[2]
sys.path[:0] = [str(REPO / "gemma.hs_amd"), str(REPO / "oracle")]

import gemma_hip as gh  # noqa: E402
import pyoracle as orc  # noqa: E402

# preset, weight seed, q4, centred codes, prompt length, generated tokens,
# forced tokens, steps with layer dumps
CASES = {
    "tiny": dict(preset="tiny", seed=7, q4=False, centered=False, n_prompt=16, n_gen=32, n_forced=32,
                 dump=(0, 15, 46, 78)),
    "gemma3-1b": dict(preset="gemma3-1b", seed=1234, q4=True, centered=False, n_prompt=128, n_gen=64,
                      n_forced=64, dump=(0, 127, 190, 254)),
    "gemma3-1b-centered": dict(preset="gemma3-1b", seed=1234, q4=True, centered=True, n_prompt=128,
                               n_gen=64, n_forced=64, dump=(0, 127, 190, 254), min_distinct_forced=48),
    # an untied output.weight LM head (src/Gemma/Model.hs:412-414, 988)
    # breaks the tied model's repeated-token fixed point: its 64 greedy ids
    # vary
    "gemma3-1b-untied": dict(preset="gemma3-1b", seed=1234, q4=True, centered=True, untied=True, n_prompt=128,
                             n_gen=64, n_forced=32, dump=(0, 127, 160, 220), min_distinct_greedy=32,
                             min_distinct_forced=24),
}
# C5: prefilled cache of kv_pos positions (gh_synth_kv seed kv_seed, N(0, 1)),
# then n_gen greedy steps from one seeded token and n_forced teacher-forced
# steps; centred codes, so the forced argmaxes vary
PREFILLED = {
    "gemma3-4b": dict(preset="gemma3-4b", seed=1234, q4=True, centered=True, kv_seed=5, kv_pos=4096, n_gen=32,
                      n_forced=32, dump=(0, 16, 31, 63), min_distinct_forced=24),
}
PROMPT_SEED = 1


def build_oracle(cfg, seed, q4, centered=False, untied=False):
    om = orc.OracleModel(cfg)
    for name, dtype, arr in gh.synth_tensors(cfg, seed, q4, centered=centered, untied=untied):
        om.set_tensor(name, arr, dtype)
    return om


def top8(logits):
    o = np.argsort(-logits, kind="stable")[:8]
    return o.astype(np.int32), logits[o]


def run_from_zero(name, case):
    cfg = gh.preset(case["preset"])
    prompt = gh.synth_tokens(PROMPT_SEED, "prompt", case["n_prompt"], cfg.vocab)
    t0 = time.time()
    om = build_oracle(cfg, case["seed"], case["q4"], case["centered"], case.get("untied", False))
    print(f"weights ready in {time.time() - t0:.1f}s", flush=True)
    n_greedy = case["n_prompt"] + case["n_gen"] - 1
    forced = gh.synth_tokens(PROMPT_SEED + 1, "forced", case["n_forced"], cfg.vocab)
    n_steps = n_greedy + case["n_forced"]
    ids, margins, layers, top_idx, top_val = [], [], {}, {}, {}
    f_ids, f_margins = [], []
    topk_idx, topk_val = [], []  # every step from the last prompt token on
    tok = int(prompt[0])
    t0 = time.time()
    for pos in range(n_steps):
        want = pos in case["dump"]
        logits, lay, best = om.step(tok, pos, want_layers=want)
        if want:
            layers[pos] = lay
            top_idx[pos], top_val[pos] = top8(logits)
        srt = np.sort(logits)
        if pos + 1 >= case["n_prompt"]:
            i8, v8 = top8(logits)
            topk_idx.append(i8)
            topk_val.append(v8)
        if pos + 1 < case["n_prompt"]:
            tok = int(prompt[pos + 1])
        elif pos < n_greedy:
            ids.append(best)
            margins.append(float(srt[-1] - srt[-2]))
            tok = best if pos + 1 < n_greedy else int(forced[0])
        else:
            f_ids.append(best)
            f_margins.append(float(srt[-1] - srt[-2]))
            k = pos - n_greedy + 1
            tok = int(forced[k]) if k < len(forced) else -1
        if pos % 32 == 0:
            print(f"step {pos}/{n_steps} {time.time() - t0:.1f}s", flush=True)
    dump = np.array(sorted(layers), np.int32)
    distinct = len(set(ids) | set(f_ids))
    need = case.get("min_distinct_forced", 0)
    assert len(set(f_ids)) >= need, f"{name}: {len(set(f_ids))} distinct forced argmaxes, need {need}"
    need = case.get("min_distinct_greedy", 0)
    assert len(set(ids)) >= need, f"{name}: {len(set(ids))} distinct greedy ids, need {need}: {ids}"
    out = REPO / "tests" / "golden" / f"{name}.npz"
    np.savez_compressed(
        out, config=np.frombuffer(bytes(cfg), np.uint8), seed=np.int64(case["seed"]),
        q4=np.int32(case["q4"]), centered=np.int32(case["centered"]), untied=np.int32(case.get("untied", False)),
        prompt=prompt,
        ids=np.array(ids, np.int32), margins=np.array(margins, np.float32), forced=forced,
        forced_ids=np.array(f_ids, np.int32), forced_margins=np.array(f_margins, np.float32),
        dump_steps=dump, topk_idx=np.stack(topk_idx), topk_val=np.stack(topk_val),
        layers=np.stack([layers[p] for p in dump]), top_idx=np.stack([top_idx[p] for p in dump]),
        top_val=np.stack([top_val[p] for p in dump]))
    print(f"wrote {out}; min greedy margin {min(margins):.3g}, min forced margin {min(f_margins):.3g}; "
          f"{len(set(ids))} distinct greedy ids, {len(set(f_ids))} distinct forced argmaxes, "
          f"{distinct} distinct compared argmaxes; {time.time() - t0:.1f}s")


def run_prefilled(name, case):
    cfg = gh.preset(case["preset"])
    n0, n_gen, n_forced = case["kv_pos"], case["n_gen"], case["n_forced"]
    cfg.max_seq = n0 + n_gen + n_forced
    t0 = time.time()
    om = build_oracle(cfg, case["seed"], case["q4"], case["centered"])
    width = cfg.n_kv_heads * cfg.head_dim
    for l in range(cfg.n_layers):
        k, v = gh.synth_kv(case["kv_seed"], l, n0, width, 1.0)
        om.set_kv(l, k, v)
    print(f"weights and cache ready in {time.time() - t0:.1f}s", flush=True)
    first = gh.synth_tokens(PROMPT_SEED, "c5", 1, cfg.vocab)
    forced = gh.synth_tokens(PROMPT_SEED + 1, "c5-forced", n_forced, cfg.vocab)
    tok = int(first[0])
    ids, margins, f_ids, f_margins, layers, topk_idx, topk_val = [], [], [], [], [], [], []
    t0 = time.time()
    for i in range(n_gen + n_forced):
        logits, lay, best = om.step(tok, n0 + i, want_layers=i in case["dump"])
        if i in case["dump"]:
            layers.append(lay)
        i8, v8 = top8(logits)
        topk_idx.append(i8)
        topk_val.append(v8)
        srt = np.sort(logits)
        if i < n_gen:
            ids.append(best)
            margins.append(float(srt[-1] - srt[-2]))
            tok = best if i + 1 < n_gen else int(forced[0])
        else:
            f_ids.append(best)
            f_margins.append(float(srt[-1] - srt[-2]))
            k = i - n_gen + 1
            tok = int(forced[k]) if k < n_forced else -1
        print(f"step {n0 + i} {time.time() - t0:.1f}s", flush=True)
    need = case.get("min_distinct_forced", 0)
    assert len(set(f_ids)) >= need, f"{name}: {len(set(f_ids))} distinct forced argmaxes, need {need}"
    out = REPO / "tests" / "golden" / f"{name}.npz"
    np.savez_compressed(
        out, config=np.frombuffer(bytes(cfg), np.uint8), seed=np.int64(case["seed"]), q4=np.int32(case["q4"]),
        centered=np.int32(case["centered"]), kv_seed=np.int64(case["kv_seed"]), kv_pos=np.int32(n0), first=first,
        ids=np.array(ids, np.int32), margins=np.array(margins, np.float32), forced=forced,
        forced_ids=np.array(f_ids, np.int32), forced_margins=np.array(f_margins, np.float32),
        dump_steps=np.array(case["dump"], np.int32), topk_idx=np.stack(topk_idx), topk_val=np.stack(topk_val),
        layers=np.stack(layers))
    print(f"wrote {out}; {len(set(ids))} distinct greedy ids, {len(set(f_ids))} distinct forced argmaxes, "
          f"min greedy margin {min(margins):.3g}, min forced margin {min(f_margins):.3g}; {time.time() - t0:.1f}s")


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--config", default="gemma3-1b", choices=sorted(CASES) + sorted(PREFILLED))
    ap.add_argument("--threads", type=int, default=8)
    a = ap.parse_args(argv)
    orc.set_threads(a.threads)
    if a.config in CASES:
        run_from_zero(a.config, CASES[a.config])
    else:
        run_prefilled(a.config, PREFILLED[a.config])


if __name__ == "__main__":
    main()
