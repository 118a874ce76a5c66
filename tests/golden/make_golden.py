"""Write the committed oracle fixtures for the full-model parity tests.

  python tests/golden/make_golden.py [--config gemma3-1b|tiny] [--threads N]

For a config it regenerates the seeded synthetic weights (gh_synth_*; the
same bytes a GPU box regenerates), runs the C oracle over a seeded prompt
with greedy decoding, and stores
  - the generated ids and top-1/top-2 logit margins per generated token,
  - a teacher-forced phase after it (seeded input tokens, not the argmax)
    with the argmax and margin of every step -- random tied-embedding
    models fall into a repeated-token fixed point under pure greedy
    decoding, so this phase is what checks many distinct argmaxes,
  - the hidden state after every layer at a few steps,
  - the top-8 logits at those steps,
in tests/golden/<config>.npz.  The oracle is the checker here; nothing in
the product reads these files.
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

# (preset, weight seed, q4, prompt length, generated tokens, steps with layer dumps)
CASES = {
    "tiny": dict(preset="tiny", seed=7, q4=False, n_prompt=16, n_gen=32, n_forced=32, dump=(0, 15, 46, 78)),
    "gemma3-1b": dict(preset="gemma3-1b", seed=1234, q4=True, n_prompt=128, n_gen=64, n_forced=64,
                      dump=(0, 127, 190, 254)),
}
PROMPT_SEED = 1


def build_oracle(cfg, seed, q4):
    om = orc.OracleModel(cfg)
    for name, dtype, arr in gh.synth_tensors(cfg, seed, q4):
        om.set_tensor(name, arr, dtype)
    return om


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--config", default="gemma3-1b", choices=sorted(CASES))
    ap.add_argument("--threads", type=int, default=8)
    a = ap.parse_args(argv)
    case = CASES[a.config]
    orc.set_threads(a.threads)
    cfg = gh.preset(case["preset"])
    prompt = gh.synth_tokens(PROMPT_SEED, "prompt", case["n_prompt"], cfg.vocab)
    t0 = time.time()
    om = build_oracle(cfg, case["seed"], case["q4"])
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
            o = np.argsort(-logits, kind="stable")[:8]
            top_idx[pos], top_val[pos] = o.astype(np.int32), logits[o]
        srt = np.sort(logits)
        if pos + 1 >= case["n_prompt"]:
            o = np.argsort(-logits, kind="stable")[:8]
            topk_idx.append(o.astype(np.int32))
            topk_val.append(logits[o])
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
    out = REPO / "tests" / "golden" / f"{a.config}.npz"
    np.savez_compressed(
        out, config=np.frombuffer(bytes(cfg), np.uint8), seed=np.int64(case["seed"]),
        q4=np.int32(case["q4"]), prompt=prompt, ids=np.array(ids, np.int32),
        margins=np.array(margins, np.float32), forced=forced, forced_ids=np.array(f_ids, np.int32),
        forced_margins=np.array(f_margins, np.float32), dump_steps=dump,
        topk_idx=np.stack(topk_idx), topk_val=np.stack(topk_val),
        layers=np.stack([layers[p] for p in dump]), top_idx=np.stack([top_idx[p] for p in dump]),
        top_val=np.stack([top_val[p] for p in dump]))
    print(f"wrote {out}; min greedy margin {min(margins):.3g}, min forced margin {min(f_margins):.3g}, "
          f"{len(set(f_ids))} distinct forced argmaxes; {time.time() - t0:.1f}s")


if __name__ == "__main__":
    main()
