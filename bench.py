"""Decode benchmark: Gemma-3-1B-shaped Q4_0 batch-1 greedy decode on one MI355X.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]

A step is one decode token through the whole model (26 layers + LM head +
on-device argmax).  The seeded synthetic weights are generated on the host,
uploaded once, and stay resident in HBM; a seeded 128-token prompt is fed
one token per step (untimed, as in the reference's generation loop); W
warmup steps run on a scratch cache, and exactly K timed greedy steps
(HIP events on the step stream, device-synchronised on both sides) are
centred on C3's mean position 256: positions 128..383 at the default K =
256, 246..265 at K = 20.

Prints ONE JSON line with tok/s; per-kernel-kind execution times measured
inside real decode steps at C3's positions 128..383 (gh_profile_steps: the
step's kernels launched eagerly in order, each timed by its own dispatch's
begin and end timestamps, the quantity a rocprofv3 kernel trace reports;
every layer's weights are cold there, as in the decode loop); the roofline
of gate/up, the per-layer kernel with the largest share of the step (the LM
head, the largest single matvec, beside it); the kernel plan in use
(gh_model_plan); and the CPU baseline (bounded samples on the host cores).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path[:0] = [str(REPO / "gemma.hs_amd"), str(REPO / "oracle")]

METRIC = "decode tok/s, Gemma-3-1B Q4_0 batch 1; Q4 matvec HBM GB/s vs peak"
HBM_PEAK_GBPS = 8000.0
WEIGHT_SEED = 1234
PROMPT_SEED = 1
N_PROMPT = 128
C3_MEAN_POSITION = 256  # C3: prompt 128, greedy generation at positions 128..383
# HBM bytes per launch from two rocprofv3 --pmc passes (FETCH_SIZE, then
# WRITE_SIZE, each scaled by bytes / counter of a 256 MiB device copy) over
# replays of each kernel kind at position 257 (kernel_profile run --prompt
# 256 --prefill-prompt): profiles/step_kernels_gemma3-1b_decode_c3.md,
# gate/up 9,641,342 fetched + 170,496 written, the LM head 172,293,019 +
# 1,179,657.
GATE_UP_TRAFFIC_BYTES = 9_811_838
LM_HEAD_TRAFFIC_BYTES = 173_472_676
TRAFFIC_PROFILE = "profiles/step_kernels_gemma3-1b_decode_c3.md"
# the in-step kernel timings: C3's decode positions 128..383
PROFILE_STEPS = 256


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def host_cpu() -> dict:
    """The host's CPU model (lscpu's 'Model name', from /proc/cpuinfo), its
    logical CPU count and the threads this process may use: the pool sets
    OMP_NUM_THREADS to the box's CPU share, which os.cpu_count() does not see."""
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    n = os.cpu_count() or 1
    share = int(os.environ.get("OMP_NUM_THREADS") or n)
    try:
        share = min(share, len(os.sched_getaffinity(0)))
    except AttributeError:
        pass
    return {"cpu_model": model, "logical_cpus": n, "threads": max(1, min(n, share))}


def cpu_baseline(cfg, seconds: float) -> dict:
    """The CPU baseline on the host cores, on a bounded sample of the same
    workload (greedy decode of the seeded gemma3-1b Q4_0 model from position
    1, about `seconds` of CPU work per leg):
      - the headline leg: the PyTorch-CPU restatement (oracle/torch_ref.py),
        Q4_0 dequantised to f32 once (untimed), every thread of the box's
        share (torch.set_num_threads);
      - beside it, the C oracle (oracle/gemma_oracle.c, OpenMP) on the same
        threads, reading the Q4_0 bytes directly.
    The reference's own path (the WGSL shaders on Dawn's SwiftShader CPU
    adapter) does not exist in this image."""
    import gemma_hip as gh
    import pyoracle as orc
    host = host_cpu()
    threads = host["threads"]
    tensors = list(gh.synth_tensors(cfg, WEIGHT_SEED, True))
    prompt = gh.synth_tokens(PROMPT_SEED, "prompt", N_PROMPT, cfg.vocab)

    def run(step, label):
        step(int(prompt[0]), 0)  # warm caches / page in
        t0 = time.perf_counter()
        n, tok = 0, int(prompt[1])
        while time.perf_counter() - t0 < seconds:
            tok = step(tok, n + 1)
            n += 1
        dt = time.perf_counter() - t0
        log(f"  cpu baseline ({label}, {threads} threads): {n} steps in {dt:.1f} s -> {n / dt:.2f} tok/s")
        return n, dt

    orc.set_threads(threads)
    om = orc.OracleModel(cfg)
    for name, dtype, arr in tensors:
        om.set_tensor(name, arr, dtype)
    on, odt = run(lambda t, p: om.step(t, p)[2], "C oracle")
    om.close()
    oracle_leg = {"value": round(on / odt, 3), "unit": "tok/s", "cores": threads, "kind": "port",
                  "sample": f"{on} greedy steps at positions 1..{on} ({odt:.1f} s), oracle/gemma_oracle.c"}
    try:
        import torch
        import torch_ref
    except ImportError as e:  # torch absent on the box: the C-oracle leg is the baseline
        return {**oracle_leg, "host": host, "torch_leg": f"not run: {e}"}
    torch.set_num_threads(threads)
    t0 = time.perf_counter()
    tm = torch_ref.TorchModel(cfg, tensors, max_seq=N_PROMPT + 4096)
    prep = time.perf_counter() - t0
    tn, tdt = run(lambda t, p: tm.step(t, p)[1], "PyTorch-CPU")
    del tm
    return {"value": round(tn / tdt, 3), "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"{tn} greedy decode steps of the seeded gemma3-1b Q4_0 model at positions 1..{tn} "
                      f"({tdt:.1f} s; oracle/torch_ref.py, PyTorch {torch.__version__} on {threads} threads, "
                      f"weights dequantised to f32 once in {prep:.1f} s, untimed); the per-step cost is the "
                      f"weight pass, position-independent at these lengths",
            "host": host, "torch_version": torch.__version__, "c_oracle": oracle_leg}


def extras_c2_matvec(gh, ctx) -> dict:
    """C2: one Q4_0 matvec at the three Gemma-3-1B shapes, x ~ N(0, 1),
    rotating over >= 2 GiB of device copies of the weights so the 256 MB
    Infinity Cache cannot serve repeated reads.  Each call is
    gh_q4_0_matvec (the op-level runLinearQ4 path: split-K matvec plus its
    partial-sum kernel when the plan splits columns), captured into one
    graph with a call per copy and replayed; the time is per call."""
    import numpy as np
    out = {}
    for rows, cols, name in ((6912, 1152, "gate"), (1152, 6912, "down"), (262144, 1152, "lm_head")):
        raw = gh.synth_q4_0(7, f"c2.{name}", 0.01, rows, cols)
        wbytes = rows * cols // 32 * 18
        copies = -(-(2 << 30) // wbytes)
        ts = [gh.Q4Tensor(ctx, raw, rows, cols) for _ in range(copies)]
        x = gh.DeviceBuffer.from_numpy(ctx, np.random.default_rng(3).normal(size=cols).astype(np.float32))
        y = gh.DeviceBuffer(ctx, 4 * rows)
        for t in ts:
            gh._lib.check(gh.lib().gh_q4_0_matvec(t.h, x.ptr, y.ptr, 0, 0.0))
        # one graph holding one call per copy, replayed (no per-call launch cost)
        ctx.capture_begin()
        for t in ts:
            gh._lib.check(gh.lib().gh_q4_0_matvec(t.h, x.ptr, y.ptr, 0, 0.0))
        reps = max(1, 256 // copies)
        us = ctx.capture_replay(reps) * 1e3 / copies
        algo = wbytes + 4 * cols + 4 * rows
        out[f"{rows}x{cols}"] = {"avg_us": round(us, 3), "bytes": algo, "gbps": round(algo / us / 1e3, 1),
                                 "frac": round(algo / us / 1e3 / HBM_PEAK_GBPS, 4), "copies": copies}
        for t in ts:
            t.close()
        x.free()
        y.free()
        log(f"  C2 {rows}x{cols}: {us:.2f} us, {algo / us / 1e3:.0f} GB/s ({copies} copies)")
    return out


def extras_c4_attention(gh, ctx) -> dict:
    """C4: one decode query (4 q heads, 1 kv head, head_dim 256) over a
    K/V cache of 8192 or 32768 N(0, 1) positions, global (whole cache) and
    local (last 512), scale 1/16: gh_attention_decode (split-K attention
    plus its merge kernel).  The cache exists in enough copies to hold
    >= 512 MiB (32 of the 8192-position cache, 8 of the 32768 one), one call
    per copy is captured into a graph and the graph replayed, so no call
    finds its K/V in the 256 MB Infinity Cache."""
    import numpy as np
    out = {}
    rng = np.random.default_rng(4)
    hd, nq, nkv = 256, 4, 1
    q = gh.DeviceBuffer.from_numpy(ctx, rng.normal(size=nq * hd).astype(np.float32))
    o = gh.DeviceBuffer(ctx, 4 * nq * hd)
    for L in (8192, 32768):
        cache_bytes = 2 * L * nkv * hd * 4
        copies = max(4, -(-(512 << 20) // cache_bytes))
        kv = [(gh.DeviceBuffer.from_numpy(ctx, rng.normal(size=L * nkv * hd).astype(np.float32)),
               gh.DeviceBuffer.from_numpy(ctx, rng.normal(size=L * nkv * hd).astype(np.float32)))
              for _ in range(copies)]
        for kind, pb in (("global", 0), ("local", L - 512)):
            def call(k, v):
                gh._lib.check(gh.lib().gh_attention_decode(ctx.h, q.ptr, k.ptr, v.ptr, nq, nkv, hd, pb, L, 0, o.ptr))
            call(*kv[0])
            ctx.capture_begin()
            for k, v in kv:
                call(k, v)
            reps = max(2, 64 // copies)
            us = ctx.capture_replay(reps) * 1e3 / copies
            algo = 2 * (L - pb) * nkv * hd * 4 + 8 * nq * hd
            out[f"L{L}_{kind}"] = {"avg_us": round(us, 3), "bytes": algo, "gbps": round(algo / us / 1e3, 1),
                                   "frac": round(algo / us / 1e3 / HBM_PEAK_GBPS, 4), "copies": copies}
            log(f"  C4 L={L} {kind}: {us:.2f} us, {algo / us / 1e3:.0f} GB/s ({copies} copies)")
        for k, v in kv:
            k.free()
            v.free()
    q.free()
    o.free()
    return out


def in_step_kernels(gh, model, kv, n_steps: int) -> dict:
    """Execution time of every step kernel kind inside n_steps real greedy
    decode steps from the cache's position (gh_profile_steps: eager launches
    in the step's order, each timed by its own dispatch timestamps)."""
    stats = gh.profile_steps(model, kv, n_steps)
    return {st.name: st for st in stats}


def extras_c5_gemma3_4b(gh, ctx, steps: int = 256, warmup: int = 8) -> dict:
    """C5: Gemma-3-4B-shaped Q4_0 decode (34 layers, hidden 2560, 8 q / 4 kv
    heads, window 1024) with seeded synthetic weights; the KV cache holds
    seeded N(0, 1) K/V (gh_kv_synth, in place of running a prefill) up to
    the prompt token, and the timed greedy steps run at C5's positions
    4096..4351.  The in-step kernel timings (and the step's algorithmic
    bytes) come from a second cache of the same kind, at C5's mean
    position."""
    cfg = gh.preset("gemma3-4b")
    p0, n_prof = 4096, 8
    n0 = p0 - 1 - warmup  # the prompt token at n0, the warmup steps, then p0 .. p0 + steps - 1
    mid = p0 + steps // 2 - n_prof // 2  # profiled steps centred on the timed steps' mean position
    cfg.max_seq = max(p0 + steps, mid + n_prof) + 8
    model = gh.GemmaModel(ctx, cfg)
    model.synth(WEIGHT_SEED, q4=True)
    kv = gh.KVCache(model, cfg.max_seq)
    kv.synth(5, n0)
    prompt = gh.synth_tokens(PROMPT_SEED, "c5", 1, cfg.vocab)
    ms, _ = gh.bench_decode(model, kv, prompt, warmup, steps)
    tok_s = steps / (ms / 1e3)
    del kv
    kv = gh.KVCache(model, cfg.max_seq)
    kv.synth(5, mid)
    timings = in_step_kernels(gh, model, kv, n_prof)
    step_bytes = sum(t.bytes_per_launch * t.launches for t in timings.values()) / n_prof
    log(f"  C5 gemma3-4b @ {p0}..{p0 + steps - 1}: {tok_s:.1f} tok/s")
    out = {"value": round(tok_s, 2), "unit": "tok/s", "ms_per_step": round(ms / steps, 4), "steps": steps,
           "timed_positions": [p0, p0 + steps - 1], "profiled_positions": [mid, mid + n_prof - 1],
           "step_algorithmic_bytes": int(step_bytes),
           "step_frac_of_hbm_peak": round(step_bytes / (ms / steps * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
           "lm_head_gbps": round(timings["lm_head"].gbps, 1),
           "kernels_in_step": {t.name: {"avg_us": round(t.avg_us, 3), "gbps": round(t.gbps, 1),
                                        "per_step": t.launches // n_prof,
                                        "step_us": round(t.avg_us * t.launches / n_prof, 1)}
                               for t in timings.values()}}
    del kv, model
    return out


MFMA_FP16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 (and bf16) MFMA


def extras_f2_prefill(gh, ctx, model, sizes=(128, 512), reps: int = 5) -> dict:
    """f2: batched prefill of a seeded prompt on the C3 model (gh_prefill):
    wall time between two HIP events on the context stream (host launches
    included), median of `reps`, and the per-kernel profile of one more run.
    GEMM flops = 2 * tokens * rows * cols of the fused matrix; each Q4_0
    GEMM issues 2 fp16 MFMAs per product (hi and lo parts of the
    activations against the exact (q - 8) weights), so its MFMA utilisation
    is 2x the flop rate / the fp16 dense peak."""
    cfg = model.cfg
    H, F, hd = cfg.hidden, cfg.ffn, cfg.head_dim
    shapes = {"pf_qkv": ((cfg.n_heads + 2 * cfg.n_kv_heads) * hd, H), "pf_o": (H, cfg.n_heads * hd),
              "pf_gate_up": (2 * F, H), "pf_down": (H, F)}
    out = {}
    for n in sizes:
        prompt = gh.synth_tokens(PROMPT_SEED, "prefill", n, cfg.vocab)
        kv = gh.KVCache(model, n + 8)
        gh.prefill(model, kv, prompt, want_logits=False)  # warm-up (buffers, code)
        times = []
        for _ in range(reps):
            kv.reset()
            ctx.timer_start()
            gh.prefill(model, kv, prompt, want_logits=False)
            times.append(ctx.timer_stop())
        ms = sorted(times)[len(times) // 2]
        kv.reset()
        stats = gh.profile_prefill(model, kv, prompt)
        kern = {}
        gemm_ms = 0.0
        for st in stats:
            e = {"launches": st.launches, "total_us": round(st.total_ms * 1e3, 1)}
            if st.name in shapes:
                r, c = shapes[st.name]
                fl = 2.0 * n * r * c * st.launches
                tf = fl / (st.total_ms * 1e-3) / 1e12
                e["tflops"] = round(tf, 1)
                e["mfma_util"] = round(2 * tf / MFMA_FP16_PEAK_TFLOPS, 4)
                gemm_ms += st.total_ms
            kern[st.name] = e
        layer_flops = 2.0 * n * sum(r * c for r, c in shapes.values())
        tok_s = n / (ms * 1e-3)
        log(f"  f2 prefill {n} tokens: {ms:.3f} ms -> {tok_s:.0f} tok/s (GEMMs {gemm_ms:.3f} ms of events)")
        out[str(n)] = {"ms": round(ms, 4), "tok_s": round(tok_s, 1),
                       "gemm_tflops": round(layer_flops * cfg.n_layers / (gemm_ms * 1e-3) / 1e12, 1),
                       "kernels": kern}
        del kv
    return out


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extras", action="store_true", help="skip the C2/C4/C5 measurements")
    a = ap.parse_args(argv)
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build runs on one GPU only; multi-GPU runs (--gpus > 1) are not "
              "part of it (independent sequences would run one per GPU with no exchange)", file=sys.stderr)
        return 2

    import numpy as np

    import gemma_hip as gh

    cfg = gh.preset("gemma3-1b")
    t0 = time.time()
    ctx = gh.Context(0)
    model = gh.GemmaModel(ctx, cfg)
    model.synth(WEIGHT_SEED, q4=True)
    log(f"model ready in {time.time() - t0:.1f}s")
    prompt = gh.synth_tokens(PROMPT_SEED, "prompt", N_PROMPT, cfg.vocab)
    # C3 generates at positions 128..383 (mean 256).  The K timed steps are
    # centred on that mean, from s0 = max(128, 256 - K/2): with the default
    # K = 256 exactly C3's positions.  The W warmup steps run on a scratch
    # cache of the same model; the timed cache is fed the prompt and
    # advanced to s0 with untimed greedy steps, then K steps are timed.
    s0 = max(N_PROMPT, C3_MEAN_POSITION - a.steps // 2)
    if a.warmup > 0:
        gh.bench_decode(model, gh.KVCache(model, N_PROMPT + a.warmup + 8), prompt, a.warmup - 1, 1)
    kv = gh.KVCache(model, s0 + a.steps + 8)
    ms, ids = gh.bench_decode(model, kv, prompt, s0 - N_PROMPT, a.steps)
    tok_s = a.steps / (ms / 1e3)
    log(f"decode: {a.steps} steps at positions {s0}..{s0 + a.steps - 1} in {ms:.3f} ms -> {tok_s:.1f} tok/s")

    # kernel execution times inside real decode steps at C3's positions
    # 128..383: a second cache fed the prompt, then PROFILE_STEPS eager greedy
    # steps, each kernel timed by its own dispatch timestamps
    kv_p = gh.KVCache(model, N_PROMPT + PROFILE_STEPS + 8)
    gh.generate(model, kv_p, prompt, 1)
    pos0 = len(kv_p)
    timings = in_step_kernels(gh, model, kv_p, PROFILE_STEPS)
    del kv_p
    for t in timings.values():
        log(f"  {t.name:10s} x{t.launches // PROFILE_STEPS:3d}/step avg {t.avg_us:8.2f} us  {t.gbps:8.1f} GB/s")
    step_bytes = sum(t.bytes_per_launch * t.launches for t in timings.values()) / PROFILE_STEPS
    kernel_us = sum(t.total_ms for t in timings.values()) * 1e3 / PROFILE_STEPS
    # roofline kernel: gate/up (26 launches per token, the largest share of
    # the step); algorithmic bytes per launch = the fused [gate | up] Q4_0
    # weights (2 x 6912 x 1152 / 32 x 18 B) + the input and the output rows
    gu, lm = timings["gate_up"], timings["lm_head"]
    roofline = {"bound": "hbm", "achieved": round(gu.gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                "frac": round(gu.gbps / HBM_PEAK_GBPS, 4), "traffic": GATE_UP_TRAFFIC_BYTES,
                "traffic_source": f"rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE (copy-calibrated) at position 257: "
                                  f"{TRAFFIC_PROFILE}",
                "kernel": "gate_up", "bytes_per_launch": int(gu.bytes_per_launch), "avg_us": round(gu.avg_us, 3),
                "timing": f"dispatch begin/end timestamps of every gate/up launch in {PROFILE_STEPS} real decode "
                          f"steps at positions {pos0}..{pos0 + PROFILE_STEPS - 1} ({gu.launches} launches)",
                "lm_head": {"achieved": round(lm.gbps, 1), "frac": round(lm.gbps / HBM_PEAK_GBPS, 4),
                            "traffic": LM_HEAD_TRAFFIC_BYTES, "bytes_per_launch": int(lm.bytes_per_launch),
                            "avg_us": round(lm.avg_us, 3)}}
    # the box's practical ceiling: 1 GiB read once per launch (non-temporal 16 B loads)
    sr_gbps, sr_us = gh.stream_read_gbps(ctx, 1 << 30, 20)
    log(f"  stream read 1 GiB: {sr_us:.1f} us -> {sr_gbps:.1f} GB/s")
    roofline["measured_stream_read"] = {"gbps": round(sr_gbps, 1), "bytes": 1 << 30, "avg_us": round(sr_us, 2),
                                        "gate_up_frac": round(gu.gbps / sr_gbps, 4),
                                        "lm_head_frac": round(lm.gbps / sr_gbps, 4)}

    out = {
        "metric": METRIC, "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": round(ms / a.steps, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "gemma3-1b Q4_0 greedy decode, batch 1", "weights": "seeded synthetic Q4_0",
                   "prompt_tokens": N_PROMPT, "timed_positions": [s0, s0 + a.steps - 1],
                   "warmup_note": "W greedy steps on a scratch cache of the same model, before the timed cache",
                   "global_batch": 1, "parallelism": "single-gpu",
                   "step_algorithmic_bytes": int(step_bytes),
                   "step_frac_of_hbm_peak": round(step_bytes / (ms / a.steps * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)},
        "plan": model.plan(),
        "roofline": roofline,
        "kernels": {t.name: {"avg_us": round(t.avg_us, 3), "gbps": round(t.gbps, 1),
                             "frac": round(t.gbps / HBM_PEAK_GBPS, 4), "per_step": t.launches // PROFILE_STEPS,
                             "step_us": round(t.total_ms * 1e3 / PROFILE_STEPS, 1)}
                    for t in timings.values()},
        "kernels_note": f"dispatch begin-to-end intervals inside eager decode steps at positions {pos0}.."
                        f"{pos0 + PROFILE_STEPS - 1}; each includes that kernel's launch by the command processor, "
                        f"so their sum, {kernel_us:.1f} us per step, compares with the {1e3 * ms / a.steps:.1f} us "
                        f"of a timed graph step",
    }
    if not a.no_extras:
        out["extras"] = {"c2_matvec_rotating_2GiB": extras_c2_matvec(gh, ctx),
                         "c4_attention": extras_c4_attention(gh, ctx),
                         "c5_gemma3_4b_prefilled_4096": extras_c5_gemma3_4b(gh, ctx),
                         "f2_prefill_gemma3_1b": extras_f2_prefill(gh, ctx, model)}
    if not a.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(cfg, a.cpu_seconds)
    else:
        out["cpu_baseline"] = None
    print(json.dumps(out), flush=True)
    del np
    return 0


if __name__ == "__main__":
    sys.exit(main())
