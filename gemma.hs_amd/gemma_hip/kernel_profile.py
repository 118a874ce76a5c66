"""Hardware-counter driver and summariser for the step kernels.

Driver (run under rocprofv3 on the GPU box, eagerly: GH_NO_GRAPH=1):

  python -m gemma_hip.kernel_profile run [--kernel all|KIND] [--config gemma3-1b] [--reps 20]
                                         [--prompt 8] [--prefill-prompt] [--kv-synth N] [--copy-mib 256]
                                         [--manifest FILE]
  python -m gemma_hip.kernel_profile run --prefill 128 [--reps 5] [--copy-mib 256]
  python -m gemma_hip.kernel_profile run --attention 32768 [--reps 20] [--copy-mib 256] [--copies 8]
  python -m gemma_hip.kernel_profile run --decode 64 [--prompt 128] [--start 224] [--copy-mib 256]
  python -m gemma_hip.kernel_profile exchange [--wgs 8 64 128 256] [--rounds 2000]
  python -m gemma_hip.kernel_profile phases [--config gemma3-1b] [--prompt 128] [--reps 20] [--kernel KIND]

It builds the seeded model of the config and decodes a short prompt.  Then,
for each step-kernel kind asked for, it launches a separator (two launches
of the stream-read kernel over 4 KiB, a kernel that appears nowhere else)
and replays that kind `reps` times at the cache's position (gh_time_kernel,
the launches bench.py times).  Last comes one more separator and a
device-to-device copy of `copy-mib` MiB: the calibration kernel for the
byte counters, which reads and writes exactly that many bytes.  With
--prefill N it instead runs `reps` prefills of a seeded N-token prompt;
with --attention L, `reps` op-level attention decodes (4 q heads, 1 kv head,
head_dim 256, global over L positions: the C4 case), rotating over `copies`
K/V caches so that replays do not hit the 256 MB Infinity Cache.  With
--decode N the kernels are measured where they run: a seeded `prompt`-token
prompt and greedy steps up to position `start` (graph replays), then N
greedy decode steps launched eagerly in the step's order (gh_profile_steps,
the measurement bench.py's roofline comes from); the summariser assigns
each dispatch its kernel kind by its place in the step's launch sequence,
which the manifest records.  The manifest (JSON) lists the segments in
order.  `exchange` needs no profiler: it prints the
cost of one all-to-all word exchange among n co-resident workgroups
(gh_time_exchange, the persistent step's synchronisation).  `phases` needs
no profiler either: it loads libgemma_hip_marks.so (the step kernels built
with phase timestamps, build.py) and prints, per step-kernel kind, when
each workgroup reaches each phase of its latency chain (medians over the
workgroups of the last replayed launch, us since the workgroup started).

Summariser (on any host, from rocprofv3's CSV output):

  python -m gemma_hip.kernel_profile summarize --manifest FILE [--fetch DIR] [--write DIR] [--sq DIR]
                                               [--trace DIR]

It splits each run's dispatches at the separators, averages every counter
over each segment's dispatches, scales FETCH_SIZE / WRITE_SIZE (KiB per
dispatch) by the bytes / counter reading of the calibration copy, and
prints a Markdown table per segment: HBM traffic against the algorithmic
bytes, and the SQ counters (waves, wave cycles, busy cycles, wait cycles,
VMEM / VALU / LDS instructions per wave).
"""
from __future__ import annotations

import argparse
import csv
import ctypes as C
import json
import sys
from collections import defaultdict
from pathlib import Path

from . import (GemmaModel, KVCache, Context, DeviceBuffer, STEP_KERNELS, bench_decode, prefill, preset,
               profile_steps, stream_read_gbps, synth_tokens, time_kernel)
from ._lib import check, lib

HIP_MEMCPY_D2D = 3
SEPARATOR = "k_stream_read"  # preceded by a fill of its buffer (__amd_rocclr_fillBufferAligned), skipped too
CALIBRATION = "__amd_rocclr_copyBuffer"


def _hip():
    # the HIP runtime the library is linked against (already loaded)
    return C.CDLL("libamdhip64.so")


def device_copy(n_bytes: int) -> None:
    """One device-to-device copy of n_bytes (plus a fill of the source)."""
    hip = _hip()
    src, dst = C.c_void_p(), C.c_void_p()
    for p in (src, dst):
        rc = hip.hipMalloc(C.byref(p), C.c_size_t(n_bytes))
        if rc != 0:
            raise RuntimeError(f"hipMalloc({n_bytes}) failed: {rc}")
    try:
        if hip.hipMemset(src, 1, C.c_size_t(n_bytes)) != 0:
            raise RuntimeError("hipMemset failed")
        if hip.hipDeviceSynchronize() != 0:
            raise RuntimeError("hipDeviceSynchronize failed")
        if hip.hipMemcpy(dst, src, C.c_size_t(n_bytes), HIP_MEMCPY_D2D) != 0:
            raise RuntimeError("hipMemcpy D2D failed")
        if hip.hipDeviceSynchronize() != 0:
            raise RuntimeError("hipDeviceSynchronize failed")
    finally:
        hip.hipFree(src)
        hip.hipFree(dst)


def run(a) -> int:
    cfg = preset(a.config)
    ctx = Context(0)
    segments = []
    replay_pos = None

    def separator():
        stream_read_gbps(ctx, 4096, 1)

    if a.attention > 0:
        import numpy as np
        L, hd, nq, nkv = a.attention, 256, 4, 1
        rng = np.random.default_rng(4)
        # inputs uploaded once, the K/V cache in `copies` copies; each rep is
        # one gh_attention_decode on device pointers (the attention kernel
        # and its merge, nothing else) over the next copy
        q = DeviceBuffer.from_numpy(ctx, rng.normal(size=nq * hd).astype(np.float32))
        kvs = [(DeviceBuffer.from_numpy(ctx, rng.normal(size=L * nkv * hd).astype(np.float32)),
                DeviceBuffer.from_numpy(ctx, rng.normal(size=L * nkv * hd).astype(np.float32)))
               for _ in range(max(1, a.copies))]
        o = DeviceBuffer(ctx, 4 * nq * hd)
        k, v = kvs[0]
        check(lib().gh_attention_decode(ctx.h, q.ptr, k.ptr, v.ptr, nq, nkv, hd, 0, L, 0, o.ptr))  # scratch
        separator()
        for i in range(a.reps):
            k, v = kvs[i % len(kvs)]
            check(lib().gh_attention_decode(ctx.h, q.ptr, k.ptr, v.ptr, nq, nkv, hd, 0, L, 0, o.ptr))
        # one unit = the attention kernel + its merge (two dispatches)
        segments.append({"name": f"attention_c4_L{L}", "reps": a.reps, "dispatches_per_unit": 2,
                         "bytes_per_launch": 2 * L * nkv * hd * 4 + 8 * nq * hd})
    else:
        model = GemmaModel(ctx, cfg)
        model.synth(1234, q4=True)
        if a.prefill > 0:
            toks = synth_tokens(1, "prefill", a.prefill, cfg.vocab)
            kv = KVCache(model, a.prefill + 8)
            separator()
            for _ in range(a.reps):
                kv.reset()
                prefill(model, kv, toks, want_logits=False)
            segments.append({"name": f"prefill_{a.prefill}", "reps": a.reps, "by_kernel": True})
        elif a.decode > 0:
            start = max(a.start, a.prompt)
            kv = KVCache(model, start + a.decode + 8)
            bench_decode(model, kv, synth_tokens(1, "prompt", a.prompt, cfg.vocab), start - a.prompt, 1)
            pos0 = len(kv)
            separator()
            stats = profile_steps(model, kv, a.decode)
            seq = [k for _ in range(cfg.n_layers) for k in ("qkv", "attention", "o_proj", "gate_up", "down")]
            seq += ["final_norm", "lm_head", "finish"]
            launches = {st.name: st.launches for st in stats}
            assert sum(launches.values()) == len(seq) * a.decode, (launches, len(seq))
            segments.append({"name": "decode", "steps": a.decode, "positions": [pos0, pos0 + a.decode - 1],
                             "sequence": seq,
                             "kinds": {st.name: {"bytes_per_launch": int(st.bytes_per_launch),
                                                 "event_avg_us": round(st.avg_us, 3)} for st in stats}})
        else:
            kv = KVCache(model, a.kv_synth + a.prompt + 8)
            if a.kv_synth > 0:  # the C5 start: a prefilled cache of that many positions
                kv.synth(5, a.kv_synth)
            toks = synth_tokens(1, "prompt", a.prompt, cfg.vocab)
            if a.prefill_prompt:  # one batched pass (a few hundred dispatches), then one step
                prefill(model, kv, toks[:-1], want_logits=False)
                bench_decode(model, kv, toks[-1:], 0, 1)
            else:
                bench_decode(model, kv, toks, 0, 1)
            replay_pos = len(kv)
            kinds = STEP_KERNELS if a.kernel == "all" else (a.kernel,)
            for kind in kinds:
                separator()
                t = time_kernel(model, kv, kind, a.reps)
                segments.append({"name": kind, "reps": a.reps, "launches_per_step": t.launches_per_step,
                                 "bytes_per_launch": int(t.bytes_per_launch), "event_avg_us": round(t.avg_us, 3)})
    separator()
    device_copy(a.copy_mib << 20)
    man = {"config": a.config,
           "position": replay_pos if a.prefill == 0 and a.attention == 0 and a.decode == 0 else None,
           "copy_bytes": a.copy_mib << 20, "segments": segments}
    if a.manifest:
        Path(a.manifest).write_text(json.dumps(man, indent=1))
    print(json.dumps(man), flush=True)
    return 0


def _dispatches(d: Path):
    """{dispatch id: (kernel name, {counter: value}, duration ns)} of a rocprofv3 CSV directory."""
    files = list(d.glob("**/*counter_collection.csv"))
    out = {}
    if files:
        for row in csv.DictReader(open(files[0])):
            i = int(row["Dispatch_Id"])
            name, ctrs, dur = out.get(i, (row["Kernel_Name"], {}, 0))
            ctrs[row["Counter_Name"]] = ctrs.get(row["Counter_Name"], 0.0) + float(row["Counter_Value"])
            dur = int(row["End_Timestamp"]) - int(row["Start_Timestamp"])
            out[i] = (name, ctrs, dur)
        return out
    files = list(d.glob("**/*kernel_trace.csv"))
    for row in csv.DictReader(open(files[0])):
        i = int(row["Dispatch_Id"])
        out[i] = (row["Kernel_Name"], {}, int(row["End_Timestamp"]) - int(row["Start_Timestamp"]))
    return out


def _segments(disp, n_seg):
    """Split dispatches at separator launches: [(kernel dispatches of segment k)], calibration copies."""
    order = sorted(disp)
    groups, cur, seen_sep = [], None, False
    for i in order:
        name = disp[i][0]
        if "__amd_rocclr_fill" in name:  # the separator's buffer fill
            continue
        if name.startswith(SEPARATOR) or SEPARATOR in name:
            if not seen_sep or cur:
                cur = []
                groups.append(cur)
            seen_sep = True
            continue
        if cur is not None:
            cur.append(i)
    segs = groups[:n_seg]
    tail = groups[n_seg] if len(groups) > n_seg else []
    cal = [i for i in tail if CALIBRATION in disp[i][0]]
    return segs, cal


def _units(man, segs, disp):
    """(row name, dispatch ids, algorithmic bytes per unit, dispatches per
    unit, event avg us) of every summarised row: one per segment, or one per
    kernel kind of a decode segment, whose dispatches take their kind from
    their place in the recorded step sequence (the runtime's copy kernels of
    the step state, __amd_rocclr_*, left out)."""
    out = []
    for k, s in enumerate(man["segments"]):
        seg = segs[k] if k < len(segs) else []
        if "sequence" in s:
            seg = [i for i in seg if not disp[i][0].startswith("__amd_rocclr")]
            seq = s["sequence"]
            if len(seg) != len(seq) * s["steps"]:
                raise SystemExit(f"decode segment: {len(seg)} dispatches, expected {len(seq)} x {s['steps']}")
            for kind in dict.fromkeys(seq):
                ids = [seg[i] for i in range(len(seg)) if seq[i % len(seq)] == kind]
                info = s["kinds"].get(kind, {})
                out.append((kind, ids, info.get("bytes_per_launch"), 1, info.get("event_avg_us")))
        elif s.get("by_kernel"):  # one row per kernel of the segment
            names = {}
            for i in seg:
                names.setdefault(disp[i][0].split("(")[0].replace("void gh::", ""), []).append(i)
            for kname, ids in names.items():
                out.append((f"{s['name']}: {kname}", ids, None, 1, None))
        else:
            out.append((s["name"], seg, s.get("bytes_per_launch"), s.get("dispatches_per_unit", 1),
                        s.get("event_avg_us")))
    return out


def summarize(a) -> int:
    man = json.loads(Path(a.manifest).read_text())
    n = len(man["segments"])
    rows = defaultdict(dict)
    factors = {}
    names = []
    passes = [("fetch", a.fetch), ("write", a.write)] + [("sq", d) for d in (a.sq or [])] + [("trace", a.trace)]
    for label, d in passes:
        if not d:
            continue
        disp = _dispatches(Path(d))
        segs, cal = _segments(disp, n)
        units = _units(man, segs, disp)
        names = [(u[0], u[2], u[3], u[4]) for u in units]
        for name, seg, _, _, _ in units:
            if not seg:
                continue
            r = rows[name]
            ctr_sum = defaultdict(float)
            for i in seg:
                for c, v in disp[i][1].items():
                    ctr_sum[c] += v
            r.setdefault("dispatches", len(seg))
            r.setdefault("kernels", sorted({disp[i][0].split("(")[0] for i in seg}))
            for c, v in ctr_sum.items():
                r[c] = v / len(seg)
                r["sum:" + c] = v
            if label == "trace":
                r["trace_avg_us"] = sum(disp[i][2] for i in seg) / len(seg) / 1e3
        for c in ("FETCH_SIZE", "WRITE_SIZE"):
            vals = [disp[i][1][c] for i in cal if c in disp[i][1]]
            if vals:
                factors[c] = man["copy_bytes"] / max(vals)
    print(f"Calibration: {man['copy_bytes']} B device copy; bytes per counter unit: "
          + ", ".join(f"{c} {f:.5f}" for c, f in factors.items()))
    print()
    print("| segment | dispatches | algorithmic B / launch | FETCH B / launch | WRITE B / launch | traffic / algorithmic |")
    print("|---|---|---|---|---|---|")
    for name, algo, per, _ in names:
        r = rows.get(name, {})
        fb = r["FETCH_SIZE"] * factors["FETCH_SIZE"] * per if "FETCH_SIZE" in r and "FETCH_SIZE" in factors else None
        wb = r["WRITE_SIZE"] * factors["WRITE_SIZE"] * per if "WRITE_SIZE" in r and "WRITE_SIZE" in factors else None
        ratio = (fb + wb) / algo if fb is not None and wb is not None and algo else None
        f = lambda x: f"{x:,.0f}" if x is not None else "-"
        print(f"| {name} | {r.get('dispatches', '-')} | {f(algo)} | {f(fb)} | {f(wb)} | "
              + (f"{ratio:.3f} |" if ratio is not None else "- |"))
    sq = [c for c in ("SQ_WAVES", "SQ_WAVE_CYCLES", "SQ_BUSY_CYCLES", "SQ_WAIT_INST_ANY", "SQ_INSTS_VMEM_RD",
                      "SQ_INSTS_VALU", "SQ_INSTS_LDS", "SQ_ACTIVE_INST_VALU", "SQ_INSTS_MFMA",
                      "SQ_VALU_MFMA_BUSY_CYCLES", "SQ_LDS_BANK_CONFLICT", "SQ_WAIT_ANY", "SQ_ACTIVE_INST_LDS")
          if any(c in r for r in rows.values())]
    if sq:
        print()
        print("| segment | " + " | ".join(sq) + " | wait / wave cycles | VALU / wave | VMEM rd / wave |")
        print("|---|" + "---|" * (len(sq) + 3))
        for name, _, _, _ in names:
            r = rows.get(name, {})
            waves = r.get("SQ_WAVES") or 1.0
            cells = [f"{r.get(c, 0):,.0f}" for c in sq]
            wait = r.get("SQ_WAIT_INST_ANY", 0) / max(r.get("SQ_WAVE_CYCLES", 0), 1)
            print(f"| {name} | " + " | ".join(cells) +
                  f" | {wait:.3f} | {r.get('SQ_INSTS_VALU', 0) / waves:.1f} | {r.get('SQ_INSTS_VMEM_RD', 0) / waves:.1f} |")
        mf = [(name, rows.get(name, {})) for name, _, _, _ in names if rows.get(name, {}).get("SQ_INSTS_MFMA")]
        if mf:
            print()
            print("| segment | MFMA instructions (sum) | VALU / MFMA | LDS / MFMA | LDS bank-conflict cycles / LDS "
                  "instruction |")
            print("|---|---|---|---|---|")
            for name, r in mf:
                m = r["sum:SQ_INSTS_MFMA"]
                bc = (f"{r['sum:SQ_LDS_BANK_CONFLICT'] / max(r.get('sum:SQ_INSTS_LDS', 0), 1):.3f}"
                      if "sum:SQ_LDS_BANK_CONFLICT" in r else "-")
                print(f"| {name} | {m:,.0f} | {r.get('sum:SQ_INSTS_VALU', 0) / m:.2f} | "
                      f"{r.get('sum:SQ_INSTS_LDS', 0) / m:.2f} | {bc} |")
    if any("trace_avg_us" in r for r in rows.values()):
        print()
        print("| segment | kernels | traced avg us / unit | algorithmic GB/s | of 8 TB/s | dispatch-event avg us "
              "(same run) |")
        print("|---|---|---|---|---|---|")
        for name, algo, per, ev in names:
            r = rows.get(name, {})
            if "trace_avg_us" not in r:
                continue
            us = r["trace_avg_us"] * per
            gbps = algo / (us * 1e3) if algo else None
            print(f"| {name} | {', '.join(r['kernels'])} | {us:.3f} | "
                  + (f"{gbps:.0f} | {gbps / 8000:.3f} |" if gbps else "- | - |")
                  + (f" {ev:.3f} |" if ev is not None else " - |"))
    return 0


# Phase points of the step kernels (GH_MARK slots in kernels.hip): the
# matvec work items (mv_item_valu, mv_item_multi_v, mq_item_v with the
# residual-norm prologue's own points) and the step attention.
MATVEC_SLOTS = {6: "norm reduced", 7: "residual out", 1: "prologue done", 2: "slice in LDS", 3: "dots done",
                4: "rows reduced", 5: "epilogue done"}
ATTN_SLOTS = {1: "loads issued", 2: "q/k/v in LDS", 4: "rounds done", 5: "wave states merged",
              6: "state written"}
MARKS_TUS = (1, 5, 6, 7)
MARK_WAVES, MARK_SLOTS, MARK_MAXWG = 8, 16, 8192
TICK_US = 0.01  # s_memrealtime runs at 100 MHz


def phases(a) -> int:
    import os
    import numpy as np
    marks = Path(__file__).resolve().parent / "libgemma_hip_marks.so"
    if not marks.exists():
        raise SystemExit(f"{marks} is not built (python gemma.hs_amd/build.py)")
    os.environ["GEMMA_HIP_LIB"] = str(marks)
    L = lib()
    fetch = {tu: getattr(L, f"gh_marks_fetch_tu{tu}") for tu in MARKS_TUS}
    clear = {tu: getattr(L, f"gh_marks_clear_tu{tu}") for tu in MARKS_TUS}
    for f in fetch.values():
        f.argtypes, f.restype = [C.c_void_p, C.c_size_t], C.c_int
    for f in clear.values():
        f.argtypes, f.restype = [], C.c_int
    cfg = preset(a.config)
    ctx = Context(0)
    model = GemmaModel(ctx, cfg)
    model.synth(1234, q4=True)
    kv = KVCache(model, a.prompt + 8)
    bench_decode(model, kv, synth_tokens(1, "prompt", a.prompt, cfg.vocab), 0, 1)
    print(f"{a.config}, position {len(kv)}; medians over the workgroups of the last replayed launch, "
          f"us since each workgroup's start (wave 0)")
    print()
    buf = np.zeros((MARK_MAXWG, MARK_WAVES, MARK_SLOTS), np.uint64)
    kinds = [k for k in STEP_KERNELS if k not in ("final_norm", "lm_head")] if a.kernel == "all" else [a.kernel]
    for kind in kinds:
        for f in clear.values():
            if f() != 0:
                raise RuntimeError("gh_marks_clear failed")
        t = time_kernel(model, kv, kind, a.reps)
        got = []
        for tu, f in fetch.items():
            buf[:] = 0
            if f(buf.ctypes.data, buf.nbytes) != 0:
                raise RuntimeError("gh_marks_fetch failed")
            used = np.nonzero(buf[:, 0, 0])[0]
            if len(used):
                got.append(buf[used].astype(np.int64))
        if not got:
            print(f"| {kind} | no marks |")
            continue
        b = max(got, key=len)  # the kind's kernels live in one unit
        t0 = b[:, 0, 0].min()
        labels = ATTN_SLOTS if kind == "attention" else MATVEC_SLOTS
        cols = [(sl, lab) for sl, lab in labels.items() if (b[:, 0, sl] > 0).any()]
        print(f"**{kind}** ({t.avg_us:.2f} us per replayed launch, {len(b)} workgroups; start of the last "
              f"workgroup {np.max(b[:, 0, 0] - t0) * TICK_US:.2f} us after the first)")
        print()
        print("| " + " | ".join(lab for _, lab in cols) + " | workgroup done |")
        print("|" + "---|" * (len(cols) + 1))
        cells = []
        for sl, _ in cols:
            v = b[:, 0, sl]
            ok = v > 0
            cells.append(f"{np.median((v[ok] - b[ok, 0, 0]) * TICK_US):.2f}")
        done = b.max(axis=(1, 2))
        cells.append(f"{np.median((done - b[:, 0, 0]) * TICK_US):.2f}")
        print("| " + " | ".join(cells) + " |")
        print()
        # the launch's span: when the workgroups finish, counted from the
        # first workgroup's start (the kernel's tail beyond the median chain)
        fin = (done - t0) * TICK_US
        last = int(np.argmax(done))
        print(f"Workgroups done, us after the first one started: p50 {np.median(fin):.2f}, "
              f"p90 {np.percentile(fin, 90):.2f}, last {fin.max():.2f} (that workgroup started "
              f"{(b[last, 0, 0] - t0) * TICK_US:.2f} us in and ran {(done[last] - b[last, 0, 0]) * TICK_US:.2f} us)")
        print()
    return 0


def exchange(a) -> int:
    """Cost of one all-to-all word exchange among n co-resident workgroups
    (gh_time_exchange), for each n of --wgs: a markdown table."""
    from . import time_exchange
    ctx = Context(0)
    time_exchange(ctx, 8, 100)  # warm-up (code object load)
    print("| workgroups | rounds | us per exchange (median of 5 runs) |")
    print("|---|---|---|")
    for n in a.wgs:
        us = sorted(time_exchange(ctx, n, a.rounds) for _ in range(5))
        print(f"| {n} | {a.rounds} | {us[2]:.3f} |")
    return 0


def main(argv=None) -> int:
    argv = list(sys.argv[1:] if argv is None else argv)
    if not argv or argv[0] not in ("run", "summarize", "exchange", "phases"):
        argv = ["run", *argv]
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd")
    r = sub.add_parser("run")
    r.add_argument("--kernel", default="all", choices=("all",) + STEP_KERNELS)
    r.add_argument("--config", default="gemma3-1b")
    r.add_argument("--reps", type=int, default=20)
    r.add_argument("--copy-mib", type=int, default=256)
    r.add_argument("--prompt", type=int, default=8)
    r.add_argument("--kv-synth", type=int, default=0, help="fill the cache with this many positions first")
    r.add_argument("--prefill", type=int, default=0, help="time N-token prefills instead of step kernels")
    r.add_argument("--attention", type=int, default=0, help="op-level C4 attention over L positions")
    r.add_argument("--copies", type=int, default=1, help="K/V cache copies the attention reps rotate over")
    r.add_argument("--decode", type=int, default=0, help="profile N eager decode steps in the step's order")
    r.add_argument("--prefill-prompt", action="store_true",
                   help="feed all but the last prompt token by batched prefill (kernel replays at a late position "
                        "with few dispatches before them)")
    r.add_argument("--start", type=int, default=0, help="--decode: first profiled position (after the prompt)")
    r.add_argument("--manifest", default="")
    ph = sub.add_parser("phases")
    ph.add_argument("--config", default="gemma3-1b")
    ph.add_argument("--prompt", type=int, default=128)
    ph.add_argument("--reps", type=int, default=20)
    ph.add_argument("--kernel", default="all", choices=("all",) + STEP_KERNELS)
    x = sub.add_parser("exchange")
    x.add_argument("--wgs", type=int, nargs="+", default=[8, 64, 128, 256])
    x.add_argument("--rounds", type=int, default=2000)
    s = sub.add_parser("summarize")
    s.add_argument("--manifest", required=True)
    for k in ("fetch", "write", "trace"):
        s.add_argument(f"--{k}", default="")
    s.add_argument("--sq", action="append", help="an SQ counter pass (may be given more than once)")
    a = ap.parse_args(argv)
    if a.cmd == "exchange":
        return exchange(a)
    if a.cmd == "phases":
        return phases(a)
    return run(a) if a.cmd == "run" else summarize(a)


if __name__ == "__main__":
    sys.exit(main())
