"""Single-kernel driver for hardware-counter runs.

  python -m gemma_hip.kernel_profile [--kernel lm_head] [--reps 20] [--copy-mib 256]
  python -m gemma_hip.kernel_profile --prefill 128 [--reps 5] [--copy-mib 256]

It builds the seeded gemma3-1b Q4_0 model and decodes a short prompt. Then it
replays one step-kernel kind `reps` times at the cache's position
(gh_time_kernel, the same launches bench.py times). With --prefill N it
instead runs `reps` prefills of a seeded N-token prompt (gh_prefill, as
bench.py's prefill extras do). Last, it copies a device buffer of
`copy-mib` MiB once with hipMemcpy device-to-device.

That copy is the calibration kernel for byte counters: it reads and writes
exactly copy-mib MiB, so FETCH_SIZE / WRITE_SIZE of the kernel under study
scale by what the counters read for it.

The run is kept short and free of graph launches, so counter collection
sees only plain kernel dispatches.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import sys

from . import GemmaModel, KVCache, Context, STEP_KERNELS, bench_decode, prefill, preset, synth_tokens, time_kernel

HIP_MEMCPY_D2D = 3


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


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--kernel", default="lm_head", choices=STEP_KERNELS)
    ap.add_argument("--reps", type=int, default=20)
    ap.add_argument("--copy-mib", type=int, default=256)
    ap.add_argument("--prompt", type=int, default=8)
    ap.add_argument("--prefill", type=int, default=0, help="time N-token prefills instead of a step kernel")
    a = ap.parse_args(argv)
    cfg = preset("gemma3-1b")
    ctx = Context(0)
    model = GemmaModel(ctx, cfg)
    model.synth(1234, q4=True)
    if a.prefill > 0:
        toks = synth_tokens(1, "prefill", a.prefill, cfg.vocab)
        kv = KVCache(model, a.prefill + 8)
        ms = []
        for _ in range(a.reps):
            kv.reset()
            ctx.timer_start()
            prefill(model, kv, toks, want_logits=False)
            ms.append(ctx.timer_stop())
        device_copy(a.copy_mib << 20)
        print(json.dumps({"prefill_tokens": a.prefill, "reps": a.reps, "ms": [round(x, 4) for x in ms],
                          "copy_bytes": a.copy_mib << 20}), flush=True)
        return 0
    kv = KVCache(model, a.prompt + 8)
    bench_decode(model, kv, synth_tokens(1, "prompt", a.prompt, cfg.vocab), 0, 1)
    t = time_kernel(model, kv, a.kernel, a.reps)
    device_copy(a.copy_mib << 20)
    print(json.dumps({"kernel": t.name, "reps": a.reps, "avg_us": round(t.avg_us, 3),
                      "bytes_per_launch": int(t.bytes_per_launch), "gbps": round(t.gbps, 1),
                      "copy_bytes": a.copy_mib << 20}), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
