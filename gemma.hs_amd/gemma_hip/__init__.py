"""Python host binding of libgemma_hip (MI355X decode step of gemma.hs).

The names mirror the reference's Haskell API so that code and tests read
alike:

  Gemma.Model.GemmaConfig / gemma3_1BConfig   -> GemmaConfig, preset()
  Gemma.Model.loadGemmaModelFromGGUF          -> GemmaModel.load_gguf
  Gemma.Model.runGemmaInferenceCached         -> runGemmaInferenceCached
  Gemma.Model.runGemmaInferenceCachedWithLayer0 -> runGemmaInferenceCachedWithLayer0
  Gemma.KVCache (initKVCache, cacheLength)    -> KVCache
  Gemma.Layers.LinearQ4.runLinearQ4           -> runLinearQ4
  app/Main.hs sampleToken                     -> on-device argmax inside the step

Everything runs through the C ABI of include/gemma_hip.h; there is no CPU
fallback: without libgemma_hip.so (or without a GPU) the calls raise.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from ._lib import (DTYPE_F16, DTYPE_F32, DTYPE_Q4_0, FLAG_IEEE_SCALES, FLAG_POST_ATTN_NORM,
                   FLAG_POST_FFN_NORM, FLAG_QK_NORM, FLAG_ZERO_CENTERED, MODE_GEMMA3, MODE_REF,
                   GemmaHipError, GhConfig, GhKernelStat, check, lib)

GemmaConfig = GhConfig

__all__ = [
    "GemmaConfig", "GemmaHipError", "Context", "DeviceBuffer", "Q4Tensor", "GemmaModel", "KVCache",
    "preset", "runLinearQ4", "runGemmaInferenceCached", "runGemmaInferenceCachedWithLayer0",
    "generate", "prefill", "bench_decode", "profile_steps", "profile_prefill", "sample_logits", "time_kernel", "KernelTiming", "STEP_KERNELS", "synth_f32", "synth_q4_0", "synth_tokens",
    "tensor_list", "synth_tensors", "synth_kv", "center_q4_0", "device_count", "DTYPE_F32", "DTYPE_F16", "DTYPE_Q4_0",
    "MODE_GEMMA3", "MODE_REF", "FLAG_QK_NORM", "FLAG_POST_ATTN_NORM", "FLAG_POST_FFN_NORM",
    "FLAG_ZERO_CENTERED", "FLAG_IEEE_SCALES",
]


def _ptr(a: np.ndarray) -> C.c_void_p:
    return C.c_void_p(a.ctypes.data)


def device_count() -> int:
    n = C.c_int32()
    check(lib().gh_device_count(C.byref(n)))
    return n.value


def preset(name: str) -> GemmaConfig:
    """Config presets: 'tiny', 'gemma3-1b' (src/Gemma/Model.hs:213-237), 'gemma3-4b'."""
    c = GemmaConfig()
    check(lib().gh_config_preset(name.encode(), C.byref(c)))
    return c


# ---------------------------------------------------------------- context
class Context:
    """createContext / waitAll of the Dawn layer (src/Gemma/Model.hs:419)."""

    def __init__(self, device: int = 0):
        h = C.c_void_p()
        check(lib().gh_ctx_create(device, C.byref(h)))
        self.h = h

    def sync(self) -> None:
        check(lib().gh_ctx_sync(self.h))

    def timer_start(self) -> None:
        """Record the start event of gh_timer_start on the context stream."""
        check(lib().gh_timer_start(self.h))

    def timer_stop(self) -> float:
        """ms since timer_start, measured with HIP events on the stream."""
        ms = C.c_float()
        check(lib().gh_timer_stop(self.h, C.byref(ms)))
        return ms.value

    def capture_begin(self) -> None:
        """Start capturing the context stream: launch-only op calls enqueue
        into a graph instead of running (gh_capture_begin)."""
        check(lib().gh_capture_begin(self.h))

    def capture_replay(self, n_replays: int) -> float:
        """End the capture, replay the graph n_replays times between two
        HIP events; returns ms per replay (gh_capture_replay)."""
        ms = C.c_float()
        check(lib().gh_capture_replay(self.h, n_replays, C.byref(ms)))
        return ms.value

    def close(self) -> None:
        """Destroy the context handle.  Models, caches and Q4_0 tensors made
        on it stay usable; the library frees the context when the last of
        them is closed (handles close in any order)."""
        if self.h:
            lib().gh_ctx_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class DeviceBuffer:
    """createTensorWithData / fromGPU equivalents (device memory owned by the library)."""

    def __init__(self, ctx: Context, nbytes: int):
        self.ctx = ctx
        self.nbytes = int(nbytes)
        h = C.c_void_p()
        check(lib().gh_buf_alloc(ctx.h, self.nbytes, C.byref(h)))
        self.ptr = h

    @classmethod
    def from_numpy(cls, ctx: Context, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(ctx, a.nbytes)
        b.upload(a)
        return b

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        check(lib().gh_buf_upload(self.ctx.h, self.ptr, _ptr(a), a.nbytes))

    def numpy(self, dtype=np.float32, count: int | None = None) -> np.ndarray:
        dt = np.dtype(dtype)
        n = self.nbytes // dt.itemsize if count is None else count
        out = np.empty(n, dtype=dt)
        check(lib().gh_buf_download(self.ctx.h, _ptr(out), self.ptr, out.nbytes))
        return out

    def free(self) -> None:
        if self.ptr:
            lib().gh_buf_free(self.ctx.h, self.ptr)
            self.ptr = None


# ---------------------------------------------------------------- Q4_0
class Q4Tensor:
    """A GGUF Q4_0 matrix resident on the device (repacked on upload)."""

    def __init__(self, ctx: Context, raw: np.ndarray, rows: int, cols: int, ieee_scales: bool = False):
        raw = np.ascontiguousarray(raw).view(np.uint8)
        if raw.nbytes < rows * (cols // 32) * 18:
            raise ValueError("raw Q4_0 buffer too small")
        h = C.c_void_p()
        check(lib().gh_q4_0_upload(ctx.h, _ptr(raw), rows, cols, FLAG_IEEE_SCALES if ieee_scales else 0,
                                   C.byref(h)))
        self.ctx, self.h, self.rows, self.cols = ctx, h, rows, cols

    def dequant(self) -> np.ndarray:
        out = DeviceBuffer(self.ctx, 4 * self.rows * self.cols)
        try:
            check(lib().gh_q4_0_dequant(self.h, out.ptr))
            return out.numpy().reshape(self.rows, self.cols)
        finally:
            out.free()

    def matvec(self, x: np.ndarray, softcap: bool = False, cap: float = 30.0) -> np.ndarray:
        xb = DeviceBuffer.from_numpy(self.ctx, np.asarray(x, dtype=np.float32))
        yb = DeviceBuffer(self.ctx, 4 * self.rows)
        try:
            check(lib().gh_q4_0_matvec(self.h, xb.ptr, yb.ptr, int(softcap), float(cap)))
            return yb.numpy()
        finally:
            xb.free()
            yb.free()

    def close(self) -> None:
        if self.h:
            lib().gh_q4_0_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def runLinearQ4(ctx: Context, weights_q4: np.ndarray, x: np.ndarray, n_rows: int, n_cols: int,
                softcap: bool = False, cap: float = 30.0) -> np.ndarray:
    """runLinearQ4 (src/Gemma/Layers/LinearQ4.hs:41-48): raw GGUF bytes as
    little-endian uint32 words, x[n_cols] -> y[n_rows]."""
    words = np.ascontiguousarray(weights_q4)
    if words.dtype != np.uint32:
        b = words.view(np.uint8)
        pad = (-b.nbytes) % 4
        words = np.concatenate([b, np.zeros(pad, np.uint8)]).view(np.uint32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(n_rows, dtype=np.float32)
    check(lib().gh_linear_q4(ctx.h, _ptr(words), words.size, _ptr(x), n_rows, n_cols, int(softcap),
                             float(cap), _ptr(y)))
    return y


# ---------------------------------------------------------------- ops
def _dev(ctx, a):
    return DeviceBuffer.from_numpy(ctx, np.ascontiguousarray(a, dtype=np.float32))


def rmsnorm(ctx: Context, x, w, eps: float = 1e-6, zero_centered: bool = True) -> np.ndarray:
    xb, wb, yb = _dev(ctx, x), _dev(ctx, w), DeviceBuffer(ctx, 4 * len(x))
    check(lib().gh_rmsnorm(ctx.h, xb.ptr, wb.ptr, len(x), eps, int(zero_centered), yb.ptr))
    out = yb.numpy()
    for b in (xb, wb, yb):
        b.free()
    return out


def qk_norm(ctx: Context, x, w, n_heads: int, head_dim: int, eps: float = 1e-6,
            zero_centered: bool = True) -> np.ndarray:
    xb, wb, yb = _dev(ctx, x), _dev(ctx, w), DeviceBuffer(ctx, 4 * n_heads * head_dim)
    check(lib().gh_qk_norm(ctx.h, xb.ptr, wb.ptr, n_heads, head_dim, eps, int(zero_centered), yb.ptr))
    out = yb.numpy()
    for b in (xb, wb, yb):
        b.free()
    return out


def rope(ctx: Context, x, n_heads: int, head_dim: int, theta: float, pos: int) -> np.ndarray:
    xb = _dev(ctx, x)
    check(lib().gh_rope(ctx.h, xb.ptr, n_heads, head_dim, theta, pos))
    out = xb.numpy()
    xb.free()
    return out


def attention_decode(ctx: Context, q, k_cache, v_cache, nq: int, nkv: int, head_dim: int,
                     p_begin: int, p_end: int, n_splits: int = 0) -> np.ndarray:
    qb, kb, vb = _dev(ctx, q), _dev(ctx, k_cache), _dev(ctx, v_cache)
    ob = DeviceBuffer(ctx, 4 * nq * head_dim)
    try:
        check(lib().gh_attention_decode(ctx.h, qb.ptr, kb.ptr, vb.ptr, nq, nkv, head_dim, p_begin, p_end,
                                        n_splits, ob.ptr))
        return ob.numpy()
    finally:
        for b in (qb, kb, vb, ob):
            b.free()


def sample_logits(ctx: Context, logits, temperature: float, seed: int, counter: int, top_k: int = 0) -> int:
    """Draw from softmax(logits / T) with Philox4x32-10 (key seed, counter);
    temperature 0 is the argmax (gh_sample_logits).  top_k > 0 restricts the
    draw to the top_k largest logits, drawn in rank order
    (gh_sample_logits_top_k)."""
    lb = _dev(ctx, logits)
    t = C.c_int32()
    try:
        if top_k:
            check(lib().gh_sample_logits_top_k(ctx.h, lb.ptr, len(logits), float(temperature), int(top_k), int(seed),
                                               int(counter), C.byref(t)))
        else:
            check(lib().gh_sample_logits(ctx.h, lb.ptr, len(logits), float(temperature), int(seed), int(counter),
                                         C.byref(t)))
        return t.value
    finally:
        lb.free()


def gelu_mul(ctx: Context, g, u) -> np.ndarray:
    gb, ub, hb = _dev(ctx, g), _dev(ctx, u), DeviceBuffer(ctx, 4 * len(g))
    check(lib().gh_gelu_mul(ctx.h, gb.ptr, ub.ptr, len(g), hb.ptr))
    out = hb.numpy()
    for b in (gb, ub, hb):
        b.free()
    return out


def argmax(ctx: Context, v) -> int:
    vb = _dev(ctx, v)
    idx = C.c_int32()
    try:
        check(lib().gh_argmax(ctx.h, vb.ptr, len(v), C.byref(idx)))
    finally:
        vb.free()
    return idx.value


# ---------------------------------------------------------------- synthetic data
def synth_f32(seed: int, name: str, sigma: float, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    check(lib().gh_synth_f32(seed, name.encode(), sigma, _ptr(out), n))
    return out


def synth_q4_0(seed: int, name: str, scale_sigma: float, rows: int, cols: int) -> np.ndarray:
    out = np.empty(rows * (cols // 32) * 18, dtype=np.uint8)
    check(lib().gh_synth_q4_0(seed, name.encode(), scale_sigma, rows, cols, _ptr(out)))
    return out


def synth_tokens(seed: int, name: str, n: int, vocab: int) -> np.ndarray:
    out = np.empty(n, dtype=np.int32)
    check(lib().gh_synth_tokens(seed, name.encode(), n, vocab, _ptr(out)))
    return out


def synth_kv(seed: int, layer: int, n_pos: int, width: int, sigma: float = 1.0):
    """(K, V) [n_pos, width] of one layer as KVCache.synth fills it (gh_synth_kv)."""
    k = np.empty((n_pos, width), np.float32)
    v = np.empty((n_pos, width), np.float32)
    check(lib().gh_synth_kv(seed, layer, n_pos, width, sigma, _ptr(k), _ptr(v)))
    return k, v


def center_q4_0(raw: np.ndarray) -> np.ndarray:
    """Zero-mean variant of raw Q4_0 blocks: code 0 becomes 8, so the codes
    have mean 8 and q - 8 mean 0.  Uniform codes give every row a common
    -0.5 * d offset per block, which makes a random deep model's argmax
    almost independent of its input; the centred codes do not."""
    b = np.ascontiguousarray(raw, np.uint8).reshape(-1, 18).copy()
    q = b[:, 2:]
    lo, hi = q & 15, q >> 4
    lo[lo == 0] = 8
    hi[hi == 0] = 8
    b[:, 2:] = lo | (hi << 4)
    return b.reshape(-1)


def flat_scales_q4_0(raw: np.ndarray, d: float) -> np.ndarray:
    """Raw Q4_0 blocks with every block's fp16 scale set to d (rounded to
    fp16).  With |N(0, s)| scales a row's norm varies by about 12 % over 36
    blocks, so among 262144 LM-head rows one stands ~50 % above the rest and
    wins the greedy argmax from most states; equal scales leave no such
    row."""
    b = np.ascontiguousarray(raw, np.uint8).reshape(-1, 18).copy()
    b[:, :2] = np.array([d], np.float16).view(np.uint8)
    return b.reshape(-1)


def tensor_list(cfg: GemmaConfig, untied: bool = False):
    """(name, kind, shape) of every tensor a config needs; kind 'mat' or 'vec'.
    GGUF names; the same order gh_synth_model uses.  untied: with an
    output.weight LM head (last), which gh_synth_model does not make."""
    H, hd, F = cfg.hidden, cfg.head_dim, cfg.ffn
    out = [("token_embd.weight", "mat", (cfg.vocab, H)), ("output_norm.weight", "vec", (H,))]
    for l in range(cfg.n_layers):
        p = f"blk.{l}."
        out += [
            (p + "attn_norm.weight", "vec", (H,)),
            (p + "attn_q.weight", "mat", (cfg.n_heads * hd, H)),
            (p + "attn_k.weight", "mat", (cfg.n_kv_heads * hd, H)),
            (p + "attn_v.weight", "mat", (cfg.n_kv_heads * hd, H)),
            (p + "attn_q_norm.weight", "vec", (hd,)),
            (p + "attn_k_norm.weight", "vec", (hd,)),
            (p + "attn_output.weight", "mat", (H, cfg.n_heads * hd)),
            (p + "post_attention_norm.weight", "vec", (H,)),
            (p + "ffn_norm.weight", "vec", (H,)),
            (p + "ffn_gate.weight", "mat", (F, H)),
            (p + "ffn_up.weight", "mat", (F, H)),
            (p + "ffn_down.weight", "mat", (H, F)),
            (p + "post_ffw_norm.weight", "vec", (H,)),
        ]
    if untied:
        out.append(("output.weight", "mat", (cfg.vocab, H)))
    return out


def synth_tensors(cfg: GemmaConfig, seed: int, q4: bool, w_sigma: float = 0.02,
                  scale_sigma: float = 0.01, norm_sigma: float = 0.02, centered: bool = False,
                  untied: bool = False):
    """Yield (name, dtype, array) with exactly the bytes gh_synth_model uploads
    (centered: Q4_0 codes through center_q4_0; untied: plus an output.weight
    LM head from the same seed, whose Q4_0 blocks all have the scale
    scale_sigma: flat_scales_q4_0)."""
    for name, kind, shape in tensor_list(cfg, untied):
        if kind == "vec":
            yield name, DTYPE_F32, synth_f32(seed, name, norm_sigma, shape[0])
        elif q4:
            raw = synth_q4_0(seed, name, scale_sigma, shape[0], shape[1])
            if name == "output.weight":
                raw = flat_scales_q4_0(raw, scale_sigma)
            yield name, DTYPE_Q4_0, center_q4_0(raw) if centered else raw
        else:
            yield name, DTYPE_F32, synth_f32(seed, name, w_sigma, shape[0] * shape[1])


# ---------------------------------------------------------------- model
class GemmaModel:
    """GemmaModel (src/Gemma/Model.hs:243-257) with device-resident weights."""

    def __init__(self, ctx: Context, cfg: GemmaConfig, handle=None):
        self.ctx = ctx
        if handle is None:
            h = C.c_void_p()
            check(lib().gh_model_create(ctx.h, C.byref(cfg), C.byref(h)))
            handle = h
        self.h = handle
        self.cfg = self.config()

    @classmethod
    def load_gguf(cls, ctx: Context, path: str, max_seq: int = 0) -> "GemmaModel":
        """loadGemmaModelFromGGUF (src/Gemma/Model.hs:908)."""
        h = C.c_void_p()
        check(lib().gh_model_load_gguf(ctx.h, str(path).encode(), max_seq, C.byref(h)))
        return cls(ctx, None, handle=h)

    def config(self) -> GemmaConfig:
        c = GemmaConfig()
        check(lib().gh_model_config(self.h, C.byref(c)))
        return c

    def set_tensor(self, name: str, a: np.ndarray, dtype: int) -> None:
        a = np.ascontiguousarray(a)
        check(lib().gh_model_set_tensor(self.h, name.encode(), dtype, _ptr(a), a.nbytes))

    def synth(self, seed: int, q4: bool, w_sigma: float = 0.02, scale_sigma: float = 0.01,
              norm_sigma: float = 0.02, centered: bool = False, untied: bool = False) -> None:
        """The tensors of synth_tensors with the same arguments (gh_synth_model
        for the plain case)."""
        if centered or untied:
            for name, dtype, arr in synth_tensors(self.cfg, seed, q4, w_sigma, scale_sigma, norm_sigma,
                                                  centered, untied):
                self.set_tensor(name, arr, dtype)
            return
        check(lib().gh_synth_model(self.h, seed, int(q4), w_sigma, scale_sigma, norm_sigma))

    def check(self) -> None:
        check(lib().gh_model_check(self.h))

    def plan(self) -> str:
        """gh_model_plan: the step's kernel plan and the GH_* switches set."""
        n = C.c_size_t(0)
        check(lib().gh_model_plan(self.h, None, 0, C.byref(n)))
        buf = C.create_string_buffer(n.value + 1)
        check(lib().gh_model_plan(self.h, buf, n.value + 1, None))
        return buf.value.decode()

    def close(self) -> None:
        if self.h:
            lib().gh_model_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class KVCache:
    """Gemma.KVCache handle (src/Gemma/KVCache.hs:45-82): device K/V plus the length."""

    def __init__(self, model: GemmaModel, max_seq: int = 0):
        h = C.c_void_p()
        check(lib().gh_kv_create(model.h, max_seq, C.byref(h)))
        self.model, self.h = model, h

    def cacheLength(self) -> int:
        n = C.c_int32()
        check(lib().gh_kv_length(self.h, C.byref(n)))
        return n.value

    __len__ = cacheLength

    def synth(self, seed: int, n_pos: int, sigma: float = 1.0) -> None:
        """Fill positions [0, n_pos) with seeded N(0, sigma) K/V (a stand-in
        for a prefilled context; gh_kv_synth) and set the length to n_pos."""
        check(lib().gh_kv_synth(self.h, seed, n_pos, sigma))

    def set_sampling(self, temperature: float, seed: int = 0) -> None:
        """Next-token rule of this cache's steps: temperature 0 = greedy
        (sampleToken, app/Main.hs:488-507); > 0 = draw from softmax(l / T)
        with Philox keyed by seed, counter = position (gh_kv_set_sampling)."""
        check(lib().gh_kv_set_sampling(self.h, float(temperature), int(seed)))

    def set_top_k(self, top_k: int) -> None:
        """Restrict sampled steps to the top_k largest logits, 1..64, drawn in
        rank order; 0 = every logit (gh_kv_set_top_k)."""
        check(lib().gh_kv_set_top_k(self.h, int(top_k)))

    def reset(self) -> None:
        check(lib().gh_kv_reset(self.h))

    def truncate(self, n: int) -> None:
        """Rewind to the first n positions (gh_kv_truncate)."""
        check(lib().gh_kv_truncate(self.h, int(n)))

    def close(self) -> None:
        if self.h:
            lib().gh_kv_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def runGemmaInferenceCached(model: GemmaModel, token: int, cache: KVCache | None = None,
                            want_logits: bool = True):
    """One decode step (src/Gemma/Model.hs:1313-1437).  Returns
    (logits or None, cache, greedy next token)."""
    if cache is None:
        cache = KVCache(model)
    logits = np.empty(model.cfg.vocab, np.float32) if want_logits else None
    nxt = C.c_int32()
    check(lib().gh_step(model.h, cache.h, int(token), _ptr(logits) if want_logits else None, None,
                        C.byref(nxt)))
    return logits, cache, nxt.value


def runGemmaInferenceCachedWithLayer0(model: GemmaModel, token: int, cache: KVCache | None = None):
    """Step that also returns the hidden state after every layer
    (generalises src/Gemma/Model.hs:1441): (logits, cache, layers[L, H], next)."""
    if cache is None:
        cache = KVCache(model)
    c = model.cfg
    logits = np.empty(c.vocab, np.float32)
    layers = np.empty((c.n_layers, c.hidden), np.float32)
    nxt = C.c_int32()
    check(lib().gh_step(model.h, cache.h, int(token), _ptr(logits), _ptr(layers), C.byref(nxt)))
    return logits, cache, layers, nxt.value


def prefill(model: GemmaModel, cache: KVCache, tokens, want_logits: bool = True, want_layers: bool = False):
    """Batched prefill: the prompt tokens at the cache's next positions in one
    pass per layer (Q4_0 GEMMs on MFMA) instead of one decode step per token
    (the prompt loop of app/Main.hs:426-436).  Returns (logits, layers[L, H],
    next token) of the last token, as runGemmaInferenceCachedWithLayer0 would
    after stepping the tokens one by one; logits / layers are None unless
    asked for."""
    t = np.ascontiguousarray(tokens, dtype=np.int32)
    c = model.cfg
    logits = np.empty(c.vocab, np.float32) if want_logits else None
    layers = np.empty((c.n_layers, c.hidden), np.float32) if want_layers else None
    nxt = C.c_int32()
    check(lib().gh_prefill(model.h, cache.h, _ptr(t), len(t), _ptr(logits) if want_logits else None,
                           _ptr(layers) if want_layers else None, C.byref(nxt)))
    return logits, layers, nxt.value


def generate(model: GemmaModel, cache: KVCache, prompt, n_gen: int, prefill: bool = False) -> np.ndarray:
    """Generation loop on device (app/Main.hs:372-463): greedy, or sampled per
    KVCache.set_sampling.  prefill=True feeds the prompt as one batched
    prefill instead of token by token."""
    p = np.ascontiguousarray(prompt, dtype=np.int32)
    ids = np.empty(n_gen, np.int32)
    fn = lib().gh_generate_prefill if prefill else lib().gh_generate
    check(fn(model.h, cache.h, _ptr(p), len(p), n_gen, _ptr(ids)))
    return ids


def bench_decode(model: GemmaModel, cache: KVCache, prompt, n_warmup: int, n_steps: int):
    """(ms for n_steps timed greedy steps, ids[n_warmup + n_steps + 1])."""
    p = np.ascontiguousarray(prompt, dtype=np.int32)
    ids = np.empty(n_warmup + n_steps + 1, np.int32)
    ms = C.c_float()
    check(lib().gh_bench_decode(model.h, cache.h, _ptr(p), len(p), n_warmup, n_steps, C.byref(ms),
                                _ptr(ids)))
    return ms.value, ids


@dataclass
class KernelStat:
    name: str
    launches: int
    total_ms: float
    bytes_per_launch: float

    @property
    def avg_us(self) -> float:
        return 1e3 * self.total_ms / max(1, self.launches)

    @property
    def gbps(self) -> float:
        return self.bytes_per_launch / (self.avg_us * 1e-6) / 1e9 if self.total_ms > 0 else 0.0


def profile_steps(model: GemmaModel, cache: KVCache, n_steps: int) -> list[KernelStat]:
    """Per-kernel event timing over n_steps greedy steps (replaces the
    reference's gpu_print_profile_stats hook)."""
    arr = (GhKernelStat * 32)()
    n = C.c_int32()
    check(lib().gh_profile_steps(model.h, cache.h, n_steps, arr, 32, C.byref(n)))
    return [KernelStat(arr[i].name.decode(), arr[i].launches, arr[i].total_ms, arr[i].bytes)
            for i in range(n.value)]


def profile_prefill(model: GemmaModel, cache: KVCache, tokens) -> list[KernelStat]:
    """gh_prefill of the tokens with per-kernel event timing (the cache
    advances as with prefill)."""
    t = np.ascontiguousarray(tokens, dtype=np.int32)
    arr = (GhKernelStat * 32)()
    n = C.c_int32()
    check(lib().gh_prefill_profile(model.h, cache.h, _ptr(t), len(t), arr, 32, C.byref(n)))
    return [KernelStat(arr[i].name.decode(), arr[i].launches, arr[i].total_ms, arr[i].bytes)
            for i in range(n.value)]


STEP_KERNELS = ("qkv", "attention", "o_proj", "gate_up", "down", "final_norm", "lm_head")


@dataclass
class KernelTiming:
    name: str
    avg_us: float            # HIP-event time per launch, launches back to back
    bytes_per_launch: float  # algorithmic HBM bytes per launch
    launches_per_step: int

    @property
    def gbps(self) -> float:
        return self.bytes_per_launch / (self.avg_us * 1e-6) / 1e9 if self.avg_us > 0 else 0.0


def time_kernel(model: GemmaModel, cache: KVCache, name: str, n_reps: int = 50) -> KernelTiming:
    """Replay only the step kernels called `name` at the cache's current
    position n_reps times between two HIP events (model and cache state are
    unchanged); see gh_time_kernel."""
    us, nb, per = C.c_double(), C.c_double(), C.c_int32()
    check(lib().gh_time_kernel(model.h, cache.h, name.encode(), n_reps, C.byref(us), C.byref(nb), C.byref(per)))
    return KernelTiming(name, us.value, nb.value, per.value)


def time_exchange(ctx: Context, n_wg: int, rounds: int = 2000) -> float:
    """Microseconds per all-to-all exchange of one self-validating word per
    workgroup among n_wg co-resident workgroups (gh_time_exchange), the
    synchronisation the persistent step uses between its phases."""
    us = C.c_double()
    check(lib().gh_time_exchange(ctx.h, n_wg, rounds, C.byref(us)))
    return us.value


def stream_read_gbps(ctx: Context, nbytes: int = 1 << 30, n_reps: int = 20) -> tuple[float, float]:
    """Measured stream-read peak of ctx's device: nbytes read once per
    launch, n_reps launches back to back (gh_time_stream_read).  Returns
    (GB/s, average microseconds per launch)."""
    us = C.c_double()
    check(lib().gh_time_stream_read(ctx.h, nbytes, n_reps, C.byref(us)))
    return nbytes / (us.value * 1e-6) / 1e9, us.value
