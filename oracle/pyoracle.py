"""ctypes binding of oracle/build/liboracle.so -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module, and only as the checker (or the timed CPU baseline).
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "build" / "liboracle.so"

F32, Q4_0 = 0, 2
MODE_GEMMA3, MODE_REF = 0, 1
QK_NORM, POST_ATTN_NORM, POST_FFN_NORM, ZERO_CENTERED, IEEE_SCALES = 1, 2, 4, 8, 16


class OrcConfig(C.Structure):
    _fields_ = [
        ("vocab", C.c_int32), ("hidden", C.c_int32), ("n_layers", C.c_int32),
        ("n_heads", C.c_int32), ("n_kv_heads", C.c_int32), ("head_dim", C.c_int32),
        ("ffn", C.c_int32), ("max_seq", C.c_int32), ("sliding_window", C.c_int32),
        ("global_every", C.c_int32), ("rope_theta_local", C.c_float),
        ("rope_theta_global", C.c_float), ("rms_eps", C.c_float), ("mode", C.c_int32),
        ("flags", C.c_int32),
    ]


_P = C.c_void_p
_SIG = {
    "orc_f16_to_f32": (C.c_float, [C.c_uint16, C.c_int]),
    "orc_q4_0_dequant": (None, [_P, C.c_size_t, C.c_int, _P]),
    "orc_q4_0_matvec": (None, [_P, _P, C.c_int, C.c_int, C.c_int, _P]),
    "orc_q4_0_matvec_f64": (None, [_P, _P, C.c_int, C.c_int, C.c_int, _P, _P]),
    "orc_f32_matvec": (None, [_P, _P, C.c_int, C.c_int, _P]),
    "orc_rmsnorm_tree": (None, [_P, _P, C.c_int, C.c_float, C.c_int, _P]),
    "orc_rmsnorm_seq": (None, [_P, _P, C.c_int, C.c_float, C.c_int, _P]),
    "orc_qk_norm": (None, [_P, _P, C.c_int, C.c_int, C.c_float, C.c_int, _P]),
    "orc_rope": (None, [_P, C.c_int, C.c_int, C.c_float, C.c_int, _P]),
    "orc_attention": (None, [_P, _P, _P, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, _P]),
    "orc_gelu_tanh": (C.c_float, [C.c_float]),
    "orc_geglu": (None, [_P, _P, C.c_int, _P]),
    "orc_argmax": (C.c_int32, [_P, C.c_int]),
    "orc_softcap": (None, [_P, C.c_int, C.c_float]),
    "orc_model_create": (_P, [C.POINTER(OrcConfig)]),
    "orc_model_destroy": (None, [_P]),
    "orc_model_set_tensor": (C.c_int, [_P, C.c_char_p, C.c_int, _P, C.c_size_t]),
    "orc_model_reset": (None, [_P]),
    "orc_model_set_kv": (C.c_int, [_P, C.c_int, C.c_int, _P, _P]),
    "orc_step": (C.c_int, [_P, C.c_int32, C.c_int32, _P, _P]),
    "orc_generate": (C.c_int, [_P, _P, C.c_int, C.c_int, _P, _P]),
    "orc_set_threads": (None, [C.c_int]),
    "orc_philox4x32_10": (None, [_P, _P, _P]),
    "orc_philox_uniform": (C.c_float, [C.c_uint64, C.c_uint64]),
    "orc_sample": (C.c_int32, [_P, C.c_int, C.c_float, C.c_float, C.POINTER(C.c_double)]),
    "orc_sample_top_k": (C.c_int32, [_P, C.c_int, C.c_float, C.c_int, C.c_float, C.POINTER(C.c_double)]),
}

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(f"{LIB_PATH} not built; run `python gemma.hs_amd/build.py --only oracle`")
        L = C.CDLL(str(LIB_PATH))
        for n, (r, a) in _SIG.items():
            f = getattr(L, n)
            f.restype = r
            f.argtypes = a
        _lib = L
    return _lib


def _p(a):
    return C.c_void_p(a.ctypes.data) if a is not None else None


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def set_threads(n: int) -> None:
    lib().orc_set_threads(int(n))


def f16_to_f32(h: int, ftz: bool = True) -> float:
    return lib().orc_f16_to_f32(h, int(ftz))


def q4_0_dequant(raw: np.ndarray, ftz: bool = True) -> np.ndarray:
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    nb = raw.size // 18
    out = np.empty(nb * 32, np.float32)
    lib().orc_q4_0_dequant(_p(raw), nb, int(ftz), _p(out))
    return out


def q4_0_matvec(raw, x, rows, cols, ftz=True) -> np.ndarray:
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    x = f32(x)
    y = np.empty(rows, np.float32)
    lib().orc_q4_0_matvec(_p(raw), _p(x), rows, cols, int(ftz), _p(y))
    return y


def q4_0_matvec_f64(raw, x, rows, cols, ftz=True):
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    x = f32(x)
    y = np.empty(rows, np.float64)
    ay = np.empty(rows, np.float64)
    lib().orc_q4_0_matvec_f64(_p(raw), _p(x), rows, cols, int(ftz), _p(y), _p(ay))
    return y, ay


def f32_matvec(w, x) -> np.ndarray:
    w = f32(w)
    x = f32(x)
    y = np.empty(w.shape[0], np.float32)
    lib().orc_f32_matvec(_p(w), _p(x), w.shape[0], w.shape[1], _p(y))
    return y


def rmsnorm_tree(x, w, eps=1e-6, zc=True):
    x, w = f32(x), f32(w)
    y = np.empty_like(x)
    lib().orc_rmsnorm_tree(_p(x), _p(w), x.size, eps, int(zc), _p(y))
    return y


def rmsnorm_seq(x, w, eps=1e-6, zc=True):
    x, w = f32(x), f32(w)
    y = np.empty_like(x)
    lib().orc_rmsnorm_seq(_p(x), _p(w), x.size, eps, int(zc), _p(y))
    return y


def qk_norm(x, w, n_heads, hd, eps=1e-6, zc=True):
    x, w = f32(x), f32(w)
    y = np.empty_like(x)
    lib().orc_qk_norm(_p(x), _p(w), n_heads, hd, eps, int(zc), _p(y))
    return y


def rope(x, n_heads, hd, theta, pos):
    x = f32(x)
    y = np.empty_like(x)
    lib().orc_rope(_p(x), n_heads, hd, theta, pos, _p(y))
    return y


def attention(q, kc, vc, nq, nkv, hd, p_begin, p_end):
    q, kc, vc = f32(q), f32(kc), f32(vc)
    out = np.empty(nq * hd, np.float32)
    lib().orc_attention(_p(q), _p(kc), _p(vc), nq, nkv, hd, p_begin, p_end, _p(out))
    return out


def gelu_tanh(x: float) -> float:
    return lib().orc_gelu_tanh(x)


def geglu(g, u):
    g, u = f32(g), f32(u)
    h = np.empty_like(g)
    lib().orc_geglu(_p(g), _p(u), g.size, _p(h))
    return h


def argmax(v) -> int:
    v = f32(v)
    return lib().orc_argmax(_p(v), v.size)


def softcap(y, cap):
    y = f32(y).copy()
    lib().orc_softcap(_p(y), y.size, cap)
    return y


def config_from(gh_cfg) -> OrcConfig:
    """Copy a gemma_hip GemmaConfig (same field layout) into an OrcConfig."""
    c = OrcConfig()
    for name, _ in OrcConfig._fields_:
        setattr(c, name, getattr(gh_cfg, name))
    return c


class OracleModel:
    def __init__(self, cfg):
        self.cfg = cfg if isinstance(cfg, OrcConfig) else config_from(cfg)
        self.h = lib().orc_model_create(C.byref(self.cfg))

    def set_tensor(self, name: str, a: np.ndarray, dtype: int) -> None:
        a = np.ascontiguousarray(a)
        rc = lib().orc_model_set_tensor(self.h, name.encode(), dtype, _p(a), a.nbytes)
        if rc != 0:
            raise ValueError(f"oracle set_tensor({name}) -> {rc}")

    def reset(self) -> None:
        lib().orc_model_reset(self.h)

    def set_kv(self, layer: int, k: np.ndarray, v: np.ndarray) -> None:
        """Positions [0, len(k)) of a layer's K/V cache ([n_pos, nkv*hd] each)."""
        k, v = f32(k), f32(v)
        rc = lib().orc_model_set_kv(self.h, layer, k.shape[0], _p(k), _p(v))
        if rc != 0:
            raise ValueError(f"oracle set_kv({layer}) -> {rc}")

    def step(self, token: int, pos: int, want_layers: bool = False):
        c = self.cfg
        logits = np.empty(c.vocab, np.float32)
        layers = np.empty((c.n_layers, c.hidden), np.float32) if want_layers else None
        r = lib().orc_step(self.h, token, pos, _p(logits), _p(layers))
        if r < 0:
            raise ValueError(f"oracle step -> {r}")
        return logits, layers, r

    def generate(self, prompt, n_gen: int):
        p = np.ascontiguousarray(prompt, dtype=np.int32)
        ids = np.empty(n_gen, np.int32)
        margins = np.empty(n_gen, np.float32)
        r = lib().orc_generate(self.h, _p(p), len(p), n_gen, _p(ids), _p(margins))
        if r < 0:
            raise ValueError(f"oracle generate -> {r}")
        return ids, margins

    def close(self):
        if self.h:
            lib().orc_model_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def philox4x32_10(ctr, key) -> np.ndarray:
    c = np.ascontiguousarray(ctr, dtype=np.uint32)
    k = np.ascontiguousarray(key, dtype=np.uint32)
    out = np.empty(4, dtype=np.uint32)
    lib().orc_philox4x32_10(_p(c), _p(k), _p(out))
    return out


def philox_uniform(seed: int, counter: int) -> float:
    return float(lib().orc_philox_uniform(seed, counter))


def sample(logits, temperature: float, u: float):
    """(index, margin): inversion draw of u from softmax(logits / T); margin
    = distance of u * total to the nearest cumulative boundary / total."""
    x = f32(logits)
    m = C.c_double()
    i = lib().orc_sample(_p(x), len(x), temperature, u, C.byref(m))
    return int(i), m.value


def sample_top_k(logits, temperature: float, k: int, u: float):
    """(index, margin): inversion draw of u from softmax(logits / T) over the
    k largest logits (value descending, then lower index), in rank order."""
    x = f32(logits)
    m = C.c_double()
    i = lib().orc_sample_top_k(_p(x), len(x), temperature, int(k), u, C.byref(m))
    return int(i), m.value
