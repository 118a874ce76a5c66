"""ctypes loader for libgemma_hip.so and the C-ABI signatures of include/gemma_hip.h."""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libgemma_hip.so"

GH_OK = 0
ERRORS = {
    -1: "GH_ERR_INVALID",
    -2: "GH_ERR_HIP",
    -3: "GH_ERR_OOM",
    -4: "GH_ERR_STATE",
    -5: "GH_ERR_RANGE",
    -6: "GH_ERR_NAN",
    -7: "GH_ERR_FORMAT",
    -8: "GH_ERR_NOT_FOUND",
}
DTYPE_F32, DTYPE_F16, DTYPE_Q4_0 = 0, 1, 2
MODE_GEMMA3, MODE_REF = 0, 1
FLAG_QK_NORM, FLAG_POST_ATTN_NORM, FLAG_POST_FFN_NORM, FLAG_ZERO_CENTERED, FLAG_IEEE_SCALES = 1, 2, 4, 8, 16


class GemmaHipError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"{ERRORS.get(code, code)}: {msg}")
        self.code = code
        self.name = ERRORS.get(code, str(code))


class GhConfig(C.Structure):
    _fields_ = [
        ("vocab", C.c_int32), ("hidden", C.c_int32), ("n_layers", C.c_int32),
        ("n_heads", C.c_int32), ("n_kv_heads", C.c_int32), ("head_dim", C.c_int32),
        ("ffn", C.c_int32), ("max_seq", C.c_int32), ("sliding_window", C.c_int32),
        ("global_every", C.c_int32), ("rope_theta_local", C.c_float),
        ("rope_theta_global", C.c_float), ("rms_eps", C.c_float), ("mode", C.c_int32),
        ("flags", C.c_int32),
    ]

    def as_dict(self) -> dict:
        return {k: getattr(self, k) for k, _ in self._fields_}

    def copy(self) -> "GhConfig":
        c = GhConfig()
        C.pointer(c)[0] = self
        return c


class GhKernelStat(C.Structure):
    _fields_ = [("name", C.c_char * 32), ("launches", C.c_int32), ("total_ms", C.c_double),
                ("bytes", C.c_double)]


_P = C.c_void_p
_F = C.POINTER(C.c_float)
_I32 = C.POINTER(C.c_int32)

# name: (restype, argtypes)
SIGNATURES = {
    "gh_last_error": (C.c_char_p, []),
    "gh_version": (C.c_char_p, []),
    "gh_device_count": (C.c_int, [_I32]),
    "gh_ctx_create": (C.c_int, [C.c_int, C.POINTER(_P)]),
    "gh_ctx_destroy": (C.c_int, [_P]),
    "gh_ctx_release": (None, [_P]),
    "gh_model_release": (None, [_P]),
    "gh_kv_release": (None, [_P]),
    "gh_q4_0_release": (None, [_P]),
    "gh_ctx_sync": (C.c_int, [_P]),
    "gh_buf_alloc": (C.c_int, [_P, C.c_size_t, C.POINTER(_P)]),
    "gh_buf_free": (C.c_int, [_P, _P]),
    "gh_buf_upload": (C.c_int, [_P, _P, _P, C.c_size_t]),
    "gh_buf_download": (C.c_int, [_P, _P, _P, C.c_size_t]),
    "gh_q4_0_upload": (C.c_int, [_P, _P, C.c_int64, C.c_int64, C.c_int, C.POINTER(_P)]),
    "gh_q4_0_free": (C.c_int, [_P]),
    "gh_q4_0_dequant": (C.c_int, [_P, _P]),
    "gh_q4_0_matvec": (C.c_int, [_P, _P, _P, C.c_int, C.c_float]),
    "gh_linear_q4": (C.c_int, [_P, _P, C.c_size_t, _P, C.c_int, C.c_int, C.c_int, C.c_float, _P]),
    "gh_rmsnorm": (C.c_int, [_P, _P, _P, C.c_int, C.c_float, C.c_int, _P]),
    "gh_qk_norm": (C.c_int, [_P, _P, _P, C.c_int, C.c_int, C.c_float, C.c_int, _P]),
    "gh_rope": (C.c_int, [_P, _P, C.c_int, C.c_int, C.c_float, C.c_int]),
    "gh_attention_decode": (C.c_int, [_P, _P, _P, _P, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                      C.c_int, _P]),
    "gh_attention_decode_noalloc": (C.c_int, [_P, _P, _P, _P, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                              C.c_int, _P]),
    "gh_gelu_mul": (C.c_int, [_P, _P, _P, C.c_int, _P]),
    "gh_argmax": (C.c_int, [_P, _P, C.c_int, _I32]),
    "gh_config_preset": (C.c_int, [C.c_char_p, C.POINTER(GhConfig)]),
    "gh_model_create": (C.c_int, [_P, C.POINTER(GhConfig), C.POINTER(_P)]),
    "gh_model_destroy": (C.c_int, [_P]),
    "gh_model_set_tensor": (C.c_int, [_P, C.c_char_p, C.c_int, _P, C.c_size_t]),
    "gh_model_check": (C.c_int, [_P]),
    "gh_model_config": (C.c_int, [_P, C.POINTER(GhConfig)]),
    "gh_model_plan": (C.c_int, [_P, C.c_char_p, C.c_size_t, C.POINTER(C.c_size_t)]),
    "gh_model_load_gguf": (C.c_int, [_P, C.c_char_p, C.c_int32, C.POINTER(_P)]),
    "gh_gguf_inspect": (C.c_int, [C.c_char_p, C.POINTER(GhConfig)]),
    "gh_kv_create": (C.c_int, [_P, C.c_int32, C.POINTER(_P)]),
    "gh_kv_destroy": (C.c_int, [_P]),
    "gh_kv_reset": (C.c_int, [_P]),
    "gh_kv_length": (C.c_int, [_P, _I32]),
    "gh_kv_truncate": (C.c_int, [_P, C.c_int32]),
    "gh_step": (C.c_int, [_P, _P, C.c_int32, _P, _P, _I32]),
    "gh_generate": (C.c_int, [_P, _P, _P, C.c_int32, C.c_int32, _P]),
    "gh_prefill": (C.c_int, [_P, _P, _P, C.c_int32, _P, _P, _I32]),
    "gh_generate_prefill": (C.c_int, [_P, _P, _P, C.c_int32, C.c_int32, _P]),
    "gh_bench_decode": (C.c_int, [_P, _P, _P, C.c_int32, C.c_int32, C.c_int32, _F, _P]),
    "gh_profile_steps": (C.c_int, [_P, _P, C.c_int32, C.POINTER(GhKernelStat), C.c_int32, _I32]),
    "gh_prefill_profile": (C.c_int, [_P, _P, _P, C.c_int32, C.POINTER(GhKernelStat), C.c_int32, _I32]),
    "gh_capture_begin": (C.c_int, [_P]),
    "gh_capture_replay": (C.c_int, [_P, C.c_int32, C.POINTER(C.c_float)]),
    "gh_timer_start": (C.c_int, [_P]),
    "gh_timer_stop": (C.c_int, [_P, C.POINTER(C.c_float)]),
    "gh_kv_synth": (C.c_int, [_P, C.c_uint64, C.c_int32, C.c_float]),
    "gh_kv_set_sampling": (C.c_int, [_P, C.c_float, C.c_uint64]),
    "gh_sample_logits": (C.c_int, [_P, _P, C.c_int, C.c_float, C.c_uint64, C.c_uint64, _I32]),
    "gh_sample_logits_top_k": (C.c_int, [_P, _P, C.c_int, C.c_float, C.c_int32, C.c_uint64, C.c_uint64, _I32]),
    "gh_kv_set_top_k": (C.c_int, [_P, C.c_int32]),
    "gh_time_kernel": (C.c_int, [_P, _P, C.c_char_p, C.c_int32, C.POINTER(C.c_double), C.POINTER(C.c_double), _I32]),
    "gh_time_stream_read": (C.c_int, [_P, C.c_size_t, C.c_int32, C.POINTER(C.c_double)]),
    "gh_time_exchange": (C.c_int, [_P, C.c_int32, C.c_int32, C.POINTER(C.c_double)]),
    "gh_synth_f32": (C.c_int, [C.c_uint64, C.c_char_p, C.c_float, _P, C.c_size_t]),
    "gh_synth_q4_0": (C.c_int, [C.c_uint64, C.c_char_p, C.c_float, C.c_int64, C.c_int64, _P]),
    "gh_synth_tokens": (C.c_int, [C.c_uint64, C.c_char_p, C.c_int32, C.c_int32, _P]),
    "gh_synth_kv": (C.c_int, [C.c_uint64, C.c_int32, C.c_int32, C.c_int32, C.c_float, _P, _P]),
    "gh_synth_model": (C.c_int, [_P, C.c_uint64, C.c_int, C.c_float, C.c_float, C.c_float]),
}

_lib = None


def lib():
    """Load libgemma_hip.so once; raise if it is not built (no fallback path)."""
    global _lib
    if _lib is None:
        path = os.environ.get("GEMMA_HIP_LIB", str(LIB_PATH))
        if not Path(path).exists():
            raise ImportError(
                f"libgemma_hip.so not found at {path}; build it with "
                "`python gemma.hs_amd/build.py` (there is no CPU fallback)")
        L = C.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc: int) -> None:
    if rc != GH_OK:
        msg = lib().gh_last_error()
        raise GemmaHipError(rc, msg.decode() if msg else "")
