"""Minimal GGUF v3 writer for tests (synthetic Gemma-3 files).

Layout per the GGUF v3 format read by src/Gemma/GGUF.hs:186-239: magic,
version 3, tensor count, metadata count, metadata key/values, tensor infos
(name, dims innermost first, ggml type, offset), data section aligned to
general.alignment (32).
"""
from __future__ import annotations

import struct

import numpy as np

GGML = {"f32": 0, "f16": 1, "q4_0": 2, "q4_1": 3}
T_U32, T_I32, T_F32, T_STR, T_ARR = 4, 5, 6, 8, 9


def _s(b: bytearray, s: str) -> None:
    e = s.encode()
    b += struct.pack("<Q", len(e)) + e


def write_gguf(path, meta: dict, tensors: list, version: int = 3, magic: int = 0x46554747,
               truncate: int | None = None) -> None:
    """meta: key -> (type, value); tensors: (name, kind, rows, cols or None, bytes)."""
    b = bytearray()
    b += struct.pack("<IIQQ", magic, version, len(tensors), len(meta))
    for k, (t, v) in meta.items():
        _s(b, k)
        b += struct.pack("<I", t)
        if t == T_U32:
            b += struct.pack("<I", v)
        elif t == T_I32:
            b += struct.pack("<i", v)
        elif t == T_F32:
            b += struct.pack("<f", v)
        elif t == T_STR:
            _s(b, v)
        elif t == T_ARR:  # array of strings
            b += struct.pack("<IQ", T_STR, len(v))
            for s in v:
                _s(b, s)
        else:
            raise ValueError(t)
    off = 0
    datas = []
    for name, kind, rows, cols, data in tensors:
        _s(b, name)
        dims = [rows] if cols is None else [cols, rows]
        b += struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        b += struct.pack("<IQ", GGML[kind], off)
        data = bytes(np.ascontiguousarray(data).view(np.uint8))
        datas.append((off, data))
        off += (len(data) + 31) // 32 * 32
    pad = (-len(b)) % 32
    b += b"\0" * pad
    base = len(b)
    body = bytearray(off)
    for o, d in datas:
        body[o:o + len(d)] = d
    b += body
    assert len(b) - base == off
    if truncate is not None:
        b = b[:truncate]
    with open(path, "wb") as f:
        f.write(b)


def gemma3_meta(cfg) -> dict:
    return {
        "general.architecture": (T_STR, "gemma3"),
        "gemma3.block_count": (T_U32, cfg.n_layers),
        "gemma3.embedding_length": (T_U32, cfg.hidden),
        "gemma3.feed_forward_length": (T_U32, cfg.ffn),
        "gemma3.attention.head_count": (T_U32, cfg.n_heads),
        "gemma3.attention.head_count_kv": (T_U32, cfg.n_kv_heads),
        "gemma3.attention.key_length": (T_U32, cfg.head_dim),
        "gemma3.attention.value_length": (T_U32, cfg.head_dim),
        "gemma3.rope.freq_base": (T_F32, cfg.rope_theta_global),
        "gemma3.attention.sliding_window": (T_U32, cfg.sliding_window),
        "gemma3.attention.layer_norm_rms_epsilon": (T_F32, cfg.rms_eps),
        "tokenizer.ggml.tokens": (T_ARR, [f"t{i}" for i in range(8)]),
    }


def random_q4_1(rows: int, cols: int, seed: int, subnormal_frac: float = 0.02) -> np.ndarray:
    """Raw Q4_1 bytes (20-byte blocks: fp16 d, fp16 m, 16 code bytes) with
    random codes, d ~ |N(0, 0.01)| (some fp16 subnormal), m ~ N(0, 0.02)."""
    rng = np.random.default_rng(seed)
    nb = rows * cols // 32
    b = rng.integers(0, 256, size=(nb, 20), dtype=np.uint8)
    d = np.abs(rng.normal(0, 0.01, nb)).astype(np.float16)
    sub = rng.random(nb) < subnormal_frac
    d[sub] = rng.integers(1, 1024, size=int(sub.sum())).astype(np.uint16).view(np.float16)
    b[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    b[:, 2:4] = rng.normal(0, 0.02, nb).astype(np.float16).view(np.uint8).reshape(nb, 2)
    return b.reshape(-1)


def synth_gguf(path, cfg, seed: int, q4: bool, embd_q4_1: bool = False, norms_f16: bool = False,
               untied: bool = False, head_f16: bool = False, **kw) -> None:
    """The seeded synthetic model of gemma_hip.synth_tensors as a GGUF file;
    embd_q4_1 replaces token_embd with random Q4_1 blocks, norms_f16 stores
    the norm vectors as F16 (with a few subnormal values); untied adds an
    output.weight LM head (Q4_0, or F16 values of N(0, 0.02) with head_f16)."""
    import gemma_hip as gh
    shapes = {n: (k, s) for n, k, s in gh.tensor_list(cfg, untied)}
    tensors = []
    for name, dtype, arr in gh.synth_tensors(cfg, seed, q4, untied=untied):
        if name == "output.weight" and head_f16:
            kind, shape = shapes[name]
            h = gh.synth_f32(seed, name, 0.02, shape[0] * shape[1]).astype(np.float16)
            tensors.append((name, "f16", shape[0], shape[1], h))
            continue
        kind, shape = shapes[name]
        if kind == "vec":
            if norms_f16:
                h = np.asarray(arr, np.float32).astype(np.float16)
                h[::97] = np.uint16(0x0203).view(np.float16)  # a subnormal: 0 after FTZ
                tensors.append((name, "f16", shape[0], None, h))
            else:
                tensors.append((name, "f32", shape[0], None, arr))
        elif name == "token_embd.weight" and embd_q4_1:
            tensors.append((name, "q4_1", shape[0], shape[1], random_q4_1(shape[0], shape[1], seed + 1)))
        else:
            tensors.append((name, "q4_0" if dtype == gh.DTYPE_Q4_0 else "f32", shape[0], shape[1], arr))
    write_gguf(path, gemma3_meta(cfg), tensors, **kw)
