"""Independent float64 restatement of a Gemma-3 decode step, written from the
Hugging Face Gemma3 formulation (Gemma3RMSNorm with (1 + w), rotate_half
RoPE, repeat_kv GQA, sliding-window mask q - kv < W, gelu_pytorch_tanh) with
numpy vector ops.  Used only to cross-check the C oracle, whose code follows
the reference's WGSL loops instead.
"""
from __future__ import annotations

import numpy as np


def q4_0_dequant_np(raw: np.ndarray, rows: int, cols: int, ftz: bool = True) -> np.ndarray:
    """llama.cpp dequantize_row_q4_0: y[j] = ((qs[j] & 15) - 8) d,
    y[j + 16] = ((qs[j] >> 4) - 8) d; d is the block's fp16 scale."""
    b = np.ascontiguousarray(raw, np.uint8).reshape(rows * (cols // 32), 18)
    d16 = b[:, :2].copy().view(np.float16).reshape(-1)
    d = d16.astype(np.float64)
    if ftz:
        sub = (b[:, 1] & 0x7C) == 0
        d = np.where(sub, np.copysign(0.0, d), d)
    qs = b[:, 2:].astype(np.int64)
    q = np.concatenate([qs & 15, qs >> 4], axis=1) - 8
    return (q * d[:, None]).reshape(rows, cols)


def rms_norm(x, w, eps, zc=True):
    x = np.asarray(x, np.float64)
    y = x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    return y * ((1.0 + w) if zc else w)


def rotate_half(x):
    h = x.shape[-1] // 2
    return np.concatenate([-x[..., h:], x[..., :h]], axis=-1)


def rope(x, pos, theta):
    """x [..., heads, hd]: HF apply_rotary_pos_emb with cos/sin = cat(freqs, freqs)."""
    hd = x.shape[-1]
    inv = 1.0 / theta ** (np.arange(0, hd, 2, dtype=np.float64) / hd)
    ang = pos * inv
    emb = np.concatenate([ang, ang])
    return x * np.cos(emb) + rotate_half(x) * np.sin(emb)


def gelu_tanh(x):
    return 0.5 * x * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (x + 0.044715 * x ** 3)))


def attention(q, K, V, nq, nkv):
    """q [nq, hd], K/V [L, nkv, hd] -> [nq, hd] (repeat_kv + softmax)."""
    rep = nq // nkv
    Kx = np.repeat(K, rep, axis=1)  # [L, nq, hd]
    Vx = np.repeat(V, rep, axis=1)
    hd = q.shape[-1]
    s = np.einsum("hd,lhd->hl", q, Kx) / np.sqrt(hd)
    s = s - s.max(axis=1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=1, keepdims=True)
    return np.einsum("hl,lhd->hd", p, Vx)


class NumpyGemma:
    """Weights given as dense float64 matrices (dequantised if Q4_0)."""

    def __init__(self, cfg, tensors: dict):
        self.c = cfg
        self.t = tensors
        L, nkv, hd = cfg.n_layers, cfg.n_kv_heads, cfg.head_dim
        self.K = [np.zeros((cfg.max_seq, nkv, hd)) for _ in range(L)]
        self.V = [np.zeros((cfg.max_seq, nkv, hd)) for _ in range(L)]

    def is_global(self, l):
        ge = self.c.global_every
        return ge <= 0 or (l + 1) % ge == 0

    def step(self, tok, pos):
        c, t = self.c, self.t
        H, nq, nkv, hd = c.hidden, c.n_heads, c.n_kv_heads, c.head_dim
        eps = c.rms_eps
        E = t["token_embd.weight"]
        x = E[tok] * np.sqrt(H)
        layers = []
        for l in range(c.n_layers):
            p = f"blk.{l}."
            glob = self.is_global(l)
            theta = c.rope_theta_global if glob else c.rope_theta_local
            xn = rms_norm(x, t[p + "attn_norm.weight"], eps)
            q = (t[p + "attn_q.weight"] @ xn).reshape(nq, hd)
            k = (t[p + "attn_k.weight"] @ xn).reshape(nkv, hd)
            v = (t[p + "attn_v.weight"] @ xn).reshape(nkv, hd)
            q = rms_norm(q, t[p + "attn_q_norm.weight"], eps)
            k = rms_norm(k, t[p + "attn_k_norm.weight"], eps)
            q, k = rope(q, pos, theta), rope(k, pos, theta)
            self.K[l][pos], self.V[l][pos] = k, v
            lo = 0
            if not glob and c.sliding_window > 0:
                lo = max(0, pos + 1 - c.sliding_window)
            o = attention(q, self.K[l][lo:pos + 1], self.V[l][lo:pos + 1], nq, nkv).reshape(-1)
            a = rms_norm(t[p + "attn_output.weight"] @ o, t[p + "post_attention_norm.weight"], eps)
            x1 = x + a
            n2 = rms_norm(x1, t[p + "ffn_norm.weight"], eps)
            h = gelu_tanh(t[p + "ffn_gate.weight"] @ n2) * (t[p + "ffn_up.weight"] @ n2)
            d = rms_norm(t[p + "ffn_down.weight"] @ h, t[p + "post_ffw_norm.weight"], eps)
            x = x1 + d
            layers.append(x.copy())
        logits = t.get("output.weight", E) @ rms_norm(x, t["output_norm.weight"], eps)
        return logits, np.stack(layers)
