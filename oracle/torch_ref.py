"""PyTorch-CPU restatement of gemma.hs's decode step -- TEST INFRASTRUCTURE ONLY.

Only tests/ and bench.py's cpu_baseline leg may import this module: it is
the benchmark's CPU baseline, a PyTorch restatement on all host cores (the
reference's own path, Dawn's SwiftShader adapter, does not exist in this
image), and a second checker beside the C oracle.  Nothing in the product
imports it.

The arithmetic contract is the one oracle/gemma_oracle.c restates (each
step cites the same reference lines): f32 everywhere; Q4_0 weights
dequantised once to f32, (q - 8) * d with subnormal d flushed to zero
(src/Gemma/GGUF.hs:726-820); zero-centred RMSNorm x / sqrt(mean(x^2) + eps)
* (1 + w) (src/Gemma/Layers/RMSNorm.hs:45-154); split-half RoPE with
1 / pow(theta, 2i / hd) (src/Gemma/Layers/AttentionGPU.hs:68-115); GQA
attention with scale 1 / sqrt(hd) (AttentionGPU.hs:292-423); GELU-tanh
with the +-10 clamp (src/Gemma/Layers/MLP.hs:384-447).  Summation orders
are torch's, so it agrees with the C oracle to a relative 1e-5 or so, not
bit for bit (tests/test_oracle.py checks it against the C oracle).
"""
from __future__ import annotations

import numpy as np
import torch

ZERO_CENTERED, QK_NORM, POST_ATTN_NORM, POST_FFN_NORM, IEEE_SCALES = 8, 1, 2, 4, 16
MODE_REF = 1


def q4_0_to_f32(raw: np.ndarray, rows: int, cols: int, ftz: bool = True) -> torch.Tensor:
    """GGUF Q4_0 rows [rows][cols/32 blocks of 18 bytes] -> f32 [rows, cols]."""
    b = np.ascontiguousarray(raw, np.uint8).reshape(rows, cols // 32, 18)
    d16 = b[:, :, 0:2].copy().view(np.float16)[..., 0]
    if ftz:
        sub = (d16.view(np.uint16) & 0x7C00) == 0
        d16 = np.where(sub, np.copysign(np.float16(0), d16), d16)
    d = d16.astype(np.float32)
    qs = b[:, :, 2:]
    q = np.concatenate([qs & 15, qs >> 4], axis=2).astype(np.float32)  # elements 0-15 low, 16-31 high nibbles
    w = (q - 8.0) * d[:, :, None]
    return torch.from_numpy(w.reshape(rows, cols))


def _norm(x: torch.Tensor, w: torch.Tensor, eps: float, zc: bool) -> torch.Tensor:
    rms = torch.sqrt(torch.mean(x * x) + eps)
    return (x / rms) * ((1.0 + w) if zc else w)


def _gelu_tanh(x: torch.Tensor) -> torch.Tensor:
    t = torch.clamp(0.7978845608 * (x + 0.044715 * x * x * x), -10.0, 10.0)
    return x * 0.5 * (1.0 + torch.tanh(t))


class TorchModel:
    """A whole model on the CPU: cfg is a gemma_hip GemmaConfig; tensors an
    iterable of (GGUF name, gemma_hip dtype code, array) as
    gemma_hip.synth_tensors yields them."""

    def __init__(self, cfg, tensors, max_seq: int | None = None):
        self.c = cfg
        self.max_seq = max_seq or cfg.max_seq
        self.zc = bool(cfg.flags & ZERO_CENTERED)
        ftz = not (cfg.flags & IEEE_SCALES)
        H, hd, nq, nkv, F = cfg.hidden, cfg.head_dim, cfg.n_heads, cfg.n_kv_heads, cfg.ffn
        shapes = {"attn_q": (nq * hd, H), "attn_k": (nkv * hd, H), "attn_v": (nkv * hd, H),
                  "attn_output": (H, nq * hd), "ffn_gate": (F, H), "ffn_up": (F, H), "ffn_down": (H, F)}
        self.t = {}
        for name, dtype, arr in tensors:
            kind = name.split(".")[-2] if name.startswith("blk.") else name.split(".")[0]
            if name in ("token_embd.weight", "output.weight"):
                rc = (cfg.vocab, H)
            elif kind in shapes:
                rc = shapes[kind]
            else:
                self.t[name] = torch.from_numpy(np.ascontiguousarray(arr, np.float32).copy())
                continue
            if dtype == 2:
                self.t[name] = q4_0_to_f32(arr, rc[0], rc[1], ftz)
            else:
                self.t[name] = torch.from_numpy(np.ascontiguousarray(arr, np.float32).reshape(rc).copy())
        self.kc = torch.zeros(cfg.n_layers, self.max_seq, nkv, hd)
        self.vc = torch.zeros(cfg.n_layers, self.max_seq, nkv, hd)
        half = hd // 2
        e = np.arange(half, dtype=np.float32) * np.float32(2) / np.float32(hd)
        self.inv_freq = {t: torch.from_numpy((np.float32(1) / np.power(np.float32(th), e, dtype=np.float32))
                                             .astype(np.float32))
                         for t, th in (("local", cfg.rope_theta_local), ("global", cfg.rope_theta_global))}

    def _rope(self, x: torch.Tensor, pos: int, which: str) -> torch.Tensor:
        half = x.shape[-1] // 2
        a = torch.tensor(float(pos), dtype=torch.float32) * self.inv_freq[which]
        c, s = torch.cos(a), torch.sin(a)
        x0, x1 = x[..., :half], x[..., half:]
        return torch.cat([x0 * c - x1 * s, x0 * s + x1 * c], dim=-1)

    def step(self, token: int, pos: int):
        """One decode step at position pos: (logits [vocab], argmax)."""
        c, T = self.c, self.t
        H, hd, nq, nkv = c.hidden, c.head_dim, c.n_heads, c.n_kv_heads
        G, eps, zc = nq // nkv, c.rms_eps, self.zc
        x = T["token_embd.weight"][token] * torch.sqrt(torch.tensor(float(H), dtype=torch.float32))
        for l in range(c.n_layers):
            p = f"blk.{l}."
            glob = c.global_every <= 0 or (l + 1) % c.global_every == 0
            pb, pe = 0, pos + 1
            if c.mode == MODE_REF:
                which = "global"
                if c.sliding_window > 0:
                    pe = min(pe, c.sliding_window)
            else:
                which = "global" if glob else "local"
                if not glob and c.sliding_window > 0:
                    pb = max(0, pe - c.sliding_window)
            xn = _norm(x, T[p + "attn_norm.weight"], eps, zc)
            q = (T[p + "attn_q.weight"] @ xn).view(nq, hd)
            k = (T[p + "attn_k.weight"] @ xn).view(nkv, hd)
            v = (T[p + "attn_v.weight"] @ xn).view(nkv, hd)
            if (c.flags & QK_NORM) and p + "attn_q_norm.weight" in T:
                q = torch.stack([_norm(q[h], T[p + "attn_q_norm.weight"], eps, zc) for h in range(nq)])
                k = torch.stack([_norm(k[h], T[p + "attn_k_norm.weight"], eps, zc) for h in range(nkv)])
            q, k = self._rope(q, pos, which), self._rope(k, pos, which)
            self.kc[l, pos], self.vc[l, pos] = k, v
            K, V = self.kc[l, pb:pe], self.vc[l, pb:pe]  # [n, nkv, hd]
            o = torch.empty(nq, hd)
            for h in range(nq):
                s = (K[:, h // G] @ q[h]) * (1.0 / float(np.sqrt(np.float32(hd))))
                pr = torch.softmax(s, dim=0)
                o[h] = pr @ V[:, h // G]
            a = T[p + "attn_output.weight"] @ o.reshape(-1)
            if (c.flags & POST_ATTN_NORM) and p + "post_attention_norm.weight" in T:
                a = _norm(a, T[p + "post_attention_norm.weight"], eps, zc)
            x1 = x + a
            wffn = T.get(p + "ffn_norm.weight", T.get(p + "post_attention_norm.weight"))
            n2 = _norm(x1, wffn, eps, zc)
            h_ = _gelu_tanh(T[p + "ffn_gate.weight"] @ n2) * (T[p + "ffn_up.weight"] @ n2)
            d = T[p + "ffn_down.weight"] @ h_
            if (c.flags & POST_FFN_NORM) and p + "post_ffw_norm.weight" in T:
                d = _norm(d, T[p + "post_ffw_norm.weight"], eps, zc)
            x = x1 + d
        xn = _norm(x, T["output_norm.weight"], eps, zc)
        # untied output.weight when present, else the tied embedding
        # (src/Gemma/Model.hs:412-414)
        logits = T.get("output.weight", T["token_embd.weight"]) @ xn
        return logits, int(torch.argmax(logits))
