"""Independent GGUF v3 reader for the tests (numpy, no library code).

It reads a file as the GGUF v3 format lays it out (src/Gemma/GGUF.hs:186-239):
magic, version, counts, metadata key/values, tensor infos (name, dims
innermost first, ggml type, offset) and the data section at the next
multiple of general.alignment.  The GPU test of gh_model_load_gguf feeds
what this returns to the oracle, so the loader is checked against a second
reading of the same bytes, not against the tensors that wrote the file.
"""
from __future__ import annotations

import struct

import numpy as np

GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q4_1 = 0, 1, 2, 3
_SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}


class GGUF:
    def __init__(self, path):
        self.buf = open(path, "rb").read()
        self.off = 0
        magic, version, n_t, n_kv = self._u("<IIQQ")
        if magic != 0x46554747 or version != 3:
            raise ValueError("not a GGUF v3 file")
        self.meta = {}
        for _ in range(n_kv):
            key = self._str()
            (t,) = self._u("<I")
            self.meta[key] = self._value(t)
        self.infos = {}
        for _ in range(n_t):
            name = self._str()
            (nd,) = self._u("<I")
            dims = list(self._u("<" + "Q" * nd)) if nd else []
            t, offset = self._u("<IQ")
            self.infos[name] = (dims, t, offset)
        align = int(self.meta.get("general.alignment", 32))
        self.data0 = (self.off + align - 1) // align * align

    def _u(self, fmt):
        v = struct.unpack_from(fmt, self.buf, self.off)
        self.off += struct.calcsize(fmt)
        return v

    def _str(self):
        (n,) = self._u("<Q")
        s = self.buf[self.off:self.off + n].decode()
        self.off += n
        return s

    def _value(self, t):
        if t == 8:
            return self._str()
        if t == 9:
            et, cnt = self._u("<IQ")
            return [self._value(et) for _ in range(cnt)]
        (v,) = self._u(_SCALAR[t])
        return v

    def tensor(self, name):
        """(dtype code as gh/orc take it: 0 f32, 1 f16, 2 Q4_0 raw bytes, array)."""
        dims, t, offset = self.infos[name]
        ne = int(np.prod(dims)) if dims else 1
        start = self.data0 + offset
        if t == GGML_F32:
            return 0, np.frombuffer(self.buf, np.float32, ne, start).copy()
        if t == GGML_F16:
            return 0, half_ftz(np.frombuffer(self.buf, np.uint16, ne, start))
        if t == GGML_Q4_0:
            return 2, np.frombuffer(self.buf, np.uint8, ne // 32 * 18, start).copy()
        if t == GGML_Q4_1:
            return 0, q4_1_dequant(np.frombuffer(self.buf, np.uint8, ne // 32 * 20, start))
        raise ValueError(f"ggml type {t}")


def half_ftz(h: np.ndarray) -> np.ndarray:
    """fp16 bit patterns to f32 with subnormals flushed to a signed zero, as
    halfToFloat (src/Gemma/GGUF.hs:797-820) decodes them."""
    h = np.asarray(h, np.uint16)
    f = h.view(np.float16).astype(np.float32)
    sub = ((h & 0x7C00) == 0) & ((h & 0x03FF) != 0)
    f[sub] = np.where(h[sub] & 0x8000, np.float32(-0.0), np.float32(0.0))
    return f


def q4_1_dequant(raw: np.ndarray) -> np.ndarray:
    """Q4_1 blocks to f32 in loadQ4_1Tensor's order (src/Gemma/GGUF.hs:762-795):
    element i of a block is code byte i // 2, low nibble for even i, high
    for odd i; value q * d + m, with d and m through half_ftz."""
    b = np.asarray(raw, np.uint8).reshape(-1, 20)
    d = half_ftz(b[:, 0:2].copy().view(np.uint16)[:, 0])
    m = half_ftz(b[:, 2:4].copy().view(np.uint16)[:, 0])
    codes = b[:, 4:]
    q = np.empty((b.shape[0], 32), np.float32)
    q[:, 0::2] = codes & 0x0F
    q[:, 1::2] = codes >> 4
    return (q * d[:, None] + m[:, None]).astype(np.float32).reshape(-1)
