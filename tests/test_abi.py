"""C-ABI checks that need no GPU: the library loads, exports every symbol
include/gemma_hip.h declares, host-only entry points (presets, synthetic
data, GGUF parsing) behave, and error codes are forced from the host."""
from __future__ import annotations

import re

import numpy as np
import pytest

import gemma_hip as gh
from conftest import REPO
from gguf_writer import gemma3_meta, synth_gguf, write_gguf

HEADER = REPO / "include" / "gemma_hip.h"


def declared_symbols():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(gh_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    L = gh.lib()
    syms = declared_symbols()
    assert len(syms) >= 40
    missing = [s for s in syms if not hasattr(L, s)]
    assert not missing, missing
    # and the Python binding declares a signature for each
    from gemma_hip._lib import SIGNATURES
    assert set(syms) <= set(SIGNATURES), set(syms) - set(SIGNATURES)


def test_version_and_presets():
    assert b"gfx950" in gh.lib().gh_version()
    c = gh.preset("gemma3-1b")
    assert (c.vocab, c.hidden, c.n_layers, c.n_heads, c.n_kv_heads, c.head_dim, c.ffn) == \
        (262144, 1152, 26, 4, 1, 256, 6912)
    assert (c.sliding_window, c.global_every, c.rope_theta_local, c.rope_theta_global) == (512, 6, 1e4, 1e6)
    t = gh.preset("tiny")
    assert (t.vocab, t.hidden, t.n_layers, t.n_heads, t.n_kv_heads, t.head_dim, t.ffn) == \
        (1024, 128, 2, 4, 1, 32, 512)
    f = gh.preset("gemma3-4b")
    assert (f.hidden, f.n_layers, f.n_heads, f.n_kv_heads, f.ffn, f.sliding_window) == (2560, 34, 8, 4, 10240, 1024)
    with pytest.raises(gh.GemmaHipError) as e:
        gh.preset("gemma3-27b")
    assert e.value.name == "GH_ERR_NOT_FOUND"


def test_synth_is_deterministic_and_distributed_as_specified():
    a = gh.synth_q4_0(1234, "blk.0.ffn_gate.weight", 0.01, 6912, 1152)
    b = gh.synth_q4_0(1234, "blk.0.ffn_gate.weight", 0.01, 6912, 1152)
    c = gh.synth_q4_0(1234, "blk.0.ffn_up.weight", 0.01, 6912, 1152)
    assert np.array_equal(a, b) and not np.array_equal(a, c)
    blk = a.reshape(-1, 18)
    scales = blk[:, :2].copy().view(np.float16).astype(np.float64).ravel()
    assert np.all(scales >= 0)
    # |N(0, 0.01)|: mean 0.01*sqrt(2/pi); fraction below the fp16 normal range ~0.49 %
    assert abs(scales.mean() - 0.01 * np.sqrt(2 / np.pi)) < 2e-4
    sub = np.mean((blk[:, 1] & 0x7C) == 0)
    assert 0.003 < sub < 0.007
    codes = np.concatenate([blk[:, 2:] & 15, blk[:, 2:] >> 4]).ravel()
    counts = np.bincount(codes, minlength=16) / codes.size
    assert np.all(np.abs(counts - 1 / 16) < 2e-3)
    x = gh.synth_f32(7, "w", 0.02, 200000)
    assert abs(x.std() - 0.02) < 5e-4 and abs(x.mean()) < 5e-4
    t = gh.synth_tokens(1, "prompt", 128, 262144)
    assert t.min() >= 0 and t.max() < 262144 and len(set(t.tolist())) > 120
    assert np.array_equal(t, gh.synth_tokens(1, "prompt", 128, 262144))


def test_synth_rounds_scales_to_nearest_even_fp16():
    """Scales are |N| values rounded to fp16 RNE: re-rounding the fp16 value
    through numpy is the identity and the distribution of the last bit is even."""
    a = gh.synth_q4_0(5, "s", 0.01, 2048, 1152).reshape(-1, 18)
    h = a[:, :2].copy().view(np.uint16).ravel()
    f = h.view(np.float16)
    assert np.array_equal(f.astype(np.float32).astype(np.float16).view(np.uint16), h)


def test_synth_rejects_bad_shapes():
    with pytest.raises(gh.GemmaHipError):
        gh.synth_q4_0(1, "x", 0.01, 4, 33)


def test_context_without_device_reports_hip_error():
    if gh.device_count() > 0:
        pytest.skip("a device is visible; this checks the no-device error path")
    with pytest.raises(gh.GemmaHipError) as e:
        gh.Context(0)
    assert e.value.name == "GH_ERR_HIP" and "no HIP device" in str(e.value)


def _inspect(path):
    import ctypes as C
    c = gh.GemmaConfig()
    gh._lib.check(gh.lib().gh_gguf_inspect(str(path).encode(), C.byref(c)))
    return c


def test_gguf_inspect_config_from_metadata(tmp_path):
    cfg = gh.preset("tiny")
    cfg.sliding_window = 7
    p = tmp_path / "tiny.gguf"
    synth_gguf(p, cfg, 3, q4=False)
    c = _inspect(p)
    assert (c.vocab, c.hidden, c.n_layers, c.n_heads, c.n_kv_heads, c.head_dim, c.ffn) == \
        (cfg.vocab, cfg.hidden, cfg.n_layers, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.ffn)
    # vocab from token_embd's shape, not the (8-entry) tokenizer array
    assert c.vocab == 1024 and c.sliding_window == 7 and c.global_every == 6
    assert c.rope_theta_global == cfg.rope_theta_global and c.rope_theta_local == 1e4


@pytest.mark.parametrize("bad", ["magic", "version", "truncated", "missing_meta", "missing_embd"])
def test_gguf_malformed_files_are_rejected(tmp_path, bad):
    cfg = gh.preset("tiny")
    cfg.n_layers = 1
    p = tmp_path / "bad.gguf"
    meta = gemma3_meta(cfg)
    emb = ("token_embd.weight", "f32", cfg.vocab, cfg.hidden, np.zeros(cfg.vocab * cfg.hidden, np.float32))
    tensors = [emb]
    kw = {}
    if bad == "magic":
        kw["magic"] = 0x12345678
    elif bad == "version":
        kw["version"] = 2
    elif bad == "truncated":
        kw["truncate"] = 40
    elif bad == "missing_meta":
        del meta["gemma3.block_count"]
    elif bad == "missing_embd":
        tensors = []
    write_gguf(p, meta, tensors, **kw)
    with pytest.raises(gh.GemmaHipError) as e:
        _inspect(p)
    want = "GH_ERR_NOT_FOUND" if bad == "missing_embd" else "GH_ERR_FORMAT"
    assert e.value.name == want, str(e.value)
    with pytest.raises(gh.GemmaHipError) as e:
        _inspect(tmp_path / "does-not-exist.gguf")
    assert e.value.name == "GH_ERR_NOT_FOUND"


def test_q4_1_reader_known_answers():
    """tests/gguf_reader.py's Q4_1 decode (the oracle side of the GGUF Q4_1
    load) on closed forms: d = 1, m = 0.5 and code byte j holding nibbles
    (2j mod 16, 2j+1 mod 16) give element i = (i mod 16) + 0.5 -- the
    reference's interleaved order (src/Gemma/GGUF.hs:762-795), which the
    split order of Q4_0 would read as 2j, 2j+16 -- and a subnormal d is
    flushed, leaving m."""
    from gguf_reader import q4_1_dequant, half_ftz
    blk = np.zeros((2, 20), np.uint8)
    blk[:, 0:2] = np.array([1.0], np.float16).view(np.uint8)
    blk[:, 2:4] = np.array([0.5], np.float16).view(np.uint8)
    j = np.arange(16)
    blk[:, 4:] = (((2 * j + 1) % 16) << 4) | ((2 * j) % 16)
    blk[1, 0:2] = np.array([0x0005], np.uint16).view(np.uint8)  # subnormal d
    got = q4_1_dequant(blk.reshape(-1)).reshape(2, 32)
    np.testing.assert_array_equal(got[0], (np.arange(32) % 16) + 0.5)
    np.testing.assert_array_equal(got[1], np.full(32, 0.5, np.float32))
    h = np.array([0x0001, 0x8200, 0x3C00, 0x0400, 0x7C00], np.uint16)
    f = half_ftz(h)
    assert f[0] == 0.0 and f[1] == 0.0 and np.signbit(f[1]) and f[2] == 1.0
    assert f[3] == np.float32(2.0 ** -14) and np.isinf(f[4])


def test_gguf_q4_1_tensors_parse_and_ragged_rows_are_rejected(tmp_path):
    """A Q4_1 token_embd is accepted by the parser (it is dequantised on
    load); a Q4_1 tensor whose rows are not whole 32-element blocks is
    GH_ERR_FORMAT."""
    from gguf_writer import random_q4_1
    cfg = gh.preset("tiny")
    p = tmp_path / "q41.gguf"
    synth_gguf(p, cfg, 3, q4=True, embd_q4_1=True, norms_f16=True)
    assert _inspect(p).vocab == cfg.vocab
    meta = gemma3_meta(cfg)
    bad = random_q4_1(4, 32, 1)
    write_gguf(p, meta, [("token_embd.weight", "f32", cfg.vocab, cfg.hidden, np.zeros(cfg.vocab * cfg.hidden, np.float32)),
                         ("blk.0.attn_q.weight", "q4_1", 4, 48, np.resize(bad, 4 * 48 // 32 * 20 + 20))])
    with pytest.raises(gh.GemmaHipError) as e:
        _inspect(p)
    assert e.value.name == "GH_ERR_FORMAT"


def test_tensor_list_matches_header_names():
    names = {n.split(".", 2)[-1] if n.startswith("blk.") else n for n, _, _ in gh.tensor_list(gh.preset("tiny"))}
    text = HEADER.read_text()
    for n in names:
        stem = n.replace(".weight", "")
        assert stem in text, n


def test_cpp_host_api_header_compiles_and_test_library_exports_its_entry(tmp_path):
    """gemma.hs_amd/host/Gemma.hpp (the C++ mirror of the reference's Haskell
    API over the C ABI) compiles on its own, and build() produced the host-API
    test library with its entry point (run on the GPU by
    tests/test_gpu_host_api.py)."""
    import shutil
    import subprocess
    cxx = shutil.which("g++") or "c++"
    src = tmp_path / "use.cpp"
    src.write_text('#include "Gemma.hpp"\n'
                   'int main() { gemma::GemmaConfig c = gemma::preset("tiny"); return c.vocab == 1024 ? 0 : 1; }\n')
    exe = tmp_path / "use"
    r = subprocess.run([cxx, "-std=c++17", "-Wall", "-Werror", f"-I{REPO / 'include'}",
                        f"-I{REPO / 'gemma.hs_amd' / 'host'}", str(src), "-o", str(exe),
                        f"-L{REPO / 'gemma.hs_amd' / 'gemma_hip'}", "-lgemma_hip",
                        f"-Wl,-rpath,{REPO / 'gemma.hs_amd' / 'gemma_hip'}", "-Wl,--allow-shlib-undefined"],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    import ctypes
    t = ctypes.CDLL(str(REPO / "tests" / "cpp" / "libhost_api_test.so"))
    assert hasattr(t, "gh_host_api_tests")


# ---------------------------------------------------------------- GGUF fuzzing
_FUZZ_DRIVER = r"""
import ctypes as C, sys, numpy as np
sys.path[:0] = [sys.argv[1], sys.argv[2]]
import gemma_hip as gh
path, n = sys.argv[3], int(sys.argv[4])
base = open(path, 'rb').read()
rng = np.random.default_rng(int(sys.argv[5]))
codes = {}
def inspect(blob):
    with open(path + '.m', 'wb') as f:
        f.write(blob)
    c = gh.GemmaConfig()
    rc = gh.lib().gh_gguf_inspect((path + '.m').encode(), C.byref(c))
    codes[rc] = codes.get(rc, 0) + 1
    return rc
# every truncation point of the header, metadata and tensor infos, then some in the data
hdr = int(sys.argv[6])
for cut in list(range(0, hdr + 40)) + list(range(hdr, len(base), max(1, (len(base) - hdr) // 64))):
    rc = inspect(base[:cut])
    assert rc != 0 or cut >= len(base), cut
# random corruption of bytes in the first 2 KB (1 to 8 bytes per trial)
for _ in range(n):
    b = bytearray(base)
    for _ in range(int(rng.integers(1, 9))):
        i = int(rng.integers(0, min(len(b), 2048)))
        b[i] = int(rng.integers(0, 256))
    inspect(bytes(b))
print(sorted(codes.items()))
"""


def _gguf_header_len(path) -> int:
    """Offset of the data section of a GGUF file written by write_gguf."""
    b = open(path, "rb").read()
    import struct
    n_t, n_kv = struct.unpack_from("<QQ", b, 8)
    off = 24

    def s(o):
        (k,) = struct.unpack_from("<Q", b, o)
        return o + 8 + k
    for _ in range(n_kv):
        off = s(off)
        (t,) = struct.unpack_from("<I", b, off)
        off += 4
        if t == 8:
            off = s(off)
        elif t == 9:
            et, cnt = struct.unpack_from("<IQ", b, off)
            off += 12
            for _ in range(cnt):
                off = s(off)
        else:
            off += 4
    for _ in range(n_t):
        off = s(off)
        (nd,) = struct.unpack_from("<I", b, off)
        off += 4 + 8 * nd + 4 + 8
    return off


def test_gguf_parser_survives_truncation_and_corruption(tmp_path):
    """Every truncation of the header/metadata/tensor-info region, and 400
    seeded random corruptions of the first 2 KB, return an error code or a
    config -- never a crash (run in a child process, so a crash fails the
    test instead of the session)."""
    import subprocess
    import sys
    cfg = gh.preset("tiny")
    cfg.n_layers = 1
    p = tmp_path / "tiny.gguf"
    synth_gguf(p, cfg, 3, q4=True)
    hdr = _gguf_header_len(p)
    r = subprocess.run([sys.executable, "-c", _FUZZ_DRIVER, str(REPO / "gemma.hs_amd"), str(REPO / "oracle"),
                        str(p), "400", "7", str(hdr)], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, (r.returncode, r.stdout[-2000:], r.stderr[-2000:])


def _raw_gguf(meta: bytes, n_kv: int, tinfo: bytes, n_t: int, data: bytes = b"") -> bytes:
    import struct
    b = struct.pack("<IIQQ", 0x46554747, 3, n_t, n_kv) + meta + tinfo
    b += b"\0" * ((-len(b)) % 32)
    return b + data


def _kv_u32(key: str, v: int) -> bytes:
    import struct
    k = key.encode()
    return struct.pack("<Q", len(k)) + k + struct.pack("<II", 4, v)


def _tensor(name: str, dims, ggml_type: int, offset: int) -> bytes:
    import struct
    n = name.encode()
    return (struct.pack("<Q", len(n)) + n + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
            + struct.pack("<IQ", ggml_type, offset))


def _gemma_meta_bytes():
    cfg = gh.preset("tiny")
    keys = {"gemma3.block_count": 1, "gemma3.embedding_length": cfg.hidden, "gemma3.feed_forward_length": cfg.ffn,
            "gemma3.attention.head_count": 4, "gemma3.attention.head_count_kv": 1,
            "gemma3.attention.key_length": 32}
    import struct
    b = b"".join(_kv_u32(k, v) for k, v in keys.items())
    k = b"gemma3.rope.freq_base"
    b += struct.pack("<Q", len(k)) + k + struct.pack("<If", 6, 10000.0)
    return b, len(keys) + 1


@pytest.mark.parametrize("case", ["huge_string", "array_count_overflow", "huge_offset", "offset_plus_size_wraps",
                                  "dims_product_overflows", "q4_row_not_block_multiple", "bad_alignment",
                                  "huge_alignment", "count_not_integer", "negative_count", "tensor_past_end"])
def test_gguf_malformed_sizes_are_format_errors(tmp_path, case):
    """Sizes and offsets taken from the file that would wrap a 64-bit bound
    check, or exceed the file, are GH_ERR_FORMAT (src/Gemma/GGUF.hs:186-239
    reads with bounds-checked ByteString slices)."""
    import struct
    meta, n_kv = _gemma_meta_bytes()
    H, V = 128, 1024
    emb_bytes = V * H // 32 * 18
    tinfo = _tensor("token_embd.weight", [H, V], 2, 0)
    n_t = 1
    data = b"\0" * emb_bytes
    if case == "huge_string":
        meta += struct.pack("<Q", 0xFFFFFFFFFFFFFFF0) + b"x"
        n_kv += 1
    elif case == "array_count_overflow":
        k = b"x.arr"
        meta += struct.pack("<Q", len(k)) + k + struct.pack("<IIQ", 9, 12, 0x2000000000000001)
        n_kv += 1
    elif case == "huge_offset":
        tinfo = _tensor("token_embd.weight", [H, V], 2, 0xFFFFFFFFFFFFFF00)
    elif case == "offset_plus_size_wraps":
        tinfo += _tensor("blk.0.attn_norm.weight", [1 << 40, 1 << 8], 0, 0xFFFFFFFFFFFF0000)
        n_t += 1
    elif case == "dims_product_overflows":
        tinfo += _tensor("blk.0.attn_q.weight", [1 << 33, 1 << 33, 1 << 33], 2, 0)
        n_t += 1
    elif case == "q4_row_not_block_multiple":
        tinfo += _tensor("blk.0.attn_q.weight", [48, 64], 2, 0)  # 3072 weights, rows of 48
        n_t += 1
    elif case == "bad_alignment":
        meta += _kv_u32("general.alignment", 3)
        n_kv += 1
    elif case == "huge_alignment":
        k = b"general.alignment"
        meta += struct.pack("<Q", len(k)) + k + struct.pack("<IQ", 10, 1 << 62)
        n_kv += 1
    elif case == "count_not_integer":
        k = b"gemma3.block_count"
        meta = meta.replace(_kv_u32("gemma3.block_count", 1), struct.pack("<Q", len(k)) + k + struct.pack("<If", 6, 1.5))
    elif case == "negative_count":
        k = b"gemma3.attention.head_count"
        meta = meta.replace(_kv_u32("gemma3.attention.head_count", 4), struct.pack("<Q", len(k)) + k + struct.pack("<Ii", 5, -4))
    elif case == "tensor_past_end":
        data = data[:-1]
    p = tmp_path / f"{case}.gguf"
    p.write_bytes(_raw_gguf(meta, n_kv, tinfo, n_t, data))
    with pytest.raises(gh.GemmaHipError) as e:
        _inspect(p)
    assert e.value.name == "GH_ERR_FORMAT", (case, str(e.value))
