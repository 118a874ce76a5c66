// GGUF v3 reader: configFromGGUF (src/Gemma/Model.hs:843-902) and
// loadGemmaModelFromGGUF (src/Gemma/Model.hs:908-1234), with the tensor
// format of src/Gemma/GGUF.hs:186-239 (header, metadata, tensor infos,
// aligned data section).  Differences from the reference, on purpose:
//  - vocab comes from the token_embd.weight shape (the reference reads the
//    tokenizer array it skipped while parsing and so always gets 256000);
//  - the Q4_0 projections and the LM head reach the device (the reference
//    uploads zero placeholders); the LM head is output.weight when the file
//    has one (src/Gemma/Model.hs:988), else the tied token_embd.weight.
// Q4_1 tensors are dequantised to f32 on load, as the reference's getTensor
// does for the embedding and the norms (src/Gemma/GGUF.hs:649-656,762-795).
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cmath>
#include <cstring>
#include <map>
#include <new>
#include <string>

#include "common.h"

using namespace gh;

namespace {

enum : uint32_t { GGML_F32 = 0, GGML_F16 = 1, GGML_Q4_0 = 2, GGML_Q4_1 = 3 };
// a tensor the loader dequantises to f32 before gh_model_set_tensor
constexpr int DT_Q4_1_HOST = 100;

struct Meta {
    uint32_t type = 0;
    double num = 0.0;  // numeric scalars
    std::string str;
    uint64_t arr_len = 0;
};

struct TInfo {
    std::vector<uint64_t> dims;
    uint32_t type = 0;
    uint64_t offset = 0;
};

// Every size and offset below comes from the file, so each bound check is
// written so that it cannot wrap: remaining bytes are n - off (off <= n
// always holds), and products of file values go through mul_ok.
bool mul_ok(uint64_t a, uint64_t b, uint64_t* out) { return !__builtin_mul_overflow(a, b, out); }

struct Reader {
    const uint8_t* p;
    size_t n, off = 0;
    bool ok = true;
    bool need(uint64_t k) {
        if (!ok || k > (uint64_t)(n - off)) ok = false;
        return ok;
    }
    template <class T>
    T get() {
        T v{};
        if (need(sizeof(T))) {
            std::memcpy(&v, p + off, sizeof(T));
            off += sizeof(T);
        }
        return v;
    }
    std::string str() {
        uint64_t len = get<uint64_t>();
        if (!need(len)) return {};
        std::string s((const char*)p + off, (size_t)len);
        off += len;
        return s;
    }
};

size_t scalar_size(uint32_t t) {
    switch (t) {
        case 0: case 1: case 7: return 1;
        case 2: case 3: return 2;
        case 4: case 5: case 6: return 4;
        case 10: case 11: case 12: return 8;
        default: return 0;
    }
}

double scalar_value(Reader& r, uint32_t t) {
    switch (t) {
        case 0: return r.get<uint8_t>();
        case 1: return r.get<int8_t>();
        case 2: return r.get<uint16_t>();
        case 3: return r.get<int16_t>();
        case 4: return r.get<uint32_t>();
        case 5: return r.get<int32_t>();
        case 6: return r.get<float>();
        case 7: return r.get<uint8_t>();
        case 10: return (double)r.get<uint64_t>();
        case 11: return (double)r.get<int64_t>();
        case 12: return r.get<double>();
        default: r.ok = false; return 0;
    }
}

bool read_value(Reader& r, uint32_t t, Meta& m) {
    m.type = t;
    if (t == 8) {
        m.str = r.str();
    } else if (t == 9) {
        uint32_t et = r.get<uint32_t>();
        uint64_t cnt = r.get<uint64_t>();
        m.arr_len = cnt;
        if (et == 8) {
            for (uint64_t i = 0; i < cnt && r.ok; ++i) r.str();
        } else if (et == 9) {
            return false;  // nested arrays are not used by GGUF models
        } else {
            const uint64_t es = scalar_size(et);
            uint64_t bytes = 0;
            if (!es || !mul_ok(es, cnt, &bytes) || !r.need(bytes)) return false;
            r.off += bytes;
        }
    } else {
        m.num = scalar_value(r, t);
    }
    return r.ok;
}

struct Mapped {
    void* p = MAP_FAILED;
    size_t n = 0;
    int fd = -1;
    ~Mapped() {
        if (p != MAP_FAILED) munmap(p, n);
        if (fd >= 0) close(fd);
    }
};

struct TData {
    int dtype;
    uint64_t off;    // from the start of the file
    uint64_t bytes;  // off + bytes <= file size
};

struct Parsed {
    Mapped mp;
    std::map<std::string, Meta> meta;
    std::map<std::string, TInfo> tens;
    std::map<std::string, TData> data;  // validated extent and dtype of every tensor
    uint64_t data0 = 0;
    gh_config cfg{};
};

// dtype and byte size of a tensor, with overflow-checked products; Q4_0
// rows (the innermost dimension) must hold whole 32-weight blocks.
int tensor_bytes(const std::string& name, const TInfo& ti, int* dtype, uint64_t* bytes) {
    uint64_t ne = 1;
    for (uint64_t d : ti.dims)
        if (d == 0 || d > (1ull << 40) || !mul_ok(ne, d, &ne) || ne > (1ull << 48))
            return set_error(GH_ERR_FORMAT, "tensor '%s' has an implausible shape", name.c_str());
    if (ti.type == GGML_F32) {
        *dtype = GH_DTYPE_F32;
        *bytes = ne * 4;
    } else if (ti.type == GGML_F16) {
        *dtype = GH_DTYPE_F16;
        *bytes = ne * 2;
    } else if (ti.type == GGML_Q4_0) {
        if (ti.dims.empty() || ti.dims[0] % 32)
            return set_error(GH_ERR_FORMAT, "Q4_0 tensor '%s': row length not a multiple of 32", name.c_str());
        *dtype = GH_DTYPE_Q4_0;
        *bytes = ne / 32 * 18;
    } else if (ti.type == GGML_Q4_1) {
        if (ti.dims.empty() || ti.dims[0] % 32)
            return set_error(GH_ERR_FORMAT, "Q4_1 tensor '%s': row length not a multiple of 32", name.c_str());
        *dtype = DT_Q4_1_HOST;
        *bytes = ne / 32 * 20;
    } else {
        return set_error(GH_ERR_FORMAT, "tensor '%s' has unsupported ggml type %u", name.c_str(), ti.type);
    }
    return GH_OK;
}

// Parse header, metadata and tensor infos; build the config (configFromGGUF).
int parse_gguf(const char* path, int32_t max_seq, Parsed& P) {
    Mapped& mp = P.mp;
    mp.fd = open(path, O_RDONLY);
    if (mp.fd < 0) return set_error(GH_ERR_NOT_FOUND, "cannot open '%s'", path);
    struct stat stt;
    if (fstat(mp.fd, &stt) != 0 || stt.st_size < 24) return set_error(GH_ERR_FORMAT, "'%s' is too small for GGUF", path);
    mp.n = (size_t)stt.st_size;
    mp.p = mmap(nullptr, mp.n, PROT_READ, MAP_PRIVATE, mp.fd, 0);
    if (mp.p == MAP_FAILED) return set_error(GH_ERR_FORMAT, "mmap of '%s' failed", path);
    Reader r{(const uint8_t*)mp.p, mp.n};
    // src/Gemma/GGUF.hs:244-265: magic 0x46554747, version 3
    const uint32_t magic = r.get<uint32_t>(), version = r.get<uint32_t>();
    if (magic != 0x46554747u) return set_error(GH_ERR_FORMAT, "invalid GGUF magic 0x%08x", magic);
    if (version != 3) return set_error(GH_ERR_FORMAT, "unsupported GGUF version %u (only 3)", version);
    const uint64_t n_tensors = r.get<uint64_t>(), n_kv = r.get<uint64_t>();
    if (n_tensors > (1u << 20) || n_kv > (1u << 20)) return set_error(GH_ERR_FORMAT, "implausible GGUF counts");
    for (uint64_t i = 0; i < n_kv; ++i) {
        std::string key = r.str();
        uint32_t t = r.get<uint32_t>();
        Meta m;
        if (!r.ok || !read_value(r, t, m)) return set_error(GH_ERR_FORMAT, "truncated GGUF metadata at '%s'", key.c_str());
        P.meta[key] = m;
    }
    for (uint64_t i = 0; i < n_tensors; ++i) {
        std::string name = r.str();
        TInfo ti;
        uint32_t nd = r.get<uint32_t>();
        if (nd > 4) return set_error(GH_ERR_FORMAT, "tensor '%s' has %u dims", name.c_str(), nd);
        for (uint32_t d = 0; d < nd; ++d) ti.dims.push_back(r.get<uint64_t>());
        ti.type = r.get<uint32_t>();
        ti.offset = r.get<uint64_t>();
        if (!r.ok) return set_error(GH_ERR_FORMAT, "truncated GGUF tensor infos");
        P.tens[name] = ti;
    }
    uint64_t align = 32;
    auto ia = P.meta.find("general.alignment");
    if (ia != P.meta.end()) {
        const double a = ia->second.num;
        if (!(a >= 1 && a <= (1 << 20)) || ((uint64_t)a & ((uint64_t)a - 1)))
            return set_error(GH_ERR_FORMAT, "general.alignment %g is not a power of two up to 2^20", a);
        align = (uint64_t)a;
    }
    P.data0 = (r.off + align - 1) / align * align;
    if (P.data0 > mp.n) return set_error(GH_ERR_FORMAT, "GGUF data section starts past the end of the file");
    for (auto& kvp : P.tens) {
        TData td{};
        GH_CHECK(tensor_bytes(kvp.first, kvp.second, &td.dtype, &td.bytes));
        const uint64_t room = mp.n - P.data0;
        if (kvp.second.offset > room || td.bytes > room - kvp.second.offset)
            return set_error(GH_ERR_FORMAT, "tensor '%s' extends past the end of the file", kvp.first.c_str());
        td.off = P.data0 + kvp.second.offset;
        P.data[kvp.first] = td;
    }

    auto num = [&](const char* key, bool required, double def, double& v) -> int {
        auto it = P.meta.find(key);
        if (it == P.meta.end() || it->second.type == 8 || it->second.type == 9) {
            if (required) return set_error(GH_ERR_FORMAT, "missing or invalid metadata: %s", key);
            v = def;
            return GH_OK;
        }
        v = it->second.num;
        return GH_OK;
    };
    // integer fields: whole numbers in [0, 2^30] (gh_model_create checks the rest)
    auto count = [&](const char* key, bool required, double def, int& out) -> int {
        double v = 0;
        GH_CHECK(num(key, required, def, v));
        if (!(v >= 0 && v <= (double)(1 << 30)) || v != (double)(int64_t)v)
            return set_error(GH_ERR_FORMAT, "metadata %s = %g is not a count", key, v);
        out = (int)v;
        return GH_OK;
    };
    gh_config& c = P.cfg;
    double v;
    GH_CHECK(count("gemma3.block_count", true, 0, c.n_layers));
    GH_CHECK(count("gemma3.embedding_length", true, 0, c.hidden));
    GH_CHECK(count("gemma3.feed_forward_length", true, 0, c.ffn));
    GH_CHECK(count("gemma3.attention.head_count", true, 0, c.n_heads));
    GH_CHECK(count("gemma3.attention.head_count_kv", true, 0, c.n_kv_heads));
    GH_CHECK(count("gemma3.attention.key_length", true, 0, c.head_dim));
    GH_CHECK(num("gemma3.rope.freq_base", true, 0, v)); c.rope_theta_global = (float)v;
    GH_CHECK(count("gemma3.attention.sliding_window", false, 512, c.sliding_window));
    GH_CHECK(num("gemma3.attention.layer_norm_rms_epsilon", false, 1e-6, v)); c.rms_eps = (float)v;
    if (!(c.rope_theta_global > 0.0f) || !(c.rms_eps > 0.0f) || !std::isfinite(c.rope_theta_global))
        return set_error(GH_ERR_FORMAT, "rope.freq_base and layer_norm_rms_epsilon must be positive");
    c.rope_theta_local = 10000.0f;
    c.global_every = 6;
    c.mode = GH_MODE_GEMMA3;
    c.flags = GH_FLAG_QK_NORM | GH_FLAG_POST_ATTN_NORM | GH_FLAG_POST_FFN_NORM | GH_FLAG_ZERO_CENTERED;
    c.max_seq = max_seq > 0 ? max_seq : 2048;
    auto te = P.tens.find("token_embd.weight");
    if (te == P.tens.end() || te->second.dims.size() != 2)
        return set_error(GH_ERR_NOT_FOUND, "missing tensor token_embd.weight");
    if (te->second.dims[1] > (1u << 30)) return set_error(GH_ERR_FORMAT, "token_embd.weight has too many rows");
    c.vocab = (int)te->second.dims[1];
    if ((int64_t)te->second.dims[0] != c.hidden)
        return set_error(GH_ERR_FORMAT, "token_embd.weight width %llu != embedding_length %d",
                         (unsigned long long)te->second.dims[0], c.hidden);
    auto ow = P.tens.find("output.weight");
    if (ow != P.tens.end() && (ow->second.dims.size() != 2 || (int64_t)ow->second.dims[0] != c.hidden ||
                               (int64_t)ow->second.dims[1] != c.vocab))
        return set_error(GH_ERR_FORMAT, "output.weight is not %d x %d, the shape of token_embd.weight", c.vocab,
                         c.hidden);
    return GH_OK;
}

// parse_gguf behind a catch: an allocation failure (a huge metadata string
// or count that passes the bounds checks on a huge file) must not unwind
// through the C ABI
int parse_safe(const char* path, int32_t max_seq, Parsed& P) {
    try {
        return parse_gguf(path, max_seq, P);
    } catch (const std::bad_alloc&) {
        return set_error(GH_ERR_OOM, "out of host memory while parsing '%s'", path);
    } catch (...) {
        return set_error(GH_ERR_FORMAT, "malformed GGUF file '%s'", path);
    }
}

// Q4_1 blocks (fp16 d, fp16 m, 16 code bytes) to f32 as loadQ4_1Tensor
// (src/Gemma/GGUF.hs:762-795) computes them: element i of a block is the low
// nibble of code byte i/2 for even i and the high nibble for odd i (not the
// split order of Q4_0), value q*d + m, with d and m through halfToFloat
// (subnormals flushed to zero unless ieee).
void q4_1_to_f32(const uint8_t* src, uint64_t n_blocks, bool ieee, float* out) {
    for (uint64_t b = 0; b < n_blocks; ++b) {
        const uint8_t* blk = src + b * 20;
        uint16_t hd, hm;
        std::memcpy(&hd, blk, 2);
        std::memcpy(&hm, blk + 2, 2);
        const float d = f16_to_f32(hd, !ieee), m = f16_to_f32(hm, !ieee);
        for (int i = 0; i < 32; ++i) {
            const uint8_t byte = blk[4 + i / 2];
            const int q = (i & 1) ? byte >> 4 : byte & 0x0F;
            out[b * 32 + i] = (float)q * d + m;  // q*d is exact in f32
        }
    }
}

}  // namespace

extern "C" int gh_gguf_inspect(const char* path, gh_config* out) {
    if (!path || !out) return set_error(GH_ERR_INVALID, "null argument");
    Parsed P;
    GH_CHECK(parse_safe(path, 0, P));
    *out = P.cfg;
    return GH_OK;
}

extern "C" int gh_model_load_gguf(gh_ctx* ctx, const char* path, int32_t max_seq, gh_model** out) {
    if (!ctx || !path || !out) return set_error(GH_ERR_INVALID, "null argument");
    Parsed P;
    GH_CHECK(parse_safe(path, max_seq, P));
    gh_model* m = nullptr;
    GH_CHECK(gh_model_create(ctx, &P.cfg, &m));
    for (auto& kvp : P.data) {
        const std::string& name = kvp.first;
        const TData& td = kvp.second;  // extent checked against the file by parse_gguf
        const uint8_t* src = (const uint8_t*)P.mp.p + td.off;
        int rc;
        if (td.dtype == DT_Q4_1_HOST) {
            std::vector<float> f32;
            try {
                f32.resize(td.bytes / 20 * 32);
            } catch (const std::bad_alloc&) {
                gh_model_destroy(m);
                return set_error(GH_ERR_OOM, "out of host memory dequantising '%s'", name.c_str());
            }
            q4_1_to_f32(src, td.bytes / 20, (P.cfg.flags & GH_FLAG_IEEE_SCALES) != 0, f32.data());
            rc = gh_model_set_tensor(m, name.c_str(), GH_DTYPE_F32, f32.data(), f32.size() * 4);
        } else {
            rc = gh_model_set_tensor(m, name.c_str(), td.dtype, src, td.bytes);
        }
        if (rc == GH_ERR_NOT_FOUND) continue;  // tensors the decode step does not use (e.g. rope_freqs)
        if (rc != GH_OK) {
            gh_model_destroy(m);
            return rc;
        }
    }
    int rc = gh_model_check(m);
    if (rc != GH_OK) {
        gh_model_destroy(m);
        return rc;
    }
    *out = m;
    return GH_OK;
}
