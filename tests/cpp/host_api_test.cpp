// Checks of the C++ host API (gemma.hs_amd/host/Gemma.hpp) on the GPU
// against the C oracle (oracle/gemma_oracle.h), written the way the
// reference's own tests use its Haskell API (test/GemmaSpec.hs,
// test/Gemma/Layers/DequantQ4GGUFSpec.hs).  Built as a shared library by
// gemma.hs_amd/build.py; tests/test_gpu_host_api.py calls gh_host_api_tests
// in-process.  The oracle is the checker only.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <sstream>
#include <string>
#include <vector>

#include "Gemma.hpp"
#include "gemma_oracle.h"

namespace {

struct Failure {
    std::string what;
};

void require(bool ok, const std::string& what) {
    if (!ok) throw Failure{what};
}

double rel_err(const float* a, const float* b, size_t n) {
    double num = 0.0, den = 1e-30;
    for (size_t i = 0; i < n; ++i) {
        num = std::fmax(num, std::fabs((double)a[i] - (double)b[i]));
        den = std::fmax(den, std::fabs((double)b[i]));
    }
    return num / den;
}

// The tensors gh_synth_model uploads, in its order, with the same bytes
// (GGUF names; f32 norm vectors, f32 or Q4_0 matrices).
struct Tensor {
    std::string name;
    int dtype;
    std::vector<unsigned char> bytes;
};

std::vector<Tensor> synth_tensors(const gemma::GemmaConfig& c, uint64_t seed, bool q4) {
    const int H = c.hidden, hd = c.head_dim, F = c.ffn;
    struct Item {
        std::string name;
        bool mat;
        int rows, cols;
    };
    std::vector<Item> items = {{"token_embd.weight", true, c.vocab, H}, {"output_norm.weight", false, H, 1}};
    for (int l = 0; l < c.n_layers; ++l) {
        const std::string p = "blk." + std::to_string(l) + ".";
        std::vector<Item> layer = {{p + "attn_norm.weight", false, H, 1},
                                   {p + "attn_q.weight", true, c.n_heads * hd, H},
                                   {p + "attn_k.weight", true, c.n_kv_heads * hd, H},
                                   {p + "attn_v.weight", true, c.n_kv_heads * hd, H},
                                   {p + "attn_q_norm.weight", false, hd, 1},
                                   {p + "attn_k_norm.weight", false, hd, 1},
                                   {p + "attn_output.weight", true, H, c.n_heads * hd},
                                   {p + "post_attention_norm.weight", false, H, 1},
                                   {p + "ffn_norm.weight", false, H, 1},
                                   {p + "ffn_gate.weight", true, F, H},
                                   {p + "ffn_up.weight", true, F, H},
                                   {p + "ffn_down.weight", true, H, F},
                                   {p + "post_ffw_norm.weight", false, H, 1}};
        items.insert(items.end(), layer.begin(), layer.end());
    }
    std::vector<Tensor> out;
    for (const Item& it : items) {
        Tensor t{it.name, GH_DTYPE_F32, {}};
        if (it.mat && q4) {
            t.dtype = GH_DTYPE_Q4_0;
            t.bytes.resize((size_t)it.rows * (it.cols / 32) * 18);
            gemma::check(gh_synth_q4_0(seed, it.name.c_str(), 0.01f, it.rows, it.cols, t.bytes.data()));
        } else {
            const size_t n = (size_t)it.rows * it.cols;
            t.bytes.resize(n * sizeof(float));
            gemma::check(gh_synth_f32(seed, it.name.c_str(), it.mat ? 0.02f : 0.02f, (float*)t.bytes.data(), n));
        }
        out.push_back(std::move(t));
    }
    return out;
}

orc_model* oracle_model(const gemma::GemmaConfig& c, uint64_t seed, bool q4) {
    orc_config oc;
    static_assert(sizeof(oc) == sizeof(c), "orc_config and gh_config share their layout");
    std::memcpy(&oc, &c, sizeof(oc));
    orc_model* om = orc_model_create(&oc);
    require(om != nullptr, "orc_model_create");
    for (const Tensor& t : synth_tensors(c, seed, q4))
        require(orc_model_set_tensor(om, t.name.c_str(), t.dtype, t.bytes.data(), t.bytes.size()) == 0,
                "oracle set_tensor " + t.name);
    return om;
}

// top_k outside 0..64 is GH_ERR_RANGE
void threw_range(gemma::KVCache& kv) {
    bool threw = false;
    try {
        gemma::setSampling(kv, 1.0f, 0, 65);
    } catch (const gemma::GemmaError& e) {
        threw = e.code == GH_ERR_RANGE;
    }
    require(threw, "top_k 65: GH_ERR_RANGE");
}

// runGemmaInferenceCached / ...WithLayer0 step by step against the oracle:
// logits and every layer within 1e-4 relative, the argmax equal, the cache
// one position longer per step (test/GemmaSpec.hs:599-644 in spirit).
void steps_match_oracle(std::ostringstream& log, const gemma::Context& ctx, const char* preset, bool q4,
                        int n_prompt, int n_gen) {
    const gemma::GemmaConfig cfg = gemma::preset(preset);
    gemma::GemmaModel model(ctx, cfg);
    model.synth(7, q4);
    orc_model* om = oracle_model(cfg, 7, q4);
    std::vector<float> ologits(cfg.vocab), olayers((size_t)cfg.n_layers * cfg.hidden);
    std::vector<int> seq;
    for (int i = 0; i < n_prompt; ++i) seq.push_back((i * 131 + 17) % cfg.vocab);
    std::optional<gemma::KVCache> cache;
    for (int pos = 0; pos < n_prompt + n_gen - 1; ++pos) {
        const int tok = seq[pos];
        const int obest = orc_step(om, tok, pos, ologits.data(), olayers.data());
        require(obest >= 0, "oracle step");
        std::vector<float> logits, layer0;
        if (pos % 2 == 0) {
            auto [l, kv, l0] = gemma::runGemmaInferenceCachedWithLayer0(model, {tok}, cache);
            logits = std::move(l);
            layer0 = std::move(l0);
            cache = kv;
            require(rel_err(layer0.data(), olayers.data(), cfg.hidden) < 1e-4, "layer 0 at pos " + std::to_string(pos));
        } else {
            auto [l, kv] = gemma::runGemmaInferenceCached(model, {tok}, cache);
            logits = std::move(l);
            cache = kv;
        }
        require(rel_err(logits.data(), ologits.data(), cfg.vocab) < 1e-4, "logits at pos " + std::to_string(pos));
        require(gemma::sampleToken(logits) == obest, "argmax at pos " + std::to_string(pos));
        require(gemma::cacheLength(*cache) == pos + 1, "cacheLength at pos " + std::to_string(pos));
        if (pos + 1 >= n_prompt) seq.push_back(obest);
    }
    require(gemma::maxCacheSize(*cache) == gemma::defaultCacheSize, "fresh cache capacity");
    // generate on the device, prompt token by token and batched: the oracle's ids
    std::vector<int> prompt(seq.begin(), seq.begin() + n_prompt), want(seq.begin() + n_prompt, seq.end());
    gemma::KVCache kv1 = gemma::initKVCache(model, 64), kv2 = gemma::initKVCache(model, 64);
    const std::vector<int> ids = gemma::generate(model, kv1, prompt, (int)want.size());
    const std::vector<int> idp = gemma::generate(model, kv2, prompt, (int)want.size(), true);
    require(ids == want, "generate ids");
    require(idp == want, "generate ids after prefill");
    require(gemma::cacheLength(kv1) == n_prompt + (int)want.size() - 1, "cache length after generate");
    gemma::resetCache(kv1);
    require(gemma::cacheLength(kv1) == 0, "resetCache");
    // sampling extension: top-1 at any temperature is the greedy rule; a
    // seeded draw reproduces itself
    gemma::setSampling(kv1, 1.7f, 11, 1);
    require(gemma::generate(model, kv1, prompt, (int)want.size()) == want, "top-1 sampling = greedy ids");
    gemma::KVCache ka = gemma::initKVCache(model, 64), kb = gemma::initKVCache(model, 64);
    gemma::setSampling(ka, 1.3f, 5, 16);
    gemma::setSampling(kb, 1.3f, 5, 16);
    require(gemma::generate(model, ka, prompt, (int)want.size()) == gemma::generate(model, kb, prompt, (int)want.size()),
            "seeded top-k generation reproduces");
    threw_range(kv1);
    orc_model_destroy(om);
    log << preset << (q4 ? " q4" : " f32") << ": " << (n_prompt + n_gen - 1) << " steps, generate and prefill ok\n";
}

// The reference's error behaviour: more than one token is an error
// (src/Gemma/Model.hs:1321-1324); a full cache is GH_ERR_RANGE.
void errors(std::ostringstream& log, const gemma::Context& ctx) {
    gemma::GemmaModel model(ctx, gemma::preset("tiny"));
    model.synth(3, false);
    gemma::KVCache kv = gemma::initKVCache(model, 2);
    bool threw = false;
    try {
        gemma::runGemmaInferenceCached(model, {1, 2}, kv);
    } catch (const gemma::GemmaError& e) {
        threw = e.code == GH_ERR_INVALID && std::string(e.what()) == "Cached inference requires single token, got 2";
    }
    require(threw, "two tokens: error");
    require(gemma::cacheLength(kv) == 0, "cache unchanged after the error");
    gemma::runGemmaInferenceCached(model, {1}, kv);
    gemma::runGemmaInferenceCached(model, {2}, kv);
    threw = false;
    try {
        gemma::runGemmaInferenceCached(model, {3}, kv);
    } catch (const gemma::GemmaError& e) {
        threw = e.code == GH_ERR_RANGE;
    }
    require(threw, "full cache: GH_ERR_RANGE");
    log << "errors ok\n";
}

// runLinearQ4 (src/Gemma/Layers/LinearQ4.hs:41-48) on raw GGUF words against
// the oracle's Q4_0 matvec, with and without the soft-cap.
void linear_q4(std::ostringstream& log, const gemma::Context& ctx) {
    const int rows = 200, cols = 96;
    std::vector<unsigned char> raw((size_t)rows * (cols / 32) * 18);
    gemma::check(gh_synth_q4_0(11, "linear", 0.01f, rows, cols, raw.data()));
    std::vector<uint32_t> words((raw.size() + 3) / 4, 0u);
    std::memcpy(words.data(), raw.data(), raw.size());
    std::vector<float> x(cols);
    gemma::check(gh_synth_f32(11, "x", 1.0f, x.data(), x.size()));
    std::vector<float> want(rows);
    orc_q4_0_matvec(raw.data(), x.data(), rows, cols, 1, want.data());
    const std::vector<float> y = gemma::runLinearQ4(ctx, words, x, rows, cols, false, 30.0f);
    require(rel_err(y.data(), want.data(), rows) < 1e-5, "runLinearQ4");
    orc_softcap(want.data(), rows, 30.0f);
    const std::vector<float> yc = gemma::runLinearQ4(ctx, words, x, rows, cols, true, 30.0f);
    require(rel_err(yc.data(), want.data(), rows) < 1e-5, "runLinearQ4 with soft-cap");
    log << "runLinearQ4 ok\n";
}

}  // namespace

// 0 when every check passes; the log (or the failed check) goes to `log`.
extern "C" int gh_host_api_tests(char* log, int log_len) {
    std::ostringstream out;
    int rc = 0;
    try {
        gemma::Context ctx(0);
        errors(out, ctx);
        linear_q4(out, ctx);
        steps_match_oracle(out, ctx, "tiny", false, 6, 8);
        steps_match_oracle(out, ctx, "tiny", true, 5, 6);
    } catch (const Failure& f) {
        out << "FAILED: " << f.what << "\n";
        rc = 1;
    } catch (const gemma::GemmaError& e) {
        out << "FAILED with GemmaError " << e.code << ": " << e.what() << "\n";
        rc = 2;
    }
    std::snprintf(log, (size_t)log_len, "%s", out.str().c_str());
    return rc;
}
