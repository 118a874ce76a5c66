// Gemma.hpp -- C++ host API over libgemma_hip's C ABI (include/gemma_hip.h).
//
// The reference's host side is Haskell (src/Gemma/*.hs), and no GHC exists
// here.  This header mirrors that API in C++: the names, the argument
// meaning and the error behaviour, so that a C++ caller (or a test) reads
// like the reference:
//   Gemma.Model        loadGemmaModelFromGGUF, configFromGGUF,
//                      runGemmaInferenceCached, runGemmaInferenceCachedWithLayer0
//   Gemma.KVCache      KVCache, initKVCache, cacheLength, resetCache, maxCacheSize
//   Gemma.Layers.LinearQ4  runLinearQ4
//   app/Main.hs        sampleToken, the generate loop
// Where the reference calls `error`, these functions throw GemmaError (code
// and message from gh_last_error).  Header-only; link with -lgemma_hip.
#pragma once

#include <cstdint>
#include <memory>
#include <optional>
#include <stdexcept>
#include <string>
#include <tuple>
#include <utility>
#include <vector>

#include "gemma_hip.h"

namespace gemma {

// The `error` calls of the reference (e.g. src/Gemma/Model.hs:1321-1324).
struct GemmaError : std::runtime_error {
    int code;
    GemmaError(int c, const std::string& msg) : std::runtime_error(msg), code(c) {}
};

inline void check(int rc) {
    if (rc != GH_OK) throw GemmaError(rc, gh_last_error());
}

// GemmaConfig (src/Gemma/Model.hs:106-129): the C ABI's gh_config.
using GemmaConfig = gh_config;

inline GemmaConfig preset(const std::string& name) {
    GemmaConfig c{};
    check(gh_config_preset(name.c_str(), &c));
    return c;
}
// gemma3_1BConfig (src/Gemma/Model.hs:213-237)
inline GemmaConfig gemma3_1BConfig() { return preset("gemma3-1b"); }

// configFromGGUF (src/Gemma/Model.hs:843): the config from a GGUF file's
// metadata, vocab from the token_embd shape.
inline GemmaConfig configFromGGUF(const std::string& path) {
    GemmaConfig c{};
    check(gh_gguf_inspect(path.c_str(), &c));
    return c;
}

// The Dawn Context (createContext, src/Gemma/Model.hs:419): one device, one
// stream.  Destroying it releases it: models and caches made on it keep it
// alive until they are destroyed.
class Context {
  public:
    explicit Context(int device = 0) {
        gh_ctx* c = nullptr;
        check(gh_ctx_create(device, &c));
        h_.reset(c, [](gh_ctx* p) { gh_ctx_destroy(p); });
    }
    gh_ctx* get() const { return h_.get(); }
    std::shared_ptr<gh_ctx> handle() const { return h_; }
    // waitAll (src/Gemma/Model.hs:1432)
    void waitAll() const { check(gh_ctx_sync(h_.get())); }

  private:
    std::shared_ptr<gh_ctx> h_;
};

// GemmaModel (src/Gemma/Model.hs:243-257): device-resident weights.
class GemmaModel {
  public:
    GemmaModel(const Context& ctx, const GemmaConfig& cfg) : ctx_(ctx.handle()) {
        gh_model* m = nullptr;
        check(gh_model_create(ctx.get(), &cfg, &m));
        adopt(m);
    }
    // one named tensor (GGUF names: token_embd.weight, blk.N.attn_q.weight, ...)
    void setTensor(const std::string& name, int dtype, const void* data, size_t nbytes) {
        check(gh_model_set_tensor(h_.get(), name.c_str(), dtype, data, nbytes));
    }
    // seeded synthetic weights (the benchmark and test models)
    void synth(uint64_t seed, bool q4) { check(gh_synth_model(h_.get(), seed, q4 ? 1 : 0, 0.02f, 0.01f, 0.02f)); }
    const GemmaConfig& gmConfig() const { return cfg_; }
    gh_model* get() const { return h_.get(); }
    std::shared_ptr<gh_model> handle() const { return h_; }

  private:
    GemmaModel() = default;
    // members: the context share is declared first, so it is released last
    void adopt(gh_model* m) {
        h_.reset(m, [](gh_model* p) { gh_model_destroy(p); });
        check(gh_model_config(m, &cfg_));
    }
    std::shared_ptr<gh_ctx> ctx_;  // keeps the context alive while the model is
    std::shared_ptr<gh_model> h_;
    GemmaConfig cfg_{};
    friend GemmaModel loadGemmaModelFromGGUF(const Context&, const std::string&, int);
};

// loadGemmaModelFromGGUF (src/Gemma/Model.hs:908): every tensor of the file
// uploaded, Q4_0 repacked, the LM head tied to token_embd.
inline GemmaModel loadGemmaModelFromGGUF(const Context& ctx, const std::string& path, int maxSeq = 2048) {
    gh_model* m = nullptr;
    check(gh_model_load_gguf(ctx.get(), path.c_str(), maxSeq, &m));
    GemmaModel g;
    g.ctx_ = ctx.handle();
    g.adopt(m);
    return g;
}

// The capacity runGemmaInferenceCached gives a fresh cache
// (initKVCache ... 2048, src/Gemma/Model.hs:1328).
constexpr int defaultCacheSize = 2048;

// KVCache (src/Gemma/KVCache.hs:45-67).  The reference returns a new cache
// value from every step; here the K/V live on the device and a step updates
// them in place, so copies of a KVCache share one cache.
class KVCache {
  public:
    gh_kv* get() const { return h_.get(); }

  private:
    std::shared_ptr<gh_model> m_;  // the model outlives its caches (declared first: destroyed last)
    std::shared_ptr<gh_kv> h_;
    int max_len_ = 0;
    friend KVCache initKVCache(const GemmaModel&, int);
    friend int maxCacheSize(const KVCache&);
};

// initKVCache (src/Gemma/KVCache.hs:78-82): an empty cache for the model's
// layers, KV heads and head_dim, with maxSeqLen positions.
inline KVCache initKVCache(const GemmaModel& model, int maxSeqLen = defaultCacheSize) {
    gh_kv* kv = nullptr;
    check(gh_kv_create(model.get(), maxSeqLen, &kv));
    KVCache c;
    c.m_ = model.handle();
    c.h_.reset(kv, [](gh_kv* p) { gh_kv_destroy(p); });
    c.max_len_ = maxSeqLen;
    return c;
}

// maxCacheSize (src/Gemma/KVCache.hs:154-155): the cache's capacity.
inline int maxCacheSize(const KVCache& cache) { return cache.max_len_; }

// cacheLength (src/Gemma/KVCache.hs:146-147)
inline int cacheLength(const KVCache& cache) {
    int32_t n = 0;
    check(gh_kv_length(cache.get(), &n));
    return n;
}

// resetCache (src/Gemma/KVCache.hs:150-151): length 0 (all layers at once).
inline void resetCache(KVCache& cache) { check(gh_kv_reset(cache.get())); }

// Next-token rule of this cache's steps and generations; no reference
// counterpart (sampleWithTemperature is an argmax, app/Main.hs:492-507).
// temperature 0: the first maximum; > 0: a Philox draw (key seed, counter =
// position) from softmax(logits / temperature), over the topK largest logits
// in rank order when 1 <= topK <= 64 (0: all).
inline void setSampling(KVCache& cache, float temperature, uint64_t seed, int topK = 0) {
    check(gh_kv_set_sampling(cache.get(), temperature, seed));
    check(gh_kv_set_top_k(cache.get(), topK));
}

// runGemmaInferenceCached (src/Gemma/Model.hs:1313-1437): one token through
// the model at position cacheLength; returns the logits [vocab] and the
// cache, one position longer.  Like the reference: exactly one token, else
// an error; no cache means a fresh 2048-position one.
inline std::pair<std::vector<float>, KVCache> runGemmaInferenceCached(const GemmaModel& model,
                                                                     const std::vector<int>& tokenIds,
                                                                     std::optional<KVCache> mCache) {
    if (tokenIds.size() != 1)
        throw GemmaError(GH_ERR_INVALID, "Cached inference requires single token, got " + std::to_string(tokenIds.size()));
    KVCache cache = mCache ? *mCache : initKVCache(model, defaultCacheSize);
    std::vector<float> logits(model.gmConfig().vocab);
    int32_t next = 0;
    check(gh_step(model.get(), cache.get(), tokenIds[0], logits.data(), nullptr, &next));
    return {std::move(logits), cache};
}

// runGemmaInferenceCachedWithLayer0 (src/Gemma/Model.hs:1441-1444): also the
// hidden state after layer 0, the reference's per-layer parity hook.
inline std::tuple<std::vector<float>, KVCache, std::vector<float>> runGemmaInferenceCachedWithLayer0(
    const GemmaModel& model, const std::vector<int>& tokenIds, std::optional<KVCache> mCache) {
    if (tokenIds.size() != 1)
        throw GemmaError(GH_ERR_INVALID, "Cached inference requires single token, got " + std::to_string(tokenIds.size()));
    const GemmaConfig& c = model.gmConfig();
    KVCache cache = mCache ? *mCache : initKVCache(model, defaultCacheSize);
    std::vector<float> logits(c.vocab), layers((size_t)c.n_layers * c.hidden);
    int32_t next = 0;
    check(gh_step(model.get(), cache.get(), tokenIds[0], logits.data(), layers.data(), &next));
    layers.resize(c.hidden);  // layer 0
    return {std::move(logits), cache, std::move(layers)};
}

// Every layer's hidden state of the step (generalises the layer-0 hook).
inline std::tuple<std::vector<float>, std::vector<float>, int> stepWithLayers(const GemmaModel& model, int token,
                                                                              KVCache& cache) {
    const GemmaConfig& c = model.gmConfig();
    std::vector<float> logits(c.vocab), layers((size_t)c.n_layers * c.hidden);
    int32_t next = 0;
    check(gh_step(model.get(), cache.get(), token, logits.data(), layers.data(), &next));
    return {std::move(logits), std::move(layers), next};
}

// runLinearQ4 (src/Gemma/Layers/LinearQ4.hs:41-48): y = W x for raw GGUF
// Q4_0 bytes packed into 32-bit words; soft-cap sigma*tanh(y/sigma) when
// applySoftCap.
inline std::vector<float> runLinearQ4(const Context& ctx, const std::vector<uint32_t>& weights,
                                      const std::vector<float>& input, int nRows, int nCols, bool applySoftCap,
                                      float softCapSigma) {
    if ((int)input.size() != nCols) throw GemmaError(GH_ERR_INVALID, "runLinearQ4: input length != nCols");
    std::vector<float> y(nRows);
    check(gh_linear_q4(ctx.get(), weights.data(), weights.size(), input.data(), nRows, nCols, applySoftCap ? 1 : 0,
                       softCapSigma, y.data()));
    return y;
}

// sampleToken (app/Main.hs:488-507): the first maximum (V.maxIndex).
inline int sampleToken(const std::vector<float>& logits) {
    int best = 0;
    for (int i = 1; i < (int)logits.size(); ++i)
        if (logits[i] > logits[best]) best = i;
    return best;
}

// The generation loop of app/Main.hs:372-463 on the device: the prompt
// (token by token, or batched with prefill), then nGen ids.
inline std::vector<int> generate(const GemmaModel& model, KVCache& cache, const std::vector<int>& prompt, int nGen,
                                 bool prefill = false) {
    std::vector<int32_t> p(prompt.begin(), prompt.end()), ids(nGen);
    check(prefill ? gh_generate_prefill(model.get(), cache.get(), p.data(), (int32_t)p.size(), nGen, ids.data())
                  : gh_generate(model.get(), cache.get(), p.data(), (int32_t)p.size(), nGen, ids.data()));
    return std::vector<int>(ids.begin(), ids.end());
}

// Batched prefill of the prompt (replaces the token-by-token goPrompt loop,
// app/Main.hs:426-436): the last token's logits and next token.
inline std::pair<std::vector<float>, int> prefill(const GemmaModel& model, KVCache& cache,
                                                  const std::vector<int>& tokens) {
    std::vector<int32_t> t(tokens.begin(), tokens.end());
    std::vector<float> logits(model.gmConfig().vocab);
    int32_t next = 0;
    check(gh_prefill(model.get(), cache.get(), t.data(), (int32_t)t.size(), logits.data(), nullptr, &next));
    return {std::move(logits), next};
}

}  // namespace gemma
