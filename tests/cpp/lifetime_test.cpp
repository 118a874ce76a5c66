// Lifetime checks of libgemma_hip's C ABI on the CPU, linked against
// hip_stub.cpp / kernel_stub.cpp and built with AddressSanitizer by
// tests/test_lifetime.py.
//
//   lifetime_test          every destroy order of context, model, cache and
//                          Q4_0 tensor is free of use-after-free and leaks;
//                          a model and its cache keep working after their
//                          context's destroy; a second destroy, or a call on
//                          a destroyed or never-created handle, is
//                          GH_ERR_STATE
//   lifetime_test exit     only the order in which Python finalisers ran at
//                          interpreter exit when a model outlived its
//                          context (context first, then model, then cache)
//   lifetime_test race     one thread steps (and takes a greedy sample)
//                          while another creates and destroys caches, Q4_0
//                          tensors and models on the same context, as a
//                          garbage collector's finaliser thread does; a
//                          watchdog fails the run if the two deadlock
#include <atomic>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <thread>
#include <vector>

#include "gemma_hip.h"

#define CHECK(c)                                                                                   \
    do {                                                                                           \
        if (!(c)) {                                                                                \
            std::fprintf(stderr, "FAIL %s:%d: %s (last error: %s)\n", __FILE__, __LINE__, #c,     \
                         gh_last_error());                                                         \
            return 1;                                                                              \
        }                                                                                          \
    } while (0)

namespace {

struct Handles {
    gh_ctx* ctx = nullptr;
    gh_model* m = nullptr;
    gh_kv* kv = nullptr;
    gh_q4* t = nullptr;
};

int make(Handles& h) {
    CHECK(gh_ctx_create(0, &h.ctx) == GH_OK);
    gh_config c;
    CHECK(gh_config_preset("tiny", &c) == GH_OK);
    CHECK(gh_model_create(h.ctx, &c, &h.m) == GH_OK);
    CHECK(gh_synth_model(h.m, 7, 1, 0.02f, 0.01f, 0.02f) == GH_OK);
    CHECK(gh_kv_create(h.m, 16, &h.kv) == GH_OK);
    std::vector<uint8_t> raw(64 * 18, 0);
    CHECK(gh_q4_0_upload(h.ctx, raw.data(), 64, 32, 0, &h.t) == GH_OK);
    int32_t next = -1;
    CHECK(gh_step(h.m, h.kv, 3, nullptr, nullptr, &next) == GH_OK);
    return 0;
}

int destroy(Handles& h, char what) {
    switch (what) {
        case 'c': return gh_ctx_destroy(h.ctx);
        case 'm': return gh_model_destroy(h.m);
        case 'k': return gh_kv_destroy(h.kv);
        default: return gh_q4_0_free(h.t);
    }
}

int any_order() {
    const char* orders[] = {"cmkt", "ckmt", "mckt", "mkct", "kcmt", "kmct", "tcmk", "ctkm"};
    for (const char* order : orders) {
        Handles h;
        if (make(h)) return 1;
        for (const char* p = order; *p; ++p) {
            CHECK(destroy(h, *p) == GH_OK);
            const bool model_open = !std::strchr(order, 'm') || std::strchr(p + 1, 'm');
            const bool kv_open = std::strchr(p + 1, 'k') != nullptr;
            if (*p == 'c' && model_open && kv_open) {
                // the context is released, not freed: its model still steps
                int32_t next = -1;
                CHECK(gh_step(h.m, h.kv, 5, nullptr, nullptr, &next) == GH_OK);
            }
            if (*p == 'm' && kv_open) {
                int32_t next = -1;
                CHECK(gh_step(h.m, h.kv, 5, nullptr, nullptr, &next) == GH_ERR_STATE);
                int32_t len = -1;
                CHECK(gh_kv_length(h.kv, &len) == GH_OK && len >= 1);
            }
        }
        for (char w : {'c', 'm', 'k', 't'}) CHECK(destroy(h, w) == GH_ERR_STATE);
    }
    // gh_kv_truncate rewinds within [0, length]; gh_model_plan reports the
    // step's plan (graph mode, five phases, the tied head) and its length
    {
        Handles h;
        if (make(h)) return 1;
        char plan[512];
        size_t n = 0;
        CHECK(gh_model_plan(h.m, plan, sizeof plan, &n) == GH_OK && n > 0 && n < sizeof plan);
        CHECK(std::strncmp(plan, "step=", 5) == 0 && std::strstr(plan, " gate_up=S") && std::strstr(plan, " lm=tied") &&
              std::strstr(plan, " env="));
        char small[8];
        size_t n2 = 0;
        CHECK(gh_model_plan(h.m, small, sizeof small, &n2) == GH_OK && n2 == n && std::strlen(small) == 7);
        CHECK(gh_model_plan(h.m, nullptr, 4, &n2) == GH_ERR_INVALID);
        int32_t len = -1;
        CHECK(gh_kv_truncate(h.kv, 2) == GH_ERR_RANGE);
        CHECK(gh_kv_truncate(h.kv, -1) == GH_ERR_RANGE);
        CHECK(gh_kv_truncate(h.kv, 0) == GH_OK && gh_kv_length(h.kv, &len) == GH_OK && len == 0);
        for (char w : {'k', 'm', 't', 'c'}) CHECK(destroy(h, w) == GH_OK);
    }
    // handles that were never returned by the library
    int local = 0;
    CHECK(gh_model_destroy(reinterpret_cast<gh_model*>(&local)) == GH_ERR_STATE);
    CHECK(gh_kv_length(reinterpret_cast<gh_kv*>(&local), &local) == GH_ERR_STATE);
    CHECK(gh_ctx_sync(reinterpret_cast<gh_ctx*>(&local)) == GH_ERR_STATE);
    // a handle of the wrong kind
    Handles h;
    if (make(h)) return 1;
    CHECK(gh_kv_destroy(reinterpret_cast<gh_kv*>(h.m)) == GH_ERR_STATE);
    gh_kv_release(h.kv);
    gh_model_release(h.m);
    gh_q4_0_release(h.t);
    gh_ctx_release(h.ctx);
    gh_ctx_release(h.ctx);  // void: a second release is ignored
    return 0;
}

// Concurrent use and destruction on one context (finalisers run on their
// own thread under a -threaded RTS, gemma.cabal:102).
int race() {
    Handles h;
    if (make(h)) return 1;
    void* buf = nullptr;
    CHECK(gh_buf_alloc(h.ctx, 1024 * sizeof(float), &buf) == GH_OK);
    std::atomic<bool> done{false};
    std::atomic<int> failed{0};
    std::thread watchdog([&] {
        for (int i = 0; i < 600 && !done.load(); ++i) std::this_thread::sleep_for(std::chrono::milliseconds(100));
        if (!done.load()) {
            std::fprintf(stderr, "DEADLOCK: stepping and destroying threads did not finish in 60 s\n");
            std::fflush(stderr);
            std::_Exit(3);
        }
    });
    const int iters = 300;
    std::thread stepper([&] {
        for (int i = 0; i < iters; ++i) {
            int32_t next = -1, tok = -1, len = -1;
            if (gh_kv_truncate(h.kv, 0) != GH_OK) failed = 1;
            if (gh_step(h.m, h.kv, (i * 7) % 1024, nullptr, nullptr, &next) != GH_OK) failed = 2;
            if (gh_sample_logits(h.ctx, (const float*)buf, 1024, 0.0f, 1, 0, &tok) != GH_OK) failed = 3;
            if (gh_kv_length(h.kv, &len) != GH_OK || len != 1) failed = 4;
        }
    });
    std::thread finaliser([&] {
        gh_config c;
        if (gh_config_preset("tiny", &c) != GH_OK) failed = 10;
        std::vector<uint8_t> raw(64 * 18, 0);
        for (int i = 0; i < iters; ++i) {
            gh_kv* kv2 = nullptr;
            if (gh_kv_create(h.m, 8, &kv2) != GH_OK) failed = 11;
            gh_q4* t2 = nullptr;
            if (gh_q4_0_upload(h.ctx, raw.data(), 64, 32, 0, &t2) != GH_OK) failed = 12;
            gh_kv_release(kv2);
            gh_q4_0_release(t2);
            if (i % 30 == 0) {
                gh_model* m2 = nullptr;
                if (gh_model_create(h.ctx, &c, &m2) != GH_OK) failed = 13;
                gh_kv* kv3 = nullptr;
                if (gh_kv_create(m2, 4, &kv3) != GH_OK) failed = 14;
                gh_model_release(m2);  // released first: freed with its cache
                gh_kv_release(kv3);
            }
        }
    });
    stepper.join();
    finaliser.join();
    done = true;
    watchdog.join();
    CHECK(failed.load() == 0);
    CHECK(gh_buf_free(h.ctx, buf) == GH_OK);
    for (char w : {'t', 'c', 'k', 'm'}) CHECK(destroy(h, w) == GH_OK);
    return 0;
}

// gh_model_create rejects configurations the kernels do not support, and
// creates nothing for them.
int config_checks() {
    gh_ctx* ctx = nullptr;
    CHECK(gh_ctx_create(0, &ctx) == GH_OK);
    gh_config base;
    CHECK(gh_config_preset("gemma3-4b", &base) == GH_OK);
    gh_model* m = nullptr;
    CHECK(gh_model_create(ctx, &base, &m) == GH_OK && m);
    CHECK(gh_model_destroy(m) == GH_OK);
    auto rejects = [&](void (*edit)(gh_config&)) {
        gh_config c = base;
        edit(c);
        gh_model* bad = nullptr;
        return gh_model_create(ctx, &c, &bad) == GH_ERR_INVALID && bad == nullptr;
    };
    CHECK(rejects([](gh_config& c) { c.hidden = 3104; }));
    CHECK(rejects([](gh_config& c) { c.hidden = 1000; }));
    CHECK(rejects([](gh_config& c) { c.head_dim = 64; }));
    CHECK(rejects([](gh_config& c) { c.n_kv_heads = 3; }));
    CHECK(rejects([](gh_config& c) { c.n_heads = 48; }));  // group 12
    CHECK(rejects([](gh_config& c) { c.sliding_window = -1; }));
    CHECK(rejects([](gh_config& c) { c.global_every = -6; }));
    CHECK(rejects([](gh_config& c) { c.rope_theta_local = 0.0f; }));
    CHECK(rejects([](gh_config& c) { c.rope_theta_global = -1e6f; }));
    CHECK(rejects([](gh_config& c) { c.rope_theta_global = 1.0f / 0.0f; }));
    CHECK(rejects([](gh_config& c) { c.rms_eps = -1e-6f; }));
    CHECK(rejects([](gh_config& c) { c.rms_eps = 0.0f / 0.0f; }));
    CHECK(rejects([](gh_config& c) { c.mode = 7; }));
    CHECK(rejects([](gh_config& c) { c.max_seq = 0; }));
    gh_config wide = base;
    wide.hidden = 3072;
    CHECK(gh_model_create(ctx, &wide, &m) == GH_OK);
    CHECK(gh_model_destroy(m) == GH_OK);
    CHECK(gh_ctx_destroy(ctx) == GH_OK);
    return 0;
}

}  // namespace

int main(int argc, char** argv) {
    if (argc > 1 && std::strcmp(argv[1], "config") == 0) {
        if (config_checks()) return 1;
        std::printf("config ok\n");
        return 0;
    }
    if (argc > 1 && std::strcmp(argv[1], "race") == 0) {
        if (race()) return 1;
        std::printf("race ok\n");
        return 0;
    }
    if (argc > 1 && std::strcmp(argv[1], "exit") == 0) {
        Handles h;
        if (make(h)) return 1;
        gh_q4_0_free(h.t);
        gh_ctx_destroy(h.ctx);
        gh_model_destroy(h.m);
        gh_kv_destroy(h.kv);
        std::printf("exit order ok\n");
        return 0;
    }
    if (any_order()) return 1;
    std::printf("lifetime ok\n");
    return 0;
}
