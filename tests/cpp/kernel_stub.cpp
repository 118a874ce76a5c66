// No-op stand-ins for the kernel launchers of kernels.hip, so the host code
// of libgemma_hip links and runs on the CPU against hip_stub.cpp (lifetime
// tests only; never part of the product).
#include "../../gemma.hs_amd/csrc/common.h"

namespace gh {

int Profiler::kind_of(const char* name) {
    for (size_t i = 0; i < names.size(); ++i)
        if (names[i] == name) return (int)i;
    names.push_back(name);
    return (int)names.size() - 1;
}
int enqueue_step(gh_model*, gh_kv*, Sink&, int) { return GH_OK; }
int persistent_supported(const gh_model*) { return 0; }
int enqueue_persistent(gh_model*, gh_kv*, Sink&, int) { return GH_OK; }
size_t persistent_land(const gh_model*) { return 0; }
int launch_interleave_gu(const DMat&, int, int, const DMat&, hipStream_t) { return GH_OK; }
int pf_splits(const DMat&, int, int* kb_per) {
    if (kb_per) *kb_per = 1;
    return 1;
}
int enqueue_prefill(gh_model*, gh_kv*, Sink&, int, int, bool) { return GH_OK; }
int launch_q4_dequant(const DMat&, float*, hipStream_t) { return GH_OK; }
int launch_matvec_plain(const DMat&, const Plan&, const float*, float*, float*, int, float, hipStream_t) { return GH_OK; }
int launch_rmsnorm(const float*, const float*, int, float, int, float*, hipStream_t) { return GH_OK; }
int launch_qk_norm(const float*, const float*, int, int, float, int, float*, hipStream_t) { return GH_OK; }
int launch_rope(float*, int, int, const float*, hipStream_t) { return GH_OK; }
int launch_attention(const float*, const float*, const float*, int, int, int, int, int, int, float*, float*,
                     hipStream_t) {
    return GH_OK;
}
int launch_gelu_mul(const float*, const float*, int, float*, hipStream_t) { return GH_OK; }
int launch_argmax(const float*, int, unsigned long long*, hipStream_t) { return GH_OK; }
int launch_stream_read(const void*, size_t, float*, hipStream_t) { return GH_OK; }
int launch_xchg_probe(uint64_t*, int, int, int*, unsigned long long*, hipStream_t) { return GH_OK; }
int attn_noalloc_scratch(float** out) {
    static float buf[16];
    *out = buf;
    return GH_OK;
}
int launch_sample_logits(const float*, int, float, int, uint64_t, uint64_t, float*, int32_t*, hipStream_t) { return GH_OK; }

}  // namespace gh
