// Phase-timestamp build of the decode-step kernels (a measurement tool, not
// part of libgemma_hip): kernels.hip compiled with GH_MARK(slot) recording
// the wave's s_memrealtime (100 MHz) into LDS at each phase point and
// GH_MARK_END() copying the workgroup's marks to a device buffer at the
// kernel's end, so the marks add no global store that an s_waitcnt inside
// the kernel would wait on.  build.py --marks compiles this file once per
// step translation unit (GH_TU 1: attention, 5-7: the matvec phases) and
// links them with the library's other objects into libgemma_hip_marks.so.
// Each translation unit is its own code object with its own buffer, read
// and cleared through gh_marks_fetch_tu<N> / gh_marks_clear_tu<N>.
//
// Layout: marks[workgroup][wave][slot], u64 ticks, 0 = slot not reached.
// Workgroups past GH_MARK_MAXWG and waves past GH_MARK_WAVES are not
// recorded.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>

#define GH_MARK_MAXWG 8192
#define GH_MARK_WAVES 8
#define GH_MARK_SLOTS 16
__device__ unsigned long long gh_marks_buf[GH_MARK_MAXWG * GH_MARK_WAVES * GH_MARK_SLOTS];
__shared__ unsigned long long gh_mk_lds[GH_MARK_WAVES][GH_MARK_SLOTS];
#define GH_MARK(slot)                                                                       \
    do {                                                                                    \
        const int w_ = threadIdx.x >> 6;                                                    \
        if ((threadIdx.x & 63) == 0 && w_ < GH_MARK_WAVES) {                                \
            if ((slot) == 0)                                                                \
                for (int q_ = 1; q_ < GH_MARK_SLOTS; ++q_) gh_mk_lds[w_][q_] = 0;           \
            gh_mk_lds[w_][slot] = __builtin_amdgcn_s_memrealtime();                         \
        }                                                                                   \
    } while (0)
#define GH_MARK_END()                                                                        \
    do {                                                                                     \
        const int w_ = threadIdx.x >> 6;                                                     \
        if ((threadIdx.x & 63) == 0 && w_ < GH_MARK_WAVES && blockIdx.x < GH_MARK_MAXWG)     \
            for (int q_ = 0; q_ < GH_MARK_SLOTS; ++q_)                                       \
                gh_marks_buf[(blockIdx.x * GH_MARK_WAVES + w_) * GH_MARK_SLOTS + q_] = gh_mk_lds[w_][q_]; \
    } while (0)
#include "../kernels.hip"

#define GH_MARKS_CAT2(a, b) a##b
#define GH_MARKS_CAT(a, b) GH_MARKS_CAT2(a, b)
#define GH_MARKS_BYTES (sizeof(unsigned long long) * GH_MARK_MAXWG * GH_MARK_WAVES * GH_MARK_SLOTS)

// Copy this unit's marks to host (at most `bytes`); 0 or -2 (HIP error).
extern "C" int GH_MARKS_CAT(gh_marks_fetch_tu, GH_TU)(void* host, size_t bytes) {
    if (bytes > GH_MARKS_BYTES) bytes = GH_MARKS_BYTES;
    return hipMemcpyFromSymbol(host, HIP_SYMBOL(gh_marks_buf), bytes, 0, hipMemcpyDeviceToHost) == hipSuccess ? 0 : -2;
}

// Zero this unit's marks.
extern "C" int GH_MARKS_CAT(gh_marks_clear_tu, GH_TU)(void) {
    static void* zeros = nullptr;
    if (!zeros && !(zeros = calloc(1, GH_MARKS_BYTES))) return -3;
    return hipMemcpyToSymbol(HIP_SYMBOL(gh_marks_buf), zeros, GH_MARKS_BYTES, 0, hipMemcpyHostToDevice) == hipSuccess
               ? 0
               : -2;
}
