// Host-only stand-in for the HIP runtime calls of libgemma_hip's host code,
// for CPU tests of its object lifetimes (built with AddressSanitizer by
// tests/test_lifetime.py; never part of the product).
//
// Device memory is host memory; streams, events and graphs are heap
// objects that each call dereferences, as the runtime does with its own
// objects, so a call through a destroyed stream is a heap-use-after-free
// that AddressSanitizer reports.  Kernel launches are the no-op launchers
// in kernel_stub.cpp.
#include <hip/hip_runtime_api.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <set>

namespace {

constexpr unsigned kStreamMagic = 0x57EA4u, kEventMagic = 0xE7E27u, kGraphMagic = 0x6A4Fu;

struct StubObj {
    unsigned magic;
};

std::mutex& mu() {
    static auto* m = new std::mutex();
    return *m;
}
std::set<void*>& live_allocs() {
    static auto* s = new std::set<void*>();
    return *s;
}

// Reads the object's first word: a use-after-free under AddressSanitizer.
hipError_t touch(const void* o, unsigned magic) {
    if (!o) return hipSuccess;  // the null (default) stream
    return static_cast<const StubObj*>(o)->magic == magic ? hipSuccess : hipErrorInvalidHandle;
}

void* obj(unsigned magic) { return new StubObj{magic}; }

hipError_t dev_alloc(void** p, size_t n) {
    if (!p) return hipErrorInvalidValue;
    *p = std::malloc(n ? n : 1);
    std::lock_guard<std::mutex> g(mu());
    live_allocs().insert(*p);
    return hipSuccess;
}

hipError_t dev_free(void* p) {
    if (!p) return hipSuccess;
    {
        std::lock_guard<std::mutex> g(mu());
        if (!live_allocs().erase(p)) {
            std::fprintf(stderr, "hip_stub: free of a pointer that is not a live allocation: %p\n", p);
            std::abort();
        }
    }
    std::free(p);
    return hipSuccess;
}

}  // namespace

extern "C" {

hipError_t hipGetDeviceCount(int* n) {
    *n = 1;
    return hipSuccess;
}
hipError_t hipSetDevice(int d) { return d == 0 ? hipSuccess : hipErrorInvalidDevice; }
hipError_t hipDeviceSynchronize(void) { return hipSuccess; }
hipError_t hipDeviceGetAttribute(int* v, hipDeviceAttribute_t, int) {
    *v = 256;
    return hipSuccess;
}
const char* hipGetErrorString(hipError_t) { return "hip_stub error"; }
hipError_t hipGetLastError(void) { return hipSuccess; }

hipError_t hipMalloc(void** p, size_t n) { return dev_alloc(p, n); }
hipError_t hipFree(void* p) { return dev_free(p); }
hipError_t hipMallocAsync(void** p, size_t n, hipStream_t s) {
    if (touch(s, kStreamMagic) != hipSuccess) return hipErrorInvalidHandle;
    return dev_alloc(p, n);
}
hipError_t hipFreeAsync(void* p, hipStream_t s) {
    if (touch(s, kStreamMagic) != hipSuccess) return hipErrorInvalidHandle;
    return dev_free(p);
}
hipError_t hipHostMalloc(void** p, size_t n, unsigned int) { return dev_alloc(p, n); }
hipError_t hipHostFree(void* p) { return dev_free(p); }

hipError_t hipMemcpy(void* d, const void* s, size_t n, hipMemcpyKind) {
    std::memcpy(d, s, n);
    return hipSuccess;
}
hipError_t hipMemcpyAsync(void* d, const void* s, size_t n, hipMemcpyKind, hipStream_t st) {
    if (touch(st, kStreamMagic) != hipSuccess) return hipErrorInvalidHandle;
    std::memcpy(d, s, n);
    return hipSuccess;
}
hipError_t hipMemset(void* d, int v, size_t n) {
    std::memset(d, v, n);
    return hipSuccess;
}
hipError_t hipMemsetAsync(void* d, int v, size_t n, hipStream_t st) {
    if (touch(st, kStreamMagic) != hipSuccess) return hipErrorInvalidHandle;
    std::memset(d, v, n);
    return hipSuccess;
}

hipError_t hipStreamCreateWithFlags(hipStream_t* s, unsigned int) {
    *s = (hipStream_t)obj(kStreamMagic);
    return hipSuccess;
}
hipError_t hipStreamDestroy(hipStream_t s) {
    hipError_t e = touch(s, kStreamMagic);
    delete (StubObj*)s;
    return e;
}
hipError_t hipStreamSynchronize(hipStream_t s) { return touch(s, kStreamMagic); }
hipError_t hipStreamIsCapturing(hipStream_t s, hipStreamCaptureStatus* st) {
    *st = hipStreamCaptureStatusNone;
    return touch(s, kStreamMagic);
}
hipError_t hipStreamBeginCapture(hipStream_t s, hipStreamCaptureMode) { return touch(s, kStreamMagic); }
hipError_t hipStreamEndCapture(hipStream_t s, hipGraph_t* g) {
    *g = (hipGraph_t)obj(kGraphMagic);
    return touch(s, kStreamMagic);
}

hipError_t hipEventCreate(hipEvent_t* e) {
    *e = (hipEvent_t)obj(kEventMagic);
    return hipSuccess;
}
hipError_t hipEventDestroy(hipEvent_t e) {
    hipError_t r = touch(e, kEventMagic);
    delete (StubObj*)e;
    return r;
}
hipError_t hipEventRecord(hipEvent_t e, hipStream_t s) {
    if (touch(s, kStreamMagic) != hipSuccess) return hipErrorInvalidHandle;
    return touch(e, kEventMagic);
}
hipError_t hipEventSynchronize(hipEvent_t e) { return touch(e, kEventMagic); }
hipError_t hipEventElapsedTime(float* ms, hipEvent_t a, hipEvent_t b) {
    *ms = 0.0f;
    if (touch(a, kEventMagic) != hipSuccess) return hipErrorInvalidHandle;
    return touch(b, kEventMagic);
}

hipError_t hipGraphCreate(hipGraph_t* g, unsigned int) {
    *g = (hipGraph_t)obj(kGraphMagic);
    return hipSuccess;
}
hipError_t hipGraphDestroy(hipGraph_t g) {
    hipError_t r = touch(g, kGraphMagic);
    delete (StubObj*)g;
    return r;
}
hipError_t hipGraphInstantiate(hipGraphExec_t* ge, hipGraph_t g, hipGraphNode_t*, char*, size_t) {
    *ge = (hipGraphExec_t)obj(kGraphMagic);
    return touch(g, kGraphMagic);
}
hipError_t hipGraphExecDestroy(hipGraphExec_t ge) {
    hipError_t r = touch(ge, kGraphMagic);
    delete (StubObj*)ge;
    return r;
}
hipError_t hipGraphLaunch(hipGraphExec_t ge, hipStream_t s) {
    if (touch(s, kStreamMagic) != hipSuccess) return hipErrorInvalidHandle;
    return touch(ge, kGraphMagic);
}
hipError_t hipGraphExecKernelNodeSetParams(hipGraphExec_t ge, hipGraphNode_t, const hipKernelNodeParams*) {
    return touch(ge, kGraphMagic);
}

}  // extern "C"
