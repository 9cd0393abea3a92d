// probes.hip -- launch-floor probes (libdmhip_diag.so, declared in
// include/dmhip_diag.h).  Measurement only: the product library does not
// contain them.
//
// probe_read_kernel: each 256-thread workgroup streams 16 KB with four
// 16-byte loads per lane issued before any use, folds them into a checksum
// and writes only if it equals `magic` (never, in practice), so the loads
// cannot be dropped.
#include <hip/hip_runtime.h>

#include "../../../include/dmhip_diag.h"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__global__ void probe_empty_kernel() {}

__global__ void __launch_bounds__(256) probe_read_kernel(const u32x4 *__restrict__ src, size_t n16,
                                                         uint32_t magic, uint32_t *sink) {
    const size_t base = (size_t)blockIdx.x * 1024 + threadIdx.x;
    u32x4 v[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const size_t i = base + 256 * j;
        v[j] = i < n16 ? src[i] : u32x4{0, 0, 0, 0};
    }
    uint32_t h = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) h += v[j][0] ^ v[j][1] ^ v[j][2] ^ v[j][3];
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) h ^= __shfl_xor(h, m, 64);
    if (h == magic) sink[0] = h;
}

// Times `launches` calls of body(stream, i) after three untimed ones; the
// stream and events are the probe's own.
template <class Body>
int time_launches(size_t launches, double *us, Body body) {
    if (!us || launches == 0) return (int)hipErrorInvalidValue;
    hipStream_t s = nullptr;
    hipEvent_t a = nullptr, b = nullptr;
    hipError_t e = hipStreamCreate(&s);
    if (e == hipSuccess) e = hipEventCreate(&a);
    if (e == hipSuccess) e = hipEventCreate(&b);
    for (size_t i = 0; e == hipSuccess && i < 3; i++) e = body(s, i);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e == hipSuccess) e = hipEventRecord(a, s);
    for (size_t i = 0; e == hipSuccess && i < launches; i++) e = body(s, i);
    if (e == hipSuccess) e = hipEventRecord(b, s);
    if (e == hipSuccess) e = hipEventSynchronize(b);
    float ms = 0.0f;
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, a, b);
    if (e == hipSuccess) *us = (double)ms * 1e3 / (double)launches;
    if (a) (void)hipEventDestroy(a);
    if (b) (void)hipEventDestroy(b);
    if (s) (void)hipStreamDestroy(s);
    return (int)e;
}

}  // namespace

extern "C" {

int dmhip_diag_time_empty(uint32_t workgroups, uint32_t threads, size_t launches, double *us) {
    if (workgroups == 0 || threads == 0 || threads > 1024 || threads % 64) return (int)hipErrorInvalidValue;
    return time_launches(launches, us, [&](hipStream_t s, size_t) {
        hipLaunchKernelGGL(probe_empty_kernel, dim3(workgroups), dim3(threads), 0, s);
        return hipGetLastError();
    });
}

int dmhip_diag_time_read(const void *const *sources, size_t count, size_t n, size_t launches, double *us) {
    if (!sources || count == 0 || n == 0 || n % 16) return (int)hipErrorInvalidValue;
    for (size_t i = 0; i < count; i++)
        if (!sources[i] || ((uintptr_t)sources[i] & 15u)) return (int)hipErrorInvalidValue;
    const size_t n16 = n / 16, groups = (n16 + 1023) / 1024;
    if (groups > 0x7fffffffu) return (int)hipErrorInvalidValue;
    uint32_t *sink = nullptr;
    hipError_t e = hipMalloc(&sink, 256);
    if (e != hipSuccess) return (int)e;
    const int r = time_launches(launches, us, [&](hipStream_t s, size_t i) {
        hipLaunchKernelGGL(probe_read_kernel, dim3((uint32_t)groups), dim3(256), 0, s,
                           (const u32x4 *)sources[i % count], n16, 0x9e3779b9u, sink);
        return hipGetLastError();
    });
    (void)hipFree(sink);
    return r;
}

}  // extern "C"
