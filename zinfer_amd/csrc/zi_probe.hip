// zi_probe.hip -- a plain streaming read, the achievable-bandwidth reference
// that bench.py times beside the sampling kernels (`--path readfloor`).  Not
// part of the sampling ABI: it is built into its own libzi_probe.so.
//
// Each 1024-thread workgroup reads 8 16-byte vectors per thread (128 KiB,
// every load issued before any is used, non-temporal like the sampling
// stream) and writes one max per wave, so the kernel moves the buffer's bytes
// once and almost nothing else.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {
constexpr int kThreads = 1024;
constexpr int kNV = 8;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(kThreads) void read_kernel(const uint4 *src, int64_t nvec, float *out) {
    const int64_t base = (int64_t)blockIdx.x * kThreads * kNV;
    u32x4 r[kNV];
#pragma unroll
    for (int j = 0; j < kNV; ++j) {
        int64_t q = base + (int64_t)j * kThreads + threadIdx.x;
        q = q < nvec ? q : nvec - 1;
        r[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(src + q));
    }
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < kNV; ++j)
        m = fmaxf(m, fmaxf(fmaxf(__uint_as_float(r[j].x), __uint_as_float(r[j].y)),
                           fmaxf(__uint_as_float(r[j].z), __uint_as_float(r[j].w))));
    for (int o = 32; o; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    if ((threadIdx.x & 63) == 0) out[(int64_t)blockIdx.x * (kThreads / 64) + threadIdx.x / 64] = m;
}
}  // namespace

// Reads `bytes` (a multiple of 16, src 16-byte aligned) on `stream`; out
// needs ceil(bytes / 131072) * 16 floats.  Returns a hipError_t value.
extern "C" int32_t zi_probe_read(const void *src, int64_t bytes, float *out, void *stream) {
    if (!src || !out || bytes < 16 || (bytes & 15) || ((uintptr_t)src & 15)) return (int32_t)hipErrorInvalidValue;
    const int64_t nvec = bytes / 16;
    const int64_t per = (int64_t)kThreads * kNV;
    const int grid = (int)((nvec + per - 1) / per);
    hipLaunchKernelGGL(read_kernel, dim3(grid), dim3(kThreads), 0, (hipStream_t)stream,
                       reinterpret_cast<const uint4 *>(src), nvec, out);
    return (int32_t)hipGetLastError();
}
