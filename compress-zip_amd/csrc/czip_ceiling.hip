// Measured ceilings of the two resources the path's rooflines are priced
// against, beside the published peaks: HBM bandwidth (a plain streaming copy)
// and dense int8 MFMA throughput (v_mfma_i32_16x16x64_i8 chains with no
// memory traffic).  A measurement library of its own (libczip_ceiling.so),
// loaded by the benchmark only; the path's library does not contain it.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>

typedef int v4i __attribute__((ext_vector_type(4)));

// dst[i] = src[i] over n 16-byte words: a grid-stride loop of 16-byte loads
// and stores, two words in flight per thread
__global__ __launch_bounds__(256) void k_copy16(const uint4* __restrict__ src, uint4* __restrict__ dst, size_t n) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    for (; i + stride < n; i += 2 * stride) {
        const uint4 a = src[i], b = src[i + stride];
        dst[i] = a;
        dst[i + stride] = b;
    }
    if (i < n) dst[i] = src[i];
}

// NC independent accumulator chains per wave, `iters` rounds of NC MFMAs on
// register operands; the sums are stored so that nothing is dead
template <int NC>
__global__ __launch_bounds__(256) void k_mfma_i8(int iters, int* __restrict__ out) {
    const int lane = threadIdx.x & 63;
    const v4i a = {lane * 3 + 1, lane ^ 0x5A5A5A5A, lane * 0x01010101, 7};
    const v4i b = {lane ^ 0x33333333, lane * 5 + 2, 0x0F0F0F0F, lane};
    v4i c[NC];
#pragma unroll
    for (int k = 0; k < NC; k++) c[k] = (v4i){k, 0, 0, 0};
    for (int it = 0; it < iters; it++) {
#pragma unroll
        for (int k = 0; k < NC; k++) c[k] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c[k], 0, 0, 0);
    }
    int s = 0;
#pragma unroll
    for (int k = 0; k < NC; k++) s += c[k][0] + c[k][1] + c[k][2] + c[k][3];
    out[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = s;
}

namespace {
constexpr int MFMA_CHAINS = 8;

int timed_ms(hipEvent_t a, hipEvent_t b, float* ms) {
    if (hipEventSynchronize(b) != hipSuccess) return -1;
    return hipEventElapsedTime(ms, a, b) == hipSuccess ? 0 : -1;
}
}  // namespace

extern "C" {

// Copy `bytes` (a multiple of 16) `reps` times after one untimed pass; *gbs =
// (read + written bytes) / time of the timed passes.  0 on success.
int czc_copy_gbs(size_t bytes, int reps, double* gbs) {
    if (bytes < 16 || bytes % 16 != 0 || reps < 1 || !gbs) return -2;
    void *src = nullptr, *dst = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    int rc = -1;
    if (hipMalloc(&src, bytes) != hipSuccess || hipMalloc(&dst, bytes) != hipSuccess) goto done;
    if (hipMemset(src, 1, bytes) != hipSuccess || hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess)
        goto done;
    {
        const size_t n = bytes / 16;
        const dim3 grid(256 * 16), block(256);
        hipLaunchKernelGGL(k_copy16, grid, block, 0, 0, (const uint4*)src, (uint4*)dst, n);
        hipEventRecord(e0, 0);
        for (int r = 0; r < reps; r++) hipLaunchKernelGGL(k_copy16, grid, block, 0, 0, (const uint4*)src, (uint4*)dst, n);
        hipEventRecord(e1, 0);
        float ms = 0;
        if (hipGetLastError() != hipSuccess || timed_ms(e0, e1, &ms)) goto done;
        *gbs = 2.0 * (double)bytes * reps / (ms * 1e-3) / 1e9;
        rc = 0;
    }
done:
    if (e0) hipEventDestroy(e0);
    if (e1) hipEventDestroy(e1);
    if (src) hipFree(src);
    if (dst) hipFree(dst);
    return rc;
}

// Dense int8 MFMA rate: `waves_per_simd` waves on each of the device's SIMDs
// (4 per CU), each issuing iters x 8 independent 16x16x64 MFMAs (32768 ops
// each).  *tops = ops / time of one timed launch after an untimed one.
int czc_mfma_i8_tops(int iters, int waves_per_simd, double* tops) {
    if (iters < 1 || waves_per_simd < 1 || waves_per_simd > 8 || !tops) return -2;
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1)
        return -1;
    const int blocks = cus * waves_per_simd;  // 4 waves per workgroup: one per SIMD
    int* out = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    int rc = -1;
    if (hipMalloc(&out, (size_t)blocks * 256 * sizeof(int)) != hipSuccess) goto done;
    if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) goto done;
    {
        hipLaunchKernelGGL(k_mfma_i8<MFMA_CHAINS>, dim3(blocks), dim3(256), 0, 0, iters, out);
        hipEventRecord(e0, 0);
        hipLaunchKernelGGL(k_mfma_i8<MFMA_CHAINS>, dim3(blocks), dim3(256), 0, 0, iters, out);
        hipEventRecord(e1, 0);
        float ms = 0;
        if (hipGetLastError() != hipSuccess || timed_ms(e0, e1, &ms)) goto done;
        const double ops = (double)blocks * 4 * iters * MFMA_CHAINS * (16.0 * 16 * 64 * 2);
        *tops = ops / (ms * 1e-3) / 1e12;
        rc = 0;
    }
done:
    if (e0) hipEventDestroy(e0);
    if (e1) hipEventDestroy(e1);
    if (out) hipFree(out);
    return rc;
}

}  // extern "C"
