// Measured ceilings of the two resources the path's rooflines are priced
// against, beside the published peaks: HBM bandwidth (a plain streaming copy)
// and dense int8 MFMA throughput (independent MFMA chains with no memory
// traffic), for both int8 shapes: v_mfma_i32_32x32x32_i8, which reaches the
// published rate, and v_mfma_i32_16x16x64_i8, the one the path's kernels
// issue (measured on MI355X: ~4.8 vs ~4.0 POP/s; the smaller instruction pays
// the same per-instruction issue cost for half the work).  A measurement
// library of its own (libczip_ceiling.so), loaded by the benchmark only; the
// path's library does not contain it.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// dst[i] = src[i] over n 16-byte words: a grid-stride loop of 16-byte loads
// and stores (one word in flight per thread over 4 workgroups per CU: the
// fastest of the grid sizes and unrollings measured on MI355X)
__global__ __launch_bounds__(256) void k_copy16(const uint4* __restrict__ src, uint4* __restrict__ dst, size_t n) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) dst[i] = src[i];
}

// the sum of n 16-byte words, a grid-stride loop of 16-byte loads (read-only
// traffic: HBM reads without the write turnarounds of a copy); one word per
// workgroup is stored so that nothing is dead
__global__ __launch_bounds__(256) void k_read16(const uint4* __restrict__ src, size_t n, unsigned* __restrict__ out) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    unsigned acc = 0;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const uint4 v = src[i];
        acc += v.x ^ v.y ^ v.z ^ v.w;
    }
    if (acc == 0x9E3779B9u) out[blockIdx.x] = acc;  // practically never taken, but not provably dead
}

// NC independent accumulator chains per wave, `iters` rounds of NC MFMAs on
// register operands; the sums are stored so that nothing is dead
template <int NC>
__global__ __launch_bounds__(256) void k_mfma_i8_16(int iters, int* __restrict__ out) {
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
template <int NC>
__global__ __launch_bounds__(256) void k_mfma_i8_32(int iters, int* __restrict__ out) {
    const int lane = threadIdx.x & 63;
    const v4i a = {lane * 3 + 1, lane ^ 0x5A5A5A5A, lane * 0x01010101, 7};
    const v4i b = {lane ^ 0x33333333, lane * 5 + 2, 0x0F0F0F0F, lane};
    v16i c[NC];
#pragma unroll
    for (int k = 0; k < NC; k++) {
        c[k] = (v16i){};
        c[k][0] = k;
    }
    for (int it = 0; it < iters; it++) {
#pragma unroll
        for (int k = 0; k < NC; k++) c[k] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c[k], 0, 0, 0);
    }
    int s = 0;
#pragma unroll
    for (int k = 0; k < NC; k++)
#pragma unroll
        for (int j = 0; j < 16; j++) s += c[k][j];
    out[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = s;
}

namespace {
constexpr int CHAINS_16 = 16;  // independent 16x16x64 accumulators per wave
constexpr int CHAINS_32 = 4;   // independent 32x32x32 accumulators per wave

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
        int dev = 0, cus = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1)
            goto done;
        const dim3 grid(4 * cus), block(256);
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

// Read `bytes` (a multiple of 16) `reps` times after one untimed pass; *gbs =
// bytes read / time of the timed passes.  0 on success.
int czc_read_gbs(size_t bytes, int reps, double* gbs) {
    if (bytes < 16 || bytes % 16 != 0 || reps < 1 || !gbs) return -2;
    void* src = nullptr;
    unsigned* out = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    int rc = -1;
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1)
        return -1;
    if (hipMalloc(&src, bytes) != hipSuccess || hipMalloc(&out, (size_t)cus * 8 * sizeof(unsigned)) != hipSuccess) goto done;
    if (hipMemset(src, 1, bytes) != hipSuccess || hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess)
        goto done;
    {
        const size_t n = bytes / 16;
        const dim3 grid(8 * cus), block(256);
        hipLaunchKernelGGL(k_read16, grid, block, 0, 0, (const uint4*)src, n, out);
        hipEventRecord(e0, 0);
        for (int r = 0; r < reps; r++) hipLaunchKernelGGL(k_read16, grid, block, 0, 0, (const uint4*)src, n, out);
        hipEventRecord(e1, 0);
        float ms = 0;
        if (hipGetLastError() != hipSuccess || timed_ms(e0, e1, &ms)) goto done;
        *gbs = (double)bytes * reps / (ms * 1e-3) / 1e9;
        rc = 0;
    }
done:
    if (e0) hipEventDestroy(e0);
    if (e1) hipEventDestroy(e1);
    if (src) hipFree(src);
    if (out) hipFree(out);
    return rc;
}

// Dense int8 MFMA rate: `waves_per_simd` waves on each of the device's SIMDs
// (4 per CU), each issuing iters rounds of independent MFMAs of one shape:
// shape 16 = 16 chains of v_mfma_i32_16x16x64_i8 (32768 ops each), shape 32
// = 4 chains of v_mfma_i32_32x32x32_i8 (65536 ops each).  *tops = ops / time
// of one timed launch after an untimed one.
int czc_mfma_i8_tops(int shape, int iters, int waves_per_simd, double* tops) {
    if ((shape != 16 && shape != 32) || iters < 1 || waves_per_simd < 1 || waves_per_simd > 8 || !tops) return -2;
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
        for (int r = 0; r < 2; r++) {
            if (r == 1) hipEventRecord(e0, 0);
            if (shape == 16) hipLaunchKernelGGL(k_mfma_i8_16<CHAINS_16>, dim3(blocks), dim3(256), 0, 0, iters, out);
            else hipLaunchKernelGGL(k_mfma_i8_32<CHAINS_32>, dim3(blocks), dim3(256), 0, 0, iters, out);
        }
        hipEventRecord(e1, 0);
        float ms = 0;
        if (hipGetLastError() != hipSuccess || timed_ms(e0, e1, &ms)) goto done;
        const double ops = shape == 16 ? (double)blocks * 4 * iters * CHAINS_16 * (16.0 * 16 * 64 * 2)
                                       : (double)blocks * 4 * iters * CHAINS_32 * (32.0 * 32 * 32 * 2);
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
