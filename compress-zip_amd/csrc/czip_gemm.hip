// int8 MFMA GEMMs with fused epilogues (linear.rs:12-31 + model.rs:280-300).
#include "czip_device.h"
#include "czip_kernels.h"

namespace czip {

// ---------------------------------------------------------------------------
// int8 GEMM C = A * W^T on v_mfma_i32_16x16x64_i8 with fused epilogues.
// Block tile 128x128x64, 4 waves in 2x2, each wave 64x64 = 4x4 MFMA tiles.
// MFMA operand layout: lane l supplies row (l % 16) and the 16 bytes of K at
// (l / 16) * 16; A and W use the same K mapping, so the dot product is exact
// whatever the hardware's K order.  Result: lane l holds rows 4*(l/16)+r,
// column l % 16 of each 16x16 tile.
// ---------------------------------------------------------------------------
constexpr int BM = 128, BN = 128, BK = 64, LDSK = BK + 16;

__device__ __forceinline__ void load_tile(const int8_t* __restrict__ src, int rows_total, int ld, int row0, int k0,
                                          int8_t* lds, int tid) {
    // 128 rows x 64 bytes: thread t -> row t/2, bytes (t%2)*32 .. +32
    int r = tid >> 1, c = (tid & 1) * 32;
    int4 v0 = make_int4(0, 0, 0, 0), v1 = v0;
    if (row0 + r < rows_total) {
        const int4* g = (const int4*)(src + (size_t)(row0 + r) * ld + k0 + c);
        v0 = g[0];
        v1 = g[1];
    }
    int4* l = (int4*)(lds + r * LDSK + c);
    l[0] = v0;
    l[1] = v1;
}

template <int EPI>
__global__ __launch_bounds__(256) void k_gemm(GemmArgs a) {
    __shared__ __attribute__((aligned(16))) int8_t As[BM * LDSK];
    __shared__ __attribute__((aligned(16))) int8_t Ws[BN * LDSK];
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int wm = wave >> 1, wn = wave & 1;
    // N tiles vary fastest so consecutive workgroups reuse the same A rows from L2
    const int ntn = (a.N + BN - 1) / BN;
    const int m0 = (int)(blockIdx.x / ntn) * BM, n0 = (int)(blockIdx.x % ntn) * BN;

    v4i acc[4][4];
    for (int i = 0; i < 4; i++)
        for (int j = 0; j < 4; j++) acc[i][j] = (v4i){0, 0, 0, 0};

    for (int k0 = 0; k0 < a.K; k0 += BK) {
        load_tile(a.A, a.M, a.K, m0, k0, As, tid);
        load_tile(a.W, a.N, a.K, n0, k0, Ws, tid);
        __syncthreads();
        v4i af[4], bf[4];
        const int lr = lane & 15, lk = (lane >> 4) * 16;
        for (int i = 0; i < 4; i++) af[i] = *(const v4i*)(As + (wm * 64 + i * 16 + lr) * LDSK + lk);
        for (int j = 0; j < 4; j++) bf[j] = *(const v4i*)(Ws + (wn * 64 + j * 16 + lr) * LDSK + lk);
        for (int i = 0; i < 4; i++)
            for (int j = 0; j < 4; j++) acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
        __syncthreads();
    }

    const int col_base = n0 + wn * 64;  // 64-aligned, one head / one gate-up group
    if (col_base >= a.N) return;
    const int lc = lane & 15, lrow = (lane >> 4) * 4;
#pragma unroll
    for (int i = 0; i < 4; i++) {
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int row = m0 + wm * 64 + i * 16 + lrow + r;
            if (row >= a.M) continue;
            if (EPI == EPI_RAW) {
#pragma unroll
                for (int j = 0; j < 4; j++) a.out32[(size_t)row * a.ldo + col_base + j * 16 + lc] = acc[i][j][r];
            } else if (EPI == EPI_REQ) {
#pragma unroll
                for (int j = 0; j < 4; j++)
                    a.out8[(size_t)row * a.ldo + col_base + j * 16 + lc] = (int8_t)requant(acc[i][j][r], a.mult, a.shift);
            } else if (EPI == EPI_REGLU) {
                // W rows were permuted so that a 64-row group holds 32 gate rows then the
                // matching 32 up rows: output feature f = col_base/2 + j*16 + lc.
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    int g = requant(acc[i][j][r], a.mult, a.shift);
                    int u = requant(acc[i][j + 2][r], a.mult, a.shift);
                    int gr = g > 0 ? g : 0;
                    a.out8[(size_t)row * a.ldo + (col_base >> 1) + j * 16 + lc] = (int8_t)clamp127(sra_rne32(gr * u, 7));
                }
            } else {  // EPI_QKV
                const int p = a.pos >= 0 ? a.pos : row % a.T, b = a.pos >= 0 ? row : row / a.T;
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const int i32 = j * 16 + lc;  // rotary pair (i32, i32 + 32)
                    const int xv = requant(acc[i][j][r], a.mult, a.shift);
                    const int yv = requant(acc[i][j + 2][r], a.mult, a.shift);
                    const int c = a.rcos[p * 32 + i32], s = a.rsin[p * 32 + i32];
                    const int xr = (int)((unsigned)(xv * c) - (unsigned)(yv * s));
                    const int yr = (int)((unsigned)(xv * s) + (unsigned)(yv * c));
                    if (col_base < a.d) {
                        // Q: attention.rs:53-83 (>>15 then NET_SHIFT=1, two roundings)
                        int8_t* q = a.out8 + (size_t)row * a.ldo + col_base;
                        q[i32] = (int8_t)clamp127(sra_rne32(sra_rne32(xr, 15), 1));
                        q[i32 + 32] = (int8_t)clamp127(sra_rne32(sra_rne32(yr, 15), 1));
                    } else {
                        const int kcol = col_base - a.d;
                        int g, isv;
                        if (a.kv_mode == 1) { isv = kcol >= 64 * a.G; g = (isv ? kcol - 64 * a.G : kcol) >> 6; }
                        else { isv = kcol >= 64; g = 0; }
                        if (!isv) {
                            // K: attention.rs:29-50
                            size_t off = (((size_t)b * a.KH + g) * a.T + p) * 64;
                            a.kc[off + i32] = (int8_t)clamp127(sra_rne32(xr, 15));
                            a.kc[off + i32 + 32] = (int8_t)clamp127(sra_rne32(yr, 15));
                        } else if (a.pos >= 0) {
                            // V of a decode step: key-major like K
                            size_t off = (((size_t)b * a.KH + g) * a.T + p) * 64;
                            a.vc[off + i32] = (int8_t)xv;
                            a.vc[off + i32 + 32] = (int8_t)yv;
                        } else {
                            // V, stored dim-major for the prefill PV operand
                            size_t off = (((size_t)b * a.KH + g) * 64) * a.TP + p;
                            a.vc[off + (size_t)i32 * a.TP] = (int8_t)xv;
                            a.vc[off + (size_t)(i32 + 32) * a.TP] = (int8_t)yv;
                        }
                    }
                }
            }
        }
    }
}

void launch_gemm(const GemmArgs& a, int epi, hipStream_t s) {
    dim3 grid((unsigned)(((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN)));
    switch (epi) {
        case EPI_RAW: hipLaunchKernelGGL(k_gemm<EPI_RAW>, grid, dim3(256), 0, s, a); break;
        case EPI_REQ: hipLaunchKernelGGL(k_gemm<EPI_REQ>, grid, dim3(256), 0, s, a); break;
        case EPI_QKV: hipLaunchKernelGGL(k_gemm<EPI_QKV>, grid, dim3(256), 0, s, a); break;
        default: hipLaunchKernelGGL(k_gemm<EPI_REGLU>, grid, dim3(256), 0, s, a); break;
    }
}


}  // namespace czip
