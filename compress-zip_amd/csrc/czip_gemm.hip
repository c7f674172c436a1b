// int8 MFMA GEMMs with fused epilogues (linear.rs:12-31 + model.rs:280-300).
#include "czip_device.h"
#include "czip_kernels.h"

namespace czip {

// ---------------------------------------------------------------------------
// int8 GEMM C = A * W^T on v_mfma_i32_16x16x64_i8 with fused epilogues.
// Block tile 128 (rows of A) x 128 (rows of W) x 64, 4 waves in 2x2, each
// wave 64x64 = 4x4 MFMA tiles; the K tiles are double-buffered in LDS and the
// next one is fetched into registers while the current one is multiplied.
// MFMA operand layout: lane l supplies row (l % 16) and the 16 bytes of K at
// (l / 16) * 16; A and W use the same K mapping, so the dot product is exact
// whatever the hardware's K order.  W is the first operand, so lane l holds
// output columns 4*(l/16) .. +3 (consecutive) of row l % 16 of each 16x16
// tile, and the epilogues store 4 outputs with one vector store.
// ---------------------------------------------------------------------------
constexpr int BM = 128, BN = 128, BK = 64, LDSK = BK + 16;

struct TileRegs {
    int4 v[2];
};

__device__ __forceinline__ void fetch_tile(const int8_t* __restrict__ src, int rows_total, int ld, int row0, int k0,
                                           int tid, TileRegs& t) {
    // 128 rows x 64 bytes: thread t -> row t/2, bytes (t%2)*32 .. +32
    const int r = tid >> 1, c = (tid & 1) * 32;
    t.v[0] = make_int4(0, 0, 0, 0);
    t.v[1] = t.v[0];
    if (row0 + r < rows_total) {
        const int4* g = (const int4*)(src + (size_t)(row0 + r) * ld + k0 + c);
        t.v[0] = g[0];
        t.v[1] = g[1];
    }
}

__device__ __forceinline__ void store_tile(const TileRegs& t, int8_t* lds, int tid) {
    const int r = tid >> 1, c = (tid & 1) * 32;
    int4* l = (int4*)(lds + r * LDSK + c);
    l[0] = t.v[0];
    l[1] = t.v[1];
}

// model.rs:280-300.  Fast path: |v * mult| < 2^53, so v * mult * 2^-shift is
// exact in f64 and rint rounds half to even like sra_rne_tte_s64_to_s32.
template <bool FAST>
__device__ __forceinline__ int rq(int v, const GemmArgs& a) {
    if (FAST) {
        double x = __builtin_rint((double)v * a.rq_scale);
        x = fmin(fmax(x, -127.0), 127.0);
        return (int)x;
    }
    return requant(v, a.mult, a.shift);
}

__device__ __forceinline__ unsigned pack4i(int a, int b, int c, int d) {
    return (unsigned)(a & 0xFF) | ((unsigned)(b & 0xFF) << 8) | ((unsigned)(c & 0xFF) << 16) | ((unsigned)d << 24);
}

template <int EPI, bool FAST>
__global__ __launch_bounds__(256, 2) void k_gemm(GemmArgs a) {
    __shared__ __attribute__((aligned(16))) int8_t As[2][BM * LDSK];
    __shared__ __attribute__((aligned(16))) int8_t Ws[2][BN * LDSK];
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int wm = wave >> 1, wn = wave & 1;
    // N tiles vary fastest so consecutive workgroups reuse the same A rows from L2
    const int ntn = (a.N + BN - 1) / BN;
    const int m0 = (int)(blockIdx.x / ntn) * BM, n0 = (int)(blockIdx.x % ntn) * BN;
    const int nk = a.K / BK;

    v4i acc[4][4];
    for (int i = 0; i < 4; i++)
        for (int j = 0; j < 4; j++) acc[i][j] = (v4i){0, 0, 0, 0};

    TileRegs ta, tw;
    fetch_tile(a.A, a.M, a.K, m0, 0, tid, ta);
    fetch_tile(a.W, a.N, a.K, n0, 0, tid, tw);
    store_tile(ta, As[0], tid);
    store_tile(tw, Ws[0], tid);
    __syncthreads();
    const int lr = lane & 15, lk = (lane >> 4) * 16;
    for (int kt = 0; kt < nk; kt++) {
        const int cur = kt & 1;
        if (kt + 1 < nk) {
            fetch_tile(a.A, a.M, a.K, m0, (kt + 1) * BK, tid, ta);
            fetch_tile(a.W, a.N, a.K, n0, (kt + 1) * BK, tid, tw);
        }
        v4i af[4], bf[4];
#pragma unroll
        for (int i = 0; i < 4; i++) af[i] = *(const v4i*)(As[cur] + (wm * 64 + i * 16 + lr) * LDSK + lk);
#pragma unroll
        for (int j = 0; j < 4; j++) bf[j] = *(const v4i*)(Ws[cur] + (wn * 64 + j * 16 + lr) * LDSK + lk);
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bf[j], af[i], acc[i][j], 0, 0, 0);
        if (kt + 1 < nk) {
            store_tile(ta, As[cur ^ 1], tid);
            store_tile(tw, Ws[cur ^ 1], tid);
        }
        __syncthreads();
    }

    const int col_base = n0 + wn * 64;  // 64-aligned, one head / one gate-up group
    if (col_base >= a.N) return;
    const int c4 = (lane >> 4) * 4;  // first of this lane's 4 consecutive columns in a 16-wide tile
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int row = m0 + wm * 64 + i * 16 + lr;
        if (row >= a.M) continue;
        if (EPI == EPI_RAW) {
#pragma unroll
            for (int j = 0; j < 4; j++)
                *(int4*)(a.out32 + (size_t)row * a.ldo + col_base + j * 16 + c4) =
                    make_int4(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]);
        } else if (EPI == EPI_REQ) {
#pragma unroll
            for (int j = 0; j < 4; j++)
                *(unsigned*)(a.out8 + (size_t)row * a.ldo + col_base + j * 16 + c4) =
                    pack4i(rq<FAST>(acc[i][j][0], a), rq<FAST>(acc[i][j][1], a), rq<FAST>(acc[i][j][2], a),
                           rq<FAST>(acc[i][j][3], a));
        } else if (EPI == EPI_REGLU) {
            // W rows were permuted so that a 64-row group holds 32 gate rows then the
            // matching 32 up rows: output feature f = col_base/2 + j*16 + c4 + r.
#pragma unroll
            for (int j = 0; j < 2; j++) {
                int o[4];
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int g = rq<FAST>(acc[i][j][r], a);
                    const int u = rq<FAST>(acc[i][j + 2][r], a);
                    const int gr = g > 0 ? g : 0;
                    o[r] = clamp127(rne_shr(gr * u, 7));  // reglu.rs:20-46 (|gr * u| <= 127^2)
                }
                *(unsigned*)(a.out8 + (size_t)row * a.ldo + (col_base >> 1) + j * 16 + c4) = pack4i(o[0], o[1], o[2], o[3]);
            }
        } else {  // EPI_QKV
            const int p = a.pos >= 0 ? a.pos : row % a.T, b = a.pos >= 0 ? row : row / a.T;
            const int kcol = col_base - a.d;
            int g = 0, isv = 0;
            if (kcol >= 0) {
                if (a.kv_mode == 1) { isv = kcol >= 64 * a.G; g = (isv ? kcol - 64 * a.G : kcol) >> 6; }
                else isv = kcol >= 64;
            }
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int i0 = j * 16 + c4;  // rotary pairs (i0 + r, i0 + r + 32)
                int xq[4], yq[4], xv[4], yv[4];
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    xv[r] = rq<FAST>(acc[i][j][r], a);
                    yv[r] = rq<FAST>(acc[i][j + 2][r], a);
                    const int c = a.rcos[p * 32 + i0 + r], s = a.rsin[p * 32 + i0 + r];
                    const int xr = (int)((unsigned)(xv[r] * c) - (unsigned)(yv[r] * s));
                    const int yr = (int)((unsigned)(xv[r] * s) + (unsigned)(yv[r] * c));
                    if (kcol < 0) {
                        // Q: attention.rs:53-83 (>>15 then NET_SHIFT=1, two roundings)
                        xq[r] = clamp127(rne_shr(rne_shr(xr, 15), 1));
                        yq[r] = clamp127(rne_shr(rne_shr(yr, 15), 1));
                    } else {
                        // K: attention.rs:29-50 (|xr|, |yr| <= 2 * 127 * 32768)
                        xq[r] = clamp127(rne_shr(xr, 15));
                        yq[r] = clamp127(rne_shr(yr, 15));
                    }
                }
                if (kcol < 0) {
                    int8_t* q = a.out8 + (size_t)row * a.ldo + col_base;
                    *(unsigned*)(q + i0) = pack4i(xq[0], xq[1], xq[2], xq[3]);
                    *(unsigned*)(q + i0 + 32) = pack4i(yq[0], yq[1], yq[2], yq[3]);
                } else if (!isv) {
                    int8_t* k = a.kc + (((size_t)b * a.KH + g) * a.T + p) * 64;
                    *(unsigned*)(k + i0) = pack4i(xq[0], xq[1], xq[2], xq[3]);
                    *(unsigned*)(k + i0 + 32) = pack4i(yq[0], yq[1], yq[2], yq[3]);
                } else if (a.pos >= 0) {
                    // V of a decode step: key-major like K
                    int8_t* v = a.vc + (((size_t)b * a.KH + g) * a.T + p) * 64;
                    *(unsigned*)(v + i0) = pack4i(xv[0], xv[1], xv[2], xv[3]);
                    *(unsigned*)(v + i0 + 32) = pack4i(yv[0], yv[1], yv[2], yv[3]);
                } else {
                    // V, stored dim-major for the prefill PV operand
                    int8_t* v = a.vc + (((size_t)b * a.KH + g) * 64) * a.TP + p;
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        v[(size_t)(i0 + r) * a.TP] = (int8_t)xv[r];
                        v[(size_t)(i0 + r + 32) * a.TP] = (int8_t)yv[r];
                    }
                }
            }
        }
    }
}

template <int EPI>
static void launch_epi(const GemmArgs& a, dim3 grid, hipStream_t s) {
    if (a.rq_fast)
        hipLaunchKernelGGL((k_gemm<EPI, true>), grid, dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL((k_gemm<EPI, false>), grid, dim3(256), 0, s, a);
}

void launch_gemm(const GemmArgs& a, int epi, hipStream_t s) {
    dim3 grid((unsigned)(((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN)));
    switch (epi) {
        case EPI_RAW: launch_epi<EPI_RAW>(a, grid, s); break;
        case EPI_REQ: launch_epi<EPI_REQ>(a, grid, s); break;
        case EPI_QKV: launch_epi<EPI_QKV>(a, grid, s); break;
        default: launch_epi<EPI_REGLU>(a, grid, s); break;
    }
}

}  // namespace czip
