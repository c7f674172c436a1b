// The LM head and the frequency table of a block of 64 rows, shared by the
// compress interval stage (czip_head.hip) and the decode step (czip_decode.hip):
// model.rs:470-477 + softmax_cdf.rs:85-139 with the int32 logits kept on chip.
#pragma once

#include "czip_device.h"

namespace czip {

// A workgroup owns 64 token rows and all V logits of each (16 waves, wave w
// holds columns [w*V/16, (w+1)*V/16) as CT = V/256 MFMA tiles of 16).  Lane l
// holds rows 16 i + l % 16 (i < 4) at columns 16 t + 4 (l / 16) .. +3 of its
// wave's range (t < CT).
constexpr int HBM_ROWS = 64, HNW = 16;

// E(t) (exp_q16 at table step t, lut.rs:213-235) for every step t < 4096 and
// t = 4096 standing for all larger ones: (65536 >> ip) * lut[t & 255] rounds
// to at most 1 for ip = t >> 8 >= 16, and the clamp makes it 1.  Entry 4097
// is E(0) = 65535 of a logit equal to the max (diff >= 0 in the reference,
// whatever lut[0] holds).
constexpr int ETAB_N = 4098;

constexpr int HEAD_GRID = 256;   // persistent head kernels: one workgroup (16 waves, 4 per SIMD) per CU
constexpr int HEAD_KMAX = 1024;  // the whole K of a row block staged at once (d_model <= 1024)
// NA row blocks of A (K / 64 tiles of [64][64], 64-byte permuted rows): the
// persistent compress head holds two (the one being multiplied and the next
// one arriving), the decode head one
template <int NA>
struct HeadLdsT {
    int8_t As[NA][HEAD_KMAX / 64][HBM_ROWS * 64] __attribute__((aligned(16)));
    unsigned etab[ETAB_N + 2];
    int red_a[HNW][HBM_ROWS];
    unsigned red_b[HNW][HBM_ROWS], red_c[HNW][HBM_ROWS];
    int row_i[HBM_ROWS], row_am[HBM_ROWS];
    unsigned row_Q[HBM_ROWS];
    double row_y[HBM_ROWS];
};

// The exp table of head_freqs, built once per workgroup.
template <class Lds>
__device__ __forceinline__ void head_etab_fill(Lds& L, const uint16_t* lut) {
    for (int t = threadIdx.x; t < ETAB_N; t += 64 * HNW) {
        const unsigned ip = (unsigned)t >> 8;
        const unsigned x = ip >= 16u ? 1u : ((65536u >> ip) * (unsigned)lut[t & 255] + 0x8000u) >> 16;
        L.etab[t] = t == ETAB_N - 1 ? 65535u : (x < 1u ? 1u : (x > 65535u ? 65535u : x));
    }
}

// threadIdx.x with a value the compiler cannot follow across loop iterations
__device__ __forceinline__ int opaque_tid() {
    int t = (int)threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}

// Requests the 64 x K block of A at row m0 into As by LDS DMA (no registers
// held; rows past M read as 0): each wave instruction fills 1 KB, the 16 rows
// 16 (q % 4) .. +16 of K step q / 4, lane l writing the 16 bytes at l * 16,
// i.e. row 16 (q % 4) + l / 4, slot l % 4 of the permuted row (lds64), which
// holds the row's 16-byte piece (l % 4) ^ ((row >> 1) & 3).  The caller waits
// for the loads (s_waitcnt) and then for every wave (a barrier).
__device__ __forceinline__ void head_stage_a(const int8_t* A, int M, int K, int m0, int8_t (*As)[HBM_ROWS * 64]) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int arows = M - m0 < HBM_ROWS ? M - m0 : HBM_ROWS;
    const __amdgpu_buffer_rsrc_t rA =
        __builtin_amdgcn_make_buffer_rsrc((void*)(A + (size_t)m0 * K), (short)0, arows * K, BUF_DWORD3);
    for (int q = wave; q < (K / 64) * 4; q += HNW) {
        const int kt = q >> 2, row = (q & 3) * 16 + (lane >> 2);
        const int piece = (lane & 3) ^ ((row >> 1) & 3);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rA, (__attribute__((address_space(3))) void*)(As[kt] + (q & 3) * 1024), 16,
                                                 row * K + kt * 64 + piece * 16, 0, 0, 0);
    }
}

// Logits of a row block staged in As (its K steps from LDS, each wave's W
// columns one step ahead in registers), then per row, with two block
// reductions:
//   1. max logit;
//   2. first argmax (row_am) and S = sum E(l - max) (softmax_cdf.rs:96-110,
//      coef < 2^24);
// and every element's frequency f = 1 + e*Q + floor(e*Rm / S) (Q = R / S,
// Rm = R % S, R = total - V) in place of its logit.  1 + floor(e*Rm/S) is
// the truncation of fma(e, y, 1 + 2^-30) in f64 with y = Rm / S correctly
// rounded (|y - Rm/S| <= 2^-54, y < 1): the result is below 2^16 + 2, so
// its error is < 2^16 * 2^-54 + 2^-37 < 2^-36, while a nonzero fraction of
// e*Rm/S is >= 1/S >= 2^-26 (S < 2^26).  The argmax's remainder
// (total - sum f) is left to the caller.
// tid: threadIdx.x, passed in so that a persistent caller can make it opaque
// per block (the lane-dependent addresses are then formed per block instead
// of being held in registers across the whole loop).  E0: lut[0] == 65535,
// so step 0 (where a logit equal to the max lands) already reads 65535 and
// the max needs no entry of its own.
template <int CT, bool E0, class Lds>
__device__ __forceinline__ void head_freqs(int tid, const int8_t (*As)[HBM_ROWS * 64], int K, const int8_t* W, int V,
                                           unsigned coef, unsigned total, Lds& L, v4i (&acc)[4][CT]) {
    const int wave = tid >> 6, lane = tid & 63;
    const int nb = wave * CT * 16;
    const int lr = lane & 15, c4 = (lane >> 4) * 4;
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int t = 0; t < CT; t++) acc[i][t] = (v4i){0, 0, 0, 0};
    rowblock_mma_lds<CT>(lane, K, W, V, nb, As, acc);

    // 1. row max
#pragma unroll
    for (int i = 0; i < 4; i++) {
        int mx = INT32_MIN;
#pragma unroll
        for (int t = 0; t < CT; t++)
#pragma unroll
            for (int r = 0; r < 4; r++) mx = max(mx, acc[i][t][r]);
        mx = max(mx, __shfl_xor(mx, 16, 64));
        mx = max(mx, __shfl_xor(mx, 32, 64));
        if (lane < 16) L.red_a[wave][i * 16 + lane] = mx;
    }
    __syncthreads();
    if (wave == 0) {
        int mx = L.red_a[0][lane];
#pragma unroll
        for (int w = 1; w < HNW; w++) mx = max(mx, L.red_a[w][lane]);
        L.row_i[lane] = mx;
    }
    __syncthreads();
    // 2. first argmax and S = sum of e = E(l - max).  The table step of
    // E(-n) is t = floor((n * coef + 2^23) / 2^24): for coef < 2^24 the high
    // word of n * (coef * 256) + 2^31, one 32 x 32 + 64 multiply-add; every
    // step past 4096 reads as 4096.  The lane's columns are walked from the
    // last, so the last match left is its first maximum.
    // With c = coef * 256 (< 2^31: coef < 2^23) and K = mx * c + 2^31 per
    // row, n * c + 2^31 = K - l * c: one signed 32 x 32 + 64 multiply-add of
    // the logit.  The equal-to-max case is an index (entry 4097), so every
    // element reads the table unconditionally; the argmax is kept as the
    // lane's element index k (an inline constant) and turned into a column once.
    const int negc = -(int)(coef << 8);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int mx = L.row_i[i * 16 + lr];
        const long long kr = (long long)mx * (long long)(coef << 8) + 0x80000000ll;
        int ak = 64;
        unsigned s = 0;
#pragma unroll
        for (int t = CT - 1; t >= 0; t--)
#pragma unroll
            for (int r = 3; r >= 0; r--) {
                const int l = acc[i][t][r];
                ak = l == mx ? t * 4 + r : ak;
                const unsigned st = min((unsigned)((unsigned long long)((long long)l * (long long)negc + kr) >> 32), 4096u);
                const unsigned e = L.etab[E0 || l != mx ? (int)st : ETAB_N - 1];
                acc[i][t][r] = (int)e;
                s += e;
            }
        int am = ak == 64 ? 0x7FFFFFFF : nb + (ak >> 2) * 16 + c4 + (ak & 3);
        am = min(am, __shfl_xor(am, 16, 64));
        am = min(am, __shfl_xor(am, 32, 64));
        s += (unsigned)__shfl_xor((int)s, 16, 64);
        s += (unsigned)__shfl_xor((int)s, 32, 64);
        if (lane < 16) {
            L.red_a[wave][i * 16 + lane] = am;
            L.red_b[wave][i * 16 + lane] = s;
        }
    }
    __syncthreads();
    if (wave == 0) {
        int am = L.red_a[0][lane];
        unsigned S = L.red_b[0][lane];
#pragma unroll
        for (int w = 1; w < HNW; w++) {
            am = min(am, L.red_a[w][lane]);
            S += L.red_b[w][lane];
        }
        const unsigned R = total - (unsigned)V;  // S <= 1024 * 65535 < 2^26
        const unsigned Q = R / S;
        L.row_am[lane] = am;
        L.row_Q[lane] = Q;
        L.row_y[lane] = (double)(R - Q * S) / (double)S;
    }
    __syncthreads();
    // f in place of e
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int rr = i * 16 + lr;
        const unsigned Q = L.row_Q[rr];
        const double y = L.row_y[rr];
#pragma unroll
        for (int t = 0; t < CT; t++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const unsigned e = (unsigned)acc[i][t][r];
                const unsigned q1 = (unsigned)__builtin_fma((double)e, y, 1.0 + 0x1p-30);  // 1 + floor(e*Rm/S)
                acc[i][t][r] = (int)(__umul24(e, Q) + q1);  // e < 2^16, Q < 2^15
            }
    }
}

}  // namespace czip
