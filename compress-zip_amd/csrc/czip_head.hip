// LM head fused with the logits -> coder interval stage (model.rs:470-477 +
// softmax_cdf.rs:85-139): the int32 logits of a row never leave the chip.
#include "czip_device.h"
#include "czip_kernels.h"

namespace czip {

// ---------------------------------------------------------------------------
// A workgroup owns 64 token rows and all V logits of each (16 waves, wave w
// holds columns [w*V/16, (w+1)*V/16) as CT = V/256 MFMA tiles of 16).  The
// K loop is the row GEMM's: the 64 x 64 A tile of each K step through
// double-buffered LDS, each wave's W columns straight into registers.  The
// epilogue reproduces k_cdf's mode 0 per row with three block reductions:
//   1. max logit;
//   2. first argmax, S = sum E(l - max);
//   3. sum f, f below the target and f of the target, with
//      f = 1 + e*Q + floor(e*Rm / S) (Q = R / S, Rm = R % S, R = total - V),
//      the small floor quotient exact in f64.
// Lane l holds logits of rows 16 i + l % 16 (i < 4) at columns
// 16 t + 4 (l / 16) .. +3 of its wave's range (t < CT).
// ---------------------------------------------------------------------------
constexpr int HBM_ROWS = 64, HNW = 16;

template <int CT>
__global__ __launch_bounds__(64 * HNW) void k_head_cdf(HeadCdfArgs a) {
    __shared__ __attribute__((aligned(16))) int8_t As[2][HBM_ROWS * 64];
    __shared__ unsigned lut32[256];
    __shared__ int red_a[HNW][HBM_ROWS];
    __shared__ unsigned red_b[HNW][HBM_ROWS], red_c[HNW][HBM_ROWS];
    __shared__ int row_i[HBM_ROWS], row_am[HBM_ROWS];
    __shared__ unsigned row_Q[HBM_ROWS];
    __shared__ double row_Rm[HBM_ROWS], row_inv[HBM_ROWS];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int m0 = blockIdx.x * HBM_ROWS;
    const int nb = wave * CT * 16;
    const int lr = lane & 15, c4 = (lane >> 4) * 4;
    if (tid < 256) lut32[tid] = (unsigned)a.lut[tid] << 16;

    v4i acc[4][CT];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int t = 0; t < CT; t++) acc[i][t] = (v4i){0, 0, 0, 0};
    rowblock_mma<CT>(a.A, a.M, a.K, a.W, a.V, m0, nb, As, acc);

    // targets of the lane's rows, requested before the reductions
    int tokr[4];
#pragma unroll
    for (int i = 0; i < 4; i++) tokr[i] = m0 + i * 16 + lr < a.M ? (int)a.targets[m0 + i * 16 + lr] : 0;
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
        if (lane < 16) red_a[wave][i * 16 + lane] = mx;
    }
    __syncthreads();
    if (wave == 0) {
        int mx = red_a[0][lane];
#pragma unroll
        for (int w = 1; w < HNW; w++) mx = max(mx, red_a[w][lane]);
        row_i[lane] = mx;
    }
    __syncthreads();
    // 2. first argmax and S = sum of e = E(l - max) (softmax_cdf.rs:96-110)
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int mx = row_i[i * 16 + lr];
        int am = 0x7FFFFFFF;
        unsigned s = 0;
#pragma unroll
        for (int t = 0; t < CT; t++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int col = nb + t * 16 + c4 + r;
                const int l = acc[i][t][r];
                am = (l == mx && col < am) ? col : am;
                const unsigned e = exp_q16_bf((int)((unsigned)l - (unsigned)mx), lut32, a.coef);
                acc[i][t][r] = (int)e;
                s += e;
            }
        am = min(am, __shfl_xor(am, 16, 64));
        am = min(am, __shfl_xor(am, 32, 64));
        s += (unsigned)__shfl_xor((int)s, 16, 64);
        s += (unsigned)__shfl_xor((int)s, 32, 64);
        if (lane < 16) {
            red_a[wave][i * 16 + lane] = am;
            red_b[wave][i * 16 + lane] = s;
        }
    }
    __syncthreads();
    if (wave == 0) {
        int am = red_a[0][lane];
        unsigned S = red_b[0][lane];
#pragma unroll
        for (int w = 1; w < HNW; w++) {
            am = min(am, red_a[w][lane]);
            S += red_b[w][lane];
        }
        const unsigned R = a.total - (unsigned)a.V;  // S <= 1024 * 65535 < 2^26
        const unsigned Q = R / S;
        row_am[lane] = am;
        row_Q[lane] = Q;
        row_Rm[lane] = (double)(R - Q * S);
        row_inv[lane] = 1.0 / (double)S;
    }
    __syncthreads();
    // 3. f = 1 + e*Q + floor(e*Rm/S); sum f, f below the target, f of the target.
    // floor(e*Rm/S) = floor(fma(e*Rm, 1/S, 2^-30)) in f64: e*Rm < 2^42 is exact,
    // a nonzero fraction of e*Rm/S is >= 1/S >= 2^-26, and the f64 error of the
    // product with the rounded 1/S is < 2^-35 for quotients below 2^16.
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int rr = i * 16 + lr;
        const unsigned Q = row_Q[rr];
        const double Rm = row_Rm[rr], inv = row_inv[rr];
        const int tok = tokr[i];
        unsigned fs = 0, lo = 0, ft = 0;
#pragma unroll
        for (int t = 0; t < CT; t++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int col = nb + t * 16 + c4 + r;
                const unsigned e = (unsigned)acc[i][t][r];
                const unsigned q = (unsigned)__builtin_fma((double)e * Rm, inv, 0x1p-30);
                const unsigned f = 1u + e * Q + q;
                fs += f;
                lo += col < tok ? f : 0u;
                ft += col == tok ? f : 0u;
            }
        fs += (unsigned)__shfl_xor((int)fs, 16, 64);
        fs += (unsigned)__shfl_xor((int)fs, 32, 64);
        lo += (unsigned)__shfl_xor((int)lo, 16, 64);
        lo += (unsigned)__shfl_xor((int)lo, 32, 64);
        ft += (unsigned)__shfl_xor((int)ft, 16, 64);
        ft += (unsigned)__shfl_xor((int)ft, 32, 64);
        if (lane < 16) {
            red_a[wave][rr] = (int)fs;
            red_b[wave][rr] = lo;
            red_c[wave][rr] = ft;
        }
    }
    __syncthreads();
    if (wave == 0) {
        const int row = m0 + lane;
        if (row < a.M && (row % a.T) < a.lens[row / a.T]) {
            unsigned fs = 0, lo = 0, ft = 0;
#pragma unroll
            for (int w = 0; w < HNW; w++) {
                fs += (unsigned)red_a[w][lane];
                lo += red_b[w][lane];
                ft += red_c[w][lane];
            }
            const unsigned rem = a.total - fs;  // the argmax takes the remainder
            const int tok = (int)a.targets[row], am = row_am[lane];
            if (am < tok) lo += rem;
            if (am == tok) ft += rem;
            a.out[(size_t)(a.out_row0 + row) * 2] = lo;
            a.out[(size_t)(a.out_row0 + row) * 2 + 1] = lo + ft;
        }
    }
}

bool head_cdf_supported(int V) { return V == 512 || V == 1024; }

void launch_head_cdf(const HeadCdfArgs& a, hipStream_t s) {
    dim3 grid((unsigned)((a.M + HBM_ROWS - 1) / HBM_ROWS));
    switch (a.V) {
        case 512: hipLaunchKernelGGL(k_head_cdf<2>, grid, dim3(64 * HNW), 0, s, a); break;
        default: hipLaunchKernelGGL(k_head_cdf<4>, grid, dim3(64 * HNW), 0, s, a); break;
    }
}

}  // namespace czip
