// LM head fused with the logits -> coder interval stage (model.rs:470-477 +
// softmax_cdf.rs:85-139): the int32 logits of a row never leave the chip.
#include "czip_head.h"
#include "czip_kernels.h"

namespace czip {

// ---------------------------------------------------------------------------
// Compress: the frequency table of each row (head_freqs) reduced to the
// coder interval of its target token (k_cdf's mode 0): sum f, f below the
// target and f of the target, the argmax taking the remainder total - sum f.
// ---------------------------------------------------------------------------
// Persistent: a workgroup (one per CU) walks row blocks blockIdx.x,
// + gridDim.x, ..., the next block's A arriving in LDS by DMA while the
// current one is reduced.
template <int CT, bool E0>
__global__ __launch_bounds__(64 * HNW) void k_head_cdf(HeadCdfArgs a) {
    __shared__ HeadLdsT<2> L;
    const int nblk = (a.M + HBM_ROWS - 1) / HBM_ROWS;
    head_etab_fill(L, a.lut);
    head_stage_a(a.A, a.M, a.K, (int)blockIdx.x * HBM_ROWS, L.As[0]);
    int buf = 0;
    for (int blk = (int)blockIdx.x; blk < nblk; blk += (int)gridDim.x, buf ^= 1) {
        const int tid = opaque_tid(), wave = tid >> 6, lane = tid & 63;
        const int nb = wave * CT * 16;
        const int lr = lane & 15, c4 = (lane >> 4) * 4;
        const int m0 = blk * HBM_ROWS;
        // targets of the lane's rows, requested before the reductions
        int tokr[4];
#pragma unroll
        for (int i = 0; i < 4; i++) tokr[i] = m0 + i * 16 + lr < a.M ? (int)a.targets[m0 + i * 16 + lr] : 0;
        __builtin_amdgcn_s_waitcnt(0);  // this block's A (and everything before) has landed
        __syncthreads();
        if (blk + (int)gridDim.x < nblk) head_stage_a(a.A, a.M, a.K, (blk + (int)gridDim.x) * HBM_ROWS, L.As[buf ^ 1]);
        v4i acc[4][CT];
        head_freqs<CT, E0>(tid, L.As[buf], a.K, a.W, a.V, a.coef, a.total, L, acc);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int rr = i * 16 + lr;
            // the lane's columns of tile t are nb + 16 t + c4 + (0..3): whole
            // groups below the target count in full; the group that holds the
            // target (kt = 16 t + r, r < 4; at most one per lane) gives the
            // columns before it and f(target)
            const int kt = tokr[i] - (nb + c4);
            unsigned fs = 0, lo = 0;
            v4i grp_t = acc[i][0];
#pragma unroll
            for (int t = 0; t < CT; t++) {
                const unsigned p = (unsigned)acc[i][t][0] + (unsigned)acc[i][t][1] + (unsigned)acc[i][t][2] + (unsigned)acc[i][t][3];
                fs += p;
                lo += kt >= 16 * t + 4 ? p : 0u;
                if (t > 0) grp_t = (kt >> 4) == t ? acc[i][t] : grp_t;
            }
            const int r = kt & 15;
            const bool holds = kt >= 0 && kt < 16 * CT && r < 4;
            const unsigned part = (r > 0 ? (unsigned)grp_t[0] : 0u) + (r > 1 ? (unsigned)grp_t[1] : 0u) +
                                  (r > 2 ? (unsigned)grp_t[2] : 0u);
            const unsigned fr = r == 0 ? (unsigned)grp_t[0] : r == 1 ? (unsigned)grp_t[1] : r == 2 ? (unsigned)grp_t[2] : (unsigned)grp_t[3];
            lo += holds ? part : 0u;
            unsigned ft = holds ? fr : 0u;
            fs += (unsigned)__shfl_xor((int)fs, 16, 64);
            fs += (unsigned)__shfl_xor((int)fs, 32, 64);
            lo += (unsigned)__shfl_xor((int)lo, 16, 64);
            lo += (unsigned)__shfl_xor((int)lo, 32, 64);
            ft += (unsigned)__shfl_xor((int)ft, 16, 64);
            ft += (unsigned)__shfl_xor((int)ft, 32, 64);
            if (lane < 16) {
                L.red_a[wave][rr] = (int)fs;
                L.red_b[wave][rr] = lo;
                L.red_c[wave][rr] = ft;
            }
        }
        __syncthreads();
        if (wave == 0) {
            const int row = m0 + lane;
            if (row < a.M && (row % a.T) < a.lens[row / a.T]) {
                unsigned fs = 0, lo = 0, ft = 0;
#pragma unroll
                for (int w = 0; w < HNW; w++) {
                    fs += (unsigned)L.red_a[w][lane];
                    lo += L.red_b[w][lane];
                    ft += L.red_c[w][lane];
                }
                const unsigned rem = a.total - fs;  // the argmax takes the remainder
                const int tok = (int)a.targets[row], am = L.row_am[lane];
                if (am < tok) lo += rem;
                if (am == tok) ft += rem;
                a.out[(size_t)(a.out_row0 + row) * 2] = lo;
                a.out[(size_t)(a.out_row0 + row) * 2 + 1] = lo + ft;
            }
        }
    }
}

// V = 1024 (16 waves x 4 tiles of 16 columns): the fused heads serve the
// coder paths, which feed BOS = 1022 and so need V > 1022; other vocabularies
// take the LM head GEMM + k_cdf
bool head_cdf_supported(int V) { return V == 1024; }

void launch_head_cdf(const HeadCdfArgs& a, hipStream_t s) {
    dim3 grid((unsigned)std::min((a.M + HBM_ROWS - 1) / HBM_ROWS, HEAD_GRID));
    if (a.e0) hipLaunchKernelGGL((k_head_cdf<4, true>), grid, dim3(64 * HNW), 0, s, a);
    else hipLaunchKernelGGL((k_head_cdf<4, false>), grid, dim3(64 * HNW), 0, s, a);
}

}  // namespace czip
