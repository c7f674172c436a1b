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
template <int CT>
__global__ __launch_bounds__(64 * HNW) void k_head_cdf(HeadCdfArgs a) {
    __shared__ HeadLds L;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int m0 = blockIdx.x * HBM_ROWS;
    const int nb = wave * CT * 16;
    const int lr = lane & 15, c4 = (lane >> 4) * 4;
    // targets of the lane's rows, requested before the reductions
    int tokr[4];
#pragma unroll
    for (int i = 0; i < 4; i++) tokr[i] = m0 + i * 16 + lr < a.M ? (int)a.targets[m0 + i * 16 + lr] : 0;
    v4i acc[4][CT];
    head_freqs<CT>(a.A, a.M, a.K, a.W, a.V, m0, a.lut, a.coef, a.total, L, acc);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int rr = i * 16 + lr;
        const int tok = tokr[i];
        unsigned fs = 0, lo = 0, ft = 0;
#pragma unroll
        for (int t = 0; t < CT; t++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int col = nb + t * 16 + c4 + r;
                const unsigned f = (unsigned)acc[i][t][r];
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

bool head_cdf_supported(int V) { return V == 512 || V == 1024; }

void launch_head_cdf(const HeadCdfArgs& a, hipStream_t s) {
    dim3 grid((unsigned)((a.M + HBM_ROWS - 1) / HBM_ROWS));
    switch (a.V) {
        case 512: hipLaunchKernelGGL(k_head_cdf<2>, grid, dim3(64 * HNW), 0, s, a); break;
        default: hipLaunchKernelGGL(k_head_cdf<4>, grid, dim3(64 * HNW), 0, s, a); break;
    }
}

}  // namespace czip
