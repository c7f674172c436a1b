// The FFN of one layer in one persistent kernel (model.rs:438-468 after the
// pre-FFN norm): up projection + ReGLU (reglu.rs:20-46), down projection,
// post-FFN RMSNorm + residual add, and the next pre-norm, on int8 MFMA.
//
// A workgroup of 8 waves walks strips of R = 16 RT rows.  The strip's
// normalized input (R x d bytes) sits in LDS for the whole strip, the next
// strip's arriving in a second buffer by LDS DMA; the F features go by in
// chunks of 128 (16 per wave):
//   * up: each wave multiplies the strip by its 16 gate and 16 up weight rows
//     (register-resident for the chunk, fragment-major with gate and up tiles
//     interleaved per 16 features), one row tile after the other, applies
//     requant + ReGLU to a tile while the next tile's products run, and writes
//     the 128 output bytes of each row into an LDS chunk buffer (double-buffered);
//   * down: each wave accumulates its d / 8 output columns of every strip row
//     over the chunk's 128 features, the ReGLU bytes read back from LDS.
// The ReGLU output never reaches HBM; per row the kernel reads the d input
// bytes and the int16 residual, and writes the residual and the next norm's
// input.  Weights stream from L2 once per strip per workgroup (the up rows of
// the next chunk load as soon as the last up products have read the current
// ones, during the last row tile's epilogue and the down phase; the down rows
// during the up phase; so no extra registers hold them).  The epilogue is the row GEMM's
// (rn_epilogue in czip_gemm.hip) over R rows.
#include <algorithm>

#include "czip_device.h"
#include "czip_kernels.h"

namespace czip {

constexpr int FFN_NW = 8;    // waves per workgroup
constexpr int FFN_FC = 128;  // features per chunk (16 per wave)

template <int CT, int RT, bool FU, bool FD>
__global__ __launch_bounds__(64 * FFN_NW, 1) void k_ffn(FfnArgs a) {
    constexpr int R = 16 * RT;           // rows per strip
    constexpr int D = FFN_NW * CT * 16;  // d_model
    constexpr int KS = D / 64;           // K steps of the up projection
    // two strips' input, KS tiles of [R][64] each: the current strip's, and
    // the next one's arriving by LDS DMA
    __shared__ __attribute__((aligned(16))) int8_t xs[2][KS * R * 64];
    __shared__ __attribute__((aligned(16))) int8_t rs[2][2 * R * 64];  // 2 tiles of [R][64]: a chunk's ReGLU bytes
    __shared__ unsigned red[FFN_NW][R];
    __shared__ int inv_s[R];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lr = lane & 15, lg = lane >> 4, c4 = lg * 4;
    const int nb = wave * CT * 16;  // this wave's first output column
    const int NC = a.F / FFN_FC, FK = a.F / 64;
    const int nstrips = (a.M + R - 1) / R;
    if ((int)blockIdx.x >= nstrips) return;

    const __amdgpu_buffer_rsrc_t rWu = __builtin_amdgcn_make_buffer_rsrc((void*)a.Wup, (short)0, 2 * a.F * D, BUF_DWORD3);
    const __amdgpu_buffer_rsrc_t rWd = __builtin_amdgcn_make_buffer_rsrc((void*)a.Wdf, (short)0, D * a.F, BUF_DWORD3);

    v4i wu[2][KS];    // gate / up operands of the wave's 16 features of the current chunk
    v4i wd[CT][2];    // down operands of the wave's CT column tiles, the chunk's two K steps
    auto load_wu = [&](int c) {
        const int g = c * FFN_NW + wave;
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int s = 0; s < KS; s++) wu[j][s] = __builtin_amdgcn_raw_buffer_load_b128(rWu, lane * 16, ((2 * g + j) * KS + s) * 1024, 0);
    };
    auto load_wd = [&](int c) {
#pragma unroll
        for (int i = 0; i < CT; i++)
#pragma unroll
            for (int k = 0; k < 2; k++)
                wd[i][k] = __builtin_amdgcn_raw_buffer_load_b128(rWd, lane * 16, ((wave * CT + i) * FK + 2 * c + k) * 1024, 0);
    };
    // strip s's input into xs[b] by LDS DMA (no registers held; rows past M
    // read as 0): a wave instruction fills the 16 rows 16 (q % (R / 16)) .. +16
    // of K step q / (R / 16), lane l the 16 bytes at l * 16 (row + l / 4, slot
    // l % 4 of the permuted row, which holds piece (l % 4) ^ ((row >> 1) & 3))
    auto stage_x = [&](int s, int b) {
        const int m0 = s * R;
        const __amdgpu_buffer_rsrc_t rX =
            __builtin_amdgcn_make_buffer_rsrc((void*)(a.xn + (size_t)m0 * D), (short)0, min(a.M - m0, R) * D, BUF_DWORD3);
#pragma unroll
        for (int q = wave; q < KS * (R / 16); q += FFN_NW) {
            const int ks = q / (R / 16), rq = q % (R / 16);
            const int row = rq * 16 + (lane >> 2), piece = (lane & 3) ^ ((row >> 1) & 3);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rX, (__attribute__((address_space(3))) void*)(xs[b] + ks * R * 64 + rq * 1024), 16,
                row * D + ks * 64 + piece * 16, 0, 0, 0);
        }
    };

    // the norm weights of the wave's columns
    unsigned w1r[CT], w2r[CT];
#pragma unroll
    for (int i = 0; i < CT; i++) {
        w1r[i] = *(const unsigned*)(a.w1 + nb + i * 16 + c4);
        w2r[i] = *(const unsigned*)(a.w2 + nb + i * 16 + c4);
    }
    stage_x(blockIdx.x, 0);
    load_wu(0);

    int xb = 0;  // xs buffer of the current strip
    for (int s = blockIdx.x; s < nstrips; s += gridDim.x, xb ^= 1) {
        const int m0 = s * R;
        const bool more = s + (int)gridDim.x < nstrips;
        v4i acc[RT][CT];
#pragma unroll
        for (int rt = 0; rt < RT; rt++)
#pragma unroll
            for (int i = 0; i < CT; i++) acc[rt][i] = (v4i){0, 0, 0, 0};

        __builtin_amdgcn_s_waitcnt(0);  // the strip's input (and everything before) has landed
        __syncthreads();
        if (more) stage_x(s + gridDim.x, xb ^ 1);  // its buffer was last read by the previous strip
        const int8_t* const xsb = xs[xb];
        for (int c = 0; c < NC; c++) {
            int8_t* rb = rs[c & 1];
            load_wd(c);
            // up + ReGLU of the wave's 16 features, one row tile at a time:
            // tile rt's products issue while tile rt - 1's epilogue runs, one
            // MFMA to every three epilogue VALU (scheduling groups), so that
            // the wave keeps both pipes busy (83.0 vs 85.5 ms per compress
            // step for two row tiles' products, then their epilogue; one MFMA
            // to every two or four VALU, or each K step's operand read placed
            // by the groups too, measured slower, as did no groups at all)
            auto up_mma = [&](int rt, v4i& ug, v4i& uu) {
                ug = (v4i){0, 0, 0, 0};
                uu = (v4i){0, 0, 0, 0};
#pragma unroll
                for (int ks = 0; ks < KS; ks++) {
                    const v4i a0 = *(const v4i*)(xsb + ks * R * 64 + lds64(rt * 16 + lr, lg));
                    ug = __builtin_amdgcn_mfma_i32_16x16x64_i8(wu[0][ks], a0, ug, 0, 0, 0);
                    uu = __builtin_amdgcn_mfma_i32_16x16x64_i8(wu[1][ks], a0, uu, 0, 0, 0);
                }
            };
            auto up_epi = [&](int rt, const v4i& ug, const v4i& uu) {
                int o[4];
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int gt = rq<FU>(ug[r], a.up_scale, a.up_mult, a.up_shift);
                    const int up = rq<FU>(uu[r], a.up_scale, a.up_mult, a.up_shift);
                    o[r] = clamp127(rne_shr((gt > 0 ? gt : 0) * up, 7));  // reglu.rs:20-46 (|.| <= 127^2)
                }
                // features 16 wave + c4 .. +3 of the chunk: tile wave / 4, 16-byte chunk wave % 4
                *(unsigned*)(rb + (wave >> 2) * R * 64 + lds64(rt * 16 + lr, wave & 3) + c4) = pack4i(o[0], o[1], o[2], o[3]);
            };
            v4i ugp, uup;
            up_mma(0, ugp, uup);
#pragma unroll
            for (int rt = 1; rt < RT; rt++) {
                v4i ugn, uun;
                up_mma(rt, ugn, uun);
                up_epi(rt - 1, ugp, uup);
#pragma unroll
                for (int i = 0; i < 2 * KS; i++) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
                    __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);  // three VALU
                }
                ugp = ugn;
                uup = uun;
            }
            // the last products have read the chunk's up operands: the next
            // chunk's (or the next strip's first) load during the last
            // epilogue (compress step 82.0-82.5 -> 78.4-79.5 ms against
            // loading them after the barrier)
            if (c + 1 < NC) load_wu(c + 1);
            else if (more) load_wu(0);
            up_epi(RT - 1, ugp, uup);
            __syncthreads();  // the chunk's ReGLU bytes are complete
            // down: the chunk's two K steps of 64 features
#pragma unroll
            for (int k = 0; k < 2; k++)
#pragma unroll
                for (int rt = 0; rt < RT; rt++) {
                    const v4i af = *(const v4i*)(rb + k * R * 64 + lds64(rt * 16 + lr, lg));
#pragma unroll
                    for (int i = 0; i < CT; i++) acc[rt][i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wd[i][k], af, acc[rt][i], 0, 0, 0);
                }
        }

        // epilogue: y = requant(acc); x = x_in + rmsnorm(y, w1); xn = rmsnorm(clamp(x), w2)
#pragma unroll
        for (int rt = 0; rt < RT; rt++) {
            unsigned ss = 0;
#pragma unroll
            for (int i = 0; i < CT; i++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int y = rq<FD>(acc[rt][i][r], a.dn_scale, a.dn_mult, a.dn_shift);
                    acc[rt][i][r] = y;
                    ss += (unsigned)__mul24(y, y);
                }
            ss += (unsigned)__shfl_xor((int)ss, 16, 64);
            ss += (unsigned)__shfl_xor((int)ss, 32, 64);
            if (lane < 16) red[wave][rt * 16 + lane] = ss;
        }
        __syncthreads();
        auto row_inv = [&]() {
            if (tid < R) {
                unsigned sum = 0;
#pragma unroll
                for (int w = 0; w < FFN_NW; w++) sum += red[w][tid];
                inv_s[tid] = inv_rms_q15_fast((int)(sum / (unsigned)D) + 1);  // eps_scaled = 1 (rmsnorm.rs:80-83)
            }
            __syncthreads();
        };
        row_inv();
#pragma unroll
        for (int rt = 0; rt < RT; rt++) {
            const int row = m0 + rt * 16 + lr;
            const bool live = row < a.M;
            const double inv = (double)inv_s[rt * 16 + lr] * (1.0 / 32768.0);
            unsigned ss = 0;
            uint2 xi[CT];
            const int rrow = min(row, a.M - 1);
#pragma unroll
            for (int i = 0; i < CT; i++) xi[i] = *(const uint2*)(a.x_in + (size_t)rrow * D + nb + i * 16 + c4);
#pragma unroll
            for (int i = 0; i < CT; i++) {
                int w1v[4], xo[4], xnw[4];
                unpack4s(w1r[i], w1v);
                xo[0] = (int16_t)(xi[i].x & 0xFFFFu); xo[1] = (int16_t)(xi[i].x >> 16);
                xo[2] = (int16_t)(xi[i].y & 0xFFFFu); xo[3] = (int16_t)(xi[i].y >> 16);
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    xnw[r] = xo[r] + rms_el(acc[rt][i][r], w1v[r], inv);
                    const int xc = clamp127(xnw[r]);
                    acc[rt][i][r] = xc;
                    ss += (unsigned)__mul24(xc, xc);
                }
                if (a.x_out && live)
                    *(uint2*)(a.x_out + (size_t)row * D + nb + i * 16 + c4) =
                        make_uint2(((unsigned)xnw[0] & 0xFFFFu) | ((unsigned)xnw[1] << 16),
                                   ((unsigned)xnw[2] & 0xFFFFu) | ((unsigned)xnw[3] << 16));
            }
            ss += (unsigned)__shfl_xor((int)ss, 16, 64);
            ss += (unsigned)__shfl_xor((int)ss, 32, 64);
            if (lane < 16) red[wave][rt * 16 + lane] = ss;
        }
        __syncthreads();
        row_inv();
#pragma unroll
        for (int rt = 0; rt < RT; rt++) {
            const int row = m0 + rt * 16 + lr;
            if (row >= a.M) continue;
            const double inv = (double)inv_s[rt * 16 + lr] * (1.0 / 32768.0);
#pragma unroll
            for (int i = 0; i < CT; i++) {
                int w2v[4];
                unpack4s(w2r[i], w2v);
                *(unsigned*)(a.xn_out + (size_t)row * D + nb + i * 16 + c4) =
                    pack4i(rms_el(acc[rt][i][0], w2v[0], inv), rms_el(acc[rt][i][1], w2v[1], inv),
                           rms_el(acc[rt][i][2], w2v[2], inv), rms_el(acc[rt][i][3], w2v[3], inv));
            }
        }
    }
}

// d = 384 (8 waves x 3 column tiles, 128-row strips); wider models keep the
// separate up and down kernels (their weights per strip would not fit registers)
bool ffn_supported(int d, int F) { return d == 384 && F % FFN_FC == 0 && F >= FFN_FC; }

template <int CT, int RT>
static void launch_ffn_t(const FfnArgs& a, hipStream_t s) {
    constexpr int R = 16 * RT;
    const int nstrips = (a.M + R - 1) / R;
    dim3 grid((unsigned)std::min(nstrips, 256));  // one workgroup per CU
    if (a.up_fast && a.dn_fast) hipLaunchKernelGGL((k_ffn<CT, RT, true, true>), grid, dim3(64 * FFN_NW), 0, s, a);
    else if (a.up_fast) hipLaunchKernelGGL((k_ffn<CT, RT, true, false>), grid, dim3(64 * FFN_NW), 0, s, a);
    else if (a.dn_fast) hipLaunchKernelGGL((k_ffn<CT, RT, false, true>), grid, dim3(64 * FFN_NW), 0, s, a);
    else hipLaunchKernelGGL((k_ffn<CT, RT, false, false>), grid, dim3(64 * FFN_NW), 0, s, a);
}

void launch_ffn(const FfnArgs& a, hipStream_t s) {
    if (a.M > 0 && a.d == 384) launch_ffn_t<3, 8>(a, s);
}

}  // namespace czip
