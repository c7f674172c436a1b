// Row-wise kernels: chunk preparation, embedding + RMSNorm, residual + RMSNorm,
// logits -> cumulative frequencies, and the arithmetic encoder.
#include "czip_device.h"
#include "czip_kernels.h"

namespace czip {

// ---------------------------------------------------------------------------
// Chunk preparation: inputs [BOS, t0..t_{n-2}] and targets per chunk
// (main.rs:209-226).  Padding rows get token 0 and are never read back.
// ---------------------------------------------------------------------------
__global__ void k_prep_chunks(const uint32_t* __restrict__ toks, long long n, long long chunk0, int nb, int T,
                              uint32_t* __restrict__ inp, uint32_t* __restrict__ tgt, int32_t* __restrict__ lens) {
    long long row = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (row >= (long long)nb * T) return;
    int b = (int)(row / T), p = (int)(row % T);
    long long start = (chunk0 + b) * (long long)T;
    long long len = n - start;
    if (len > T) len = T;
    if (len < 0) len = 0;
    if (p == 0) lens[b] = (int32_t)len;
    if (p < len) {
        inp[row] = p == 0 ? BOS_TOKEN : toks[start + p - 1];
        tgt[row] = toks[start + p];
    } else {
        inp[row] = 0u;
        tgt[row] = 0u;
    }
}

void launch_prep_chunks(const uint32_t* toks, int64_t n, int64_t chunk0, int nb, int T, uint32_t* inp,
                        uint32_t* tgt, int32_t* lens, hipStream_t s) {
    long long rows = (long long)nb * T;
    hipLaunchKernelGGL(k_prep_chunks, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, s, toks, (long long)n,
                       (long long)chunk0, nb, T, inp, tgt, lens);
}

// ---------------------------------------------------------------------------
// Row kernels: one wavefront per token row, d <= 1024.  Lane l owns the
// 4-element groups g = l, l + 64, ... (elements 4g .. 4g+3), so loads and
// stores are 4-byte (int8) or 16-byte (int32) vectors.
// ---------------------------------------------------------------------------
constexpr int RG = 4;  // groups per lane: d <= 64 * 4 * RG

struct RowI8 {
    int v[RG][4];
};

__device__ __forceinline__ void unpack4(unsigned w, int* o) {
    o[0] = (int)(int8_t)(w & 0xFF);
    o[1] = (int)(int8_t)((w >> 8) & 0xFF);
    o[2] = (int)(int8_t)((w >> 16) & 0xFF);
    o[3] = (int)(int8_t)(w >> 24);
}
__device__ __forceinline__ unsigned pack4(const int* v) {
    return ((unsigned)(uint8_t)(int8_t)v[0]) | ((unsigned)(uint8_t)(int8_t)v[1] << 8) |
           ((unsigned)(uint8_t)(int8_t)v[2] << 16) | ((unsigned)(uint8_t)(int8_t)v[3] << 24);
}

// rmsnorm.rs:40-75 on the wave-distributed row: y = clamp(sra_rne((x*w)*inv, 15))
__device__ __forceinline__ void rms_row(const RowI8& x, const int8_t* __restrict__ w, int d, int lane, RowI8& y) {
    const int ng = d >> 2;
    unsigned ss = 0;
#pragma unroll
    for (int j = 0; j < RG; j++)
        if (lane + 64 * j < ng)
#pragma unroll
            for (int k = 0; k < 4; k++) ss += (unsigned)(x.v[j][k] * x.v[j][k]);
    ss = wave_sum_u(ss);
    const int mean_sq = (int)(ss / (unsigned)d) + 1;  // eps_scaled = 1 (rmsnorm.rs:80-83); <= 127^2 + 1
    const int inv = inv_rms_q15_fast(mean_sq);
#pragma unroll
    for (int j = 0; j < RG; j++) {
        const int g = lane + 64 * j;
        if (g < ng) {
            int wv[4];
            unpack4(*(const unsigned*)(w + 4 * g), wv);
#pragma unroll
            for (int k = 0; k < 4; k++) {
                int tmp = (int)((unsigned)(x.v[j][k] * wv[k]) * (unsigned)inv);
                y.v[j][k] = clamp127(sra_rne32(tmp, 15));
            }
        }
    }
}

// x = E[tok] (model.rs:372-374); xn = rmsnorm(clamp(x), w) (model.rs:384-385).
// Sixteen lanes per row, four rows per wavefront: lane s of a row owns the
// 4-element groups g = s, s + 16, ... (d <= 1024: at most 16 groups), so the
// four rows' gather -> reduce -> normalize chains overlap.
__global__ __launch_bounds__(256) void k_embed_norm(const uint32_t* __restrict__ inp, const int8_t* __restrict__ embed,
                                                    const int8_t* __restrict__ w, int M, int d,
                                                    int16_t* __restrict__ x, int8_t* __restrict__ xn) {
    constexpr int G16 = 16;  // groups per lane: d <= 16 * 4 * 16
    const int row = blockIdx.x * 16 + (threadIdx.x >> 4);
    const int sl = threadIdx.x & 15;
    const bool live = row < M;
    const int ng = d >> 2;
    const int8_t* e = embed + (size_t)(live ? inp[row] : 0u) * d;
    unsigned raw[G16];
#pragma unroll
    for (int j = 0; j < G16; j++) {
        const int g = sl + 16 * j;
        raw[j] = g < ng ? *(const unsigned*)(e + 4 * g) : 0u;
    }
    unsigned ss = 0;
#pragma unroll
    for (int j = 0; j < G16; j++) {
        int v[4];
        unpack4(raw[j], v);
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int c = clamp127(v[k]);
            ss += (unsigned)(c * c);
        }
    }
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) ss += (unsigned)__shfl_xor((int)ss, o, 64);
    const int inv = inv_rms_q15_fast((int)(ss / (unsigned)d) + 1);  // eps_scaled = 1 (rmsnorm.rs:80-83)
    if (!live) return;
#pragma unroll
    for (int j = 0; j < G16; j++) {
        const int g = sl + 16 * j;
        if (g < ng) {
            int v[4], wv[4], y[4];
            unpack4(raw[j], v);
            unpack4(*(const unsigned*)(w + 4 * g), wv);
            if (x) {
                const unsigned lo = ((unsigned)v[0] & 0xFFFFu) | ((unsigned)v[1] << 16);
                const unsigned hi = ((unsigned)v[2] & 0xFFFFu) | ((unsigned)v[3] << 16);
                *(uint2*)(x + (size_t)row * d + 4 * g) = make_uint2(lo, hi);
            }
#pragma unroll
            for (int k = 0; k < 4; k++) y[k] = clamp127(rne_shr(clamp127(v[k]) * wv[k] * inv, 15));
            *(unsigned*)(xn + (size_t)row * d + 4 * g) = pack4(y);
        }
    }
}

void launch_embed_norm(const uint32_t* inp, const int8_t* embed, const int8_t* w, int M, int d, int16_t* x,
                       int8_t* xn, hipStream_t s) {
    hipLaunchKernelGGL(k_embed_norm, dim3((unsigned)((M + 15) / 16)), dim3(256), 0, s, inp, embed, w, M, d, x, xn);
}

// ---------------------------------------------------------------------------
// Epilogue of the split-K row GEMM, one wavefront per row: sum the K slices'
// int32 partials (wrapping, like the accumulator), requantize, add the
// residual (the int16 stream or the token's embedding row), both RMSNorms
// (model.rs:424-468): the same arithmetic as the fused row GEMM's epilogue.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_rn_splitk_epi(RowGemmArgs a, const int32_t* __restrict__ part, int splits) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= a.M) return;
    const int d = a.d, ng = d >> 2;
    RowI8 yi, yn, xi;
#pragma unroll
    for (int j = 0; j < RG; j++) {
        const int g = lane + 64 * j;
        if (g < ng) {
            unsigned acc[4] = {0u, 0u, 0u, 0u};
            for (int sp = 0; sp < splits; sp++) {
                const int4 v = *(const int4*)(part + ((size_t)sp * a.M + row) * d + 4 * g);
                acc[0] += (unsigned)v.x; acc[1] += (unsigned)v.y; acc[2] += (unsigned)v.z; acc[3] += (unsigned)v.w;
            }
#pragma unroll
            for (int k = 0; k < 4; k++)
                yi.v[j][k] = a.rq_fast ? clamp127(rint_fma_i32((double)(int)acc[k], a.rq_scale))
                                       : requant((int)acc[k], a.mult, a.shift);
        }
    }
    rms_row(yi, a.w1, d, lane, yn);
    const int8_t* erow = a.x_in ? nullptr : a.embed + (size_t)a.tok[row] * d;
#pragma unroll
    for (int j = 0; j < RG; j++) {
        const int g = lane + 64 * j;
        if (g < ng) {
            int xo[4];
            if (a.x_in) {
                const uint2 xv = *(const uint2*)(a.x_in + (size_t)row * d + 4 * g);
                xo[0] = (int16_t)(xv.x & 0xFFFFu); xo[1] = (int16_t)(xv.x >> 16);
                xo[2] = (int16_t)(xv.y & 0xFFFFu); xo[3] = (int16_t)(xv.y >> 16);
            } else {
                unpack4(*(const unsigned*)(erow + 4 * g), xo);
            }
            int nv[4];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                nv[k] = xo[k] + yn.v[j][k];
                xi.v[j][k] = clamp127(nv[k]);
            }
            if (a.x_out)
                *(uint2*)(a.x_out + (size_t)row * d + 4 * g) = make_uint2(((unsigned)nv[0] & 0xFFFFu) | ((unsigned)nv[1] << 16),
                                                                          ((unsigned)nv[2] & 0xFFFFu) | ((unsigned)nv[3] << 16));
        }
    }
    rms_row(xi, a.w2, d, lane, yn);
#pragma unroll
    for (int j = 0; j < RG; j++) {
        const int g = lane + 64 * j;
        if (g < ng) *(unsigned*)(a.xn + (size_t)row * d + 4 * g) = pack4(yn.v[j]);
    }
}

void launch_rn_splitk_epi(const RowGemmArgs& a, const int32_t* part, int splits, hipStream_t s) {
    hipLaunchKernelGGL(k_rn_splitk_epi, dim3((unsigned)((a.M + 3) / 4)), dim3(256), 0, s, a, part, splits);
}

// ---------------------------------------------------------------------------
// Layer 0's QKV from the per-token table.  One thread per (row, item): items
// 0 .. 8H-1 are query rotary groups (head i / 8, dims 4 (i % 8) .. +3 paired
// with +32), the next 8 NG key rotary groups, the last 16 NG value quads.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_qkv_table(QkvTabArgs a) {
    const int per_row = 8 * a.H + 24 * a.NG;
    const int idx = blockIdx.x * 256 + threadIdx.x;
    if (idx >= a.M * per_row) return;
    // idx / per_row from the host's 1 / per_row: the product is within 2^-21
    // of the quotient, whose fraction is 0 or >= 1 / per_row >= 2^-12, so a
    // 2^-13 bias truncates to it exactly (per_row < 2^12, idx < 2^31)
    const int row = (int)__builtin_fma((double)idx, a.inv_per_row, 0x1p-13), it = idx - row * per_row;
    const int b = a.pos >= 0 ? row : row / a.T, p = a.pos >= 0 ? a.pos : row - b * a.T;
    const int8_t* t = a.tab + (size_t)a.tok[row] * a.qkv_n;
    if (it >= 8 * a.H + 8 * a.NG) {  // V: dims 4 q .. 4 q + 3 of head g, in blocks of 2^vl keys (vt_off)
        const int v = it - 8 * a.H - 8 * a.NG, g = v >> 4, q = v & 15;
        const unsigned w = *(const unsigned*)(t + a.d + 64 * a.NG + 64 * g + 4 * q);
        const int vl = a.vl;
        int8_t* dst = a.vc + ((size_t)b * a.KH + g) * 64 * a.TP + vt_off(p, 4 * q, vl);
#pragma unroll
        for (int r = 0; r < 4; r++) dst[r << vl] = (int8_t)(w >> (8 * r));
        return;
    }
    const bool isq = it < 8 * a.H;
    // Q: >> 15 then NET_SHIFT = 1 (attention.rs:53-83); K: >> 15 (attention.rs:29-50)
    const double rm = isq ? 0.5 : 1.0, rb = isq ? ROPE_Q_BIAS : 0.0;
    const int hd = isq ? it >> 3 : (it - 8 * a.H) >> 3, i0 = 4 * (it & 7);
    const int col = isq ? 64 * hd : a.d + 64 * hd;
    const unsigned xw = *(const unsigned*)(t + col + i0), yw = *(const unsigned*)(t + col + i0 + 32);
    const uint2 cw = *(const uint2*)(a.rcos + p * 32 + i0), sw = *(const uint2*)(a.rsin + p * 32 + i0);
    int xq[4], yq[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int xv = (int8_t)(xw >> (8 * r)), yv = (int8_t)(yw >> (8 * r));
        const unsigned cc = r < 2 ? cw.x : cw.y, ss = r < 2 ? sw.x : sw.y;
        const int c = (int16_t)(r & 1 ? cc >> 16 : cc & 0xFFFFu), sn = (int16_t)(r & 1 ? ss >> 16 : ss & 0xFFFFu);
        const int xr = (int)((unsigned)(xv * c) - (unsigned)(yv * sn));
        const int yr = (int)((unsigned)(xv * sn) + (unsigned)(yv * c));
        xq[r] = clamp127(rope_round(xr, rm, rb));
        yq[r] = clamp127(rope_round(yr, rm, rb));
    }
    int8_t* dst = isq ? a.q8 + (size_t)row * a.d + 64 * hd : a.kc + (((size_t)b * a.KH + hd) * a.T + p) * 64;
    *(unsigned*)(dst + i0) = pack4(xq);
    *(unsigned*)(dst + i0 + 32) = pack4(yq);
}

// Prefill: a workgroup takes 16 consecutive positions p0 .. p0 + 15 of one
// chunk (p0 % 16 == 0), computes their Q and K rotary groups and gathers
// their V rows into LDS, then writes every output as contiguous 16-byte
// pieces: the 16 query rows (16 d bytes), each key head's 16 rows (1 KB) and
// each value head's 64 x 16-key block of the transposed cache (1 KB).  Keys
// past the chunk's T inside the last block get don't-care bytes (never
// weighted by the attention).
constexpr int QT_MAXD = 1024, QT_MAXG = 4;
__global__ __launch_bounds__(256) void k_qkv_table_blk(QkvTabArgs a) {
    __shared__ __attribute__((aligned(16))) int8_t qs[16 * QT_MAXD];
    __shared__ __attribute__((aligned(16))) int8_t ks[QT_MAXG * 16 * 64];
    __shared__ __attribute__((aligned(16))) int8_t vs[QT_MAXG * 16 * 64];
    __shared__ uint32_t tk[16];
    const int tid = threadIdx.x;
    const int nkb = (a.T + 15) / 16;
    const int b = blockIdx.x / nkb, p0 = (blockIdx.x - b * nkb) * 16;
    const int nrows = min(16, a.T - p0);
    const int row0 = b * a.T + p0;
    if (tid < 16) tk[tid] = tid < nrows ? a.tok[row0 + tid] : 0u;
    __syncthreads();
    // Q and K rotary groups: item = (row k, group i): group < 8H query, else key
    const int per_row = 8 * a.H + 8 * a.NG;
    // item idx = (row k, group it), advanced by 256 per pass: one division per thread
    const int kstep = 256 / per_row, istep = 256 - kstep * per_row;
    int k = tid / per_row, it = tid - k * per_row;
    for (int idx = tid; idx < 16 * per_row; idx += 256, k += kstep, it += istep) {
        if (it >= per_row) {
            it -= per_row;
            k++;
        }
        const int8_t* t = a.tab + (size_t)tk[k] * a.qkv_n;
        const bool isq = it < 8 * a.H;
        // Q: >> 15 then NET_SHIFT = 1 (attention.rs:53-83); K: >> 15 (attention.rs:29-50)
        const double rm = isq ? 0.5 : 1.0, rb = isq ? ROPE_Q_BIAS : 0.0;
        const int hd = isq ? it >> 3 : (it - 8 * a.H) >> 3, i0 = 4 * (it & 7);
        const int col = isq ? 64 * hd : a.d + 64 * hd;
        const unsigned xw = *(const unsigned*)(t + col + i0), yw = *(const unsigned*)(t + col + i0 + 32);
        const int p = min(p0 + k, a.T - 1);
        const uint2 cw = *(const uint2*)(a.rcos + p * 32 + i0), sw = *(const uint2*)(a.rsin + p * 32 + i0);
        int xq[4], yq[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int xv = (int8_t)(xw >> (8 * r)), yv = (int8_t)(yw >> (8 * r));
            const unsigned cc = r < 2 ? cw.x : cw.y, ss = r < 2 ? sw.x : sw.y;
            const int c = (int16_t)(r & 1 ? cc >> 16 : cc & 0xFFFFu), sn = (int16_t)(r & 1 ? ss >> 16 : ss & 0xFFFFu);
            const int xr = (int)((unsigned)(xv * c) - (unsigned)(yv * sn));
            const int yr = (int)((unsigned)(xv * sn) + (unsigned)(yv * c));
            xq[r] = clamp127(rope_round(xr, rm, rb));
            yq[r] = clamp127(rope_round(yr, rm, rb));
        }
        int8_t* dst = isq ? qs + k * a.d + 64 * hd : ks + (hd * 16 + k) * 64;
        *(unsigned*)(dst + i0) = pack4(xq);
        *(unsigned*)(dst + i0 + 32) = pack4(yq);
    }
    // V rows (16 bytes per item)
    for (int idx = tid; idx < 16 * a.NG * 4; idx += 256) {
        const int k = idx / (4 * a.NG), r = idx - k * 4 * a.NG, g = r >> 2, c = r & 3;
        *(uint4*)(vs + (g * 16 + k) * 64 + 16 * c) =
            *(const uint4*)(a.tab + (size_t)tk[k] * a.qkv_n + a.d + 64 * a.NG + 64 * g + 16 * c);
    }
    __syncthreads();
    // query rows: nrows * d contiguous bytes
    const int qn = nrows * a.d / 16;
    for (int i = tid; i < qn; i += 256) *(uint4*)(a.q8 + (size_t)row0 * a.d + 16 * i) = *(const uint4*)(qs + 16 * i);
    // key rows of each head: nrows * 64 contiguous bytes
    for (int i = tid; i < a.NG * nrows * 4; i += 256) {
        const int g = i / (nrows * 4), c = i - g * nrows * 4;
        *(uint4*)(a.kc + (((size_t)b * a.KH + g) * a.T + p0) * 64 + 16 * c) = *(const uint4*)(ks + g * 1024 + 16 * c);
    }
    // value blocks: dim j of head g -> the 16 keys' bytes
    for (int i = tid; i < a.NG * 64; i += 256) {
        const int g = i >> 6, j = i & 63;
        unsigned w[4];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int8_t* v = vs + (g * 16 + 4 * q) * 64 + j;
            w[q] = (unsigned)(uint8_t)v[0] | ((unsigned)(uint8_t)v[64] << 8) | ((unsigned)(uint8_t)v[128] << 16) |
                   ((unsigned)(uint8_t)v[192] << 24);
        }
        *(uint4*)(a.vc + ((size_t)b * a.KH + g) * 64 * a.TP + (size_t)(p0 >> 4) * 1024 + 16 * j) =
            make_uint4(w[0], w[1], w[2], w[3]);
    }
}

void launch_qkv_table(const QkvTabArgs& a, hipStream_t s) {
    if (a.pos < 0 && a.d <= QT_MAXD && a.NG <= QT_MAXG) {
        const int nb = a.M / a.T, nkb = (a.T + 15) / 16;
        hipLaunchKernelGGL(k_qkv_table_blk, dim3((unsigned)(nb * nkb)), dim3(256), 0, s, a);
        return;
    }
    const int per_row = 8 * a.H + 24 * a.NG;
    const long long n = (long long)a.M * per_row;
    // n < 2^31 (the caller takes the table path only then) and per_row <= 512 (d <= 1024)
    QkvTabArgs g = a;
    g.inv_per_row = 1.0 / per_row;
    hipLaunchKernelGGL(k_qkv_table, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, g);
}

// x += rmsnorm(y8, w1) (model.rs:429-434 / 463-468);
// xn = rmsnorm(clamp(x), w2) (model.rs:438-439, next layer 384-385, final 473-474)
__global__ __launch_bounds__(256) void k_resid_norm(int16_t* __restrict__ x, const int8_t* __restrict__ y8,
                                                    const int8_t* __restrict__ w1, const int8_t* __restrict__ w2,
                                                    int M, int d, int8_t* __restrict__ xn) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= M) return;
    const int ng = d >> 2;
    RowI8 yi, yn, xi;
#pragma unroll
    for (int j = 0; j < RG; j++) {
        const int g = lane + 64 * j;
        if (g < ng) unpack4(*(const unsigned*)(y8 + (size_t)row * d + 4 * g), yi.v[j]);
    }
    rms_row(yi, w1, d, lane, yn);
#pragma unroll
    for (int j = 0; j < RG; j++) {
        const int g = lane + 64 * j;
        if (g < ng) {
            // |x| <= 127 * (2 * n_layers + 1) < 2^15: the i32 sums of the reference fit int16
            uint2* px = (uint2*)(x + (size_t)row * d + 4 * g);
            const uint2 xv = *px;
            const int nv[4] = {(int16_t)(xv.x & 0xFFFFu) + yn.v[j][0], (int16_t)(xv.x >> 16) + yn.v[j][1],
                               (int16_t)(xv.y & 0xFFFFu) + yn.v[j][2], (int16_t)(xv.y >> 16) + yn.v[j][3]};
            *px = make_uint2(((unsigned)nv[0] & 0xFFFFu) | ((unsigned)nv[1] << 16),
                             ((unsigned)nv[2] & 0xFFFFu) | ((unsigned)nv[3] << 16));
#pragma unroll
            for (int k = 0; k < 4; k++) xi.v[j][k] = clamp127(nv[k]);
        }
    }
    rms_row(xi, w2, d, lane, yn);
#pragma unroll
    for (int j = 0; j < RG; j++) {
        const int g = lane + 64 * j;
        if (g < ng) *(unsigned*)(xn + (size_t)row * d + 4 * g) = pack4(yn.v[j]);
    }
}

void launch_resid_norm(int16_t* x, const int8_t* y8, const int8_t* w1, const int8_t* w2, int M, int d, int8_t* xn,
                       hipStream_t s) {
    hipLaunchKernelGGL(k_resid_norm, dim3((unsigned)((M + 3) / 4)), dim3(256), 0, s, x, y8, w1, w2, M, d, xn);
}

// ---------------------------------------------------------------------------
// Logits -> cumulative frequencies (softmax_cdf.rs:85-139).
// WPR wavefronts per row, EPL consecutive logits per lane (V <= 64*WPR*EPL).
// The frequency f = 1 + floor(e * R / S) (R = total - V) is formed exactly as
// f = 1 + e*Q + floor(e*Rm / S) with Q = R / S, Rm = R % S: e*Q < 2^31
// because S >= 65535 (the max logit weighs 65535), and the small quotient is
// an f32 estimate corrected by one exact 64-bit remainder test.
// mode 0: write (cum_lo, cum_hi) of the row's target; mode 1: write the full
// inclusive table; mode 2: targets holds the row's decoder value (the
// ((code - low + 1) * total - 1) / range of arith_coder.rs:199-203) and the
// row gets (sym, cum_lo, cum_hi) with sym the first index whose inclusive
// cumulative frequency exceeds the value, clamped to V - 1
// (bisect_cumfreqs, arith_coder.rs:225-241).
// ---------------------------------------------------------------------------
template <int WPR, int EPL>
__global__ __launch_bounds__(64 * WPR) void k_cdf(const int32_t* __restrict__ logits, int V,
                                                  const uint32_t* __restrict__ targets,
                                                  const int32_t* __restrict__ lens, int T,
                                                  const uint16_t* __restrict__ glut, unsigned coef, unsigned total,
                                                  int mode, uint32_t* __restrict__ out, long long out_row0) {
    __shared__ uint16_t lut[256];
    __shared__ int red_i[WPR];
    __shared__ unsigned red_u[WPR];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int row = blockIdx.x;
    for (int i = tid; i < 256; i += 64 * WPR) lut[i] = glut[i];
    if (lens && (row % T) >= lens[row / T]) return;  // uniform per block
    __syncthreads();
    const int i0 = tid * EPL;
    const int32_t* L = logits + (size_t)row * V;
    int lv[EPL];
    if (i0 + EPL <= V) {
#pragma unroll
        for (int k = 0; k < EPL; k += 4) {
            int4 v = *(const int4*)(L + i0 + k);
            lv[k] = v.x; lv[k + 1] = v.y; lv[k + 2] = v.z; lv[k + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int k = 0; k < EPL; k++) lv[k] = (i0 + k < V) ? L[i0 + k] : INT32_MIN;
    }
    auto bmax = [&](int v) {
        v = wave_max_i(v);
        if (WPR == 1) return v;
        if (lane == 0) red_i[wave] = v;
        __syncthreads();
        int r = red_i[0];
        for (int w = 1; w < WPR; w++) r = max(r, red_i[w]);
        __syncthreads();
        return r;
    };
    auto bmin = [&](int v) {
        v = wave_min_i(v);
        if (WPR == 1) return v;
        if (lane == 0) red_i[wave] = v;
        __syncthreads();
        int r = red_i[0];
        for (int w = 1; w < WPR; w++) r = min(r, red_i[w]);
        __syncthreads();
        return r;
    };
    auto bsum = [&](unsigned v) {
        v = wave_sum_u(v);
        if (WPR == 1) return v;
        if (lane == 0) red_u[wave] = v;
        __syncthreads();
        unsigned r = 0;
        for (int w = 0; w < WPR; w++) r += red_u[w];
        __syncthreads();
        return r;
    };
    int mx = INT32_MIN;
#pragma unroll
    for (int k = 0; k < EPL; k++) mx = max(mx, lv[k]);
    mx = bmax(mx);
    int am = 0x7FFFFFFF;
#pragma unroll
    for (int k = EPL - 1; k >= 0; k--)
        if (i0 + k < V && lv[k] == mx) am = i0 + k;
    am = bmin(am);
    unsigned e[EPL];
    unsigned ls = 0;
#pragma unroll
    for (int k = 0; k < EPL; k++) {
        e[k] = (i0 + k < V) ? exp_q16((int)((unsigned)lv[k] - (unsigned)mx), lut, coef) : 0u;
        ls += e[k];
    }
    const unsigned S = bsum(ls);  // <= 8192 * 65535 < 2^32
    const unsigned R = total - (unsigned)V;
    const unsigned Q = R / S, Rm = R - Q * S;
    const float rf = (float)Rm / (float)S;
    unsigned fl = 0;
#pragma unroll
    for (int k = 0; k < EPL; k++) {
        unsigned f = 0;
        if (i0 + k < V) {
            unsigned q = (unsigned)((float)e[k] * rf);
            const unsigned long long t = (unsigned long long)e[k] * Rm, u = (unsigned long long)q * S;
            if (t < u) q -= 1;
            else if (t - u >= S) q += 1;
            f = 1u + e[k] * Q + q;
        }
        e[k] = f;
        fl += f;
    }
    const unsigned rem = total - bsum(fl);
    if (mode == 0) {
        const int tok = (int)targets[row];
        unsigned lo = 0, ft = 0;
#pragma unroll
        for (int k = 0; k < EPL; k++) {
            lo += (i0 + k < tok) ? e[k] : 0u;
            ft += (i0 + k == tok) ? e[k] : 0u;
        }
        lo = bsum(lo);
        ft = bsum(ft);
        if (am < tok) lo += rem;
        if (am == tok) ft += rem;
        if (tid == 0) {
            out[(size_t)(out_row0 + row) * 2] = lo;
            out[(size_t)(out_row0 + row) * 2 + 1] = lo + ft;
        }
    } else {
        // exclusive scan of lane sums across the row
        unsigned incl = fl;
        for (int o = 1; o < 64; o <<= 1) {
            unsigned v = (unsigned)__shfl_up((int)incl, o, 64);
            if (lane >= o) incl += v;
        }
        unsigned excl = incl - fl;
        if (WPR > 1) {
            if (lane == 63) red_u[wave] = incl;
            __syncthreads();
            for (int w = 0; w < wave; w++) excl += red_u[w];
        }
        unsigned run = excl + (am < i0 ? rem : 0u);
        if (mode == 1) {
            uint32_t* o = out + (size_t)(out_row0 + row) * V;
#pragma unroll
            for (int k = 0; k < EPL; k++) {
                if (i0 + k < V) {
                    run += e[k] + (i0 + k == am ? rem : 0u);
                    o[i0 + k] = run;
                }
            }
        } else {
            const unsigned value = targets[row];
            int cand = 0x7FFFFFFF;
            unsigned clo = 0, chi = 0;
#pragma unroll
            for (int k = 0; k < EPL; k++) {
                if (i0 + k < V) {
                    const unsigned before = run;
                    run += e[k] + (i0 + k == am ? rem : 0u);
                    // the last symbol also takes a value at or past the total (the clamp)
                    if (cand == 0x7FFFFFFF && (value < run || i0 + k == V - 1)) {
                        cand = i0 + k;
                        clo = before;
                        chi = run;
                    }
                }
            }
            const int sym = bmin(cand);
            if (cand == sym) {
                uint32_t* o = out + (size_t)(out_row0 + row) * 3;
                o[0] = (uint32_t)sym;
                o[1] = clo;
                o[2] = chi;
            }
        }
    }
}

void launch_cdf(const int32_t* logits, int M, int V, const uint32_t* targets, const int32_t* lens, int T,
                const uint16_t* lut, unsigned coef, unsigned total, int mode, uint32_t* out, int64_t out_row0,
                hipStream_t s) {
    if (V <= 1024)
        hipLaunchKernelGGL((k_cdf<1, 16>), dim3((unsigned)M), dim3(64), 0, s, logits, V, targets, lens, T, lut, coef,
                           total, mode, out, (long long)out_row0);
    else if (V <= 4096)
        hipLaunchKernelGGL((k_cdf<4, 16>), dim3((unsigned)M), dim3(256), 0, s, logits, V, targets, lens, T, lut, coef,
                           total, mode, out, (long long)out_row0);
    else
        hipLaunchKernelGGL((k_cdf<4, 32>), dim3((unsigned)M), dim3(256), 0, s, logits, V, targets, lens, T, lut, coef,
                           total, mode, out, (long long)out_row0);
}

// ---------------------------------------------------------------------------
// Rows of a [B, T] block of coder targets for the prefill (main.rs:220-226):
// the input of row (b, p) is BOS at p = 0, else target (b, p - 1); lens are
// clamped to [0, T]; rows past a chunk's length get zeros, and so does their
// (cum_lo, cum_hi) in out (the head writes only live rows).  A live target
// >= V sets *err and reads as 0.  One thread per row.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_prep_rows(const uint32_t* __restrict__ targets,
                                                   const int32_t* __restrict__ lens_in, int B, int T, unsigned V,
                                                   uint32_t* __restrict__ inp, uint32_t* __restrict__ tgt,
                                                   int32_t* __restrict__ lens, uint32_t* __restrict__ out,
                                                   int32_t* __restrict__ err) {
    const long long r = (long long)blockIdx.x * 256 + threadIdx.x;
    if (r >= (long long)B * T) return;
    const int b = (int)(r / T), p = (int)(r - (long long)b * T);
    const int n = min(max(lens_in[b], 0), T);
    if (p == 0) lens[b] = n;
    uint32_t t = 0, prev = 0;
    if (p < n) {
        t = targets[r];
        if (t >= V) {
            atomicOr(err, 1);
            t = 0;
        }
        prev = p == 0 ? BOS_TOKEN : targets[r - 1];
        prev = prev < V ? prev : 0u;
    }
    inp[r] = prev;
    tgt[r] = t;
    *(uint2*)(out + 2 * r) = make_uint2(0u, 0u);
}

__global__ void k_zero_i32(int32_t* p) { *p = 0; }

void launch_prep_rows(const uint32_t* targets, const int32_t* lens_in, int B, int T, int V, uint32_t* inp,
                      uint32_t* tgt, int32_t* lens, uint32_t* out, int32_t* err, hipStream_t s) {
    const long long M = (long long)B * T;
    hipLaunchKernelGGL(k_zero_i32, dim3(1), dim3(1), 0, s, err);
    if (M > 0)
        hipLaunchKernelGGL(k_prep_rows, dim3((unsigned)((M + 255) / 256)), dim3(256), 0, s, targets, lens_in, B, T,
                           (unsigned)V, inp, tgt, lens, out, err);
}

// ---------------------------------------------------------------------------
// Coded chunks from their fixed-size slots to one back-to-back buffer (the
// chunk data layout of the container, file_format.rs:324-331), so that only
// the coded bytes cross PCIe.  One workgroup per chunk; lens[c] <= slot.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_pack_chunks(const uint8_t* __restrict__ src, long long slot,
                                                     const int32_t* __restrict__ lens,
                                                     const long long* __restrict__ offs, uint8_t* __restrict__ dst) {
    const int c = blockIdx.x;
    const uint8_t* s = src + (size_t)c * slot;
    uint8_t* d = dst + offs[c];
    const int n = lens[c];
    for (int i = threadIdx.x; i < n; i += 256) d[i] = s[i];
}

void launch_pack_chunks(const uint8_t* src, int64_t slot, const int32_t* lens, const int64_t* offs, int n,
                        uint8_t* dst, hipStream_t s) {
    if (n > 0)
        hipLaunchKernelGGL(k_pack_chunks, dim3((unsigned)n), dim3(256), 0, s, src, (long long)slot, lens,
                           (const long long*)offs, dst);
}

// ---------------------------------------------------------------------------
// Arithmetic encoder (arith_coder.rs:26-136), one thread per chunk.
// ---------------------------------------------------------------------------
struct BitOut {
    uint8_t* buf;
    long long cap, len;
    unsigned cur;
    int bit_pos;
    int overflow;
    __device__ void bit(unsigned b) {
        if (b) cur |= 1u << bit_pos;
        if (--bit_pos < 0) {
            if (len < cap) buf[len] = (uint8_t)cur;
            else overflow = 1;
            len++;
            cur = 0;
            bit_pos = 7;
        }
    }
};

__global__ __launch_bounds__(64) void k_encode(const uint32_t* __restrict__ lohi, const int32_t* __restrict__ lens,
                                               int nb, int T, unsigned total, uint8_t* __restrict__ out,
                                               long long slot, int32_t* __restrict__ out_lens,
                                               int32_t* __restrict__ err) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= nb) return;
    const unsigned long long MASK = 0xFFFFFFFFull, HALF = 1ull << 31, QUART = 1ull << 30;
    unsigned long long low = 0, high = MASK;
    unsigned underflow = 0;
    BitOut o{out + (size_t)c * slot, slot, 0, 0u, 7, 0};
    const double invT = 1.0 / (double)total;
    const int n = lens[c];
    const uint2* lh = (const uint2*)(lohi + (size_t)c * T * 2);
    uint2 nxt = n > 0 ? lh[0] : make_uint2(0, 0);
    for (int i = 0; i < n; i++) {
        const uint2 cur = nxt;
        if (i + 1 < n) nxt = lh[i + 1];  // prefetch the next interval
        const unsigned long long range = high - low + 1;
        high = low + udiv64_32((unsigned long long)cur.y * range, total, invT) - 1;
        low = low + udiv64_32((unsigned long long)cur.x * range, total, invT);
        for (;;) {
            if (((low ^ high) & HALF) == 0) {
                unsigned bitv = (unsigned)((low >> 31) & 1);
                o.bit(bitv);
                for (unsigned u = 0; u < underflow; u++) o.bit(bitv ^ 1u);
                underflow = 0;
                low = (low << 1) & MASK;
                high = ((high << 1) & MASK) | 1;
            } else if ((low & ~high & QUART) != 0) {
                underflow += 1;
                low = ((low << 1) ^ HALF) & MASK;
                high = (((high ^ HALF) << 1) | HALF | 1) & MASK;
            } else {
                break;
            }
        }
    }
    o.bit(1u);  // finish(): terminating bit, then flush the partial byte
    if (o.bit_pos < 7) {
        if (o.len < o.cap) o.buf[o.len] = (uint8_t)o.cur;
        else o.overflow = 1;
        o.len++;
    }
    out_lens[c] = (int32_t)o.len;
    if (o.overflow) atomicOr(err, 1);
}

void launch_encode(const uint32_t* lohi, const int32_t* lens, int nb, int T, unsigned total, uint8_t* out,
                   int64_t slot, int32_t* out_lens, int32_t* err, hipStream_t s) {
    hipLaunchKernelGGL(k_encode, dim3((unsigned)((nb + 63) / 64)), dim3(64), 0, s, lohi, lens, nb, T, total, out,
                       (long long)slot, out_lens, err);
}

}  // namespace czip
