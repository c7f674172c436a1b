// gfx950 kernels of the compress-zip integer transformer.
//
// All arithmetic is integer and bit-exact with the reference crate
// (rust/src).  Wrapping i32 arithmetic is written with unsigned types.
// Wavefronts are 64 lanes; GEMMs use v_mfma_i32_16x16x64_i8.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "czip_kernels.h"

namespace czip {

// ---------------------------------------------------------------------------
// Integer primitives (device copies of rust/src/primitives.rs)
// ---------------------------------------------------------------------------
__device__ __forceinline__ int clamp127(int x) { return x < -127 ? -127 : (x > 127 ? 127 : x); }

// primitives.rs:18-42
__device__ __forceinline__ int sra_rne32(int v, unsigned sh) {
    if (sh == 0) return v;
    unsigned sign = (unsigned)(v >> 31);
    unsigned av = ((unsigned)v ^ sign) - sign;
    unsigned q = av >> sh;
    unsigned r = av & ((1u << sh) - 1u);
    unsigned half = 1u << (sh - 1);
    q += (r > half) ? 1u : ((r == half) ? (q & 1u) : 0u);
    return (int)((q ^ sign) - sign);
}

// primitives.rs:49-73
__device__ __forceinline__ int sra_rne64(long long v, unsigned sh) {
    if (sh == 0) return (int)(v < INT32_MIN ? INT32_MIN : (v > INT32_MAX ? INT32_MAX : v));
    unsigned long long sign = (unsigned long long)(v >> 63);
    unsigned long long av = ((unsigned long long)v ^ sign) - sign;
    unsigned long long q = av >> sh;
    unsigned long long r = av & ((1ull << sh) - 1ull);
    unsigned long long half = 1ull << (sh - 1);
    q += (r > half) ? 1ull : ((r == half) ? (q & 1ull) : 0ull);
    long long so = (long long)((q ^ sign) - sign);
    return (int)(so < INT32_MIN ? INT32_MIN : (so > INT32_MAX ? INT32_MAX : so));
}

// model.rs:280-300
__device__ __forceinline__ int requant(int v, int mult, int shift) {
    long long p = (long long)v * (long long)mult;
    if (shift <= 0) return (int)(p < -127 ? -127 : (p > 127 ? 127 : p));
    return clamp127(sra_rne64(p, (unsigned)shift));
}

// primitives.rs:80-97
__device__ __forceinline__ unsigned udiv_rne(unsigned n, unsigned d) {
    if (d == 0) return 0;
    unsigned q = n / d;
    unsigned r = n - q * d;
    unsigned tr = r << 1;
    return tr > d ? q + 1 : (tr == d ? q + (q & 1u) : q);
}

// primitives.rs:192-213
__device__ __forceinline__ unsigned isqrt32(unsigned x) {
    unsigned op = x, res = 0, one = 1u << 30;
    while (one > op) one >>= 2;
    while (one != 0) {
        if (op >= res + one) { op -= res + one; res = (res >> 1) + one; }
        else res >>= 1;
        one >>= 2;
    }
    return res;
}

// rmsnorm.rs:14-30
__device__ __forceinline__ int inv_rms_q15(int mean_sq) {
    unsigned ms = mean_sq > 0 ? (unsigned)mean_sq : 1u;
    unsigned inv = udiv_rne(8388608u, isqrt32(ms << 16));
    return (int)(inv < 1u ? 1u : (inv > 32768u ? 32768u : inv));
}

// lut.rs:213-235 / softmax_cdf.rs:55-77
__device__ __forceinline__ unsigned exp_q16(int diff, const uint16_t* lut, unsigned coef) {
    if (diff >= 0) return 65535u;
    unsigned neg = 0u - (unsigned)diff;
    unsigned t = (unsigned)(((unsigned long long)neg * coef + (1ull << 23)) >> 24);
    unsigned ip = t >> 8;
    if (ip >= 31u) return 1u;
    unsigned out = ((65536u >> ip) * (unsigned)lut[t & 255u] + 0x8000u) >> 16;
    return out < 1u ? 1u : (out > 65535u ? 65535u : out);
}

// primitives.rs:163-185 (the result is formed with i32 wrap like `as i32 * sign`)
__device__ __forceinline__ int div_rne_s32_u64(int num, unsigned long long den) {
    if (den == 0) return 0;
    unsigned long long an = (unsigned long long)(num < 0 ? 0u - (unsigned)num : (unsigned)num);
    unsigned long long q = an / den;
    unsigned long long r = an - q * den;
    unsigned long long tr = r << 1;
    unsigned long long rq = tr > den ? q + 1 : (tr == den ? q + (q & 1ull) : q);
    unsigned u = (unsigned)rq;
    return (int)(num < 0 ? 0u - u : u);
}

// floor(a / d) for a < 2^62, 0 < d < 2^32, via an f64 estimate and an exact
// integer correction (the estimate is within one of the true quotient).
__device__ __forceinline__ unsigned long long udiv64_32(unsigned long long a, unsigned d, double inv_d) {
    unsigned long long q = (unsigned long long)((double)a * inv_d);
    long long r = (long long)(a - q * (unsigned long long)d);
    while (r < 0) { q -= 1; r += (long long)d; }
    while (r >= (long long)d) { q += 1; r -= (long long)d; }
    return q;
}

__device__ __forceinline__ int wave_sum_i(int v) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

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
        inp[row] = p == 0 ? 1022u : toks[start + p - 1];
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
// Row kernels: one wavefront per token row, d <= 1024.
// ---------------------------------------------------------------------------
constexpr int MAXE = 16;  // d / 64

// rmsnorm.rs:40-75 on a wave-distributed row (element i = lane + 64*j)
__device__ __forceinline__ void rms_row(const int* xi8, const int8_t* __restrict__ w, int d, int lane, int8_t* yout) {
    const int nj = d >> 6;
    unsigned ss = 0;
    for (int j = 0; j < nj; j++) ss += (unsigned)(xi8[j] * xi8[j]);
    ss = (unsigned)wave_sum_i((int)ss);
    int mean_sq = (int)(ss / (unsigned)d) + 1;  // eps_scaled = 1 (rmsnorm.rs:80-83)
    if (mean_sq < 1) mean_sq = 1;
    int inv = inv_rms_q15(mean_sq);
    for (int j = 0; j < nj; j++) {
        int i = lane + 64 * j;
        int tmp = (int)((unsigned)(xi8[j] * (int)w[i]) * (unsigned)inv);
        yout[j] = (int8_t)clamp127(sra_rne32(tmp, 15));
    }
}

// x = E[tok] (model.rs:372-374); xn = rmsnorm(clamp(x), w) (model.rs:384-385)
__global__ void k_embed_norm(const uint32_t* __restrict__ inp, const int8_t* __restrict__ embed,
                             const int8_t* __restrict__ w, int M, int d, int32_t* __restrict__ x,
                             int8_t* __restrict__ xn) {
    int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    int lane = threadIdx.x & 63;
    if (row >= M) return;
    const int8_t* e = embed + (size_t)inp[row] * d;
    int xi[MAXE];
    int8_t y[MAXE];
    const int nj = d >> 6;
    for (int j = 0; j < nj; j++) {
        int v = e[lane + 64 * j];
        x[(size_t)row * d + lane + 64 * j] = v;
        xi[j] = clamp127(v);
    }
    rms_row(xi, w, d, lane, y);
    for (int j = 0; j < nj; j++) xn[(size_t)row * d + lane + 64 * j] = y[j];
}

void launch_embed_norm(const uint32_t* inp, const int8_t* embed, const int8_t* w, int M, int d, int32_t* x,
                       int8_t* xn, hipStream_t s) {
    hipLaunchKernelGGL(k_embed_norm, dim3((unsigned)((M + 3) / 4)), dim3(256), 0, s, inp, embed, w, M, d, x, xn);
}

// x += rmsnorm(y8, w1) (model.rs:429-434 / 463-468);
// xn = rmsnorm(clamp(x), w2) (model.rs:438-439, next layer 384-385, final 473-474)
__global__ void k_resid_norm(int32_t* __restrict__ x, const int8_t* __restrict__ y8, const int8_t* __restrict__ w1,
                             const int8_t* __restrict__ w2, int M, int d, int8_t* __restrict__ xn) {
    int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    int lane = threadIdx.x & 63;
    if (row >= M) return;
    const int nj = d >> 6;
    int yi[MAXE];
    int8_t yn[MAXE];
    for (int j = 0; j < nj; j++) yi[j] = y8[(size_t)row * d + lane + 64 * j];
    rms_row(yi, w1, d, lane, yn);
    int xi[MAXE];
    for (int j = 0; j < nj; j++) {
        size_t o = (size_t)row * d + lane + 64 * j;
        int v = (int)((unsigned)x[o] + (unsigned)(int)yn[j]);
        x[o] = v;
        xi[j] = clamp127(v);
    }
    rms_row(xi, w2, d, lane, yn);
    for (int j = 0; j < nj; j++) xn[(size_t)row * d + lane + 64 * j] = yn[j];
}

void launch_resid_norm(int32_t* x, const int8_t* y8, const int8_t* w1, const int8_t* w2, int M, int d, int8_t* xn,
                       hipStream_t s) {
    hipLaunchKernelGGL(k_resid_norm, dim3((unsigned)((M + 3) / 4)), dim3(256), 0, s, x, y8, w1, w2, M, d, xn);
}

// ---------------------------------------------------------------------------
// int8 GEMM C = A * W^T on v_mfma_i32_16x16x64_i8 with fused epilogues.
// Block tile 128x128x64, 4 waves in 2x2, each wave 64x64 = 4x4 MFMA tiles.
// MFMA operand layout: lane l supplies row (l % 16) and the 16 bytes of K at
// (l / 16) * 16; A and W use the same K mapping, so the dot product is exact
// whatever the hardware's K order.  Result: lane l holds rows 4*(l/16)+r,
// column l % 16 of each 16x16 tile.
// ---------------------------------------------------------------------------
typedef int v4i __attribute__((ext_vector_type(4)));

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
                const int p = row % a.T, b = row / a.T;
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
                        } else {
                            // V, stored dim-major for the PV operand
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

// ---------------------------------------------------------------------------
// Prefill attention, exact, on MFMA.
//
// The reference walks the keys of a query row in order, rescaling the running
// sum S and the value accumulator with a rounded factor each time the running
// max strictly increases (attention.rs:205-276).  Between two such "records"
// every key's weight uses the same max, so the segment's contribution is a
// plain integer sum (S in u64, vacc modulo 2^32) that can be formed in any
// order.  Per 64-key tile the kernel therefore:
//   1. forms S^T = K Q^T with int8 MFMA and applies the score epilogue;
//   2. scans each row's keys in order for running max, records, weights
//      w = E(s - max) and segment ids (lanes own 16 consecutive keys);
//   3. for each segment j = 0..max records, accumulates O^T += V^T P_j^T on
//      int8 MFMA (P_j = weights of segment j, split into three 7-bit limbs),
//      rescaling the state at record j exactly as the reference does.
// Layout: S^T puts query row (lane % 16) in the lane and keys
// 16*blk + 4*(lane/16) + r in its registers -- which is exactly the B-operand
// layout of P^T for the PV product, so P never moves between the two MFMAs.
// One workgroup = one chunk, one head, 64 query rows (4 waves x 16 rows).
// ---------------------------------------------------------------------------
__device__ __forceinline__ int score_of(int dot, int mult) {
    int du = sra_rne32(dot, 2);                             // Q_SHIFT
    return sra_rne64((long long)du * (long long)mult, 15);  // attention.rs:233-239
}

constexpr int KLD = 80;  // LDS row stride (bytes) of the K tile and the V^T tile
constexpr unsigned NOSEG = 0xFFFFu;

__device__ __forceinline__ void wave_lds_fence() { __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront"); }

__device__ __forceinline__ int pack_limb(const unsigned* w, int shift, unsigned mask) {
    return (int)(((w[0] >> shift) & mask) | (((w[1] >> shift) & mask) << 8) | (((w[2] >> shift) & mask) << 16) |
                 (((w[3] >> shift) & mask) << 24));
}

__device__ __forceinline__ void rescale(unsigned long long& S, unsigned* vacc, unsigned e) {
    S = (S * e + 0x8000ull) >> 16;
    for (int i = 0; i < 16; i++) {
        long long pr = (long long)(int)vacc[i] * (long long)e;
        pr += pr >= 0 ? (1ll << 15) : -(1ll << 15);
        vacc[i] = (unsigned)(int)(pr >> 16);
    }
}

__global__ __launch_bounds__(256) void k_attention(AttnArgs a) {
    __shared__ uint16_t lut[256];
    __shared__ __attribute__((aligned(16))) int8_t Ks[64 * KLD];
    __shared__ __attribute__((aligned(16))) int8_t Vt[64 * KLD];
    __shared__ __attribute__((aligned(16))) unsigned scw[4][16][64];  // scores, then (w | seg << 16)
    __shared__ unsigned rec_e[4][16][64];                            // rescale factor of record j (0 = none)

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int row = lane & 15, grp = lane >> 4;
    const int q0 = blockIdx.x * 64, h = blockIdx.y, b = blockIdx.z;
    const int T = a.T, len = a.lens[b];
    if (q0 >= len) return;
    for (int i = tid; i < 256; i += 256) lut[i] = a.lut[i];
    const int D = a.H * 64;
    const int g = a.kv_mode == 1 ? (h * a.G) / a.H : 0;
    const int8_t* Kg = a.kc + ((size_t)b * a.KH + g) * T * 64;
    const int8_t* Vg = a.vc + ((size_t)b * a.KH + g) * 64 * a.TP;
    const int mult = a.score_mult[h];
    const int p = q0 + wave * 16 + row;  // this lane's query position
    const int wrow0 = q0 + wave * 16;
    const bool wave_live = wrow0 < len;
    const int wave_last = min(wrow0 + 15, len - 1);

    v4i qop = (v4i){0, 0, 0, 0};
    if (p < T) qop = *(const v4i*)(a.q + ((size_t)b * T + p) * D + h * 64 + grp * 16);

    int m = INT32_MIN;
    unsigned long long S = 0;
    unsigned vacc[16];
    for (int i = 0; i < 16; i++) vacc[i] = 0;
    if (a.sink) {  // attention.rs:211-224: the sink key's score is the initial max, weight E(0)
        const int* sk = (const int*)(a.sink + grp * 16);
        int dot = 0;
        for (int i = 0; i < 4; i++) dot = __builtin_amdgcn_sdot4(qop[i], sk[i], dot, false);
        dot += __shfl_xor(dot, 16, 64);
        dot += __shfl_xor(dot, 32, 64);
        m = score_of(dot, mult);
        S = 65535ull;
    }

    const int ntiles = (min(q0 + 63, len - 1)) / 64 + 1;
    for (int kt = 0; kt < ntiles; kt++) {
        const int t0 = kt * 64;
        __syncthreads();
        {
            const int r = tid >> 2, c = (tid & 3) * 16;
            int4 kv = make_int4(0, 0, 0, 0);
            if (t0 + r < T) kv = *(const int4*)(Kg + (size_t)(t0 + r) * 64 + c);
            *(int4*)(Ks + r * KLD + c) = kv;
            *(int4*)(Vt + r * KLD + c) = *(const int4*)(Vg + (size_t)r * a.TP + t0 + c);
        }
        __syncthreads();
        if (!wave_live || t0 > wave_last) continue;

        // 1. S^T = K Q^T, score epilogue, store row-major [row][key]
        for (int blk = 0; blk < 4; blk++) {
            v4i kop = *(const v4i*)(Ks + (blk * 16 + row) * KLD + grp * 16);
            v4i st = __builtin_amdgcn_mfma_i32_16x16x64_i8(kop, qop, (v4i){0, 0, 0, 0}, 0, 0, 0);
            int4 sv;
            sv.x = score_of(st[0], mult);
            sv.y = score_of(st[1], mult);
            sv.z = score_of(st[2], mult);
            sv.w = score_of(st[3], mult);
            *(int4*)&scw[wave][row][blk * 16 + grp * 4] = sv;
        }
        wave_lds_fence();

        // 2. in-order scan of keys [16*grp, 16*grp+16) of this row
        int sv[16];
        for (int i = 0; i < 4; i++) {
            int4 v = *(const int4*)&scw[wave][row][grp * 16 + i * 4];
            sv[i * 4] = v.x; sv[i * 4 + 1] = v.y; sv[i * 4 + 2] = v.z; sv[i * 4 + 3] = v.w;
        }
        const int kbase = t0 + grp * 16;
        int nvalid = p - kbase + 1;  // keys t <= p are visible (causal)
        nvalid = nvalid < 0 ? 0 : (nvalid > 16 ? 16 : nvalid);
        int bmax = INT32_MIN;
        for (int k = 0; k < 16; k++)
            if (k < nvalid) bmax = max(bmax, sv[k]);
        // exclusive running max from the lanes holding earlier keys of the row
        int e1 = __shfl(bmax, (lane - 16) & 63, 64), e2 = __shfl(bmax, (lane - 32) & 63, 64),
            e3 = __shfl(bmax, (lane - 48) & 63, 64);
        int cur = m;
        if (grp >= 1) cur = max(cur, e1);
        if (grp >= 2) cur = max(cur, e2);
        if (grp >= 3) cur = max(cur, e3);
        int nrec = 0;
        for (int k = 0; k < 16; k++)
            if (k < nvalid && sv[k] > cur) { nrec++; cur = sv[k]; }
        int r1 = __shfl(nrec, (lane - 16) & 63, 64), r2 = __shfl(nrec, (lane - 32) & 63, 64),
            r3 = __shfl(nrec, (lane - 48) & 63, 64);
        int seg = 0;
        if (grp >= 1) seg += r1;
        if (grp >= 2) seg += r2;
        if (grp >= 3) seg += r3;
        // replay with weights
        cur = m;
        if (grp >= 1) cur = max(cur, e1);
        if (grp >= 2) cur = max(cur, e2);
        if (grp >= 3) cur = max(cur, e3);
        unsigned wsg[16];
        for (int k = 0; k < 16; k++) {
            if (k < nvalid) {
                const int s = sv[k];
                if (s > cur) {
                    unsigned e = cur != INT32_MIN ? exp_q16((int)((unsigned)cur - (unsigned)s), lut, 378194u) : 0u;
                    rec_e[wave][row][seg] = e;
                    seg++;
                    cur = s;
                }
                unsigned w = exp_q16((int)((unsigned)s - (unsigned)cur), lut, 378194u);
                wsg[k] = w | ((unsigned)seg << 16);
            } else {
                wsg[k] = NOSEG << 16;
            }
        }
        for (int i = 0; i < 4; i++)
            *(uint4*)&scw[wave][row][grp * 16 + i * 4] = make_uint4(wsg[i * 4], wsg[i * 4 + 1], wsg[i * 4 + 2], wsg[i * 4 + 3]);
        // row-wide results: new running max and record count
        int mrow = cur;
        mrow = max(mrow, __shfl_xor(mrow, 16, 64));
        mrow = max(mrow, __shfl_xor(mrow, 32, 64));
        int nrow = nrec + __shfl_xor(nrec, 16, 64);
        nrow += __shfl_xor(nrow, 32, 64);
        int nmax = nrow;
        for (int o = 1; o < 16; o <<= 1) nmax = max(nmax, __shfl_xor(nmax, o, 64));
        m = mrow;
        wave_lds_fence();

        // 3. PV per segment. P^T operand: this lane's keys 16*blk + 4*grp + r (r fastest).
        unsigned wk[16];
        for (int blk = 0; blk < 4; blk++) {
            uint4 v = *(const uint4*)&scw[wave][row][blk * 16 + grp * 4];
            wk[blk * 4] = v.x; wk[blk * 4 + 1] = v.y; wk[blk * 4 + 2] = v.z; wk[blk * 4 + 3] = v.w;
        }
        v4i vop[4];
        for (int db = 0; db < 4; db++) {
            const int8_t* vr = Vt + (db * 16 + row) * KLD + grp * 4;
            vop[db] = (v4i){*(const int*)(vr), *(const int*)(vr + 16), *(const int*)(vr + 32), *(const int*)(vr + 48)};
        }
        for (int j = 0; j <= nmax; j++) {
            unsigned wj[16];
            unsigned sj = 0;
            for (int k = 0; k < 16; k++) {
                wj[k] = (wk[k] >> 16) == (unsigned)j ? (wk[k] & 0xFFFFu) : 0u;
                sj += wj[k];
            }
            v4i bc, bb, ba;
            for (int blk = 0; blk < 4; blk++) {
                bc[blk] = pack_limb(wj + blk * 4, 0, 127u);
                bb[blk] = pack_limb(wj + blk * 4, 7, 127u);
                ba[blk] = pack_limb(wj + blk * 4, 14, 3u);
            }
            sj += __shfl_xor(sj, 16, 64);
            sj += __shfl_xor(sj, 32, 64);
            if (j >= 1 && j <= nrow) {
                unsigned e = rec_e[wave][row][j - 1];
                if (e) rescale(S, vacc, e);
            }
            S += sj;
            for (int db = 0; db < 4; db++) {
                v4i z = (v4i){0, 0, 0, 0};
                v4i cc = __builtin_amdgcn_mfma_i32_16x16x64_i8(vop[db], bc, z, 0, 0, 0);
                v4i cb = __builtin_amdgcn_mfma_i32_16x16x64_i8(vop[db], bb, z, 0, 0, 0);
                v4i ca = __builtin_amdgcn_mfma_i32_16x16x64_i8(vop[db], ba, z, 0, 0, 0);
                for (int r = 0; r < 4; r++)
                    vacc[db * 4 + r] += ((unsigned)ca[r] << 14) + ((unsigned)cb[r] << 7) + (unsigned)cc[r];
            }
        }
    }
    if (p >= len) return;
    // normalize (attention.rs:278-285); lane holds dims 16*db + 4*grp + r
    const unsigned long long den = S == 0 ? 1ull : S;
    int8_t* o = a.out + ((size_t)b * T + p) * D + h * 64 + grp * 4;
    for (int db = 0; db < 4; db++) {
        unsigned pk = 0;
        for (int r = 0; r < 4; r++)
            pk |= ((unsigned)(uint8_t)(int8_t)clamp127(div_rne_s32_u64((int)vacc[db * 4 + r], den))) << (8 * r);
        *(unsigned*)(o + db * 16) = pk;
    }
}

void launch_attention(const AttnArgs& a, int B, hipStream_t s) {
    dim3 grid((unsigned)((a.T + 63) / 64), (unsigned)a.H, (unsigned)B);
    hipLaunchKernelGGL(k_attention, grid, dim3(256), 0, s, a);
}

// ---------------------------------------------------------------------------
// Logits -> cumulative frequencies (softmax_cdf.rs:85-139), one block per row.
// ---------------------------------------------------------------------------
constexpr int CDF_THREADS = 256;
constexpr int CDF_MAXE = 32;  // V <= 8192

template <typename T, typename Op>
__device__ __forceinline__ T block_reduce(T v, T* sh, Op op) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int o = 32; o > 0; o >>= 1) v = op(v, __shfl_xor(v, o, 64));
    if (lane == 0) sh[wave] = v;
    __syncthreads();
    T r = sh[0];
    for (int w = 1; w < CDF_THREADS / 64; w++) r = op(r, sh[w]);
    __syncthreads();
    return r;
}

__global__ __launch_bounds__(CDF_THREADS) void k_cdf(const int32_t* __restrict__ logits, int V,
                                                     const uint32_t* __restrict__ targets,
                                                     const int32_t* __restrict__ lens, int T,
                                                     const uint16_t* __restrict__ glut, unsigned coef,
                                                     unsigned total, int mode, uint32_t* __restrict__ out) {
    __shared__ uint16_t lut[256];
    __shared__ long long red[CDF_THREADS / 64];
    __shared__ unsigned scan[CDF_THREADS];
    const int row = blockIdx.x, tid = threadIdx.x;
    if (lens && (row % T) >= lens[row / T]) return;
    for (int i = tid; i < 256; i += CDF_THREADS) lut[i] = glut[i];
    const int per = (V + CDF_THREADS - 1) / CDF_THREADS;
    const int i0 = tid * per;
    const int32_t* L = logits + (size_t)row * V;
    int lv[CDF_MAXE];
    int mx = INT32_MIN;
    for (int k = 0; k < per; k++) {
        int i = i0 + k;
        lv[k] = i < V ? L[i] : INT32_MIN;
        if (i < V && lv[k] > mx) mx = lv[k];
    }
    __syncthreads();
    mx = (int)block_reduce<long long>((long long)mx, red, [](long long x, long long y) { return x > y ? x : y; });
    int am = 0x7fffffff;
    for (int k = 0; k < per; k++) {
        int i = i0 + k;
        if (i < V && lv[k] == mx && i < am) am = i;
    }
    am = (int)block_reduce<long long>((long long)am, red, [](long long x, long long y) { return x < y ? x : y; });
    unsigned e[CDF_MAXE];
    unsigned long long ls = 0;
    for (int k = 0; k < per; k++) {
        int i = i0 + k;
        e[k] = i < V ? exp_q16((int)((unsigned)lv[k] - (unsigned)mx), lut, coef) : 0u;
        ls += e[k];
    }
    const unsigned long long S =
        (unsigned long long)block_reduce<long long>((long long)ls, red, [](long long x, long long y) { return x + y; });
    const unsigned long long R = (unsigned long long)total - (unsigned long long)V;
    const double invS = 1.0 / (double)S;
    unsigned fl = 0;
    for (int k = 0; k < per; k++) {
        int i = i0 + k;
        unsigned f = 0;
        if (i < V) f = 1u + (unsigned)udiv64_32((unsigned long long)e[k] * R, (unsigned)S, invS);
        e[k] = f;  // reuse as freq
        fl += f;
    }
    // exclusive scan of per-thread sums
    scan[tid] = fl;
    __syncthreads();
    for (int o = 1; o < CDF_THREADS; o <<= 1) {
        unsigned v = tid >= o ? scan[tid - o] : 0u;
        __syncthreads();
        scan[tid] += v;
        __syncthreads();
    }
    const unsigned fsum = scan[CDF_THREADS - 1];
    const unsigned excl = scan[tid] - fl;
    const unsigned rem = total - fsum;
    if (mode == 0) {
        const int tok = (int)targets[row];
        if (tok >= i0 && tok < i0 + per) {
            unsigned lo = excl;
            for (int k = 0; k < tok - i0; k++) lo += e[k];
            unsigned f = e[tok - i0];
            if (am < tok) lo += rem;
            if (am == tok) f += rem;
            out[(size_t)row * 2] = lo;
            out[(size_t)row * 2 + 1] = lo + f;
        }
    } else {
        unsigned run = excl + (am < i0 ? rem : 0u);
        for (int k = 0; k < per; k++) {
            int i = i0 + k;
            if (i >= V) break;
            run += e[k] + (i == am ? rem : 0u);
            out[(size_t)row * V + i] = run;
        }
    }
}

void launch_cdf(const int32_t* logits, int M, int V, const uint32_t* targets, const int32_t* lens, int T,
                const uint16_t* lut, unsigned coef, unsigned total, int mode, uint32_t* out, hipStream_t s) {
    hipLaunchKernelGGL(k_cdf, dim3((unsigned)M), dim3(CDF_THREADS), 0, s, logits, V, targets, lens, T, lut, coef, total,
                       mode, out);
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

__global__ void k_encode(const uint32_t* __restrict__ lohi, const int32_t* __restrict__ lens, int nb, int T,
                         unsigned total, uint8_t* __restrict__ out, long long slot, int32_t* __restrict__ out_lens,
                         int32_t* __restrict__ err) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= nb) return;
    const unsigned long long MASK = 0xFFFFFFFFull, HALF = 1ull << 31, QUART = 1ull << 30;
    unsigned long long low = 0, high = MASK;
    unsigned underflow = 0;
    BitOut o{out + (size_t)c * slot, slot, 0, 0u, 7, 0};
    const double invT = 1.0 / (double)total;
    const int n = lens[c];
    for (int i = 0; i < n; i++) {
        const unsigned long long lo = lohi[((size_t)c * T + i) * 2], hi = lohi[((size_t)c * T + i) * 2 + 1];
        const unsigned long long range = high - low + 1;
        high = low + udiv64_32(hi * range, total, invT) - 1;
        low = low + udiv64_32(lo * range, total, invT);
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
