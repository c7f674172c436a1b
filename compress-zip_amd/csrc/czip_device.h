// Device-side integer primitives shared by the gfx950 kernels.
//
// Bit-exact copies of rust/src/primitives.rs, lut.rs and rmsnorm.rs.
// Wrapping i32 arithmetic is written with unsigned types (the reference is
// built without overflow checks, so i32 adds and multiplies wrap).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace czip {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));

constexpr unsigned ATTN_COEF_Q24 = 378194u;  // (LOG2E / 64 * 2^24 + 0.5) as u32, attention.rs:17-19
constexpr uint32_t BOS_TOKEN = 1022u;        // main.rs:222, 387

__device__ __forceinline__ int clamp127(int x) { return x < -127 ? -127 : (x > 127 ? 127 : x); }

// Byte offset of 16-byte chunk c of row r in an LDS tile of 64-byte rows, the
// chunks of a row permuted by c ^ ((r >> 1) & 3): both the MFMA operand reads
// (lane -> row l % 16, chunk l / 16) and the row-major stores (lane -> row
// l / 4, chunk l % 4) then touch every bank once per access (measured with
// the LDS bank-conflict counter on gfx950; an unpermuted 80-byte stride costs
// 4 extra cycles per read and 8 per store).
__device__ __forceinline__ int lds64(int r, int c) { return r * 64 + ((c ^ ((r >> 1) & 3)) << 4); }

// V^T caches hold each KV head's values transposed in blocks of 2^vl keys,
// [key >> vl][dim][key & (2^vl - 1)]: the PV operand (16 consecutive keys of
// one dim) is one 16-byte load with 16-key blocks (vl = 4, the prefill
// caches) and four 4-byte loads with 4-key blocks (vl = 2, the caches a
// decode step appends one key to: the step's 64 value bytes then fall in 256
// bytes instead of 1 KB).  Byte offset of (key p, dim) in a head's cache:
__device__ __forceinline__ int vt_off(int p, int dim, int vl) {
    return ((p >> vl) << (6 + vl)) + (dim << vl) + (p & ((1 << vl) - 1));
}

constexpr int BUF_DWORD3 = 0x00020000;  // word 3 of a raw buffer resource: 32-bit data format, no swizzle

// Fragment-major weights: for W [N, K] (N % 16 == 0, K % 64 == 0) the MFMA
// operand of rows 16 t .. 16 t + 15 at K step s is the 1 KB at
// (t * K / 64 + s) * 1024, lane l's 16 bytes at +16 l being W[16 t + l % 16,
// 64 s + 16 (l / 16) .. +16]: one operand load reads eight whole 128-byte
// lines (the row-major operand touches half of 16 lines, and the other half
// is gone from L1 by the next step).
//
// acc[i][t] += A[m0 + 16 i + l%16, :] . W[nb + 16 t + l%16, :] over K (a
// multiple of 64) for a workgroup that owns 64 rows of A, Wf fragment-major:
// the 64 x 64 A tile of each K step goes through double-buffered LDS (threads
// 0..255 stage 16 bytes each; rows past M read as 0 by the buffer range
// check), and each wave streams its own CT W operands straight into
// registers, in two register sets so that the next step's loads are in
// flight while the current one multiplies.  W is the first MFMA operand: lane
// l ends with columns nb + 16 t + 4 (l / 16) .. +3 of rows m0 + 16 i + l % 16.
template <int CT>
__device__ __forceinline__ void rowblock_mma(const int8_t* A, int M, int K, const int8_t* Wf, int wrows, int m0,
                                             int nb, int8_t (*As)[64 * 64], v4i (&acc)[4][CT], int ks0 = 0,
                                             int nks = -1) {
    // K steps ks0 .. ks0 + nks - 1 (all of them by default)
    const int tid = threadIdx.x, lane = tid & 63, lr = lane & 15;
    const int nkt = K / 64;
    const int nk = nks < 0 ? nkt : nks;
    const int arows = M - m0 < 64 ? M - m0 : 64;
    const __amdgpu_buffer_rsrc_t rA =
        __builtin_amdgcn_make_buffer_rsrc((void*)(A + (size_t)m0 * K), (short)0, arows * K, BUF_DWORD3);
    const __amdgpu_buffer_rsrc_t rW = __builtin_amdgcn_make_buffer_rsrc((void*)Wf, (short)0, wrows * K, BUF_DWORD3);
    const int aoff = (tid >> 2) * K + (tid & 3) * 16 + ks0 * 64;
    const int woff = (nb >> 4) * nkt * 1024 + ks0 * 1024 + lane * 16;
    v4i ra = (v4i){0, 0, 0, 0};
    auto fetch_a = [&](int k0) {
        if (tid < 256) ra = __builtin_amdgcn_raw_buffer_load_b128(rA, aoff, k0, 0);
    };
    auto store_a = [&](int buf) {
        if (tid < 256) *(v4i*)(As[buf] + lds64(tid >> 2, tid & 3)) = ra;
    };
    auto fetch_w = [&](v4i* w, int k0) {
#pragma unroll
        for (int t = 0; t < CT; t++) w[t] = __builtin_amdgcn_raw_buffer_load_b128(rW, woff + t * nkt * 1024, (k0 >> 6) * 1024, 0);
    };
    auto step = [&](int kt, const v4i* wc, v4i* wn) {
        const bool more = kt + 1 < nk;
        if (more) {
            fetch_a((kt + 1) * 64);
            fetch_w(wn, (kt + 1) * 64);
        }
        __builtin_amdgcn_sched_barrier(0);  // the next step's loads ahead of this step's MFMAs
        v4i af[4];
#pragma unroll
        for (int i = 0; i < 4; i++) af[i] = *(const v4i*)(As[kt & 1] + lds64(i * 16 + lr, lane >> 4));
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int t = 0; t < CT; t++) acc[i][t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wc[t], af[i], acc[i][t], 0, 0, 0);
        if (more) store_a((kt & 1) ^ 1);
        __syncthreads();
    };
    v4i w0[CT], w1[CT];
    fetch_a(0);
    fetch_w(w0, 0);
    store_a(0);
    __syncthreads();
    int kt = 0;
    for (; kt + 1 < nk; kt += 2) {
        step(kt, w0, w1);
        step(kt + 1, w1, w0);
    }
    if (kt < nk) step(kt, w0, w1);
}

// The K steps of rowblock_mma_full over a row block already in As (its
// caller staged it and waited for every wave): each wave's W one step ahead.
template <int CT>
__device__ __forceinline__ void rowblock_mma_lds(int lane, int K, const int8_t* Wf, int wrows, int nb,
                                                 const int8_t (*As)[64 * 64], v4i (&acc)[4][CT]) {
    const int lr = lane & 15;
    const int nkt = K / 64;
    const __amdgpu_buffer_rsrc_t rW = __builtin_amdgcn_make_buffer_rsrc((void*)Wf, (short)0, wrows * K, BUF_DWORD3);
    const int woff = (nb >> 4) * nkt * 1024 + lane * 16;
    v4i w0[CT], w1[CT];
    auto fetch_w = [&](v4i* w, int kt) {
#pragma unroll
        for (int t = 0; t < CT; t++) w[t] = __builtin_amdgcn_raw_buffer_load_b128(rW, woff + t * nkt * 1024, kt * 1024, 0);
    };
    fetch_w(w0, 0);
    auto step = [&](int kt, const v4i* wc, v4i* wn) {
        if (kt + 1 < nkt) fetch_w(wn, kt + 1);
        v4i af[4];
#pragma unroll
        for (int i = 0; i < 4; i++) af[i] = *(const v4i*)(As[kt] + lds64(i * 16 + lr, lane >> 4));
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int t = 0; t < CT; t++) acc[i][t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wc[t], af[i], acc[i][t], 0, 0, 0);
    };
    int kt = 0;
    for (; kt + 1 < nkt; kt += 2) {
        step(kt, w0, w1);
        step(kt + 1, w1, w0);
    }
    if (kt < nkt) step(kt, w0, w1);
}

// The same product with the row block's whole A (64 rows x K) staged in LDS
// at once (As: K / 64 tiles of [64][64], 64-byte permuted rows), one barrier,
// then the K steps without barriers, each wave's W one step ahead.  The
// workgroup's threads (any multiple of 64) share the staging.
template <int CT>
__device__ __forceinline__ void rowblock_mma_full(const int8_t* A, int M, int K, const int8_t* Wf, int wrows, int m0,
                                                  int nb, int8_t (*As)[64 * 64], v4i (&acc)[4][CT]) {
    const int tid = threadIdx.x, lane = tid & 63, lr = lane & 15;
    const int nkt = K / 64;
    const int arows = M - m0 < 64 ? M - m0 : 64;
    const __amdgpu_buffer_rsrc_t rA =
        __builtin_amdgcn_make_buffer_rsrc((void*)(A + (size_t)m0 * K), (short)0, arows * K, BUF_DWORD3);
    const __amdgpu_buffer_rsrc_t rW = __builtin_amdgcn_make_buffer_rsrc((void*)Wf, (short)0, wrows * K, BUF_DWORD3);
    const int woff = (nb >> 4) * nkt * 1024 + lane * 16;
    v4i w0[CT], w1[CT];
    auto fetch_w = [&](v4i* w, int kt) {
#pragma unroll
        for (int t = 0; t < CT; t++) w[t] = __builtin_amdgcn_raw_buffer_load_b128(rW, woff + t * nkt * 1024, kt * 1024, 0);
    };
    fetch_w(w0, 0);
    // chunk c: K step c / 256, row (c / 4) % 64, 16-byte piece c % 4
    for (int c = tid; c < nkt * 256; c += (int)blockDim.x) {
        const v4i x = __builtin_amdgcn_raw_buffer_load_b128(rA, ((c >> 2) & 63) * K + (c >> 8) * 64 + (c & 3) * 16, 0, 0);
        *(v4i*)(As[c >> 8] + lds64((c >> 2) & 63, c & 3)) = x;
    }
    __syncthreads();
    auto step = [&](int kt, const v4i* wc, v4i* wn) {
        if (kt + 1 < nkt) fetch_w(wn, kt + 1);
        v4i af[4];
#pragma unroll
        for (int i = 0; i < 4; i++) af[i] = *(const v4i*)(As[kt] + lds64(i * 16 + lr, lane >> 4));
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int t = 0; t < CT; t++) acc[i][t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wc[t], af[i], acc[i][t], 0, 0, 0);
    };
    int kt = 0;
    for (; kt + 1 < nkt; kt += 2) {
        step(kt, w0, w1);
        step(kt + 1, w1, w0);
    }
    if (kt < nkt) step(kt, w0, w1);
}

// rint(a * b) (round half to even) for |a * b| < 2^31, exact when a * b is
// exact in f64: adding 1.5 * 2^52 makes the ulp 1, so the FMA's single
// rounding lands on the integer, and the low word of the sum is that integer
// modulo 2^32 (the mantissa holds 2^51 + rint(a * b)).
__device__ __forceinline__ int rint_fma_i32(double a, double b) {
    const double r = __builtin_fma(a, b, 6755399441055744.0);
    return (int)(unsigned)__builtin_bit_cast(unsigned long long, r);
}

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

// sra_rne32 for 1 <= sh <= 30 and |v| < 2^31 - 2^sh: round half to even is
// symmetric, so the floor form (v + 2^(sh-1) - 1 + bit_sh(v)) >> sh equals the
// sign-magnitude one.
__device__ __forceinline__ int rne_shr(int v, int sh) { return (v + (1 << (sh - 1)) - 1 + ((v >> sh) & 1)) >> sh; }

// RoPE rounding for |v| < 2^31: sra_rne32(v, 15) (m = 1, bb = 0) or
// sra_rne32(sra_rne32(v, 15), 1) (m = 1/2, bb = B/2), B = 1.5 * 2^67, whose
// ulp is 2^15: r1 = v + B is B + 2^15 RNE(v / 2^15) exactly (its mantissa
// 1.5 * 2^52 + the quotient), and fma(r1, m, bb) is B + 2^15 times r1's
// quotient times m rounded once (half to even, as the reference's symmetric
// RNE); the low word is the result.  (An add with B held in scalar registers
// where an FMA by 2^-15 would need B copied into vector registers each time.)
__device__ __forceinline__ int rope_round(int v, double m, double bb) {
    const double r1 = (double)v + 221360928884514619392.0;  // 1.5 * 2^67
    return (int)(unsigned)__builtin_bit_cast(unsigned long long, __builtin_fma(r1, m, bb));
}
constexpr double ROPE_Q_BIAS = 110680464442257309696.0;  // bb of the query's second rounding: 0.75 * 2^67

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

// sra_rne64((i64)a * b, sh) computed in sign-magnitude form with one
// 32x32->64 multiply; identical results for every (a, b, sh in 1..31).
__device__ __forceinline__ int mul_sra_rne(int a, int b, unsigned sh) {
    const unsigned sa = (unsigned)(a >> 31), sb = (unsigned)(b >> 31);
    const unsigned ua = ((unsigned)a ^ sa) - sa, ub = ((unsigned)b ^ sb) - sb;
    const unsigned long long p = (unsigned long long)ua * ub;
    unsigned long long q = p >> sh;
    const unsigned r = (unsigned)p & ((1u << sh) - 1u), half = 1u << (sh - 1);
    q += (r > half) ? 1ull : ((r == half) ? (q & 1ull) : 0ull);
    const bool neg = (sa ^ sb) != 0u && p != 0ull;
    if (neg) return q >= 0x80000000ull ? INT32_MIN : -(int)q;
    return q > 0x7FFFFFFFull ? INT32_MAX : (int)q;
}

// model.rs:280-300
__device__ __forceinline__ int requant(int v, int mult, int shift) {
    if (shift <= 0) {
        long long p = (long long)v * (long long)mult;
        return (int)(p < -127 ? -127 : (p > 127 ? 127 : p));
    }
    if (shift < 32) return clamp127(mul_sra_rne(v, mult, (unsigned)shift));
    return clamp127(sra_rne64((long long)v * (long long)mult, (unsigned)shift));
}

// rmsnorm.rs:14-30: clamp(udiv_rne(2^23, isqrt32(mean_sq << 16)), 1, 32768)
// (primitives.rs:80-97, 192-213) for mean_sq in [1, 2^16): the integer square
// root by f64 sqrt with an exact correction, the round-half-even quotient by
// an f64 estimate with an exact remainder test (2^23 / s, s in [256, 2^16)).
// Checked against the reference algorithm on every mean_sq < 2^16.
__device__ __forceinline__ int inv_rms_q15_fast(int mean_sq) {
    const unsigned x = (unsigned)(mean_sq > 0 ? mean_sq : 1) << 16;
    unsigned long long r = (unsigned long long)__builtin_sqrt((double)x);
    if (r * r > x) r--;
    if ((r + 1) * (r + 1) <= x) r++;
    const unsigned d = (unsigned)r;
    unsigned q = (unsigned)(8388608.0 / (double)d);
    int rem = (int)(8388608u - q * d);
    if (rem < 0) { q--; rem += (int)d; }
    if (rem >= (int)d) { q++; rem -= (int)d; }
    const unsigned tr = (unsigned)rem << 1;
    const unsigned inv = tr > d ? q + 1 : (tr == d ? q + (q & 1u) : q);
    return (int)(inv < 1u ? 1u : (inv > 32768u ? 32768u : inv));
}

// model.rs:280-300.  Fast path: |v * mult| < 2^53, so v * mult * 2^-shift is
// exact in f64, and |v * mult * 2^-shift| < 2^31, so its rint (half to even,
// like sra_rne_tte_s64_to_s32) is one FMA and the clamp an integer med3.
template <bool FAST>
__device__ __forceinline__ int rq(int v, double scale, int mult, int shift) {
    if (FAST) return clamp127(rint_fma_i32((double)v, scale));
    return requant(v, mult, shift);
}

__device__ __forceinline__ unsigned pack4i(int a, int b, int c, int d) {
    return (unsigned)(a & 0xFF) | ((unsigned)(b & 0xFF) << 8) | ((unsigned)(c & 0xFF) << 16) | ((unsigned)d << 24);
}

__device__ __forceinline__ void unpack4s(unsigned w, int* o) {
    o[0] = (int)(int8_t)(w & 0xFF);
    o[1] = (int)(int8_t)((w >> 8) & 0xFF);
    o[2] = (int)(int8_t)((w >> 16) & 0xFF);
    o[3] = (int)(int8_t)(w >> 24);
}

// rmsnorm.rs:40-75 for one element: clamp(sra_rne((x * w) * inv, 15)).  |x|, |w| <= 127 and
// 1 <= inv <= 2^15, so x * w is an exact 24-bit multiply and (x * w) * (inv * 2^-15)
// is exact in f64 with |.| < 2^15: its rint (half to even) is one FMA.
__device__ __forceinline__ int rms_el(int x, int w, double inv_s15) {
    return clamp127(rint_fma_i32((double)__mul24(x, w), inv_s15));
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

// exp_q16 (lut.rs:213-235 / softmax_cdf.rs:55-77) without branches, from a
// table pre-shifted by 16 bits (lut32[i] = lut[i] << 16): for ip <= 16,
// (65536 >> ip) * lut == (lut << 16) >> ip; for 17 <= ip <= 31 both round to 0
// and clamp to 1; ip is capped at 31 like the early return.
__device__ __forceinline__ unsigned exp_q16_bf(int diff, const unsigned* lut32, unsigned coef) {
    const unsigned neg = 0u - (unsigned)diff;
    const unsigned long long pr = (unsigned long long)neg * coef + (1ull << 23);
    const unsigned t = (unsigned)(pr >> 24);
    const unsigned ip = min(t >> 8, 31u);
    const unsigned x = max(((lut32[t & 255u] >> ip) + 0x8000u) >> 16, 1u);
    return diff >= 0 ? 65535u : x;
}

// The table step of exp_q16(-neg) for a coefficient below 2^24 (coef256 =
// coef * 256): t = floor((neg * coef + 2^23) / 2^24) is the high word of
// neg * coef256 + 2^31 (one 32 x 32 + 64 multiply-add), and every t >= 4352
// (ip >= 17, result 1) gives the same result as t = 4352 (lut32[0] >> 17
// rounds to 0), so clamping t replaces clamping ip.
__device__ __forceinline__ unsigned exp_q16_t(unsigned neg, const unsigned* lut32, unsigned coef256) {
    const unsigned t = min((unsigned)(((unsigned long long)neg * coef256 + 0x80000000ull) >> 32), 4352u);
    return max(((lut32[t & 255u] >> (t >> 8)) + 0x8000u) >> 16, 1u);
}

// primitives.rs:163-185 (the result is formed with i32 wrap like `as i32 * sign`)
__device__ __forceinline__ int div_rne_s32_u64(int num, unsigned long long den) {
    if (den == 0) return 0;
    unsigned long long an = (unsigned long long)(num < 0 ? 0u - (unsigned)num : (unsigned)num);
    unsigned long long q, r;
    if (den <= 0xFFFFFFFFull) {
        unsigned q32 = (unsigned)an / (unsigned)den;
        q = q32;
        r = an - q * den;
    } else {
        q = 0;
        r = an;
    }
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
__device__ __forceinline__ unsigned wave_sum_u(unsigned v) {
    for (int o = 32; o > 0; o >>= 1) v += (unsigned)__shfl_xor((int)v, o, 64);
    return v;
}
__device__ __forceinline__ int wave_max_i(int v) {
    for (int o = 32; o > 0; o >>= 1) v = max(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ __forceinline__ int wave_min_i(int v) {
    for (int o = 32; o > 0; o >>= 1) v = min(v, __shfl_xor(v, o, 64));
    return v;
}

}  // namespace czip
