// Batched autoregressive decode (decompression): one token per stream per
// step, each stream a chunk of the .czip payload (main.rs:377-396), with an
// arithmetic decoder per stream kept on the device (arith_coder.rs:139-264).
#include "czip_device.h"
#include "czip_kernels.h"

namespace czip {

constexpr unsigned long long DMASK = 0xFFFFFFFFull, DHALF = 1ull << 31, DQUART = 1ull << 30;

__device__ __forceinline__ unsigned read_bit(const uint8_t* __restrict__ data, long long len, long long& byte_pos,
                                             int& bit_pos) {
    // arith_coder.rs:176-190 (zeros past the end of the chunk)
    if (byte_pos >= len) return 0u;
    unsigned bit = (data[byte_pos] >> bit_pos) & 1u;
    if (--bit_pos < 0) { byte_pos++; bit_pos = 7; }
    return bit;
}

// ArithDecoder::new (arith_coder.rs:153-172)
__global__ void k_dec_init(DecState st, DecStreams ds, int S) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= S) return;
    const uint8_t* data = ds.data + ds.offs[b];
    const long long len = ds.blen[b];
    long long bp = 0;
    int bi = 7;
    unsigned long long code = 0;
    for (int i = 0; i < 32; i++) code = (code << 1) | read_bit(data, len, bp, bi);
    st.low[b] = 0u;
    st.high[b] = 0xFFFFFFFFu;
    st.code[b] = (uint32_t)code;
    st.byte_pos[b] = bp;
    st.bit_pos[b] = bi;
}

void launch_dec_init(DecState st, DecStreams ds, int S, hipStream_t s) {
    hipLaunchKernelGGL(k_dec_init, dim3((unsigned)((S + 63) / 64)), dim3(64), 0, s, st, ds, S);
}

// forward input of step p (main.rs:386-388)
__global__ void k_dec_prep(DecStreams ds, int S, int p, uint32_t* __restrict__ inp) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= S) return;
    uint32_t t = 0u;
    if (p < ds.ntok[b]) t = p == 0 ? BOS_TOKEN : ds.tokens[ds.tok_offs[b] + p - 1];
    inp[b] = t;
}

void launch_dec_prep(DecStreams ds, int S, int p, uint32_t* inp, hipStream_t s) {
    hipLaunchKernelGGL(k_dec_prep, dim3((unsigned)((S + 255) / 256)), dim3(256), 0, s, ds, S, p, inp);
}

// ---------------------------------------------------------------------------
// Decode attention: one wavefront per (stream, head), query at position p.
// Per 64-key tile the lanes (= keys) form the scores and, with a wave-wide
// prefix max, the records, weights and rescale factors all at once; the
// reference's in-order update (attention.rs:227-276) then runs with
// lanes = head dims, one multiply-add per key.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int dec_score(int dot, int mult) { return mul_sra_rne(sra_rne32(dot, 2), mult, 15); }

__global__ __launch_bounds__(64) void k_attn_decode(AttnArgs a, int p) {
    __shared__ uint16_t lut[256];
    __shared__ __attribute__((aligned(16))) int8_t qs[64];
    __shared__ __attribute__((aligned(16))) int8_t vs[64 * 64];
    __shared__ unsigned wk[64];   // weight of key j
    __shared__ unsigned ek[64];   // rescale factor if key j is a record (0: no rescale)
    __shared__ int rk[64];        // key j is a record
    const int lane = threadIdx.x;
    const int b = blockIdx.x, h = blockIdx.y;
    for (int i = lane; i < 256; i += 64) lut[i] = a.lut[i];
    if (p >= a.lens[b]) return;  // stream finished (uniform)
    const int D = a.H * 64;
    qs[lane] = a.q[(size_t)b * D + h * 64 + lane];
    __syncthreads();
    const int g = a.kv_mode == 1 ? (h * a.G) / a.H : 0;
    const int8_t* K = a.kc + ((size_t)b * a.KH + g) * a.T * 64;
    const int8_t* Vr = a.vc + ((size_t)b * a.KH + g) * a.T * 64;
    const int mult = a.score_mult[h];
    const int* q4 = (const int*)qs;

    int m = INT32_MIN;
    unsigned long long S = 0;
    unsigned vacc = 0;
    if (a.sink) {  // attention.rs:211-224
        int dot = 0;
        for (int i = 0; i < 16; i++) dot = __builtin_amdgcn_sdot4(q4[i], ((const int*)a.sink)[i], dot, false);
        m = dec_score(dot, mult);
        S = 65535ull;
    }
    for (int t0 = 0; t0 <= p; t0 += 64) {
        const int t = t0 + lane;
        const int nt = min(64, p - t0 + 1);
        // stage the tile's V rows (coalesced) while forming the scores
        for (int i = 0; i < 4; i++) {
            const int r = (lane >> 2) + 16 * i, c = (lane & 3) * 16;
            int4 v = make_int4(0, 0, 0, 0);
            if (r < nt) v = *(const int4*)(Vr + (size_t)(t0 + r) * 64 + c);
            *(int4*)(vs + r * 64 + c) = v;
        }
        int s = 0;
        if (lane < nt) {
            const int* k4 = (const int*)(K + (size_t)t * 64);
            int dot = 0;
            for (int i = 0; i < 16; i++) dot = __builtin_amdgcn_sdot4(q4[i], k4[i], dot, false);
            s = dec_score(dot, mult);
        }
        // inclusive prefix max over valid keys, seeded with the running max
        int pm = lane < nt ? s : INT32_MIN;
        for (int o = 1; o < 64; o <<= 1) {
            int v = __shfl_up(pm, o, 64);
            if (lane >= o) pm = max(pm, v);
        }
        pm = max(pm, m);
        int prev = __shfl_up(pm, 1, 64);
        if (lane == 0) prev = m;
        // key lane is a record iff s > running max before it
        const bool rec = lane < nt && s > prev;
        unsigned e = 0, w = 0;
        if (lane < nt) {
            if (rec) {
                e = prev != INT32_MIN ? exp_q16((int)((unsigned)prev - (unsigned)s), lut, ATTN_COEF_Q24) : 0u;
                w = 65535u;
            } else {
                w = exp_q16((int)((unsigned)s - (unsigned)pm), lut, ATTN_COEF_Q24);
            }
        }
        wk[lane] = w;
        ek[lane] = e;
        rk[lane] = rec ? 1 : 0;
        m = __shfl(pm, 63, 64);
        __syncthreads();
        for (int j = 0; j < nt; j++) {
            if (rk[j]) {
                const unsigned ej = ek[j];
                if (ej) {
                    S = (S * ej + 0x8000ull) >> 16;
                    long long pr = (long long)(int)vacc * (long long)ej;
                    pr += pr >= 0 ? (1ll << 15) : -(1ll << 15);
                    vacc = (unsigned)(int)(pr >> 16);
                }
            }
            const unsigned wj = wk[j];
            S += wj;
            vacc += (unsigned)((int)wj * (int)vs[j * 64 + lane]);
        }
        __syncthreads();
    }
    const unsigned long long den = S == 0 ? 1ull : S;
    a.out[(size_t)b * D + h * 64 + lane] = (int8_t)clamp127(div_rne_s32_u64((int)vacc, den));
}

void launch_attn_decode(const AttnArgs& a, int S, int p, hipStream_t s) {
    hipLaunchKernelGGL(k_attn_decode, dim3((unsigned)S, (unsigned)a.H), dim3(64), 0, s, a, p);
}

// ---------------------------------------------------------------------------
// Logits -> cumulative frequencies (softmax_cdf.rs:85-139) -> one decode step
// (arith_coder.rs:195-264).  Same frequency arithmetic as the prefill CDF
// kernel; the symbol is the first index whose cumulative frequency exceeds
// value = ((code - low + 1) * total - 1) / range.
// ---------------------------------------------------------------------------
template <int WPR, int EPL>
__global__ __launch_bounds__(64 * WPR) void k_cdf_decode(const int32_t* __restrict__ logits, int V,
                                                         const uint16_t* __restrict__ glut, unsigned coef,
                                                         unsigned total, int p, DecState st, DecStreams ds) {
    __shared__ uint16_t lut[256];
    __shared__ int red_i[WPR];
    __shared__ unsigned red_u[WPR];
    __shared__ unsigned found[2];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int b = blockIdx.x;
    for (int i = tid; i < 256; i += 64 * WPR) lut[i] = glut[i];
    if (p >= ds.ntok[b]) return;  // uniform per block
    __syncthreads();
    const int i0 = tid * EPL;
    const int32_t* L = logits + (size_t)b * V;
    int lv[EPL];
#pragma unroll
    for (int k = 0; k < EPL; k++) lv[k] = (i0 + k < V) ? L[i0 + k] : INT32_MIN;
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
    unsigned f[EPL];
    unsigned ls = 0;
#pragma unroll
    for (int k = 0; k < EPL; k++) {
        f[k] = (i0 + k < V) ? exp_q16((int)((unsigned)lv[k] - (unsigned)mx), lut, coef) : 0u;
        ls += f[k];
    }
    const unsigned Ssum = bsum(ls);
    const unsigned R = total - (unsigned)V;
    const unsigned Q = R / Ssum, Rm = R - Q * Ssum;
    const float rf = (float)Rm / (float)Ssum;
    unsigned fl = 0;
#pragma unroll
    for (int k = 0; k < EPL; k++) {
        unsigned fk = 0;
        if (i0 + k < V) {
            unsigned q = (unsigned)((float)f[k] * rf);
            const unsigned long long t = (unsigned long long)f[k] * Rm, u = (unsigned long long)q * Ssum;
            if (t < u) q -= 1;
            else if (t - u >= Ssum) q += 1;
            fk = 1u + f[k] * Q + q;
        }
        f[k] = fk;
        fl += fk;
    }
    const unsigned rem = total - bsum(fl);
    // exclusive scan of the per-thread sums
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
        __syncthreads();
    }
    // decoder state
    const unsigned long long low = st.low[b], high = st.high[b], code = st.code[b];
    const unsigned long long range = high - low + 1;  // <= 2^32
    const unsigned long long value = ((code - low + 1) * (unsigned long long)total - 1) / range;
    const unsigned v32 = (unsigned)value;
    // first i with v32 < cum_i, clamped to V-1 (arith_coder.rs:225-241)
    unsigned run = excl + (am < i0 ? rem : 0u);
    int sym = 0x7FFFFFFF;
    unsigned lo_c = 0, hi_c = 0;
#pragma unroll
    for (int k = 0; k < EPL; k++) {
        if (i0 + k < V) {
            const unsigned before = run;
            run += f[k] + (i0 + k == am ? rem : 0u);
            if (sym == 0x7FFFFFFF && v32 < run) { sym = i0 + k; lo_c = before; hi_c = run; }
        }
    }
    int best = bmin(sym);
    if (best == 0x7FFFFFFF) {  // value >= total: the last symbol
        best = V - 1;
        if (i0 <= V - 1 && V - 1 < i0 + EPL) { lo_c = run - f[V - 1 - i0] - (V - 1 == am ? rem : 0u); hi_c = run; sym = V - 1; }
    }
    if (sym == best) { found[0] = lo_c; found[1] = hi_c; }
    __syncthreads();
    if (tid != 0) return;
    const unsigned long long sl = found[0], sh = found[1];
    const double invT = 1.0 / (double)total;
    unsigned long long nh = low + udiv64_32(sh * range, total, invT) - 1;
    unsigned long long nl = low + udiv64_32(sl * range, total, invT);
    unsigned long long cd = code;
    const uint8_t* data = ds.data + ds.offs[b];
    const long long len = ds.blen[b];
    long long bp = st.byte_pos[b];
    int bi = st.bit_pos[b];
    for (;;) {
        if (((nl ^ nh) & DHALF) == 0) {
            nl = (nl << 1) & DMASK;
            nh = ((nh << 1) & DMASK) | 1;
            cd = ((cd << 1) & DMASK) | read_bit(data, len, bp, bi);
        } else if ((nl & ~nh & DQUART) != 0) {
            nl = ((nl << 1) ^ DHALF) & DMASK;
            nh = (((nh ^ DHALF) << 1) | DHALF | 1) & DMASK;
            cd = (cd & DHALF) | ((cd << 1) & (DMASK >> 1)) | read_bit(data, len, bp, bi);
        } else {
            break;
        }
    }
    st.low[b] = (uint32_t)nl;
    st.high[b] = (uint32_t)nh;
    st.code[b] = (uint32_t)cd;
    st.byte_pos[b] = bp;
    st.bit_pos[b] = bi;
    ds.tokens[ds.tok_offs[b] + p] = (uint32_t)best;
}

void launch_cdf_decode(const int32_t* logits, int S, int V, const uint16_t* lut, unsigned coef, unsigned total, int p,
                       DecState st, DecStreams ds, hipStream_t s) {
    if (V <= 1024)
        hipLaunchKernelGGL((k_cdf_decode<1, 16>), dim3((unsigned)S), dim3(64), 0, s, logits, V, lut, coef, total, p,
                           st, ds);
    else if (V <= 4096)
        hipLaunchKernelGGL((k_cdf_decode<4, 16>), dim3((unsigned)S), dim3(256), 0, s, logits, V, lut, coef, total, p,
                           st, ds);
    else
        hipLaunchKernelGGL((k_cdf_decode<4, 32>), dim3((unsigned)S), dim3(256), 0, s, logits, V, lut, coef, total, p,
                           st, ds);
}

}  // namespace czip
