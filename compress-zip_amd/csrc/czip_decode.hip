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
// Decode attention (attention.rs:162-289 for one query per stream): one
// workgroup per (stream, KV group), one wavefront per head of the group.  Per
// 64-key tile the K rows and the transposed V (V^T rows, one per head dim)
// are staged in LDS once for all heads, while the next tile is fetched into
// registers.  Each wave then:
//  1. lanes = keys: scores, the running max by a wave prefix max, records,
//     weights and rescale factors, and the prefix sums of the weights;
//  2. lanes = head dims: walks the tile in groups of 4 keys; a group's
//     contribution sum(w v) comes from sdot4 over signed weight bytes
//     (w - 32896 = 256*hi + lo, plus 32896 * sum(v) of the group), and a
//     group holding records is split at them: rescale at the record, then
//     continue (the reference's in-order update, attention.rs:227-276).
// S follows the same records with segment sums taken from the prefix sums.
constexpr int DKLD = 80;              // LDS row stride of the K and V^T tiles (conflict-free 16-byte reads)
constexpr unsigned DWOFF = 32896;     // w - DWOFF = 256*hi + lo with hi, lo signed bytes

__device__ __forceinline__ int dec_score(int dot, double mscale) {
    // sra_rne64(sra_rne32(dot, 2) * mult, 15) with the i32 clamp: exact in f64
    const int du = (dot + 1 + ((dot >> 2) & 1)) >> 2;
    double r = __builtin_rint((double)du * mscale);
    r = fmin(fmax(r, -2147483648.0), 2147483647.0);
    return (int)r;
}

// rescale at a record (attention.rs:246-261): ((i64)v * e +- 2^15) >> 16
__device__ __forceinline__ unsigned dec_rescale(unsigned v, unsigned e) {
    const int vh = (int)v >> 16;
    const unsigned t = __umul24(v & 0xFFFFu, e);
    return (unsigned)__mul24(vh, (int)e) + (t >> 16) + ((t >> 15) & 1u) + (unsigned)((int)v >> 31);
}

// sum over the keys of byte mask m (0xFF per key) of w * v for one group of 4
// keys: weights hi/lo (other keys carry w = 0, i.e. bytes 0x80), values vg
__device__ __forceinline__ unsigned group_wv(unsigned hi, unsigned lo, unsigned m, int vg, unsigned vsum) {
    const unsigned h = (hi & m) | (0x80808080u & ~m), l = (lo & m) | (0x80808080u & ~m);
    const int sh = __builtin_amdgcn_sdot4((int)h, vg, 0, false), sl = __builtin_amdgcn_sdot4((int)l, vg, 0, false);
    return ((unsigned)sh << 8) + (unsigned)sl + vsum * DWOFF;
}

__global__ __launch_bounds__(1024) void k_attn_decode(AttnArgs a, int p) {
    __shared__ unsigned lut32[256];
    __shared__ __attribute__((aligned(16))) int8_t Ks[64 * DKLD];
    __shared__ __attribute__((aligned(16))) int8_t Vt[64 * DKLD];
    __shared__ __attribute__((aligned(16))) uint8_t whi[16][64], wlo[16][64];
    __shared__ unsigned ekl[16][64];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, nthr = (int)blockDim.x;
    const int b = blockIdx.x, g = blockIdx.y;
    for (int i = tid; i < 256; i += nthr) lut32[i] = (unsigned)a.lut[i] << 16;
    if (p >= a.lens[b]) return;  // stream finished (uniform)
    // heads of KV group g: h with (h * G) / H == g in GQA mode; all heads otherwise
    int h0 = 0, h1 = a.H;
    if (a.kv_mode == 1) {
        h0 = (g * a.H + a.G - 1) / a.G;
        h1 = ((g + 1) * a.H + a.G - 1) / a.G;
    }
    const int h = h0 + wave;
    const bool live = h < h1;
    const int D = a.H * 64;
    const int8_t* K = a.kc + ((size_t)b * a.KH + g) * a.T * 64;
    const int8_t* Vr = a.vc + ((size_t)b * a.KH + g) * a.T * 64;
    const double mscale = live ? (double)a.score_mult[h] * (1.0 / 32768.0) : 0.0;
    int q4[16];
    {
        const int4* qp = (const int4*)(a.q + (size_t)b * D + (live ? h : h0) * 64);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int4 v = qp[i];
            q4[4 * i] = v.x; q4[4 * i + 1] = v.y; q4[4 * i + 2] = v.z; q4[4 * i + 3] = v.w;
        }
    }
    int m = INT32_MIN;
    unsigned long long S = 0;
    unsigned vacc = 0;
    if (a.sink && live) {  // attention.rs:211-224: the sink score is the initial max, weight E(0)
        int dot = 0;
#pragma unroll
        for (int i = 0; i < 16; i++) dot = __builtin_amdgcn_sdot4(q4[i], ((const int*)a.sink)[i], dot, false);
        m = dec_score(dot, mscale);
        S = 65535ull;
    }
    // tile chunks of 16 bytes: 256 of K then 256 of V (key r, dims c .. c+15);
    // a thread holds chunks tid and tid + nthr (nthr >= 256)
    int4 pre0 = make_int4(0, 0, 0, 0), pre1 = pre0;
    auto fetch = [&](int t0) {
        const int i0 = tid, i1 = tid + nthr;
        const int8_t* base0 = i0 < 256 ? K : Vr;
        pre0 = *(const int4*)(base0 + (size_t)(t0 + ((i0 & 255) >> 2)) * 64 + (i0 & 3) * 16);
        if (i1 < 512) {
            const int8_t* base1 = i1 < 256 ? K : Vr;
            pre1 = *(const int4*)(base1 + (size_t)(t0 + ((i1 & 255) >> 2)) * 64 + (i1 & 3) * 16);
        }
    };
    auto stage = [&](int i, int4 v) {
        const int r = (i & 255) >> 2, c = (i & 3) * 16;
        if (i < 256) {
            *(int4*)(Ks + r * DKLD + c) = v;
        } else {
            const int vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int k = 0; k < 16; k++) Vt[(c + k) * DKLD + r] = (int8_t)(vv[k >> 2] >> (8 * (k & 3)));
        }
    };
    fetch(0);
    for (int t0 = 0; t0 <= p; t0 += 64) {
        __syncthreads();
        stage(tid, pre0);
        if (tid + nthr < 512) stage(tid + nthr, pre1);
        __syncthreads();
        if (t0 + 64 <= p) fetch(t0 + 64);
        if (!live) continue;
        const int nt = min(64, p - t0 + 1);
        // 1. lanes = keys
        int s = INT32_MIN;
        if (lane < nt) {
            const int* k4 = (const int*)(Ks + lane * DKLD);
            int dot = 0;
#pragma unroll
            for (int i = 0; i < 16; i++) dot = __builtin_amdgcn_sdot4(q4[i], k4[i], dot, false);
            s = dec_score(dot, mscale);
        }
        int pm = s;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int v = __shfl_up(pm, o, 64);
            if (lane >= o) pm = max(pm, v);
        }
        pm = max(pm, m);
        int prev = __shfl_up(pm, 1, 64);
        if (lane == 0) prev = m;
        const bool rec = lane < nt && s > prev;
        unsigned w = 0, e = 0;
        if (lane < nt) {
            const unsigned x = exp_q16_bf(rec ? (int)((unsigned)prev - (unsigned)s) : (int)((unsigned)s - (unsigned)pm),
                                          lut32, ATTN_COEF_Q24);
            w = rec ? 65535u : x;
            e = (rec && prev != INT32_MIN) ? x : 0u;
        }
        unsigned pw = w;  // inclusive prefix sum of the weights (< 2^22)
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const unsigned v = (unsigned)__shfl_up((int)pw, o, 64);
            if (lane >= o) pw += v;
        }
        const unsigned pe = pw - w;  // exclusive
        const unsigned long long recm = __ballot(rec);
        const unsigned wx = w ^ 0x8080u;
        whi[wave][lane] = (uint8_t)(wx >> 8);
        wlo[wave][lane] = (uint8_t)wx;
        ekl[wave][lane] = e;
        m = __shfl(pm, 63, 64);
        const unsigned total = (unsigned)__shfl((int)pw, 63, 64);
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        // 2. lanes = head dims
        int vr[16];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int4 v = *(const int4*)(Vt + lane * DKLD + 16 * i);
            vr[4 * i] = v.x; vr[4 * i + 1] = v.y; vr[4 * i + 2] = v.z; vr[4 * i + 3] = v.w;
        }
        const unsigned* hw = (const unsigned*)whi[wave];
        const unsigned* lw = (const unsigned*)wlo[wave];
        int cur = 0;  // first key of the running segment
#pragma unroll
        for (int gi = 0; gi < 16; gi++) {
            const unsigned vsum = (unsigned)__builtin_amdgcn_sdot4(vr[gi], 0x01010101, 0, false);
            const unsigned rb = (unsigned)(recm >> (4 * gi)) & 0xFu;
            if (rb == 0u) {
                vacc += group_wv(hw[gi], lw[gi], 0xFFFFFFFFu, vr[gi], vsum);
            } else {
                unsigned from = 0;  // first key of the group not yet added
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    if ((rb >> r) & 1u) {
                        const unsigned mk = (r > 0 ? (0xFFFFFFFFu >> (32 - 8 * r)) : 0u) & ~((1u << (8 * from)) - 1u);
                        vacc += group_wv(hw[gi], lw[gi], mk, vr[gi], vsum);
                        const int kr = 4 * gi + r;
                        const unsigned ej = ekl[wave][kr];
                        S += (unsigned)__builtin_amdgcn_readlane((int)pe, kr) - (unsigned)__builtin_amdgcn_readlane((int)pe, cur);
                        if (ej) {
                            vacc = dec_rescale(vacc, ej);
                            S = (S * ej + 0x8000ull) >> 16;
                        }
                        cur = kr;
                        from = (unsigned)r;
                    }
                }
                vacc += group_wv(hw[gi], lw[gi], ~((1u << (8 * from)) - 1u), vr[gi], vsum);
            }
        }
        S += total - (unsigned)__builtin_amdgcn_readlane((int)pe, cur);
    }
    if (!live) return;
    const unsigned long long den = S == 0 ? 1ull : S;
    a.out[(size_t)b * D + h * 64 + lane] = (int8_t)clamp127(div_rne_s32_u64((int)vacc, den));
}

void launch_attn_decode(const AttnArgs& a, int S, int p, hipStream_t s) {
    // waves per workgroup: the most heads any KV group has
    const int KH = a.KH;
    int waves = a.H;
    if (a.kv_mode == 1) {
        waves = 0;
        for (int g = 0; g < KH; g++) {
            const int h0 = (g * a.H + a.G - 1) / a.G, h1 = ((g + 1) * a.H + a.G - 1) / a.G;
            waves = h1 - h0 > waves ? h1 - h0 : waves;
        }
    }
    // at least 4 waves: the tile staging gives each thread at most 2 of the
    // 512 16-byte chunks of a K + V tile
    if (waves < 4) waves = 4;
    hipLaunchKernelGGL(k_attn_decode, dim3((unsigned)S, (unsigned)KH), dim3(64 * waves), 0, s, a, p);
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
