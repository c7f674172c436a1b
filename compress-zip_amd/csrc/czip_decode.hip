// Batched autoregressive decode (decompression): one token per stream per
// step, each stream a chunk of the .czip payload (main.rs:377-396), with an
// arithmetic decoder per stream kept on the device (arith_coder.rs:139-264).
#include "czip_attn_tile.h"
#include "czip_head.h"
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

// The decoder step of a decoded symbol with interval [lo, hi) (arith_coder.rs:243-262):
// narrow (low, high), then renormalize, reading the stream's bits from an
// 8-byte window: a step shifts at most 32 bits (each pass shifts a 0 into low
// and a 1 into high; after 32 of them low = 0, high = 2^32 - 1 ends the loop).
// The window comes from three aligned words of the chunk buffer (which carries
// 16 bytes of padding); bytes at or past the chunk's end read as 0
// (arith_coder.rs:176-190).
__device__ __forceinline__ void dec_advance(DecState st, DecStreams ds, int b, unsigned lo, unsigned hi, unsigned total) {
    const unsigned low = st.low[b], high = st.high[b], code = st.code[b];
    const unsigned long long range = (unsigned long long)high - low + 1;
    const double invT = 1.0 / (double)total;
    unsigned long long nh = low + udiv64_32((unsigned long long)hi * range, total, invT) - 1;
    unsigned long long nl = low + udiv64_32((unsigned long long)lo * range, total, invT);
    unsigned long long cd = code;
    const long long len = ds.blen[b];
    const long long bp = st.byte_pos[b];
    const int bi = st.bit_pos[b];
    const long long start = ds.offs[b] + bp, base = start & ~3ll;
    const unsigned* w = (const unsigned*)(ds.data + base);
    const unsigned w0 = w[0], w1 = w[1], w2 = w[2];
    const int sh = (int)(start - base) * 8;
    const unsigned long long lo64 = ((unsigned long long)w1 << 32) | w0;
    unsigned long long v = sh ? (lo64 >> sh) | ((unsigned long long)w2 << (64 - sh)) : lo64;  // bytes bp .. bp + 7
    const long long nv = len - bp;
    if (nv < 8) v = nv <= 0 ? 0ull : v & ((1ull << (8 * nv)) - 1ull);
    const unsigned long long win = __builtin_bswap64(v);  // MSB first
    int pos = 56 + bi;  // window bit of the next stream bit
    for (;;) {
        if (((nl ^ nh) & DHALF) == 0) {
            nl = (nl << 1) & DMASK;
            nh = ((nh << 1) & DMASK) | 1;
            cd = ((cd << 1) & DMASK) | ((win >> pos) & 1);
            pos--;
        } else if ((nl & ~nh & DQUART) != 0) {
            nl = ((nl << 1) ^ DHALF) & DMASK;
            nh = (((nh ^ DHALF) << 1) | DHALF | 1) & DMASK;
            cd = (cd & DHALF) | ((cd << 1) & (DMASK >> 1)) | ((win >> pos) & 1);
            pos--;
        } else {
            break;
        }
    }
    // reader position after the bits taken (it stops at the end of the chunk)
    const long long used = (long long)(7 - bi) + (56 + bi - pos);
    long long nbp = bp + used / 8;
    int nbi = 7 - (int)(used % 8);
    if (bp >= len) { nbp = bp; nbi = bi; }
    else if (nbp >= len) { nbp = len; nbi = 7; }
    st.low[b] = (uint32_t)nl;
    st.high[b] = (uint32_t)nh;
    st.code[b] = (uint32_t)cd;
    st.byte_pos[b] = nbp;
    st.bit_pos[b] = nbi;
}

// forward input of step p (main.rs:386-388), after the decoder step of step
// p - 1's symbol when the fused head left it pending (upd)
__global__ void k_dec_prep(DecStreams ds, DecState st, int S, int p, int upd, unsigned total, uint32_t* __restrict__ inp) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= S) return;
    const int n = ds.ntok[b];
    if (upd && p <= n) dec_advance(st, ds, b, st.pend_lo[b], st.pend_hi[b], total);
    uint32_t t = 0u;
    if (p < n) t = p == 0 ? BOS_TOKEN : ds.tokens[ds.tok_offs[b] + p - 1];
    inp[b] = t;
}

void launch_dec_prep(DecStreams ds, DecState st, int S, int p, bool upd, unsigned total, uint32_t* inp, hipStream_t s) {
    hipLaunchKernelGGL(k_dec_prep, dim3((unsigned)((S + 255) / 256)), dim3(256), 0, s, ds, st, S, p, upd ? 1 : 0, total,
                       inp);
}

// ---------------------------------------------------------------------------
// Decode attention (attention.rs:162-289 for one query per stream): one
// wavefront per (NS streams, KV group), four independent wavefronts per
// workgroup.  The G heads of the group (d_model <= 1024 bounds G to 16) at
// the streams' position p are the rows of attn_tile: with 2 * G <= 16, two
// streams share a wavefront (rows [0, G) and [G, 2G)), each meeting only its
// own stream's keys.  Each lane loads its own K and V^T operand fragments
// (16 bytes each) straight from the caches, one tile ahead: one stream into
// a second register set, two streams in place (the next K and V after the
// tile's passes; the V latency is covered by the scores and the scan, the K
// latency by the other waves of the SIMD).  Three waves per SIMD (168 VGPRs,
// no scratch).
// ---------------------------------------------------------------------------
template <bool GEN, int NS, int NR>
__global__ __launch_bounds__(256, 3) void k_attn_decode(AttnArgs a, int p, int G) {
    __shared__ __attribute__((aligned(16))) uint16_t etb[ETB_PAD];
    __shared__ __attribute__((aligned(16))) AttnWaveLds wl[4];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: streams, group and caches in SGPRs
    const int row = lane & 15, grp = lane >> 4;
    for (int i = tid; i < ETB_PAD / 8; i += 256) ((uint4*)etb)[i] = ((const uint4*)a.etab)[i];
    attn_wave_init(wl[wave]);
    __syncthreads();
    const int item = (int)blockIdx.x * 4 + wave;
    const int sp = item / a.KH, g = item % a.KH;
    int bs[NS];
    bool act[NS], any = false;
#pragma unroll
    for (int t = 0; t < NS; t++) {
        bs[t] = sp * NS + t;
        act[t] = bs[t] < a.B && p < a.lens[bs[t]];
        any = any || act[t];
        bs[t] = min(bs[t], a.B - 1);  // a finished or missing stream's rows are dead; its loads stay in range
    }
    if (!any) return;  // no barrier follows
    // heads of KV group g: h with (h * G) / H == g in GQA mode; all heads otherwise
    const int h0 = a.kv_mode == 1 ? (g * a.H + a.G - 1) / a.G : 0;
    const int rs = NS == 1 ? 0 : min(row / G, NS);  // the row's stream (NS: no stream)
    bool live = row < NS * G;
#pragma unroll
    for (int t = 0; t < NS; t++)
        if (rs == t) live = live && act[t];
    int b = bs[0];
#pragma unroll
    for (int t = 1; t < NS; t++) b = rs == t ? bs[t] : b;
    const int h = h0 + (row < NS * G ? row - rs * G : 0);
    const int D = a.H * 64;
    const double mscale = (double)a.score_mult[h] * (1.0 / 32768.0);
    v4i qop = (v4i){0, 0, 0, 0};
    if (live) qop = *(const v4i*)(a.q + (size_t)b * D + h * 64 + grp * 16);
    v4i qs[NS];
#pragma unroll
    for (int t = 0; t < NS; t++) qs[t] = NS == 1 || rs == t ? qop : (v4i){0, 0, 0, 0};

    AttnRows st;
    st.m = live ? attn_m_empty<GEN>() : attn_m_never<GEN>();  // dead rows: never a record
    st.S = 0;
    for (int r = 0; r < 16; r++) st.vacc[r] = 0;
    if (a.sink) {  // attention.rs:211-224: sink score is the initial max, weight E(0) = 65535
        const int* sk = (const int*)(a.sink + grp * 16);
        int dot = 0;
        for (int i = 0; i < 4; i++) dot = __builtin_amdgcn_sdot4(qop[i], sk[i], dot, false);
        dot += __shfl_xor(dot, 16, 64);
        dot += __shfl_xor(dot, 32, 64);
        if (live) {
            st.m = attn_sink_m<GEN>(dot, mscale);
            st.S = 65535u;
        }
    }

    const int ntiles = p / 64 + 1;  // keys 0..p; tile t0 + 64 <= p stays inside TP
    // buffer loads: one 32-bit offset per lane, range-checked against the
    // stream's TP * 64 bytes of K ([TP][64]) and of V^T (vt_off)
    __amdgpu_buffer_rsrc_t rk[NS], rv[NS];
#pragma unroll
    for (int t = 0; t < NS; t++) {
        const size_t base = ((size_t)bs[t] * a.KH + g) * a.TP * 64;
        rk[t] = __builtin_amdgcn_make_buffer_rsrc((void*)(a.kc + base), (short)0, a.TP * 64, BUF_DWORD3);
        rv[t] = __builtin_amdgcn_make_buffer_rsrc((void*)(a.vc + base), (short)0, a.TP * 64, BUF_DWORD3);
    }
    auto load_k = [&](int t, int blk, int t0) {
        return __builtin_amdgcn_raw_buffer_load_b128(rk[t], (t0 + kperm(blk, row)) * 64 + grp * 16, 0, 0);
    };
    auto load_k_half = [&](int t, int blk, int t0) {
        return __builtin_amdgcn_raw_buffer_load_b128(rk[t], (t0 + kperm<32>(blk, row)) * 64 + grp * 16, 0, 0);
    };
    // V^T of the decode caches in 4-key blocks (vt_off, vl = 2): the operand's
    // 16 keys of one dim are four 4-byte words, 256 bytes apart
    auto load_v = [&](int t, int db, int t0) {
        const int o = vt_off(t0 + grp * 16, db * 16 + row, 2);
        return (v4i){(int)__builtin_amdgcn_raw_buffer_load_b32(rv[t], o, 0, 0),
                     (int)__builtin_amdgcn_raw_buffer_load_b32(rv[t], o + 256, 0, 0),
                     (int)__builtin_amdgcn_raw_buffer_load_b32(rv[t], o + 512, 0, 0),
                     (int)__builtin_amdgcn_raw_buffer_load_b32(rv[t], o + 768, 0, 0)};
    };
    // a half tile's operand: keys 8 grp .. +8 of one dim, two words
    auto load_v_half = [&](int t, int db, int t0) {
        const int o = vt_off(t0 + grp * 8, db * 16 + row, 2);
        return (v4i){(int)__builtin_amdgcn_raw_buffer_load_b32(rv[t], o, 0, 0),
                     (int)__builtin_amdgcn_raw_buffer_load_b32(rv[t], o + 256, 0, 0), 0, 0};
    };
    auto nvalid_at = [&](int t0) {
        const int n = p - (t0 + grp * 16) + 1;
        return n < 0 ? 0 : (n > 16 ? 16 : n);
    };
    if constexpr (NS == 1) {
        // two register sets: the tile's operands in one while the next tile's
        // are loaded into the other; after the last tile the loads stay
        // unconditional (nothing waits on them before their use) but point
        // past the stream's cache, where the range check returns zeros
        // without reading memory
        auto tile = [&](v4i* kc, v4i* vc, v4i* kn, v4i* vn, int t0) {
            const int tn = t0 + 64 <= p ? t0 + 64 : a.TP;
            attn_tile<GEN, 1, 64>(
                [&](int, int blk) {
                    kn[blk] = load_k(0, blk, tn);
                    return kc[blk];
                },
                [&](int, int db) { return vc[db]; }, qs, 0, mscale, nvalid_at(t0), t0 + 63 > p, etb, wl[wave],
                st);
#pragma unroll
            for (int db = 0; db < 4; db++) vn[db] = load_v(0, db, tn);
        };
        v4i k0[4], v0[4], k1[4], v1[4];
#pragma unroll
        for (int blk = 0; blk < 4; blk++) k0[blk] = load_k(0, blk, 0);
#pragma unroll
        for (int db = 0; db < 4; db++) v0[db] = load_v(0, db, 0);
        int kt = 0;
        for (; kt + 1 < ntiles; kt += 2) {
            tile(k0, v0, k1, v1, kt * 64);
            tile(k1, v1, k0, v0, kt * 64 + 64);
        }
        if (kt < ntiles) tile(k0, v0, k1, v1, kt * 64);
    } else {
        // the last tile is a half tile (keys t0 .. t0 + 31) when p falls in
        // its first half.  Operands one tile ahead, all K loads before all V
        // loads, so that the scores wait for the K operands only.
        const bool half_last = (p & 63) < 32;
        const int nfull = half_last ? ntiles - 1 : ntiles;
        v4i kr[NS][4], vr[NS][4];
        auto load_full = [&](int t0) {
#pragma unroll
            for (int t = 0; t < NS; t++)
#pragma unroll
                for (int i = 0; i < 4; i++) kr[t][i] = load_k(t, i, t0);
#pragma unroll
            for (int t = 0; t < NS; t++)
#pragma unroll
                for (int i = 0; i < 4; i++) vr[t][i] = load_v(t, i, t0);
        };
        if (nfull > 0) load_full(0);
        for (int kt = 0; kt < nfull; kt++) {
            const int t0 = kt * 64;
            attn_tile<GEN, NS, 64, NR>([&](int t, int blk) { return kr[t][blk]; },
                                   [&](int t, int db) { return vr[t][db]; }, qs, rs, mscale, nvalid_at(t0),
                                   t0 + 63 > p, etb, wl[wave], st);
            // the next tile's K and V once the passes are done: no operand
            // register is live across the passes (168 VGPRs, three waves per
            // SIMD; the next K requested after the scan held 210, two waves).
            // After the last full tile the loads stay unconditional but point
            // past the stream's cache (TP keys), where the range check returns
            // zeros without reading memory (a reload of the tile itself went
            // to HBM again: ~8 KB more per stream-step).
            load_full(kt + 1 < nfull ? t0 + 64 : a.TP);
        }
        if (half_last) {
            // requested here, not in the loop: their offsets would stay live
            // across it; the latency is covered by the other waves, like a K
            const int t0 = nfull * 64;
#pragma unroll
            for (int t = 0; t < NS; t++)
#pragma unroll
                for (int i = 0; i < 2; i++) kr[t][i] = load_k_half(t, i, t0);
#pragma unroll
            for (int t = 0; t < NS; t++)
#pragma unroll
                for (int i = 0; i < 4; i++) vr[t][i] = load_v_half(t, i, t0);
            const int nv = min(max(p - (t0 + grp * 8) + 1, 0), 8);
            attn_tile<GEN, NS, 32, NR>([&](int t, int blk) { return kr[t][blk]; },
                                   [&](int t, int db) { return vr[t][db]; }, qs, rs, mscale, nv, true, etb,
                                   wl[wave], st);
        }
    }
    // each lane forms the output offset of its row (-1: no live row), read
    // per row into a scalar: out[S][H * 64] stays below 2^31 bytes (host check)
    const int rs2 = NS == 1 ? 0 : (row >= G) + (row >= 2 * G);
    bool live2 = row < NS * G;
#pragma unroll
    for (int t = 0; t < NS; t++)
        if (rs2 == t) live2 = live2 && act[t];
    const int ooff = live2 ? (rs2 == 0 ? bs[0] : bs[NS - 1]) * D + (h0 + row - rs2 * G) * 64 : -1;
    attn_normalize<NR>(st, [&](int r, int8_t v) {
        const int o = __builtin_amdgcn_readlane(ooff, r);
        if (o >= 0) a.out[o + lane] = v;
    });
}

void launch_attn_decode(const AttnArgs& a, int S, int p, hipStream_t s) {
    // heads per KV group: all of them in rust-compat mode (one KV head), H / G
    // in GQA mode (n_heads is a multiple of n_kv_heads); at most 16
    const int G = a.kv_mode == 1 ? a.H / a.G : a.H;
    AttnArgs g = a;
    g.B = S;
    const bool two = 2 * G <= 16;
    const long long waves = (long long)(two ? (S + 1) / 2 : S) * a.KH;
    dim3 grid((unsigned)((waves + 3) / 4));
    // rows in use per wave (NS G of 16), rounded up to 8, 12 or 16
    const int nr = !two ? 16 : (2 * G <= 8 ? 8 : (2 * G <= 12 ? 12 : 16));
#define CZIP_ATTN_DEC(GEN, NS, NR) hipLaunchKernelGGL((k_attn_decode<GEN, NS, NR>), grid, dim3(256), 0, s, g, p, G)
    if (!two) {
        if (a.general) CZIP_ATTN_DEC(true, 1, 16);
        else CZIP_ATTN_DEC(false, 1, 16);
    } else if (nr == 8) {
        if (a.general) CZIP_ATTN_DEC(true, 2, 8);
        else CZIP_ATTN_DEC(false, 2, 8);
    } else if (nr == 12) {
        if (a.general) CZIP_ATTN_DEC(true, 2, 12);
        else CZIP_ATTN_DEC(false, 2, 12);
    } else {
        if (a.general) CZIP_ATTN_DEC(true, 2, 16);
        else CZIP_ATTN_DEC(false, 2, 16);
    }
#undef CZIP_ATTN_DEC
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

// ---------------------------------------------------------------------------
// One decode step with the logits kept on chip: a workgroup owns 64 streams
// (the rows of head_freqs).  After the frequency table, per row:
//   - wave 0 (lane = row) forms the remainder total - sum f, the exclusive
//     prefix of the 16 wave ranges (the argmax's wave carrying the
//     remainder) and value = ((code - low + 1) * total - 1) / range, clamped
//     to total - 1 (a value >= total decodes as the last symbol, whose
//     interval ends at total: arith_coder.rs:225-241);
//   - every lane walks its 4-column groups in column order (tile, lane
//     group) from its wave's base, the lane-group prefix within a tile by two
//     shuffles, and keeps the one group whose range holds the value; that
//     group's columns give the symbol (the one column with lo <= value < hi)
//     and its interval;
//   - wave 0 stores the symbol and the interval; the next step's input
//     kernel narrows and renormalizes the decoder (arith_coder.rs:243-262).
// ---------------------------------------------------------------------------
template <int CT, bool E0>
__global__ __launch_bounds__(64 * HNW) void k_head_dec(HeadDecArgs a, DecState st, DecStreams ds) {
    __shared__ HeadLdsT<1> L;
    __shared__ unsigned row_v[HBM_ROWS], row_rem[HBM_ROWS], row_lo[HBM_ROWS], row_hi[HBM_ROWS];
    __shared__ int row_sym[HBM_ROWS];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int nb = wave * CT * 16;
    const int lr = lane & 15, grp = lane >> 4, c4 = grp * 4;
    const int m0 = blockIdx.x * HBM_ROWS;
    head_stage_a(a.A, a.M, a.K, m0, L.As[0]);
    head_etab_fill(L, a.lut);
    // decoder state of wave 0's stream, requested before the GEMM
    const int b = m0 + lane;
    bool live = false;
    unsigned low = 0, high = 0, code = 0;
    if (wave == 0 && b < a.M && a.p < ds.ntok[b]) {
        live = true;
        low = st.low[b];
        high = st.high[b];
        code = st.code[b];
    }
    __builtin_amdgcn_s_waitcnt(0);  // the block's A (and everything before) has landed
    __syncthreads();
    if (wave == 0) {
        // the decoder value (a 64-bit division) while the other waves start
        // their products, not in the one-wave section after the reductions
        const unsigned long long range = (unsigned long long)high - low + 1;  // <= 2^32
        const unsigned long long value = ((unsigned long long)(code - low) + 1) * a.total - 1;
        row_v[lane] = live ? (unsigned)min(value / range, (unsigned long long)a.total - 1) : 0u;
    }
    v4i acc[4][CT];
    head_freqs<CT, E0>(tid, L.As[0], a.K, a.W, a.V, a.coef, a.total, L, acc);
    // sum f per row and wave
#pragma unroll
    for (int i = 0; i < 4; i++) {
        unsigned fs = 0;
#pragma unroll
        for (int t = 0; t < CT; t++)
#pragma unroll
            for (int r = 0; r < 4; r++) fs += (unsigned)acc[i][t][r];
        fs += (unsigned)__shfl_xor((int)fs, 16, 64);
        fs += (unsigned)__shfl_xor((int)fs, 32, 64);
        if (lane < 16) L.red_b[wave][i * 16 + lane] = fs;
    }
    __syncthreads();
    if (wave == 0) {
        unsigned tot = 0;
#pragma unroll
        for (int w = 0; w < HNW; w++) tot += L.red_b[w][lane];
        const unsigned rem = a.total - tot;
        const int wam = L.row_am[lane] / (CT * 16);
        unsigned run = 0;
#pragma unroll
        for (int w = 0; w < HNW; w++) {
            L.red_c[w][lane] = run;
            run += L.red_b[w][lane] + (w == wam ? rem : 0u);
        }
        row_rem[lane] = rem;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int rr = i * 16 + lr;
        const unsigned v = row_v[rr], rem = row_rem[rr];
        // the argmax as (tile, element) of this lane's 4-column groups, if it is one of them
        const int amk = L.row_am[rr] - (nb + c4);
        const int am_t = amk >= 0 && (amk & 15) < 4 ? amk >> 4 : -1;
        unsigned run = L.red_c[wave][rr];
        // per tile, only the group sum (the argmax's group with the
        // remainder) and its start: the one group of the row holding v is
        // kept and searched after the loop
        int ht = -1;
        unsigned hb0 = 0u;
#pragma unroll
        for (int t = 0; t < CT; t++) {
            const unsigned g = (unsigned)acc[i][t][0] + (unsigned)acc[i][t][1] + (unsigned)acc[i][t][2] +
                               (unsigned)acc[i][t][3] + (am_t == t ? rem : 0u);
            // inclusive prefix over the four lane groups of the row, and their total
            unsigned x = g;
            const unsigned y1 = (unsigned)__shfl_up((int)x, 16, 64);
            x += grp >= 1 ? y1 : 0u;
            const unsigned y2 = (unsigned)__shfl_up((int)x, 32, 64);
            x += grp >= 2 ? y2 : 0u;
            const unsigned tile_sum = (unsigned)__shfl((int)x, lr + 48, 64);
            const unsigned b0 = run + x - g;
            const bool in = v - b0 < g;  // b0 <= v < b0 + g; every f >= 1: at most one group holds v
            ht = in ? t : ht;
            hb0 = in ? b0 : hb0;
            run += tile_sum;
        }
        if (ht >= 0) {
            // the held group's frequencies (the argmax's with the remainder)
            unsigned f[4];
#pragma unroll
            for (int r = 0; r < 4; r++) {
                unsigned e = (unsigned)acc[i][0][r];
#pragma unroll
                for (int t = 1; t < CT; t++) e = ht == t ? (unsigned)acc[i][t][r] : e;
                f[r] = e + (am_t == ht && (amk & 3) == r ? rem : 0u);
            }
            const unsigned b1 = hb0 + f[0], b2 = b1 + f[1], b3 = b2 + f[2];
            const unsigned k = (v >= b1 ? 1u : 0u) + (v >= b2 ? 1u : 0u) + (v >= b3 ? 1u : 0u);
            row_sym[rr] = nb + ht * 16 + c4 + (int)k;
            row_lo[rr] = k == 0 ? hb0 : k == 1 ? b1 : k == 2 ? b2 : b3;
            row_hi[rr] = k == 0 ? b1 : k == 1 ? b2 : k == 2 ? b3 : b3 + f[3];
        }
    }
    __syncthreads();
    if (!live) return;
    // the symbol, and its interval for the decoder step, which the next
    // step's input kernel applies (the workgroup ends here instead of
    // waiting on one wave's bit reads)
    ds.tokens[ds.tok_offs[b] + a.p] = (uint32_t)row_sym[lane];
    st.pend_lo[b] = row_lo[lane];
    st.pend_hi[b] = row_hi[lane];
}

// One workgroup per 64-stream block (not persistent like the compress head:
// with two decode lanes sharing the GPU, blocks handed to whichever CU frees
// up finish sooner than a fixed share per workgroup)
void launch_head_dec(const HeadDecArgs& a, DecState st, DecStreams ds, hipStream_t s) {
    dim3 grid((unsigned)((a.M + HBM_ROWS - 1) / HBM_ROWS));
    if (a.e0) hipLaunchKernelGGL((k_head_dec<4, true>), grid, dim3(64 * HNW), 0, s, a, st, ds);
    else hipLaunchKernelGGL((k_head_dec<4, false>), grid, dim3(64 * HNW), 0, s, a, st, ds);
}

}  // namespace czip
