// One wavefront's exact attention over one 64-key tile for 16 query rows
// (attention.rs:162-289), shared by the prefill kernel (rows = 16 consecutive
// positions of one head) and the decode kernel (rows = the heads of one KV
// group at the stream's current position).
//
// The reference walks the keys of a query row in order and, each time the
// running max strictly increases (a "record"), rescales the running sum S and
// the value accumulator with a rounded factor (attention.rs:205-276).  Between
// records every weight uses the same max, so a segment's contribution is a
// plain integer sum (S in u32, vacc modulo 2^32) that can be formed in any
// order; only the rescales must be applied in key order.  Per tile the wave:
//  1. forms S^T = K Q^T (int8 MFMA, K rows permuted so that each lane gets
//     16 consecutive keys of its row) and the score epilogue in f64, which
//     is exact: |dot / 4 * mult| < 2^49;
//  2. scans its rows' keys in order (a lane owns 16 consecutive keys of one
//     row): running max, records, one exp per key from a table in LDS.  A
//     key's weight and, at a record, the rescale factor are both
//     E(-|s - max before the key|);
//  3. for each segment index j = 0..max records, forms the segment sums of
//     all 16 rows at once, O_j^T = V^T P_j^T, on int8 MFMA.  The 16-bit
//     weights enter as two signed bytes: w - 32896 = 256*hi + lo, keys outside
//     segment j carry w = 0, and the constant 32896 * sum(v) (rows of ones
//     times V) is added back; each row's weight sum for S comes from rows of
//     ones times the weight columns;
//  4. hands O_j through LDS to a "lanes = head dims" layout and adds it to
//     every row, the rows whose record j falls in this pass rescaled first (a
//     row without a segment j adds exactly 0); S is kept with lanes = rows.
//
// Fast path (GEN false: |score| < 2^30 and lut[0] == 65535): scores are held
// as score + 2^31 in a u32 (order-preserving), "nothing seen yet" is 0, and
// the table step of a key is one multiply-add of |s - max|.  General path:
// scores in i32 with the reference's wrapping differences, INT32_MIN for
// "nothing seen yet".
#pragma once

#include "czip_device.h"
#include "czip_kernels.h"

namespace czip {

constexpr unsigned WOFF = 32896;      // w - WOFF spans [-32896, 32639] = 256*[-128,127] + [-128,127]
constexpr unsigned WB = 0x8080u;      // w ^ WB: the bytes of w - WOFF (each byte of w offset by 128)
constexpr int RS = 68;                // row stride (words) of the per-wave buffer: 16-byte accesses of 16 rows hit 64 banks

struct AttnWaveLds {
    unsigned buf[16][RS];    // per pass: the segment sums [row][dim]
    uint16_t ex[16][72];     // [row][key]: at a record key, the rescale factor ^ WB;
                             // 144-byte rows: 16-byte stores of 16 rows hit 64 banks;
                             // slot 64: factor 0 (WB), read for a row with no split left
};

// Once per wave, before its first tile.
__device__ __forceinline__ void attn_wave_init(AttnWaveLds& W) {
    const int lane = threadIdx.x & 63;
    if (lane < 16) W.ex[lane][64] = (uint16_t)WB;
}

__device__ __forceinline__ void wave_lds_fence() { __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront"); }

// The running max of a row before its first key: "nothing seen yet"
// (INT32_MIN, attention.rs:205), and a max that no score passes (rows of a
// decode wave that belong to no stream).
template <bool GEN>
__device__ __forceinline__ int attn_m_empty() { return GEN ? INT32_MIN : 0; }
template <bool GEN>
__device__ __forceinline__ int attn_m_never() { return GEN ? INT32_MAX : -1; }

// sra_rne64(sra_rne32(dot, 2) * mult, 15) (attention.rs:233-239), mscale =
// mult * 2^-15.  RNE of a quotient by 2^k is symmetric, so it is IEEE
// round-half-even.
// Fast path (|score| < 2^30, |mult| < 2^27): r1 = dot + 1.5 * 2^54, whose
// ulp is 4, is 1.5 * 2^54 + 4 du exactly (du = sra_rne32(dot, 2)); then
// fma(r1, mscale / 4, cb) with cb = 1.5 * 2^52 + 2^31 - 1.5 * 2^52 * mscale
// (exact: 1.5 * 2^37 * (2^15 - mult) + 2^31) is 1.5 * 2^52 + 2^31 +
// du * mscale rounded once at ulp 1, whose low word is score + 2^31.
// The general path rounds du * mscale in f64 (exact, |du * mult| < 2^49) and
// clamps to the i32 range.
__device__ __forceinline__ double score_bias_u(double mscale) {
    return __builtin_fma(-6755399441055744.0, mscale, 6755399441055744.0 + 2147483648.0);
}
__device__ __forceinline__ unsigned score_u(int dot, double ms4, double cbu) {
    const double r1 = (double)dot + 27021597764222976.0;  // 1.5 * 2^54
    return (unsigned)__builtin_bit_cast(unsigned long long, __builtin_fma(r1, ms4, cbu));
}
__device__ __forceinline__ int score_g(int dot, double mscale) {
    const int du = (dot + 1 + ((dot >> 2) & 1)) >> 2;
    double r = __builtin_rint((double)du * mscale);
    r = fmin(fmax(r, -2147483648.0), 2147483647.0);
    return (int)r;
}
// the row state's max after a sink of dot product `dot` (attention.rs:211-224)
template <bool GEN>
__device__ __forceinline__ int attn_sink_m(int dot, double mscale) {
    if (GEN) return score_g(dot, mscale);
    return (int)score_u(dot, mscale * 0.25, score_bias_u(mscale));
}

// |a - b| of two u32 (v_sad_u32 with a zero accumulator).  Inline asm is not
// covered by the compiler's MFMA hazard checks (an asm write to a register
// that an MFMA still in flight will write), so it is used only in the scan,
// where every MFMA result has been read (checked in the kernels' assembly).
__device__ __forceinline__ unsigned absdiff_u32(unsigned a, unsigned b) {
    unsigned r;
    asm("v_sad_u32 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
    return r;
}

// Table step of E(-n) (lut.rs:213-235): t = floor((n * coef + 2^23) / 2^24),
// every step from 4096 on reading entry 4096.  Fast path: for every u32 n,
// the high word of n * (coef * 2^8) + 2^31, one 32 x 32 + 64 multiply-add.
__device__ __forceinline__ unsigned exp_step_u(unsigned n) {
    const unsigned t = (unsigned)(((unsigned long long)n * (ATTN_COEF_Q24 << 8) + 0x80000000ull) >> 32);
    return min(t, 4096u);
}
__device__ __forceinline__ unsigned exp_step_g(unsigned n) {
    const unsigned long long t = ((unsigned long long)n * ATTN_COEF_Q24 + (1ull << 23)) >> 24;
    return t < 4096ull ? (unsigned)t : 4096u;
}

// vacc rescale at a record (attention.rs:246-261): the low 32 bits of
// ((i64)v * e + (v >= 0 ? 2^15 : -2^15)) >> 16, written as
// ((v * e + 2^15) >> 16) - (v < 0): for v < 0 the floor of (p + 2^15) / 2^16
// less one is the floor of (p - 2^15) / 2^16.
__device__ __forceinline__ unsigned rescale_v(unsigned v, unsigned e) {
    const long long p = (long long)(int)v * (long long)(int)e + 0x8000ll;  // e <= 65535
    return (unsigned)(p >> 16) + (unsigned)((int)v >> 31);
}

// S rescale at a record (attention.rs:246-250): (S * e + 0x8000) >> 16.  S is
// a sum of at most T + 1 weights <= 65535 (rescales only shrink it), so it
// fits 32 bits for T < 65536; the product is formed in 64.
__device__ __forceinline__ unsigned rescale_s(unsigned S, unsigned e) {
    return (unsigned)(((unsigned long long)S * e + 0x8000ull) >> 16);
}

// selector of v_perm_b32 that spreads bit 7 of each byte of z over the byte:
// perm(z, z << 8, .) with selectors 8..11 = sign bits 15 and 31 of the low
// operand and 15 and 31 of the high one, i.e. bits 7, 23, 15 and 31 of z;
// selector 12 gives a zero byte
constexpr unsigned SEL_B7 = 0x0B090A08u, SEL_ZERO = 0x0C0C0C0Cu;
__device__ __forceinline__ unsigned spread_b7(unsigned z, unsigned sel) { return __builtin_amdgcn_perm(z, z << 8, sel); }

__device__ __forceinline__ unsigned pick(unsigned msk, unsigned a, unsigned b) { return (a & msk) | (b & ~msk); }

// The K operand's row m of MFMA block blk holds key kperm(blk, m) of the tile,
// so that the score block's output lane (row, g) receives keys KT/4 g + 4 blk
// + (0..3): after the KT/16 blocks each lane holds KT/4 consecutive keys of
// its row, the order of the scan, with no transpose.  KT = 64 (a full tile) or
// 32 (a half tile: the last tile of a row block whose visible keys end in its
// first half).
template <int KT = 64>
__device__ __forceinline__ int kperm(int blk, int m) { return (KT / 4) * (m >> 2) + 4 * blk + (m & 3); }

// Running state of a wave's 16 rows: max m (attn_m_empty / the scan's
// representation) and weight sum S with lanes = rows (replicated over the 4
// lane groups); vacc with lanes = head dims, register index = row.
struct AttnRows {
    int m;
    unsigned S;
    unsigned vacc[16];
};

// One tile of KT keys (64, or 32 for a half tile: KT/16 score blocks, KT/4
// keys per lane and the PV products on the 16x16x32 MFMA).  kop(s, blk): the
// K operand of key kperm<KT>(blk, lane%16), head dims 16*(lane/16) .. +16;
// vop(s, db): the V^T operand of head dim 16*db + lane%16, keys
// KT/4*(lane/16) .. +KT/4 (a half tile uses its low 8 bytes; each called once
// per index, the V operands after the scan).  etb: the exp table of
// attn_etab_host in LDS.  nvalid: keys [KT/4*(lane/16), +nvalid) of the
// lane's row are visible (the others get weight 0 and are never records),
// used when diag is set.  The first NR rows of the wave are combined into
// vacc (the caller's rows among them; rows from NR on must stay without
// records, as the rows of no stream are); the caller reads only its own.
//
// NS > 1 packs NS independent key streams (decode: streams sharing nothing
// but the shape) into the wave's rows (rs: the lane's row's stream, NS for
// none).  Every product is then summed over the streams, the streams being
// consecutive slices of the contraction: the scores with the other streams'
// rows zeroed in the query operand (qs[s]: the lane's query when its row
// reads stream s, else 0), the PV products with weight 0 in the other
// streams' columns (a constant, corrected like the keys outside a segment).
// NS == 1: qs[0] is the query operand and rs is unused.
// the PV-side operand types and product of a tile of KT keys: 16 bytes of 16
// keys per lane (16x16x64) or 8 bytes of 8 keys (16x16x32)
template <int KT>
struct AttnPv {
    using Op = v4i;
    static constexpr v4i ONES = {0x01010101, 0x01010101, 0x01010101, 0x01010101};
    static __device__ __forceinline__ Op op(v4i v) { return v; }
    static __device__ __forceinline__ Op from_dw(const unsigned* d) {
        return (v4i){(int)d[0], (int)d[1], (int)d[2], (int)d[3]};
    }
    static __device__ __forceinline__ v4i mma(Op a, Op b, v4i c) {
        return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
    }
};
template <>
struct AttnPv<32> {
    using Op = long;
    static constexpr long ONES = 0x0101010101010101l;
    static __device__ __forceinline__ Op op(v4i v) {
        return (long)(((unsigned long long)(unsigned)v[1] << 32) | (unsigned)v[0]);
    }
    static __device__ __forceinline__ Op from_dw(const unsigned* d) {
        return (long)(((unsigned long long)d[1] << 32) | d[0]);
    }
    static __device__ __forceinline__ v4i mma(Op a, Op b, v4i c) {
        return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, c, 0, 0, 0);
    }
};

template <bool GEN, int NS, int KT, int NR = 16, class KOp, class VOp>
__device__ __forceinline__ void attn_tile(KOp kop, VOp vop_at, const v4i* qs, int rs, double mscale,
                                          int nvalid, bool diag, const uint16_t* etb, AttnWaveLds& W,
                                          AttnRows& st) {
    static_assert(KT == 64 || KT == 32, "a tile holds 64 or 32 keys");
    static_assert(NR >= 1 && NR <= 16, "rows in use: the first NR of 16");
    constexpr int KPL = KT / 4;   // keys per lane
    constexpr int NDW = KPL / 4;  // dwords of weight bytes per lane = score blocks
    using Pv = AttnPv<KT>;
    using Op = typename Pv::Op;
    const int lane = threadIdx.x & 63, row = lane & 15, grp = lane >> 4;

    // 1. S^T = K Q^T and the score epilogue: lane (row, grp) gets the scores
    // of keys KPL*grp .. +KPL of its row (kperm)
    unsigned sv[KPL];
    {
        const double ms4 = mscale * 0.25, cbu = score_bias_u(mscale);
#pragma unroll
        for (int blk = 0; blk < NDW; blk++) {
            v4i sc = __builtin_amdgcn_mfma_i32_16x16x64_i8(kop(0, blk), qs[0], (v4i){0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
            for (int t = 1; t < NS; t++) sc = __builtin_amdgcn_mfma_i32_16x16x64_i8(kop(t, blk), qs[t], sc, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; i++)
                sv[blk * 4 + i] = GEN ? (unsigned)score_g(sc[i], mscale) : score_u(sc[i], ms4, cbu);
        }
    }

    // 2. in-order scan of keys [KPL*grp, KPL*grp+KPL) of this row
    if (diag) {
#pragma unroll
        for (int k = 0; k < KPL; k++)
            if (k >= nvalid) sv[k] = (unsigned)attn_m_empty<GEN>();  // never a record; weight masked below
    }
    // the running max entering this lane's keys: the row's max so far and the
    // maxima of the lanes before it
    auto vmax = [](unsigned a, unsigned b) { return GEN ? (unsigned)max((int)a, (int)b) : max(a, b); };
    unsigned bmax = sv[0];
#pragma unroll
    for (int k = 1; k < KPL; k++) bmax = vmax(bmax, sv[k]);
    const unsigned e1 = (unsigned)__shfl((int)bmax, (lane - 16) & 63, 64),
                   e2 = (unsigned)__shfl((int)bmax, (lane - 32) & 63, 64),
                   e3 = (unsigned)__shfl((int)bmax, (lane - 48) & 63, 64);
    unsigned cur0 = (unsigned)st.m;
    if (grp >= 1) cur0 = vmax(cur0, e1);
    if (grp >= 2) cur0 = vmax(cur0, e2);
    if (grp >= 3) cur0 = vmax(cur0, e3);
    // weights (offset bytes, WB) and rescale factors (^ WB): one exp per key,
    // no branches, so the table reads can be in flight together
    unsigned xs[KPL], ws[KPL];  // rescale factor (or weight) of each key, and its weight (65535 at a record)
    unsigned recm = 0u;   // bit k: key k is a record
    unsigned fresh = 0u;  // bit k: key k is a record over "nothing seen": no rescale, no split
    if (GEN) {
        int M = (int)cur0;
#pragma unroll
        for (int k = 0; k < KPL; k++) {
            const int s = (int)sv[k];
            const bool rec = s > M;
            const int d = (int)(rec ? (unsigned)M - (unsigned)s : (unsigned)s - (unsigned)M);  // i32 wrap, as the reference
            const unsigned x = d >= 0 ? 65535u : ((unsigned)etb[exp_step_g(0u - (unsigned)d)] ^ WB);
            ws[k] = (rec ? 65535u : x) ^ WB;
            xs[k] = x ^ WB;
            fresh |= (rec && M == INT32_MIN ? 1u : 0u) << k;
            recm |= (rec ? 1u : 0u) << k;
            M = max(M, s);
        }
    } else {
        // three phases, so that the table reads are in flight together:
        // the running max and every key's table step, the reads, the
        // weights.  Only the lane's first key can meet "nothing seen" as a
        // record (masked keys are a suffix).
        unsigned tk[KPL];
        bool recb[KPL];
        unsigned M = cur0;
#pragma unroll
        for (int k = 0; k < KPL; k++) {
            const unsigned s = sv[k];
            recb[k] = s > M;
            tk[k] = exp_step_u(absdiff_u32(s, M));
            M = max(M, s);
            recm |= (recb[k] ? 1u : 0u) << k;
        }
        fresh = recb[0] && cur0 == 0u ? 1u : 0u;
        __builtin_amdgcn_sched_barrier(0);
        unsigned eb[KPL];
#pragma unroll
        for (int k = 0; k < KPL; k++) eb[k] = etb[tk[k]];
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int k = 0; k < KPL; k++) {
            ws[k] = recb[k] ? 0x7F7Fu : eb[k];  // a record's weight E(0) = 65535
            xs[k] = eb[k];
        }
    }
    // segments split at the records that rescale (a record over "nothing
    // seen" has nothing before it to rescale, so its segment runs on): the
    // row's splits in the tile (bit = key), their count and the splits before
    // this lane's keys
    const unsigned splm = recm & ~fresh;
    const unsigned g0 = (unsigned)__shfl((int)splm, row, 64), g1 = (unsigned)__shfl((int)splm, row + 16, 64),
                   g2 = (unsigned)__shfl((int)splm, row + 32, 64), g3 = (unsigned)__shfl((int)splm, row + 48, 64);
    // the row's splits as a KT-bit mask (bit = key of the tile) in rlo:rhi
    unsigned rlo, rhi, blo, bhi;
    if constexpr (KT == 64) {
        rlo = g0 | (g1 << 16);
        rhi = g2 | (g3 << 16);
        blo = grp == 0 ? 0u : (grp == 1 ? 0xFFFFu : 0xFFFFFFFFu);
        bhi = grp == 3 ? 0xFFFFu : 0u;
    } else {
        rlo = g0 | (g1 << 8) | (g2 << 16) | (g3 << 24);
        rhi = 0u;
        blo = (1u << (8 * grp)) - 1u;
        bhi = 0u;
    }
    const int nrow = __builtin_popcount(rlo) + __builtin_popcount(rhi);
    const unsigned seg = (unsigned)(__builtin_popcount(rlo & blo) + __builtin_popcount(rhi & bhi));
    unsigned long long rsp = ((unsigned long long)rhi << 32) | rlo;  // the splits not yet passed
    // every key's factor, read at its split's pass
#pragma unroll
    for (int h = 0; h < KPL / 8; h++) {
        uint4 e;
        e.x = __builtin_amdgcn_perm(xs[8 * h + 1], xs[8 * h], 0x05040100u);
        e.y = __builtin_amdgcn_perm(xs[8 * h + 3], xs[8 * h + 2], 0x05040100u);
        e.z = __builtin_amdgcn_perm(xs[8 * h + 5], xs[8 * h + 4], 0x05040100u);
        e.w = __builtin_amdgcn_perm(xs[8 * h + 7], xs[8 * h + 6], 0x05040100u);
        *(uint4*)&W.ex[row][grp * KPL + 8 * h] = e;
    }
    // weights as signed byte pairs (the bytes of w ^ WB) and segment bytes
    // dd = 128 + the key's segment id (splits up to and including the key,
    // <= 64): byte k of a dword = key KPL*grp + 4*i + k.  Pass j keeps
    // dd - j * 0x01010101, whose bytes never borrow (63 <= 128 + id - j <= 192),
    // so bit 7 of a byte tells id >= j.
    unsigned hi_dw[NDW], lo_dw[NDW], dd[NDW];
#pragma unroll
    for (int i = 0; i < NDW; i++) {
        const unsigned* w4 = ws + i * 4;
        const unsigned p01 = __builtin_amdgcn_perm(w4[1], w4[0], 0x05010400u);
        const unsigned p23 = __builtin_amdgcn_perm(w4[3], w4[2], 0x05010400u);
        lo_dw[i] = __builtin_amdgcn_perm(p23, p01, 0x05040100u);
        hi_dw[i] = __builtin_amdgcn_perm(p23, p01, 0x07060302u);
        const unsigned nib = (splm >> (4 * i)) & 15u;
        const unsigned ones = (nib * 0x204081u) & 0x01010101u;  // bit k of nib -> byte k
        const unsigned base = seg + (unsigned)__builtin_popcount(splm & ((1u << (4 * i)) - 1u));
        dd[i] = (ones + base) * 0x01010101u + 0x80808080u;  // byte k: 128 + base + bits 0..k of nib
    }
    if (diag) {  // invisible keys: weight 0 (bytes 0x80), in no segment (id 127: bit 7 stays set)
#pragma unroll
        for (int i = 0; i < NDW; i++) {
            const int q = nvalid - 4 * i;
            const unsigned vm = q >= 4 ? 0xFFFFFFFFu : (q <= 0 ? 0u : ((1u << (8 * q)) - 1u));
            hi_dw[i] = pick(vm, hi_dw[i], 0x80808080u);
            lo_dw[i] = pick(vm, lo_dw[i], 0x80808080u);
            dd[i] = pick(vm, dd[i], 0xFFFFFFFFu);
        }
    }
    {
        const unsigned mr = vmax(vmax(cur0, bmax), (unsigned)__shfl_xor((int)vmax(cur0, bmax), 16, 64));
        st.m = (int)vmax(mr, (unsigned)__shfl_xor((int)mr, 32, 64));
    }

    // 3. segment j of every row in pass j (MFMA column = row): O_j^T = V^T P_j^T
    int nmax = nrow;
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) nmax = max(nmax, __shfl_xor(nmax, o, 64));
    nmax = __builtin_amdgcn_readfirstlane(nmax);  // every lane holds the max over the 16 rows
    // A operand of the PV product, and the sum over the tile's KT keys (of
    // every stream) of v at head dim = lane: rows of ones times V, whose
    // output lane l holds column l % 16, i.e. dim 16 db + l % 16
    Op vop[NS][4];
    int vsum = 0;
#pragma unroll
    for (int db = 0; db < 4; db++) {
        v4i cs = {0, 0, 0, 0};
#pragma unroll
        for (int t = 0; t < NS; t++) {
            vop[t][db] = Pv::op(vop_at(t, db));
            cs = Pv::mma(Pv::ONES, vop[t][db], cs);
        }
        vsum = grp == db ? cs[0] : vsum;
    }
    // Every row's weight column for a stream other than its own reads w = 0
    // (bytes -128, like the keys outside segment j), so each row's product
    // carries -32896 * v of every key of every stream: one correction for
    // all rows.  sel[t]: the byte-mask selector of stream t's column.
    const unsigned corr = (unsigned)vsum * WOFF;
    unsigned sel[NS];
#pragma unroll
    for (int t = 0; t < NS; t++) sel[t] = NS == 1 || rs == t ? SEL_B7 : SEL_ZERO;
    for (int j = 0; j <= nmax; j++) {
        Op bhs[NS], bls[NS];
        {
            unsigned bh[NS][NDW], bl[NS][NDW];
#pragma unroll
            for (int i = 0; i < NDW; i++) {
                const unsigned dn = dd[i] - 0x01010101u;
                const unsigned m = dd[i] & ~dn;  // bit 7 of a byte: id >= j and not id >= j + 1
                dd[i] = dn;
#pragma unroll
                for (int t = 0; t < NS; t++) {
                    const unsigned msk = spread_b7(m, sel[t]);
                    bh[t][i] = pick(msk, hi_dw[i], 0x80808080u);
                    bl[t][i] = pick(msk, lo_dw[i], 0x80808080u);
                }
            }
#pragma unroll
            for (int t = 0; t < NS; t++) {
                bhs[t] = Pv::from_dw(bh[t]);
                bls[t] = Pv::from_dw(bl[t]);
            }
        }
        // sum over the row's KT keys of (w_j - 32896) (rows of ones times the
        // weight columns: output lane l holds column l % 16 = the lane's
        // row), less the other streams' columns (KT keys of -32896 each)
        v4i sh = {0, 0, 0, 0}, sl = {0, 0, 0, 0};
        // from the pass's first products to its end the wave runs at raised
        // priority: a wave that has formed its weight columns goes ahead of
        // the waves still forming theirs (or scanning a tile), whose
        // independent VALU then fills the issue slots its MFMA, LDS and
        // rescale latencies leave (prefill attention 190.5 -> 184.0 ms per
        // compress step; from the mask generation on 186.0, only up to the
        // LDS hand-over 187.2, with the tile's scores raised too 188.6)
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int t = 0; t < NS; t++) {
            sh = Pv::mma(Pv::ONES, bhs[t], sh);
            sl = Pv::mma(Pv::ONES, bls[t], sl);
        }
        const int sw = sh[0] * 256 + sl[0] + (NS - 1) * KT * (int)WOFF;
        // rescale factor of this lane's row at record j (0: none), the lowest
        // record not yet passed; row r's is read by the combine from lane r
        unsigned erow = 0u;
        if (j >= 1) {
            if constexpr (NS == 1) {
                // lowest split left, else slot 64, which holds factor 0
                // (attn_wave_init) for a row with no split left
                const unsigned key = (unsigned)__builtin_ctzg(rsp, 64);
                erow = (unsigned)W.ex[row][key] ^ WB;
                rsp &= rsp - 1ull;
            } else {
                // the two-stream decode tile keeps the 32-bit form (the 64-bit
                // one made its register allocation spill: 440 vs 415 ms)
                const int key = rlo ? __builtin_ctz(rlo) : 32 + __builtin_ctz(rhi | 0x80000000u);
                erow = j <= nrow ? (unsigned)W.ex[row][key] ^ WB : 0u;
                rhi = rlo ? rhi : rhi & (rhi - 1u);
                rlo &= rlo - 1u;
            }
        }
        // 4a. S of this lane's row (lanes = rows): rescale at record j (a
        // factor of 65536 leaves S as it is), then add segment j
        st.S = rescale_s(st.S, erow ? erow : 65536u);
        st.S += (unsigned)sw + (unsigned)KT * WOFF;
        // the high- and low-byte products of two head-dim blocks at a time are
        // independent, so their MFMAs issue back to back and one shift-add
        // joins them
#pragma unroll
        for (int d2 = 0; d2 < 4; d2 += 2) {
            v4i ah[2], al[2];
#pragma unroll
            for (int u = 0; u < 2; u++) {
                ah[u] = Pv::mma(vop[0][d2 + u], bhs[0], (v4i){0, 0, 0, 0});
                al[u] = Pv::mma(vop[0][d2 + u], bls[0], (v4i){0, 0, 0, 0});
#pragma unroll
                for (int t = 1; t < NS; t++) {
                    ah[u] = Pv::mma(vop[t][d2 + u], bhs[t], ah[u]);
                    al[u] = Pv::mma(vop[t][d2 + u], bls[t], al[u]);
                }
            }
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const v4i acc = (ah[u] << 8) + al[u];
                *(int4*)&W.buf[row][(d2 + u) * 16 + grp * 4] = make_int4(acc[0], acc[1], acc[2], acc[3]);
            }
        }
        // rows (bit r, from lane r) that rescale at record j (none in pass 0)
        const unsigned long long resc = __builtin_amdgcn_ballot_w64(erow != 0u);
        wave_lds_fence();
        // 4b. vacc (lanes = head dims).  Pass 0: every row adds its segment
        // 0.  Pass j >= 1: only the rows with a segment j, which are the rows
        // that rescale at record j (factors are at least 1); a row without
        // one has w = 0 (bytes -128) in every column, its product is exactly
        // -corr and it would add 0.
        unsigned bv[NR];
#pragma unroll
        for (int r = 0; r < NR; r++) bv[r] = W.buf[r][lane];
        if (j == 0) {
#pragma unroll
            for (int r = 0; r < NR; r++) st.vacc[r] += bv[r] + corr;
        } else {
#pragma unroll
            for (int r = 0; r < NR; r++)
                if ((resc >> r) & 1ull)
                    st.vacc[r] = rescale_v(st.vacc[r], (unsigned)__builtin_amdgcn_readlane((int)erow, r)) + bv[r] + corr;
        }
        wave_lds_fence();
        __builtin_amdgcn_s_setprio(0);
    }
}

__device__ __forceinline__ double bcast_f64(double x, int lane) {
    const unsigned long long u = __builtin_bit_cast(unsigned long long, x);
    const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)u, lane);
    const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(u >> 32), lane);
    return __builtin_bit_cast(double, ((unsigned long long)hi << 32) | lo);
}

// Normalization (attention.rs:278-285): emit(r, clamp127(div_rne(vacc[r], S_r)))
// for the 16 rows, lane = head dim, S = 0 read as 1.  div_rne
// (primitives.rs:163-185) rounds the magnitude of the quotient half to even
// and restores the sign, which is round-half-even of the signed quotient.  In f64 from
// one reciprocal per row (lanes = rows): q = rint(v * (1/S)) is within 2^-22
// of v / S (|v / S| <= 2^31), so for |v / S| <= 2^8 it is the rounded quotient
// unless that is a tie (a quotient that is no tie lies at least 1/(2S) >=
// 2^-33 from every half-integer), and beyond that the clamp decides.  r2 =
// 2 fma(-q, S, v) is exact (the remainder is an integer below 2^32 in
// magnitude) and equals +-S exactly at a tie, where the even neighbour of q
// in the direction of r2 wins: (q + (r2 > 0)) & ~1.
template <int NR = 16, class Emit>
__device__ __forceinline__ void attn_normalize(const AttnRows& st, Emit emit) {
    const double dl = (double)max(st.S, 1u);
    const double il = 1.0 / dl;
#pragma unroll
    for (int r = 0; r < NR; r++) {
        const double inv = bcast_f64(il, r), den = bcast_f64(dl, r);
        const double nf = (double)(int)st.vacc[r];
        const double q = __builtin_rint(nf * inv);
        const double r2 = 2.0 * __builtin_fma(-q, den, nf);
        const int qi = (int)q;
        const int qt = __builtin_fabs(r2) == den ? (qi + (r2 > 0.0 ? 1 : 0)) & ~1 : qi;
        emit(r, (int8_t)clamp127(qt));
    }
}

}  // namespace czip
