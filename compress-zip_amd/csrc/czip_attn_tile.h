// One wavefront's exact attention over one 64-key tile for 16 query rows
// (attention.rs:162-289), shared by the prefill kernel (rows = 16 consecutive
// positions of one head) and the decode kernel (rows = the heads of one KV
// group at the stream's current position).
//
// The reference walks the keys of a query row in order and, each time the
// running max strictly increases (a "record"), rescales the running sum S and
// the value accumulator with a rounded factor (attention.rs:205-276).  Between
// records every weight uses the same max, so a segment's contribution is a
// plain integer sum (S in u64, vacc modulo 2^32) that can be formed in any
// order; only the rescales must be applied in key order.  Per tile the wave:
//  1. forms S^T = K Q^T (int8 MFMA, K rows permuted so that each lane gets
//     16 consecutive keys of its row) and the score epilogue in f64, which
//     is exact: |dot / 4 * mult| < 2^49;
//  2. scans its rows' keys in order (a lane owns 16 consecutive keys of one
//     row): running max, records, one exp per key.  A key's weight and, at a
//     record, the rescale factor are both E(-|s - max before the key|);
//  3. for each segment index j = 0..max records, forms the segment sums of
//     all 16 rows at once, O_j^T = V^T P_j^T, on int8 MFMA.  The 16-bit
//     weights enter as two signed bytes: w - 32896 = 256*hi + lo, keys outside
//     segment j carry w = 0, and the constant 32896 * sum(v) (rows of ones
//     times V) is added back; each row's weight sum for S comes from rows of
//     ones times the weight columns;
//  4. hands O_j through LDS to a "lanes = head dims" layout and walks each
//     row's own segments: rescale at the record, then add (rows without a
//     segment j skip the pass on a ballot bit); S is kept with lanes = rows.
// INT32_MIN is the reference's "nothing seen yet" max (the fast path's scores
// stay inside +-2^30, so no score equals it).
#pragma once

#include "czip_device.h"

namespace czip {

constexpr unsigned WOFF = 32896;      // w - WOFF spans [-32896, 32639] = 256*[-128,127] + [-128,127]
constexpr int RS = 68;                // row stride (words) of the per-wave buffer: 16-byte accesses of 16 rows hit 64 banks

struct AttnWaveLds {
    unsigned buf[16][RS];    // per pass: the segment sums [row][dim]
    uint16_t ex[16][72];     // [row][key]: at a record key, the rescale factor (0: nothing to rescale);
                             // 144-byte rows: 16-byte stores of 16 rows hit 64 banks
};

__device__ __forceinline__ void wave_lds_fence() { __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront"); }

// sra_rne64(sra_rne32(dot, 2) * mult, 15) (attention.rs:233-239), mscale =
// mult * 2^-15.  RNE of a quotient by 2^k is symmetric, so it is IEEE
// round-half-even.  Fast path (|score| < 2^30, |mult| < 2^27), two FMAs
// around B = 1.5 * 2^52 (ulp 1): r1 = fma(dot, 1/4, B) = B + du exactly
// (du = sra_rne32(dot, 2)), and fma(r1, mscale, cb) with cb = B * (1 -
// mscale) (exact: 1.5 * 2^37 * (2^15 - mult)) is B + du * mscale rounded
// once, whose low word is the score.  The general path rounds du * mscale
// in f64 (exact, |du * mult| < 2^49) and clamps to the i32 range.
__device__ __forceinline__ double score_bias(double mscale) {
    return __builtin_fma(-6755399441055744.0, mscale, 6755399441055744.0);
}
template <bool GEN>
__device__ __forceinline__ int score_b(int dot, double mscale, double cb) {
    if (!GEN) {
        const double r1 = __builtin_fma((double)dot, 0.25, 6755399441055744.0);
        return (int)(unsigned)__builtin_bit_cast(unsigned long long, __builtin_fma(r1, mscale, cb));
    }
    const int du = (dot + 1 + ((dot >> 2) & 1)) >> 2;
    double r = __builtin_rint((double)du * mscale);
    r = fmin(fmax(r, -2147483648.0), 2147483647.0);
    return (int)r;
}

// exp_q16(-neg) (lut.rs:213-235) with the table pre-shifted by 16 bits.
// (65536 >> ip) * lut == (lut << 16) >> ip for ip <= 16, and both round to 0
// (then clamp to 1) for ip >= 17; ip is capped at 31 like the reference's
// early return.  neg == 0 reads lut[0], which the fast path requires to be 65535.
__device__ __forceinline__ unsigned exp_neg(unsigned neg, const unsigned* lut32) {
    const unsigned long long pr = (unsigned long long)neg * ATTN_COEF_Q24 + (1ull << 23);
    const unsigned t = (unsigned)(pr >> 24);
    const unsigned ip = min(t >> 8, 31u);
    const unsigned x = ((lut32[t & 255u] >> ip) + 0x8000u) >> 16;
    return max(x, 1u);
}

// The same for the fast path, with the table index from a difference d of
// two scores held in f64: t = floor(|d| * coef / 2^24 + 1/2) is one FMA
// (|d| < 2^32 and coef < 2^19, so the sum is exact) truncated to u32, and
// t >= 17 * 256 (ip >= 17) always gives 1, so t is capped there.
__device__ __forceinline__ unsigned exp_idx_f(double d) {
    return (unsigned)fmin(__builtin_fma(fabs(d), (double)ATTN_COEF_Q24 * 0x1p-24, 0.5), 4352.0);
}
// the value from the table word at t & 255
__device__ __forceinline__ unsigned exp_from(unsigned t, unsigned word) {
    return max(((word >> (t >> 8)) + 0x8000u) >> 16, 1u);
}

// vacc rescale at a record (attention.rs:246-261): the low 32 bits of
// ((i64)v * e + (v >= 0 ? 2^15 : -2^15)) >> 16 (one 32x32+64 multiply-add)
__device__ __forceinline__ unsigned rescale_v(unsigned v, unsigned e) {
    const int c = (int)v >= 0 ? 0x8000 : -0x8000;
    return (unsigned)(((long long)(int)v * (long long)(int)e + (long long)c) >> 16);
}

// S rescale at a record (attention.rs:246-250): (S * e + 0x8000) >> 16.  S is
// a sum of at most T + 1 weights <= 65535 (rescales only shrink it), so it
// fits 32 bits for T < 65536; the product is formed in 64.
__device__ __forceinline__ unsigned rescale_s(unsigned S, unsigned e) {
    return (unsigned)(((unsigned long long)S * e + 0x8000ull) >> 16);
}

// bit 7 of each byte of the result: that byte of x is zero (exact per byte;
// the other bits are junk)
__device__ __forceinline__ unsigned zero_bytes_b7(unsigned x) { return ~(((x & 0x7F7F7F7Fu) + 0x7F7F7F7Fu) | x); }

// selector of v_perm_b32 that spreads bit 7 of each byte of z over the byte:
// perm(z, z << 8, .) with selectors 8..11 = sign bits 15 and 31 of the low
// operand and 15 and 31 of the high one, i.e. bits 7, 23, 15 and 31 of z;
// selector 12 gives a zero byte
constexpr unsigned SEL_B7 = 0x0B090A08u, SEL_ZERO = 0x0C0C0C0Cu;
__device__ __forceinline__ unsigned spread_b7(unsigned z, unsigned sel) { return __builtin_amdgcn_perm(z, z << 8, sel); }

__device__ __forceinline__ unsigned pick(unsigned msk, unsigned a, unsigned b) { return (a & msk) | (b & ~msk); }

// The K operand's row m of MFMA block blk holds key kperm(blk, m) of the tile,
// so that the score block's output lane (row, g) receives keys 16 g + 4 blk
// + (0..3): after the 4 blocks each lane holds 16 consecutive keys of its
// row, the order of the scan, with no transpose.
__device__ __forceinline__ int kperm(int blk, int m) { return 16 * (m >> 2) + 4 * blk + (m & 3); }

// Running state of a wave's 16 rows: max m and weight sum S with
// lanes = rows (replicated over the 4 lane groups); vacc with lanes = head
// dims, register index = row.
struct AttnRows {
    int m;
    unsigned S;
    unsigned vacc[16];
};

// One 64-key tile.  kop(s, blk): the K operand of key kperm(blk, lane%16),
// head dims 16*(lane/16) .. +16; vop(s, db): the V^T operand of head dim
// 16*db + lane%16, keys 16*(lane/16) .. +16 (each called once per index);
// after_scan() runs once the scores have been scanned, before the V operands
// are read.
// nvalid: keys [16*(lane/16), +nvalid) of the lane's row are visible (the
// others get weight 0 and are never records), used when diag is set; rows
// >= nrows are not combined into vacc (their m, S and vacc are unused).
//
// NS > 1 packs NS independent key streams (decode: streams sharing nothing
// but the shape) into the wave's rows (rs: the lane's row's stream, NS for
// none).  Every product is then summed over the streams, the streams being
// consecutive slices of the contraction: the scores with the other streams'
// rows zeroed in the query operand (qs[s]: the lane's query when its row
// reads stream s, else 0), the PV products with weight 0 in the other
// streams' columns (a constant, corrected like the keys outside a segment).
// NS == 1: qs[0] is the query operand and rs is unused.
template <bool GEN, int NS, class KOp, class VOp, class After>
__device__ __forceinline__ void attn_tile(KOp kop, VOp vop_at, After after_scan, const v4i* qs, int rs, double mscale,
                                          int nvalid, bool diag, int nrows, const unsigned* lut32, AttnWaveLds& W,
                                          AttnRows& st) {
    const int lane = threadIdx.x & 63, row = lane & 15, grp = lane >> 4;

    // 1. S^T = K Q^T and the score epilogue: lane (row, grp) gets the scores
    // of keys 16*grp .. +16 of its row (kperm)
    int sv[16];
    const double cb = score_bias(mscale);
#pragma unroll
    for (int blk = 0; blk < 4; blk++) {
        v4i sc = __builtin_amdgcn_mfma_i32_16x16x64_i8(kop(0, blk), qs[0], (v4i){0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
        for (int t = 1; t < NS; t++) sc = __builtin_amdgcn_mfma_i32_16x16x64_i8(kop(t, blk), qs[t], sc, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; i++) sv[blk * 4 + i] = score_b<GEN>(sc[i], mscale, cb);
    }

    // 2. in-order scan of keys [16*grp, 16*grp+16) of this row
    if (diag) {
#pragma unroll
        for (int k = 0; k < 16; k++)
            if (k >= nvalid) sv[k] = INT32_MIN;  // never a record; weight masked below
    }
    int bmax = INT32_MIN;
#pragma unroll
    for (int k = 0; k < 16; k++) bmax = max(bmax, sv[k]);
    const int e1 = __shfl(bmax, (lane - 16) & 63, 64), e2 = __shfl(bmax, (lane - 32) & 63, 64),
              e3 = __shfl(bmax, (lane - 48) & 63, 64);
    int cur0 = st.m;
    if (grp >= 1) cur0 = max(cur0, e1);
    if (grp >= 2) cur0 = max(cur0, e2);
    if (grp >= 3) cur0 = max(cur0, e3);
    // weights and rescale factors: one exp per key, no branches, so the
    // 16 table reads can be in flight together
    unsigned xs[16], ws[16];  // rescale factor (or weight) of each key, and its weight (65535 at a record)
    unsigned recm = 0u;   // bit k: key k is a record
    unsigned fresh = 0u;  // bit k: key k is a record over "nothing seen": no rescale, no split
    int M = cur0;
    if (GEN) {
#pragma unroll
        for (int k = 0; k < 16; k++) {
            const int s = sv[k];
            const bool rec = s > M;
            const int d = (int)(rec ? (unsigned)M - (unsigned)s : (unsigned)s - (unsigned)M);  // i32 wrap, as the reference
            unsigned x = d >= 0 ? 65535u : exp_neg(0u - (unsigned)d, lut32);
            ws[k] = rec ? 65535u : x;
            const bool f = rec && M == INT32_MIN;  // a record over "nothing seen" has no rescale
            x = f ? 0u : x;
            fresh |= (f ? 1u : 0u) << k;
            xs[k] = x;
            recm |= (rec ? 1u : 0u) << k;
            M = max(M, s);
        }
    } else {
        // three phases, so that the 16 table reads are in flight together:
        // the running max (f64) and every key's table index, the reads, the
        // values.  Only the lane's first key can meet M == INT32_MIN as a
        // record (masked keys are a suffix).
        unsigned tk[16];
        bool recb[16];
        double Mf = (double)cur0;
#pragma unroll
        for (int k = 0; k < 16; k++) {
            const double sf = (double)sv[k];
            recb[k] = sf > Mf;
            tk[k] = exp_idx_f(Mf - sf);
            Mf = fmax(Mf, sf);
            recm |= (recb[k] ? 1u : 0u) << k;
        }
        fresh = recb[0] && cur0 == INT32_MIN ? 1u : 0u;
        __builtin_amdgcn_sched_barrier(0);
        unsigned word[16];
#pragma unroll
        for (int k = 0; k < 16; k++) word[k] = lut32[tk[k] & 255u];
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int k = 0; k < 16; k++) {
            const unsigned x = exp_from(tk[k], word[k]);
            ws[k] = recb[k] ? 65535u : x;
            xs[k] = k == 0 && fresh ? 0u : x;
        }
        M = max(cur0, bmax);
    }
    // segments split at the records that rescale (a record over "nothing
    // seen" has nothing before it to rescale, so its segment runs on): the
    // row's splits in the tile (bit = key), their count and the splits before
    // this lane's keys
    const unsigned splm = recm & ~fresh;
    const unsigned g0 = (unsigned)__shfl((int)splm, row, 64), g1 = (unsigned)__shfl((int)splm, row + 16, 64),
                   g2 = (unsigned)__shfl((int)splm, row + 32, 64), g3 = (unsigned)__shfl((int)splm, row + 48, 64);
    unsigned rlo = g0 | (g1 << 16), rhi = g2 | (g3 << 16);
    const int nrow = __builtin_popcount(rlo) + __builtin_popcount(rhi);
    const unsigned blo = grp == 0 ? 0u : (grp == 1 ? 0xFFFFu : 0xFFFFFFFFu), bhi = grp == 3 ? 0xFFFFu : 0u;
    const unsigned seg = (unsigned)(__builtin_popcount(rlo & blo) + __builtin_popcount(rhi & bhi));
    // every key's factor, read at its split's pass
    {
        uint4 e0, e1v;
        e0.x = xs[0] | (xs[1] << 16); e0.y = xs[2] | (xs[3] << 16); e0.z = xs[4] | (xs[5] << 16); e0.w = xs[6] | (xs[7] << 16);
        e1v.x = xs[8] | (xs[9] << 16); e1v.y = xs[10] | (xs[11] << 16); e1v.z = xs[12] | (xs[13] << 16);
        e1v.w = xs[14] | (xs[15] << 16);
        *(uint4*)&W.ex[row][grp * 16] = e0;
        *(uint4*)&W.ex[row][grp * 16 + 8] = e1v;
    }
    // weights as signed byte pairs (a record's weight is 65535) and segment
    // ids (splits up to and including the key); byte k of a dword = key
    // 16*grp + 4*i + k
    unsigned hi_dw[4], lo_dw[4], sg_dw[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const unsigned* w4 = ws + i * 4;
        const unsigned p01 = __builtin_amdgcn_perm(w4[1], w4[0], 0x05010400u);
        const unsigned p23 = __builtin_amdgcn_perm(w4[3], w4[2], 0x05010400u);
        lo_dw[i] = __builtin_amdgcn_perm(p23, p01, 0x05040100u) ^ 0x80808080u;
        hi_dw[i] = __builtin_amdgcn_perm(p23, p01, 0x07060302u) ^ 0x80808080u;
        const unsigned nib = (splm >> (4 * i)) & 15u;
        const unsigned ones = (nib * 0x204081u) & 0x01010101u;  // bit k of nib -> byte k
        const unsigned base = seg + (unsigned)__builtin_popcount(splm & ((1u << (4 * i)) - 1u));
        sg_dw[i] = (ones + base) * 0x01010101u;  // byte k: base + bits 0..k of nib (all < 256)
    }
    if (diag) {  // invisible keys: weight 0 (bytes 0x80), no segment (0xFF)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int q = nvalid - 4 * i;
            const unsigned vm = q >= 4 ? 0xFFFFFFFFu : (q <= 0 ? 0u : ((1u << (8 * q)) - 1u));
            hi_dw[i] = pick(vm, hi_dw[i], 0x80808080u);
            lo_dw[i] = pick(vm, lo_dw[i], 0x80808080u);
            sg_dw[i] = pick(vm, sg_dw[i], 0xFFFFFFFFu);
        }
    }
    {
        const int mr = max(M, __shfl_xor(M, 16, 64));
        st.m = max(mr, __shfl_xor(mr, 32, 64));
    }

    // 3. segment j of every row in pass j (MFMA column = row): O_j^T = V^T P_j^T
    after_scan();
    int nmax = nrow;
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) nmax = max(nmax, __shfl_xor(nmax, o, 64));
    // A operand of the PV product, and the sum over the tile's 64 keys (of
    // every stream) of v at head dim = lane: rows of ones times V, whose
    // output lane l holds column l % 16, i.e. dim 16 db + l % 16
    constexpr v4i ONES = {0x01010101, 0x01010101, 0x01010101, 0x01010101};
    v4i vop[NS][4];
    int vsum = 0;
#pragma unroll
    for (int db = 0; db < 4; db++) {
        v4i cs = {0, 0, 0, 0};
#pragma unroll
        for (int t = 0; t < NS; t++) {
            vop[t][db] = vop_at(t, db);
            cs = __builtin_amdgcn_mfma_i32_16x16x64_i8(ONES, vop[t][db], cs, 0, 0, 0);
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
        const unsigned jb = (unsigned)j * 0x01010101u;
        v4i bhs[NS], bls[NS];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const unsigned z = zero_bytes_b7(sg_dw[i] ^ jb);
#pragma unroll
            for (int t = 0; t < NS; t++) {
                const unsigned msk = spread_b7(z, sel[t]);
                bhs[t][i] = (int)pick(msk, hi_dw[i], 0x80808080u);
                bls[t][i] = (int)pick(msk, lo_dw[i], 0x80808080u);
            }
        }
        // sum over the row's 64 keys of (w_j - 32896) (rows of ones times the
        // weight columns: output lane l holds column l % 16 = the lane's
        // row), less the other streams' columns (64 keys of -32896 each)
        v4i sh = {0, 0, 0, 0}, sl = {0, 0, 0, 0};
#pragma unroll
        for (int t = 0; t < NS; t++) {
            sh = __builtin_amdgcn_mfma_i32_16x16x64_i8(ONES, bhs[t], sh, 0, 0, 0);
            sl = __builtin_amdgcn_mfma_i32_16x16x64_i8(ONES, bls[t], sl, 0, 0, 0);
        }
        const int sw = sh[0] * 256 + sl[0] + (NS - 1) * 64 * (int)WOFF;
        // rescale factor of this lane's row at record j (0: none), the lowest
        // record not yet passed; row r's is read by the combine from lane r
        unsigned erow = 0u;
        if (j >= 1) {
            const int key = rlo ? __builtin_ctz(rlo) : 32 + __builtin_ctz(rhi | 0x80000000u);
            erow = j <= nrow ? (unsigned)W.ex[row][key] : 0u;
            rhi = rlo ? rhi : rhi & (rhi - 1u);
            rlo &= rlo - 1u;
        }
        // 4a. S of this lane's row (lanes = rows): rescale at record j, then add segment j
        if (erow) st.S = rescale_s(st.S, erow);
        st.S += (unsigned)sw + 64u * WOFF;
#pragma unroll
        for (int db = 0; db < 4; db++) {
            v4i acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(vop[0][db], bhs[0], (v4i){0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
            for (int t = 1; t < NS; t++) acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(vop[t][db], bhs[t], acc, 0, 0, 0);
            acc = acc << 8;
#pragma unroll
            for (int t = 0; t < NS; t++) acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(vop[t][db], bls[t], acc, 0, 0, 0);
            *(int4*)&W.buf[row][db * 16 + grp * 4] = make_int4(acc[0], acc[1], acc[2], acc[3]);
        }
        // rows (bit r, from lane r) that have a segment j, and those that
        // rescale first
        const unsigned long long live = __builtin_amdgcn_ballot_w64(j <= nrow);
        const unsigned long long resc = __builtin_amdgcn_ballot_w64(erow != 0u);
        wave_lds_fence();
        // 4b. vacc (lanes = head dims): every row that has a segment j
        unsigned bv[16];
#pragma unroll
        for (int r = 0; r < 16; r++)
            if (r < nrows) bv[r] = W.buf[r][lane];
#pragma unroll
        for (int r = 0; r < 16; r++) {
            if (r < nrows && ((live >> r) & 1ull)) {
                if ((resc >> r) & 1ull)
                    st.vacc[r] = rescale_v(st.vacc[r], (unsigned)__builtin_amdgcn_readlane((int)erow, r));
                st.vacc[r] += bv[r] + corr;
            }
        }
        wave_lds_fence();
    }
}

}  // namespace czip
