// Exact causal attention of the prefill (attention.rs:162-289) on MFMA.
#include "czip_device.h"
#include "czip_kernels.h"

namespace czip {

// ---------------------------------------------------------------------------
// The reference walks the keys of a query row in order and, each time the
// running max strictly increases (a "record"), rescales the running sum S and
// the value accumulator with a rounded factor (attention.rs:205-276).  Between
// records every weight uses the same max, so a segment's contribution is a
// plain integer sum (S in u64, vacc modulo 2^32) that can be formed in any
// order; only the rescales must be applied in key order.
//
// One workgroup = one chunk, one head, 64 query rows (4 waves x 16 rows).
// Per 64-key tile each wave:
//  1. forms S^T = K Q^T (int8 MFMA) and the score epilogue;
//  2. scans its rows' keys in order: running max, records, weights
//     w = E(s - max), segment ids, rescale factors (lanes own 16 keys);
//  3. for each segment index j = 0..max records, forms the segment sums of
//     all 16 rows at once, O_j^T = V^T P_j^T, on int8 MFMA.  The 16-bit
//     weights enter as two signed bytes: w - 32896 = 256*hi + lo, keys outside
//     segment j carry w = 0, and the constant 32896 * sum(v) is added back;
//  4. hands O_j through LDS to a "lanes = head dims" layout and walks each
//     row's own segments: rescale at the record, then add (no lane waste on
//     rows that have fewer records).
// S^T puts query row (lane % 16) in the lane with keys 16*blk + 4*(lane/16) + r
// in its registers, which is the B-operand layout of P^T for the PV product.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int score_of(int dot, int mult) {
    int du = sra_rne32(dot, 2);        // Q_SHIFT
    return mul_sra_rne(du, mult, 15);  // sra_rne64((i64)du * mult, 15), attention.rs:233-239
}

constexpr int KLD = 80;           // LDS row stride (bytes) of the K tile and of the V^T tile
constexpr unsigned WOFF = 32896;  // w - WOFF spans [-32896, 32639] = 256*[-128,127] + [-128,127]

__device__ __forceinline__ void wave_lds_fence() { __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront"); }

// vacc / S rescale at a record (attention.rs:246-261)
__device__ __forceinline__ unsigned rescale_v(unsigned v, unsigned e) {
    long long pr = (long long)(int)v * (long long)e;
    pr += pr >= 0 ? (1ll << 15) : -(1ll << 15);
    return (unsigned)(int)(pr >> 16);
}

// bytes of x equal to zero -> 0xFF, others -> 0x00 (exact per byte)
__device__ __forceinline__ unsigned zero_bytes_mask(unsigned x) {
    unsigned t = ((x & 0x7F7F7F7Fu) + 0x7F7F7F7Fu) | x;
    t = ~t & 0x80808080u;
    return (t >> 7) * 0xFFu;
}

// Rows are padded to 68 words so that the 16 rows of a 16-byte access cover
// all 64 LDS banks exactly once.
constexpr int RS = 68;
struct AttnWaveLds {
    unsigned buf[16][RS];    // scores, then (w | seg << 16), then one segment's V sums
    uint16_t rec_e[16][66];  // rescale factor at record j+1 of row r (0: none)
    int nrec[16];
};

__global__ __launch_bounds__(256, 4) void k_attention(AttnArgs a) {
    __shared__ uint16_t lut[256];
    __shared__ __attribute__((aligned(16))) int8_t Ks[64 * KLD];
    __shared__ __attribute__((aligned(16))) int8_t Vt[64 * KLD];
    __shared__ __attribute__((aligned(16))) AttnWaveLds wl[4];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int row = lane & 15, grp = lane >> 4;
    const int q0 = blockIdx.x * 64, h = blockIdx.y, b = blockIdx.z;
    const int T = a.T, len = a.lens[b];
    if (q0 >= len) return;
    lut[tid] = a.lut[tid];
    AttnWaveLds& W = wl[wave];
    const int D = a.H * 64;
    const int g = a.kv_mode == 1 ? (h * a.G) / a.H : 0;
    const int8_t* Kg = a.kc + ((size_t)b * a.KH + g) * T * 64;
    const int8_t* Vg = a.vc + ((size_t)b * a.KH + g) * 64 * a.TP;
    const int mult = a.score_mult[h];
    const int p = q0 + wave * 16 + row;  // query position of this lane's row (scan / MFMA layouts)
    const int wrow0 = q0 + wave * 16;
    const bool wave_live = wrow0 < len;
    const int wave_last = min(wrow0 + 15, len - 1);

    v4i qop = (v4i){0, 0, 0, 0};
    if (p < T) qop = *(const v4i*)(a.q + ((size_t)b * T + p) * D + h * 64 + grp * 16);

    // state: running max m and weight sum S in the MFMA layout (row = lane % 16,
    // replicated over the 4 lane groups); vacc in the "lanes = dims" layout
    // (lane = head dim, register index = row)
    int m = INT32_MIN;
    unsigned long long S = 0;
    unsigned vacc[16];
    for (int r = 0; r < 16; r++) vacc[r] = 0;
    if (a.sink) {  // attention.rs:211-224: sink score is the initial max, weight E(0) = 65535
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

        // 1. S^T = K Q^T, score epilogue, stored [row][key]
#pragma unroll
        for (int blk = 0; blk < 4; blk++) {
            v4i kop = *(const v4i*)(Ks + (blk * 16 + row) * KLD + grp * 16);
            v4i st = __builtin_amdgcn_mfma_i32_16x16x64_i8(kop, qop, (v4i){0, 0, 0, 0}, 0, 0, 0);
            *(int4*)&W.buf[row][blk * 16 + grp * 4] =
                make_int4(score_of(st[0], mult), score_of(st[1], mult), score_of(st[2], mult), score_of(st[3], mult));
        }
        wave_lds_fence();

        // 2. in-order scan of keys [16*grp, 16*grp+16) of this row
        int sv[16];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            int4 v = *(const int4*)&W.buf[row][grp * 16 + i * 4];
            sv[i * 4] = v.x; sv[i * 4 + 1] = v.y; sv[i * 4 + 2] = v.z; sv[i * 4 + 3] = v.w;
        }
        int nvalid = p - (t0 + grp * 16) + 1;  // keys t <= p are visible (causal)
        nvalid = nvalid < 0 ? 0 : (nvalid > 16 ? 16 : nvalid);
        int bmax = INT32_MIN;
#pragma unroll
        for (int k = 0; k < 16; k++)
            if (k < nvalid) bmax = max(bmax, sv[k]);
        const int e1 = __shfl(bmax, (lane - 16) & 63, 64), e2 = __shfl(bmax, (lane - 32) & 63, 64),
                  e3 = __shfl(bmax, (lane - 48) & 63, 64);
        int cur0 = m;
        if (grp >= 1) cur0 = max(cur0, e1);
        if (grp >= 2) cur0 = max(cur0, e2);
        if (grp >= 3) cur0 = max(cur0, e3);
        int cur = cur0, nrec = 0;
#pragma unroll
        for (int k = 0; k < 16; k++)
            if (k < nvalid && sv[k] > cur) { nrec++; cur = sv[k]; }
        const int r1 = __shfl(nrec, (lane - 16) & 63, 64), r2 = __shfl(nrec, (lane - 32) & 63, 64),
                  r3 = __shfl(nrec, (lane - 48) & 63, 64);
        int seg = (grp >= 1 ? r1 : 0) + (grp >= 2 ? r2 : 0) + (grp >= 3 ? r3 : 0);
        cur = cur0;
        // The PV operands use this lane's 16 consecutive keys (byte k = key 16*grp + k)
        // in both A (V^T) and B (P^T), so the weights stay in registers.
        unsigned hi_dw[4] = {0, 0, 0, 0}, lo_dw[4] = {0, 0, 0, 0}, sg_dw[4] = {0, 0, 0, 0};
#pragma unroll
        for (int k = 0; k < 16; k++) {
            unsigned w = 0, sb = 0xFFu;  // invalid keys: weight 0, no segment
            if (k < nvalid) {
                const int s = sv[k];
                if (s > cur) {
                    W.rec_e[row][seg] = (uint16_t)(cur != INT32_MIN
                                                       ? exp_q16((int)((unsigned)cur - (unsigned)s), lut, ATTN_COEF_Q24)
                                                       : 0u);
                    seg++;
                    cur = s;
                    w = 65535u;
                } else {
                    w = exp_q16((int)((unsigned)s - (unsigned)cur), lut, ATTN_COEF_Q24);
                }
                sb = (unsigned)seg;
            }
            const int wq = (int)w - (int)WOFF;  // [-32896, 32639] = 256*hi + lo
            const int lo = ((wq + 128) & 255) - 128;
            const int hi = (wq - lo) >> 8;
            hi_dw[k >> 2] |= ((unsigned)hi & 255u) << (8 * (k & 3));
            lo_dw[k >> 2] |= ((unsigned)lo & 255u) << (8 * (k & 3));
            sg_dw[k >> 2] |= sb << (8 * (k & 3));
        }
        int mrow = max(cur, __shfl_xor(cur, 16, 64));
        mrow = max(mrow, __shfl_xor(mrow, 32, 64));
        m = mrow;
        int nrow = nrec + __shfl_xor(nrec, 16, 64);
        nrow += __shfl_xor(nrow, 32, 64);
        if (grp == 0) W.nrec[row] = nrow;
        int nmax = nrow;
        for (int o = 1; o < 16; o <<= 1) nmax = max(nmax, __shfl_xor(nmax, o, 64));
        wave_lds_fence();

        // 3. A operand of the PV product: V^T row (head dim 16*db + lane % 16), keys 16*grp .. +16
        v4i vop[4];
#pragma unroll
        for (int db = 0; db < 4; db++) vop[db] = *(const v4i*)(Vt + (db * 16 + row) * KLD + grp * 16);
        // 32896 * sum over the tile's 64 keys of v[key][dim = lane]
        unsigned corr;
        {
            const int* vrow = (const int*)(Vt + lane * KLD);
            int cs = 0;
#pragma unroll
            for (int i = 0; i < 16; i++) cs = __builtin_amdgcn_sdot4(vrow[i], 0x01010101, cs, false);
            corr = (unsigned)cs * WOFF;
        }
        int nr[16];
#pragma unroll
        for (int r = 0; r < 16; r++) nr[r] = __builtin_amdgcn_readfirstlane(W.nrec[r]);

        for (int j = 0; j <= nmax; j++) {
            const unsigned jb = (unsigned)j * 0x01010101u;
            v4i bh, bl;
            int sh = 0;
#pragma unroll
            for (int blk = 0; blk < 4; blk++) {
                const unsigned msk = zero_bytes_mask(sg_dw[blk] ^ jb);
                bh[blk] = (int)((hi_dw[blk] & msk) | (0x80808080u & ~msk));
                bl[blk] = (int)((lo_dw[blk] & msk) | (0x80808080u & ~msk));
                sh = __builtin_amdgcn_sdot4(bh[blk], 0x01010101, sh, false);
            }
            int sl = 0;
#pragma unroll
            for (int blk = 0; blk < 4; blk++) sl = __builtin_amdgcn_sdot4(bl[blk], 0x01010101, sl, false);
            int sw = sh * 256 + sl;  // sum over this lane's 16 keys of (w_j - 32896)
            sw += __shfl_xor(sw, 16, 64);
            sw += __shfl_xor(sw, 32, 64);
            // S of this lane's row: rescale at record j, then add segment j
            if (j >= 1 && j <= nrow) {
                const unsigned e = W.rec_e[row][j - 1];
                if (e) S = (S * e + 0x8000ull) >> 16;
            }
            S += (unsigned)(sw + 64 * (int)WOFF);
#pragma unroll
            for (int db = 0; db < 4; db++) {
                v4i acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(vop[db], bh, (v4i){0, 0, 0, 0}, 0, 0, 0);
                acc = acc << 8;
                acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(vop[db], bl, acc, 0, 0, 0);
                *(int4*)&W.buf[row][db * 16 + grp * 4] = make_int4(acc[0], acc[1], acc[2], acc[3]);
            }
            wave_lds_fence();
            // 4. lanes = dims: apply segment j of every row that has one
#pragma unroll
            for (int r = 0; r < 16; r++) {
                if (j <= nr[r]) {
                    const unsigned add = (unsigned)(int)W.buf[r][lane] + corr;
                    if (j >= 1) {
                        const unsigned e = W.rec_e[r][j - 1];
                        if (e) vacc[r] = rescale_v(vacc[r], e);
                    }
                    vacc[r] += add;
                }
            }
            wave_lds_fence();
        }
    }
    if (!wave_live) return;
    // normalize (attention.rs:278-285): lane = head dim; S of row r lives in lane r
#pragma unroll
    for (int r = 0; r < 16; r++) {
        const unsigned slo = (unsigned)__shfl((int)(unsigned)S, r, 64);
        const unsigned shi = (unsigned)__shfl((int)(unsigned)(S >> 32), r, 64);
        const int pr = wrow0 + r;
        if (pr < len) {
            const unsigned long long Sr = ((unsigned long long)shi << 32) | slo;
            const unsigned long long den = Sr == 0 ? 1ull : Sr;
            a.out[((size_t)b * T + pr) * D + h * 64 + lane] = (int8_t)clamp127(div_rne_s32_u64((int)vacc[r], den));
        }
    }
}

void launch_attention(const AttnArgs& a, int B, hipStream_t s) {
    dim3 grid((unsigned)((a.T + 63) / 64), (unsigned)a.H, (unsigned)B);
    hipLaunchKernelGGL(k_attention, grid, dim3(256), 0, s, a);
}

}  // namespace czip
