// Exact causal attention of the prefill (attention.rs:162-289) on MFMA.
#include "czip_attn_tile.h"
#include "czip_kernels.h"

namespace czip {

// ---------------------------------------------------------------------------
// One workgroup = one chunk and NWV wavefronts that share only the exp table
// (one barrier, after it is loaded).  When the head count allows, the waves
// take the same 16 query rows of NWV heads: equal tile counts, so no wave of
// a workgroup idles while another finishes.  Four heads for H a multiple of
// four: 685-688 against 728-733 ms per compress step for 8 heads at
// 1024-token chunks (two heads per workgroup: 734-737), 2,252-2,260 against
// 2,364-2,383 ms for 12 heads at 4096-token chunks (three heads: 2,337-2,348);
// else three heads for H a multiple of three: 181.5-182.3 against 183.4-183.6
// ms for the 6-head shipped model (two heads: 186.8; four waves on 64 rows of
// one head: 202.5-203.6).  Else 48 rows of one head, 16 per wave.  Each
// wave reads its K and V^T operand fragments straight from the caches
// (16-byte buffer loads; the waves of a workgroup and the workgroups of a
// chunk read the same tiles, from L1 / L2) and runs attn_tile over its rows;
// no wave waits for another.
// LDS: 8.2 KB of table + 6.5 KB of per-wave buffers per wave: 5 three-wave
// or 4 four-wave workgroups per CU (15 or 16 waves at 128 VGPRs).  For rows
// of one head, three waves per workgroup measured fastest on the 512-token
// text chunks: 189 ms per compress step against 206 with two, 210 with four,
// 237 with one and 242-248 with five, six or eight; the order in which a
// chunk's row blocks are dispatched made no difference.
// ---------------------------------------------------------------------------

// NWV wavefronts per workgroup; HWG: the waves take the same 16 rows of NWV
// heads (H a multiple of NWV), else 16 rows each of one head
template <bool GEN, int NWV, bool HWG>
__global__ __launch_bounds__(64 * NWV, 4) void k_attention(AttnArgs a) {
    constexpr int QR = HWG ? 16 : 16 * NWV;  // query rows per workgroup
    __shared__ __attribute__((aligned(16))) uint16_t etb[ETB_PAD];
    __shared__ __attribute__((aligned(16))) AttnWaveLds wl[NWV];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int row = lane & 15, grp = lane >> 4;
    // 1-D grid, XCD-aware: workgroups go round-robin over the 8 XCDs; XCD x
    // takes chunks x, x + 8, ..., all (query block, head) pairs of a chunk in a
    // row, so a chunk's K/V tiles are fetched into one L2 only.
    const int nq = (a.T + QR - 1) / QR;
    const int per_chunk = nq * (HWG ? a.H / NWV : a.H);
    const int xcd = (int)(blockIdx.x % 8u), jx = (int)(blockIdx.x / 8u);
    const int b = (jx / per_chunk) * 8 + xcd;
    if (b >= a.B) return;
    const int q0 = ((jx % per_chunk) % nq) * QR;
    const int h = HWG ? ((jx % per_chunk) / nq) * NWV + wave : (jx % per_chunk) / nq;
    const int T = a.T, len = a.lens[b];
    if (q0 >= len) return;
    for (int i = tid; i < ETB_PAD / 8; i += 64 * NWV) ((uint4*)etb)[i] = ((const uint4*)a.etab)[i];
    __syncthreads();
    const int wrow0 = HWG ? q0 : q0 + wave * 16;
    if (wrow0 >= len) return;  // no barrier follows
    AttnWaveLds& W = wl[wave];
    attn_wave_init(W);
    const int D = a.H * 64;
    const int g = a.kv_mode == 1 ? (h * a.G) / a.H : 0;
    const double mscale = (double)a.score_mult[h] * (1.0 / 32768.0);
    const int p = wrow0 + row;  // query position of this lane's row (scan / MFMA layouts)

    v4i qop = (v4i){0, 0, 0, 0};
    if (p < T) qop = *(const v4i*)(a.q + ((size_t)b * T + p) * D + h * 64 + grp * 16);

    AttnRows st;
    st.m = attn_m_empty<GEN>();
    st.S = 0;
    for (int r = 0; r < 16; r++) st.vacc[r] = 0;
    if (a.sink) {  // attention.rs:211-224: sink score is the initial max, weight E(0) = 65535
        const int* sk = (const int*)(a.sink + grp * 16);
        int dot = 0;
        for (int i = 0; i < 4; i++) dot = __builtin_amdgcn_sdot4(qop[i], sk[i], dot, false);
        dot += __shfl_xor(dot, 16, 64);
        dot += __shfl_xor(dot, 32, 64);
        st.m = attn_sink_m<GEN>(dot, mscale);
        st.S = 65535u;
    }

    const int last = min(wrow0 + 15, len - 1);  // the wave's last visible key
    const int ntiles = last / 64 + 1;
    // the last tile is a half tile (keys t0 .. t0 + 31) when the wave's
    // visible keys end in its first half
    const bool half_last = (last & 63) < 32;
    // K [T][64] and V^T [TP/16][64][16] of the chunk's KV head: buffer loads
    // with the tile offset in the scalar operand; keys past T read as 0 (the
    // resource's range check) and are never visible.
    const int8_t* Kg = a.kc + ((size_t)b * a.KH + g) * T * 64;
    const int8_t* Vg = a.vc + ((size_t)b * a.KH + g) * 64 * a.TP;
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc((void*)Kg, (short)0, T * 64, BUF_DWORD3);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc((void*)Vg, (short)0, a.TP * 64, BUF_DWORD3);
    // key kperm<KT>(blk, row) = the row's base + 4 blk; V^T of dim row (+ 16
    // db), keys 16 grp .. +16 of the tile
    const int kofs = (16 * (row >> 2) + (row & 3)) * 64 + grp * 16;
    const int vofs = grp * 1024 + row * 16;
    auto load_k = [&](int blk, int t0) { return __builtin_amdgcn_raw_buffer_load_b128(rk, kofs + blk * 256, t0 * 64, 0); };
    auto load_v = [&](int db, int t0) { return __builtin_amdgcn_raw_buffer_load_b128(rv, vofs + db * 256, t0 * 64, 0); };
    // one register set each: this tile's V^T is requested as the tile starts
    // (it arrives during the scores and the scan), the next tile's K once the
    // passes are done (the last full tile reloads itself, so the loads stay
    // unconditional)
    const int nfull = half_last ? ntiles - 1 : ntiles;
    v4i kc[4], vc[4];
    if (nfull > 0) {
#pragma unroll
        for (int blk = 0; blk < 4; blk++) kc[blk] = load_k(blk, 0);
    }
    for (int kt = 0; kt < nfull; kt++) {
        const int t0 = kt * 64;
#pragma unroll
        for (int db = 0; db < 4; db++) vc[db] = load_v(db, t0);
        const int nvalid = min(max(p - (t0 + grp * 16) + 1, 0), 16);  // keys t <= p are visible (causal)
        attn_tile<GEN, 1, 64>([&](int, int blk) { return kc[blk]; }, [&](int, int db) { return vc[db]; }, &qop, 0,
                              mscale, nvalid, t0 + 63 > wrow0, etb, W, st);
        const int tn = kt + 1 < nfull ? t0 + 64 : t0;
#pragma unroll
        for (int blk = 0; blk < 4; blk++) kc[blk] = load_k(blk, tn);
    }
    if (half_last) {
        // keys t0 .. t0 + 31, requested here rather than in the loop (their
        // offsets would stay live across it): K rows kperm<32>, V^T of keys
        // 8 grp .. +8 (8 bytes of a 16-key block)
        const int t0 = nfull * 64;
        const int ko = (8 * (row >> 2) + (row & 3)) * 64 + grp * 16, vo = (grp >> 1) * 1024 + (grp & 1) * 8 + row * 16;
#pragma unroll
        for (int blk = 0; blk < 2; blk++) kc[blk] = __builtin_amdgcn_raw_buffer_load_b128(rk, ko + blk * 256, t0 * 64, 0);
#pragma unroll
        for (int db = 0; db < 4; db++) {
            const auto x = __builtin_amdgcn_raw_buffer_load_b64(rv, vo + db * 256, t0 * 64, 0);
            vc[db] = (v4i){(int)x[0], (int)x[1], 0, 0};
        }
        const int nvalid = min(max(p - (t0 + grp * 8) + 1, 0), 8);
        attn_tile<GEN, 1, 32>([&](int, int blk) { return kc[blk]; }, [&](int, int db) { return vc[db]; }, &qop, 0,
                              mscale, nvalid, true, etb, W, st);
    }

    int8_t* const orow = a.out + ((size_t)b * T + wrow0) * D + h * 64;
    attn_normalize(st, [&](int r, int8_t v) {
        if (wrow0 + r < len) orow[(size_t)r * D + lane] = v;
    });
}

template <bool GEN, int NWV, bool HWG>
static void launch_attention_t(const AttnArgs& g, int B, hipStream_t s) {
    constexpr int QR = HWG ? 16 : 16 * NWV;
    const int nq = (g.T + QR - 1) / QR;
    dim3 grid((unsigned)(((B + 7) / 8) * 8 * nq * (HWG ? g.H / NWV : g.H)));
    hipLaunchKernelGGL((k_attention<GEN, NWV, HWG>), grid, dim3(64 * NWV), 0, s, g);
}

template <bool GEN>
static void launch_attention_g(const AttnArgs& g, int B, hipStream_t s) {
    if (g.H % 4 == 0) launch_attention_t<GEN, 4, true>(g, B, s);
    else if (g.H % 3 == 0) launch_attention_t<GEN, 3, true>(g, B, s);
    else launch_attention_t<GEN, 3, false>(g, B, s);
}

void launch_attention(const AttnArgs& a, int B, hipStream_t s) {
    AttnArgs g = a;
    g.B = B;
    if (a.general) launch_attention_g<true>(g, B, s);
    else launch_attention_g<false>(g, B, s);
}

}  // namespace czip
