// Exact causal attention of the prefill (attention.rs:162-289) on MFMA.
#include "czip_attn_tile.h"
#include "czip_kernels.h"

namespace czip {

// ---------------------------------------------------------------------------
// One workgroup = one chunk, one head, 16 * ATT_WAVES query rows (a wave per
// 16 rows).  The K / V^T tiles of 64 keys are staged in LDS once for the
// waves (the next tile is fetched into registers meanwhile); each wave runs
// attn_tile over its 16 rows.  The waves meet at a barrier per tile and their
// record passes differ, so each waits for the slowest: two waves per
// workgroup (22.5 KB of LDS, 7 workgroups per CU) lose less there than four.
// ---------------------------------------------------------------------------

// K and V^T tiles in LDS: row r (64 bytes) of the tile at r * 64, its 16-byte
// chunk c at slot c ^ swizzle.  The K tile is read in kperm order (lanes
// 0..15 take rows 16 q + 4 blk + (0..3), q = lane / 4), the V^T tile in row
// order; each swizzle spreads the 16 rows of a read, and the 4 rows x 4
// chunks of a write, over distinct 16-byte bank groups.
__device__ __forceinline__ int lds_k(int r, int c) { return r * 64 + ((c ^ ((r >> 4) & 3)) << 4); }
__device__ __forceinline__ int lds_v(int r, int c) { return r * 64 + ((c ^ ((r >> 2) & 3)) << 4); }

constexpr int ATT_WAVES = 2;  // wavefronts (16 query rows each) per workgroup

template <bool GEN, int NWV>
__global__ __launch_bounds__(64 * NWV, 4) void k_attention(AttnArgs a) {
    constexpr int QR = 16 * NWV, KPT = 4 / NWV;  // query rows per workgroup; staging loads per thread
    __shared__ unsigned lut32[256];
    __shared__ __attribute__((aligned(16))) int8_t Ks[64 * 64];
    __shared__ __attribute__((aligned(16))) int8_t Vt[64 * 64];
    __shared__ __attribute__((aligned(16))) AttnWaveLds wl[NWV];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int row = lane & 15, grp = lane >> 4;
    // 1-D grid, XCD-aware: workgroups go round-robin over the 8 XCDs; XCD x
    // takes chunks x, x + 8, ..., all (query block, head) pairs of a chunk in a
    // row, so a chunk's K/V tiles are fetched into one L2 only.
    const int nq = (a.T + QR - 1) / QR, per_chunk = nq * a.H;
    const int xcd = (int)(blockIdx.x % 8u), jx = (int)(blockIdx.x / 8u);
    const int b = (jx / per_chunk) * 8 + xcd;
    if (b >= a.B) return;
    const int q0 = ((jx % per_chunk) % nq) * QR, h = (jx % per_chunk) / nq;
    const int T = a.T, len = a.lens[b];
    if (q0 >= len) return;
    for (int i = tid; i < 256; i += 64 * NWV) lut32[i] = (unsigned)a.lut[i] << 16;
    AttnWaveLds& W = wl[wave];
    const int D = a.H * 64;
    const int g = a.kv_mode == 1 ? (h * a.G) / a.H : 0;
    const int8_t* Kg = a.kc + ((size_t)b * a.KH + g) * T * 64;
    const int8_t* Vg = a.vc + ((size_t)b * a.KH + g) * 64 * a.TP;  // [TP/16][64][16]
    const double mscale = (double)a.score_mult[h] * (1.0 / 32768.0);
    const int p = q0 + wave * 16 + row;  // query position of this lane's row (scan / MFMA layouts)
    const int wrow0 = q0 + wave * 16;
    const bool wave_live = wrow0 < len;
    const int wave_last = min(wrow0 + 15, len - 1);

    v4i qop = (v4i){0, 0, 0, 0};
    if (p < T) qop = *(const v4i*)(a.q + ((size_t)b * T + p) * D + h * 64 + grp * 16);

    AttnRows st;
    st.m = INT32_MIN;
    st.S = 0;
    for (int r = 0; r < 16; r++) st.vacc[r] = 0;
    if (a.sink) {  // attention.rs:211-224: sink score is the initial max, weight E(0) = 65535
        const int* sk = (const int*)(a.sink + grp * 16);
        int dot = 0;
        for (int i = 0; i < 4; i++) dot = __builtin_amdgcn_sdot4(qop[i], sk[i], dot, false);
        dot += __shfl_xor(dot, 16, 64);
        dot += __shfl_xor(dot, 32, 64);
        st.m = score_b<GEN>(dot, mscale, score_bias(mscale));
        st.S = 65535u;
    }

    const int ntiles = (min(q0 + QR - 1, len - 1)) / 64 + 1;
    // K / V^T tile of 64 keys: 16-byte piece c = tid + 64 NWV n -> row c/4,
    // chunk c%4; V^T is stored in blocks of 16 keys ([key/16][dim][16]).
    // Buffer loads: the tile offset is uniform, and keys past T read as 0
    // (the resource's range check).
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc((void*)Kg, (short)0, T * 64, BUF_DWORD3);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc((void*)Vg, (short)0, a.TP * 64, BUF_DWORD3);
    v4i kreg[KPT], vreg[KPT];
#pragma unroll
    for (int n = 0; n < KPT; n++) {
        const int c = tid + 64 * NWV * n, ldr = c >> 2, ldc = (c & 3) * 16;
        kreg[n] = __builtin_amdgcn_raw_buffer_load_b128(rk, ldr * 64 + ldc, 0, 0);
        vreg[n] = __builtin_amdgcn_raw_buffer_load_b128(rv, (ldc >> 4) * 1024 + ldr * 16, 0, 0);
    }
    for (int kt = 0; kt < ntiles; kt++) {
        const int t0 = kt * 64;
        __syncthreads();
#pragma unroll
        for (int n = 0; n < KPT; n++) {
            const int c = tid + 64 * NWV * n;
            *(v4i*)(Ks + lds_k(c >> 2, c & 3)) = kreg[n];
            *(v4i*)(Vt + lds_v(c >> 2, c & 3)) = vreg[n];
        }
        __syncthreads();
        if (kt + 1 < ntiles) {
#pragma unroll
            for (int n = 0; n < KPT; n++) {
                const int c = tid + 64 * NWV * n, ldr = c >> 2, ldc = (c & 3) * 16;
                kreg[n] = __builtin_amdgcn_raw_buffer_load_b128(rk, ldr * 64 + ldc, (t0 + 64) * 64, 0);
                vreg[n] = __builtin_amdgcn_raw_buffer_load_b128(rv, (ldc >> 4) * 1024 + ldr * 16, (t0 + 64) * 64, 0);
            }
        }
        if (!wave_live || t0 > wave_last) continue;
        int nvalid = p - (t0 + grp * 16) + 1;  // keys t <= p are visible (causal)
        nvalid = nvalid < 0 ? 0 : (nvalid > 16 ? 16 : nvalid);
        attn_tile<GEN, 1>([&](int, int blk) { return *(const v4i*)(Ks + lds_k(kperm(blk, row), grp)); },
                          [&](int, int db) { return *(const v4i*)(Vt + lds_v(db * 16 + row, grp)); }, [] {}, &qop, 0,
                          mscale, nvalid, t0 + 63 > wrow0, 16, lut32, W, st);
    }
    if (!wave_live) return;
    // normalize (attention.rs:278-285): lane = head dim; S of row r lives in lane r
#pragma unroll
    for (int r = 0; r < 16; r++) {
        const unsigned Sr = (unsigned)__shfl((int)st.S, r, 64);
        const int pr = wrow0 + r;
        if (pr < len) {
            const unsigned long long den = Sr == 0u ? 1ull : (unsigned long long)Sr;
            a.out[((size_t)b * T + pr) * D + h * 64 + lane] = (int8_t)clamp127(div_rne_s32_u64((int)st.vacc[r], den));
        }
    }
}

void launch_attention(const AttnArgs& a, int B, hipStream_t s) {
    AttnArgs g = a;
    g.B = B;
    constexpr int NWV = ATT_WAVES;
    dim3 grid((unsigned)(((B + 7) / 8) * 8 * ((a.T + 16 * NWV - 1) / (16 * NWV)) * a.H));
    if (a.general)
        hipLaunchKernelGGL((k_attention<true, NWV>), grid, dim3(64 * NWV), 0, s, g);
    else
        hipLaunchKernelGGL((k_attention<false, NWV>), grid, dim3(64 * NWV), 0, s, g);
}

}  // namespace czip
