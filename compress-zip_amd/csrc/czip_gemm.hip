// int8 MFMA GEMMs with fused epilogues (linear.rs:12-31 + model.rs:280-300).
#include <algorithm>
#include <cstdlib>

#include "czip_device.h"
#include "czip_kernels.h"

namespace czip {

// ---------------------------------------------------------------------------
// int8 GEMM C = A * W^T on v_mfma_i32_16x16x64_i8 with fused epilogues.
// Block tile 128 (rows of A) x 128 (rows of W) x 64, 4 waves in 2x2, each
// wave 64x64 = 4x4 MFMA tiles; the K tiles are double-buffered in LDS and the
// next one is fetched into registers while the current one is multiplied.
// MFMA operand layout: lane l supplies row (l % 16) and the 16 bytes of K at
// (l / 16) * 16; A and W use the same K mapping, so the dot product is exact
// whatever the hardware's K order.  W is the first operand, so lane l holds
// output columns 4*(l/16) .. +3 (consecutive) of row l % 16 of each 16x16
// tile, and the epilogues store 4 outputs with one vector store.
// ---------------------------------------------------------------------------
constexpr int BM = 128, BN = 128, BK = 64;
constexpr int NXCD = 8;  // XCDs of an MI355X

struct TileRegs {
    v4i v[2];
};


// The rows [row0, row0 + 128) of a row-major [rows_total, ld] int8 matrix as a
// buffer resource: rows past rows_total read as 0 (range check).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const int8_t* src, int rows_total, int ld, int row0) {
    const int rows = min(rows_total - row0, 128);
    return __builtin_amdgcn_make_buffer_rsrc((void*)(src + (size_t)row0 * ld), (short)0, rows * ld, BUF_DWORD3);
}

// 128 rows x 64 bytes at column k0: thread t -> rows t/4 and t/4 + 64, chunk t%4
__device__ __forceinline__ void fetch_tile(__amdgpu_buffer_rsrc_t r, int voff, int voff2, int k0, TileRegs& t) {
    t.v[0] = __builtin_amdgcn_raw_buffer_load_b128(r, voff, k0, 0);
    t.v[1] = __builtin_amdgcn_raw_buffer_load_b128(r, voff2, k0, 0);
}

__device__ __forceinline__ void store_tile(const TileRegs& t, int8_t* lds, int tid) {
    *(v4i*)(lds + lds64(tid >> 2, tid & 3)) = t.v[0];
    *(v4i*)(lds + lds64((tid >> 2) + 64, tid & 3)) = t.v[1];
}

template <bool FAST>
__device__ __forceinline__ int rq(int v, const GemmArgs& a) {
    return rq<FAST>(v, a.rq_scale, a.mult, a.shift);
}


// Chunk, position and RoPE cos/sin (columns c4 .. c4+3 of each 16-wide half)
// of one output row of the QKV projection.
struct QkvRow {
    int p, b;
    unsigned cs[2][2], sn[2][2];
};

__device__ __forceinline__ void qkv_row(const GemmArgs& a, int row, int c4, QkvRow& q) {
    row = min(row, a.M - 1);
    int b = (int)((float)row * (1.0f / (float)a.T));  // row < 2^24: within one of row / T
    if (b * a.T > row) b--;
    else if ((b + 1) * a.T <= row) b++;
    q.p = a.pos >= 0 ? a.pos : row - b * a.T;
    q.b = a.pos >= 0 ? row : b;
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const uint2 c = *(const uint2*)(a.rcos + q.p * 32 + j * 16 + c4);
        const uint2 sv = *(const uint2*)(a.rsin + q.p * 32 + j * 16 + c4);
        q.cs[j][0] = c.x; q.cs[j][1] = c.y;
        q.sn[j][0] = sv.x; q.sn[j][1] = sv.y;
    }
}

// Epilogue of one 16-row x 64-column tile: acc[j] holds columns
// col_base + 16 j + c4 .. +3 of `row` (col_base 64-aligned: one head / one
// gate-up group).  The caller checks row < M and col_base < N.
template <int EPI, bool FAST>
__device__ __forceinline__ void epi_tile(const GemmArgs& a, const v4i* acc, int row, int col_base, int c4,
                                         const QkvRow& q) {
    if (EPI == EPI_RAW) {
#pragma unroll
        for (int j = 0; j < 4; j++)
            *(int4*)(a.out32 + (size_t)row * a.ldo + col_base + j * 16 + c4) =
                make_int4(acc[j][0], acc[j][1], acc[j][2], acc[j][3]);
    } else if (EPI == EPI_REQ) {
#pragma unroll
        for (int j = 0; j < 4; j++)
            *(unsigned*)(a.out8 + (size_t)row * a.ldo + col_base + j * 16 + c4) =
                pack4i(rq<FAST>(acc[j][0], a), rq<FAST>(acc[j][1], a), rq<FAST>(acc[j][2], a), rq<FAST>(acc[j][3], a));
    } else if (EPI == EPI_REGLU) {
        // W rows were permuted so that a 64-row group holds 32 gate rows then the
        // matching 32 up rows: output feature f = col_base/2 + j*16 + c4 + r.
#pragma unroll
        for (int j = 0; j < 2; j++) {
            int o[4];
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int g = rq<FAST>(acc[j][r], a);
                const int u = rq<FAST>(acc[j + 2][r], a);
                const int gr = g > 0 ? g : 0;
                o[r] = clamp127(rne_shr(gr * u, 7));  // reglu.rs:20-46 (|gr * u| <= 127^2)
            }
            *(unsigned*)(a.out8 + (size_t)row * a.ldo + (col_base >> 1) + j * 16 + c4) = pack4i(o[0], o[1], o[2], o[3]);
        }
    } else {  // EPI_QKV
        const int p = q.p, b = q.b;
        const int kcol = col_base - a.d;
        int g = 0, isv = 0;
        if (kcol >= 0) {
            if (a.kv_mode == 1) { isv = kcol >= 64 * a.G; g = (isv ? kcol - 64 * a.G : kcol) >> 6; }
            else isv = kcol >= 64;
        }
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int i0 = j * 16 + c4;  // rotary pairs (i0 + r, i0 + r + 32)
            int xq[4], yq[4], xv[4], yv[4];
#pragma unroll
            for (int r = 0; r < 4; r++) {
                xv[r] = rq<FAST>(acc[j][r], a);
                yv[r] = rq<FAST>(acc[j + 2][r], a);
                const int c = (int16_t)(r & 1 ? q.cs[j][r >> 1] >> 16 : q.cs[j][r >> 1] & 0xFFFFu);
                const int sn = (int16_t)(r & 1 ? q.sn[j][r >> 1] >> 16 : q.sn[j][r >> 1] & 0xFFFFu);
                const int xr = (int)((unsigned)(xv[r] * c) - (unsigned)(yv[r] * sn));
                const int yr = (int)((unsigned)(xv[r] * sn) + (unsigned)(yv[r] * c));
                if (kcol < 0) {
                    // Q: attention.rs:53-83 (>>15 then NET_SHIFT=1, two roundings)
                    xq[r] = clamp127(rne_shr(rne_shr(xr, 15), 1));
                    yq[r] = clamp127(rne_shr(rne_shr(yr, 15), 1));
                } else {
                    // K: attention.rs:29-50 (|xr|, |yr| <= 2 * 127 * 32768)
                    xq[r] = clamp127(rne_shr(xr, 15));
                    yq[r] = clamp127(rne_shr(yr, 15));
                }
            }
            if (kcol < 0) {
                int8_t* qo = a.out8 + (size_t)row * a.ldo + col_base;
                *(unsigned*)(qo + i0) = pack4i(xq[0], xq[1], xq[2], xq[3]);
                *(unsigned*)(qo + i0 + 32) = pack4i(yq[0], yq[1], yq[2], yq[3]);
            } else if (!isv) {
                int8_t* k = a.kc + (((size_t)b * a.KH + g) * a.T + p) * 64;
                *(unsigned*)(k + i0) = pack4i(xq[0], xq[1], xq[2], xq[3]);
                *(unsigned*)(k + i0 + 32) = pack4i(yq[0], yq[1], yq[2], yq[3]);
            } else {
                // V^T in blocks of 2^vl keys (vt_off)
                const int vl = a.vl;
                int8_t* v = a.vc + ((size_t)b * a.KH + g) * 64 * a.TP + vt_off(p, 0, vl);
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    v[(i0 + r) << vl] = (int8_t)xv[r];
                    v[(i0 + r + 32) << vl] = (int8_t)yv[r];
                }
            }
        }
    }
}

template <int EPI, bool FAST>
__global__ __launch_bounds__(256, 2) void k_gemm(GemmArgs a) {
    __shared__ __attribute__((aligned(16))) int8_t As[2][BM * 64];
    __shared__ __attribute__((aligned(16))) int8_t Ws[2][BN * 64];
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int wm = wave >> 1, wn = wave & 1;
    // Workgroups are dispatched round-robin over the 8 XCDs, each with its own
    // L2: XCD x takes the A blocks m = x, x + 8, ..., all N tiles of one A block
    // back to back, so every A block is fetched from HBM by one L2 only.
    const int ntn = (a.N + BN - 1) / BN;
    const int xcd = (int)(blockIdx.x % NXCD), jx = (int)(blockIdx.x / NXCD);
    const int mt = (jx / ntn) * NXCD + xcd;
    const int m0 = mt * BM, n0 = (jx % ntn) * BN;
    if (m0 >= a.M) return;
    const int nk = a.K / BK;

    v4i acc[4][4];
    for (int i = 0; i < 4; i++)
        for (int j = 0; j < 4; j++) acc[i][j] = (v4i){0, 0, 0, 0};

    TileRegs ta, tw;
    const __amdgpu_buffer_rsrc_t rw = tile_rsrc(a.W, a.N, a.K, n0);
    const int voff = (tid >> 2) * a.K + (tid & 3) * 16, voff2 = voff + 64 * a.K;
    // A rows gathered from a table: offsets from the table's start, rows past M out of range
    const bool gather = a.a_rows != nullptr;
    const __amdgpu_buffer_rsrc_t ra =
        gather ? __builtin_amdgcn_make_buffer_rsrc((void*)a.A, (short)0, a.a_nrows * a.K, BUF_DWORD3)
               : tile_rsrc(a.A, a.M, a.K, m0);
    int aoff = voff, aoff2 = voff2;
    if (gather) {
        const int r1 = m0 + (tid >> 2), r2 = r1 + 64;
        aoff = r1 < a.M ? (int)a.a_rows[r1] * a.K + (tid & 3) * 16 : 0x7FFFFF00;
        aoff2 = r2 < a.M ? (int)a.a_rows[r2] * a.K + (tid & 3) * 16 : 0x7FFFFF00;
    }
    fetch_tile(ra, aoff, aoff2, 0, ta);
    fetch_tile(rw, voff, voff2, 0, tw);
    store_tile(ta, As[0], tid);
    store_tile(tw, Ws[0], tid);
    __syncthreads();
    const int lr = lane & 15;
    for (int kt = 0; kt < nk; kt++) {
        const int cur = kt & 1;
        if (kt + 1 < nk) {  // the next K step, fetched while this one is multiplied
            fetch_tile(ra, aoff, aoff2, (kt + 1) * BK, ta);
            fetch_tile(rw, voff, voff2, (kt + 1) * BK, tw);
        }
        __builtin_amdgcn_sched_barrier(0);  // keep the loads ahead of this step's MFMAs
        v4i af[4], bf[4];
#pragma unroll
        for (int i = 0; i < 4; i++) af[i] = *(const v4i*)(As[cur] + lds64(wm * 64 + i * 16 + lr, lane >> 4));
#pragma unroll
        for (int j = 0; j < 4; j++) bf[j] = *(const v4i*)(Ws[cur] + lds64(wn * 64 + j * 16 + lr, lane >> 4));
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bf[j], af[i], acc[i][j], 0, 0, 0);
        if (kt + 1 < nk) {
            store_tile(ta, As[cur ^ 1], tid);
            store_tile(tw, Ws[cur ^ 1], tid);
        }
        __syncthreads();
    }

    const int col_base = n0 + wn * 64;  // 64-aligned, one head / one gate-up group
    if (col_base >= a.N) return;
    const int c4 = (lane >> 4) * 4;  // first of this lane's 4 consecutive columns in a 16-wide tile
    // QKV: chunk, position and RoPE cos/sin of the lane's 4 rows, all loads
    // issued before the arithmetic
    QkvRow qr[4];
    if (EPI == EPI_QKV) {
#pragma unroll
        for (int i = 0; i < 4; i++) qkv_row(a, m0 + wm * 64 + i * 16 + lr, c4, qr[i]);
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int row = m0 + wm * 64 + i * 16 + lr;
        if (row >= a.M) continue;
        epi_tile<EPI, FAST>(a, acc[i], row, col_base, c4, qr[i]);
    }
}

// Output resources of one strip: rows past M (and, for the caches, rows whose
// offset is forced out of range) are dropped by the buffer range check.
struct WsOut {
    __amdgpu_buffer_rsrc_t o;      // out8 / out32 from the strip's first row r0
    __amdgpu_buffer_rsrc_t k, v;   // QKV: K / V^T caches from chunk b0
    int vl;                        // QKV: the V^T block exponent (vt_off)
    int r0, b0;
};

// The results of one 16 x 64 tile, packed for its stores: REQ / QKV Q and K
// the row's 16 bytes at columns 16 (lane / 16) .., REGLU its 8 bytes at
// 8 (lane / 16) .. of the 32 outputs, V the x / y bytes of the two rotary
// groups (four to a dword); off = where they go (for the caches, out of range
// for rows past M).
struct WsTile {
    unsigned d[4];
    int off;
};

// 4 x 4 dword transpose over the four 16-lane groups: on entry group g holds
// x[j] = X[g][j], on exit X[j][g] (gfx950 permlane swaps: 32 exchanges lane
// halves, 16 the odd and even 16-lane rows).
__device__ __forceinline__ void transpose4(unsigned (&x)[4]) {
    auto a = __builtin_amdgcn_permlane32_swap(x[0], x[2], false, false);
    auto b = __builtin_amdgcn_permlane32_swap(x[1], x[3], false, false);
    auto c = __builtin_amdgcn_permlane16_swap(a[0], b[0], false, false);
    auto d = __builtin_amdgcn_permlane16_swap(a[1], b[1], false, false);
    x[0] = c[0]; x[1] = c[1]; x[2] = d[0]; x[3] = d[1];
}

// 4 x 2: group g holds X[g][0], X[g][1]; on exit the 8 bytes of
// (X[2h][j], X[2h + 1][j]) with j = g / 2, h = g % 2
__device__ __forceinline__ void transpose2(unsigned& x0, unsigned& x1) {
    auto a = __builtin_amdgcn_permlane32_swap(x0, x1, false, false);
    auto c = __builtin_amdgcn_permlane16_swap(a[0], a[1], false, false);
    x0 = c[0]; x1 = c[1];
}

// Epilogue arithmetic of one tile (as epi_tile).  ROLE of a QKV wave: 0 its 64
// columns are a query head, 1 the key head g, 2 the value head g.  EPI_RAW
// stores at once (16 dwords per tile are too many to hold).
template <int EPI, bool FAST, int ROLE>
__device__ __forceinline__ void epi_ws(const GemmArgs& a, const WsOut& ro, const v4i* acc, int row, int col_base,
                                       int c4, const QkvRow& q, int g, WsTile& t) {
    if (EPI == EPI_RAW) {
#pragma unroll
        for (int j = 0; j < 4; j++)
            __builtin_amdgcn_raw_buffer_store_b128(acc[j], ro.o, ((row - ro.r0) * a.ldo + col_base + j * 16 + c4) * 4, 0, 0);
    } else if (EPI == EPI_REQ) {
#pragma unroll
        for (int j = 0; j < 4; j++)
            t.d[j] = pack4i(rq<FAST>(acc[j][0], a), rq<FAST>(acc[j][1], a), rq<FAST>(acc[j][2], a), rq<FAST>(acc[j][3], a));
        transpose4(t.d);
        t.off = (row - ro.r0) * a.ldo + col_base + c4 * 4;
    } else if (EPI == EPI_REGLU) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            int o[4];
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int gg = rq<FAST>(acc[j][r], a);
                const int u = rq<FAST>(acc[j + 2][r], a);
                const int gr = gg > 0 ? gg : 0;
                o[r] = clamp127(rne_shr(gr * u, 7));  // reglu.rs:20-46
            }
            t.d[j] = pack4i(o[0], o[1], o[2], o[3]);
        }
        transpose2(t.d[0], t.d[1]);
        t.off = (row - ro.r0) * a.ldo + (col_base >> 1) + c4 * 2;
    } else {  // EPI_QKV
        const bool valid = row < a.M;
        const int p = q.p, bl = q.b - ro.b0;
#pragma unroll
        for (int j = 0; j < 2; j++) {
            int xq[4], yq[4], xv[4], yv[4];
#pragma unroll
            for (int r = 0; r < 4; r++) {
                xv[r] = rq<FAST>(acc[j][r], a);
                yv[r] = rq<FAST>(acc[j + 2][r], a);
                if (ROLE != 2) {
                    const int c = (int16_t)(r & 1 ? q.cs[j][r >> 1] >> 16 : q.cs[j][r >> 1] & 0xFFFFu);
                    const int sn = (int16_t)(r & 1 ? q.sn[j][r >> 1] >> 16 : q.sn[j][r >> 1] & 0xFFFFu);
                    const int xr = (int)((unsigned)(xv[r] * c) - (unsigned)(yv[r] * sn));
                    const int yr = (int)((unsigned)(xv[r] * sn) + (unsigned)(yv[r] * c));
                    if (ROLE == 0) {  // attention.rs:53-83
                        xq[r] = clamp127(rne_shr(rne_shr(xr, 15), 1));
                        yq[r] = clamp127(rne_shr(rne_shr(yr, 15), 1));
                    } else {  // attention.rs:29-50
                        xq[r] = clamp127(rne_shr(xr, 15));
                        yq[r] = clamp127(rne_shr(yr, 15));
                    }
                }
            }
            if (ROLE != 2) {  // 16-column tiles: x of group j is tile j, y tile 2 + j
                t.d[j] = pack4i(xq[0], xq[1], xq[2], xq[3]);
                t.d[2 + j] = pack4i(yq[0], yq[1], yq[2], yq[3]);
            } else {
                t.d[2 * j] = pack4i(xv[0], xv[1], xv[2], xv[3]);
                t.d[2 * j + 1] = pack4i(yv[0], yv[1], yv[2], yv[3]);
            }
        }
        if (ROLE != 2) transpose4(t.d);
        if (ROLE == 0) t.off = (row - ro.r0) * a.ldo + col_base + c4 * 4;
        else if (ROLE == 1) t.off = valid ? ((bl * a.KH + g) * a.T + p) * 64 + c4 * 4 : (int)0xFFFFFF00u;
        else t.off = valid ? (bl * a.KH + g) * 64 * a.TP + vt_off(p, c4, a.vl) : (int)0xFFFF0000u;
    }
}

// The stores of one tile.
template <int EPI, int ROLE>
__device__ __forceinline__ void flush_ws(const WsOut& ro, const WsTile& t) {
    if (EPI == EPI_REQ || (EPI == EPI_QKV && ROLE != 2)) {
        __builtin_amdgcn_raw_buffer_store_b128((v4i){(int)t.d[0], (int)t.d[1], (int)t.d[2], (int)t.d[3]},
                                               EPI == EPI_QKV && ROLE == 1 ? ro.k : ro.o, t.off, 0, 0);
    } else if (EPI == EPI_REGLU) {
        __builtin_amdgcn_raw_buffer_store_b64((v2i){(int)t.d[0], (int)t.d[1]}, ro.o, t.off, 0, 0);
    } else if (EPI == EPI_QKV) {
        // V^T in blocks of 2^vl keys (vt_off): dim i of the key is at byte i << vl
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                __builtin_amdgcn_raw_buffer_store_b8((unsigned char)(t.d[2 * j] >> (8 * r)), ro.v,
                                                     t.off + ((j * 16 + r) << ro.vl), 0, 0);
                __builtin_amdgcn_raw_buffer_store_b8((unsigned char)(t.d[2 * j + 1] >> (8 * r)), ro.v,
                                                     t.off + ((j * 16 + r + 32) << ro.vl), 0, 0);
            }
    }
}

// The 16-row tiles of one SR-row strip for this wave's 64 columns, the
// epilogue arithmetic of tile i between the MFMAs of tile i + 1; the results
// stay in t for the stores.
template <int EPI, bool FAST, int KS, int SR, int ROLE>
__device__ __forceinline__ void ws_strip(const GemmArgs& a, const WsOut& ro, const v4i (&w)[4][KS],
                                         const int8_t* As, int r0, int col_base, int g, WsTile (&t)[SR / 16]) {
    const int lane = threadIdx.x & 63, lr = lane & 15, c4 = (lane >> 4) * 4;
    auto mma = [&](int i, v4i* acc) {
        v4i af[KS];
#pragma unroll
        for (int ks = 0; ks < KS; ks++) af[ks] = *(const v4i*)(As + ks * SR * 64 + lds64(i * 16 + lr, lane >> 4));
#pragma unroll
        for (int ks = 0; ks < KS; ks++)
#pragma unroll
            for (int j = 0; j < 4; j++)
                acc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(w[j][ks], af[ks], ks == 0 ? (v4i){0, 0, 0, 0} : acc[j], 0, 0, 0);
    };
    QkvRow qr[2];
    if (EPI == EPI_QKV) qkv_row(a, r0 + lr, c4, qr[0]);
    v4i acc[2][4];
    mma(0, acc[0]);
#pragma unroll
    for (int i = 0; i < SR / 16; i++) {
        if (i + 1 < SR / 16) {
            if (EPI == EPI_QKV) qkv_row(a, r0 + (i + 1) * 16 + lr, c4, qr[(i + 1) & 1]);
            mma(i + 1, acc[(i + 1) & 1]);
        }
        epi_ws<EPI, FAST, ROLE>(a, ro, acc[i & 1], r0 + i * 16 + lr, col_base, c4, qr[i & 1], g, t[i]);
        if (i + 1 < SR / 16) {
            // the next tile's products between this tile's epilogue VALU, one
            // MFMA to every three (d512 prefill: up + ReGLU 287 -> 276 ms, QKV
            // 68 -> 66.5 ms per 16M-token step)
#pragma unroll
            for (int n = 0; n < 4 * KS; n++) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
}

template <int EPI, int NT, int ROLE>
__device__ __forceinline__ void ws_flush(const WsOut& ro, const WsTile (&t)[NT]) {
#pragma unroll
    for (int i = 0; i < NT; i++) flush_ws<EPI, ROLE>(ro, t[i]);
}

// ---------------------------------------------------------------------------
// Persistent W-stationary GEMM for K = 64 KS (KS <= 8): each wave keeps its 64
// columns of W for the whole K in registers (4 x KS MFMA operands, loaded
// once), a workgroup of 4 waves owns 256 columns, and the rows of A stream
// through in strips of SR (64; 32 for QKV, whose epilogue holds more): the
// next strip is fetched into registers while the current one, double-buffered
// in LDS as KS SR x 64 tiles, is multiplied, and the strip's outputs are
// stored after the next strip is in LDS.
// Only A crosses LDS (64 B of LDS reads per 16 K MACs per lane), and no W
// byte is re-read.  Workgroups are dispatched round-robin over the 8 XCDs:
// the ncg column groups of one row worker sit on one XCD and walk the same
// strips, so each strip is fetched from HBM by one L2.
// ---------------------------------------------------------------------------
template <int EPI, bool FAST, int KS, int SR>
__global__ __launch_bounds__(256, 2) void k_gemm_ws(GemmArgs a, int ncg) {
    __shared__ __attribute__((aligned(16))) int8_t As[2][KS * SR * 64];
    constexpr int NT = SR / 16, KPT = KS * SR / 64;  // tiles per strip, staging loads per thread
    constexpr int K = KS * 64;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, lr = lane & 15;
    const int xcd = (int)(blockIdx.x % NXCD), jx = (int)(blockIdx.x / NXCD);
    const int cg = jx % ncg;
    const int worker = (jx / ncg) * NXCD + xcd, nworkers = (int)gridDim.x / ncg;
    const int nstrips = (a.M + SR - 1) / SR;
    if (worker >= nstrips) return;  // the whole workgroup
    const int col_base = cg * 256 + wave * 64;
    const bool wlive = col_base < a.N;
    // QKV: the wave's role and KV head
    int role = 0, g = 0;
    if (EPI == EPI_QKV) {
        const int kcol = col_base - a.d;
        if (kcol >= 0) {
            int isv;
            if (a.kv_mode == 1) { isv = kcol >= 64 * a.G; g = (isv ? kcol - 64 * a.G : kcol) >> 6; }
            else isv = kcol >= 64;
            role = isv ? 2 : 1;
        }
    }

    // this wave's W: w[j][ks] = rows col_base + 16 j + lane % 16, bytes 64 ks + 16 (lane / 16) .. +16
    v4i w[4][KS];
    {
        const __amdgpu_buffer_rsrc_t rW = __builtin_amdgcn_make_buffer_rsrc((void*)a.W, (short)0, a.N * K, BUF_DWORD3);
        const int woff = (col_base + lr) * K + (lane >> 4) * 16;
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int ks = 0; ks < KS; ks++) w[j][ks] = __builtin_amdgcn_raw_buffer_load_b128(rW, woff + j * 16 * K, ks * 64, 0);
    }
    WsOut ro;
    // strip staging: thread -> row (tid / 4) % SR, 16-byte chunk tid % 4 of the
    // 64-byte K steps ks = kg, kg + 64 / SR, ... (kg = tid / (4 SR))
    const int srow = (tid >> 2) % SR, sch = tid & 3, kg = (tid >> 2) / SR;
    v4i st[KPT];
    auto fetch = [&](int s) {
        const int r0 = s * SR;
        // the resource from uniform values only (a per-lane choice of resource
        // would make the compiler loop over distinct resources); with a_rows the
        // A rows are gathered from a table, rows past M out of range
        const bool gather = a.a_rows != nullptr;
        const int8_t* base = gather ? a.A : a.A + (size_t)r0 * K;
        const int nrec = gather ? a.a_nrows * K : min(a.M - r0, SR) * K;
        const __amdgpu_buffer_rsrc_t rA = __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, nrec, BUF_DWORD3);
        int off = srow * K + sch * 16;
        if (gather) off = r0 + srow < a.M ? (int)a.a_rows[r0 + srow] * K + sch * 16 : 0x7FFFFF00;
        off += kg * 64;  // per lane in the vector offset; the scalar offset stays a constant
#pragma unroll
        for (int n = 0; n < KPT; n++) st[n] = __builtin_amdgcn_raw_buffer_load_b128(rA, off, n * (64 / SR) * 64, 0);
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int n = 0; n < KPT; n++) *(v4i*)(As[buf] + (kg + n * (64 / SR)) * SR * 64 + lds64(srow, sch)) = st[n];
    };
    fetch(worker);
    store(0);
    __syncthreads();
    int cur = 0;
    for (int s = worker; s < nstrips; s += nworkers) {
        const bool more = s + nworkers < nstrips;
        if (more) fetch(s + nworkers);
        const int r0 = s * SR;
        ro.r0 = r0;
        {
            const int ob = min(a.M - r0, SR) * a.ldo * (EPI == EPI_RAW ? 4 : 1);
            if (EPI == EPI_RAW)
                ro.o = __builtin_amdgcn_make_buffer_rsrc((void*)(a.out32 + (size_t)r0 * a.ldo), (short)0, ob, BUF_DWORD3);
            else
                ro.o = __builtin_amdgcn_make_buffer_rsrc((void*)(a.out8 + (size_t)r0 * a.ldo), (short)0, ob, BUF_DWORD3);
        }
        if (EPI == EPI_QKV) {
            // the caches from the strip's first chunk: every offset of the
            // strip's rows fits 31 bits (SR rows, KH * T * 64 < 2^24 per chunk)
            const long long nb = a.pos >= 0 ? a.M : (a.M + a.T - 1) / a.T;
            ro.b0 = a.pos >= 0 ? r0 : r0 / a.T;
            const long long kb = (long long)a.KH * a.T * 64, vb = (long long)a.KH * 64 * a.TP;
            ro.k = __builtin_amdgcn_make_buffer_rsrc((void*)(a.kc + ro.b0 * kb), (short)0,
                                                     (int)min((nb - ro.b0) * kb, 0x7FFFFFFFll), BUF_DWORD3);
            ro.v = __builtin_amdgcn_make_buffer_rsrc((void*)(a.vc + ro.b0 * vb), (short)0,
                                                     (int)min((nb - ro.b0) * vb, 0x7FFFFFFFll), BUF_DWORD3);
            ro.vl = a.vl;
        }
        WsTile t[NT];
        if (wlive) {
            if (EPI != EPI_QKV || role == 0) ws_strip<EPI, FAST, KS, SR, 0>(a, ro, w, As[cur], r0, col_base, g, t);
            else if (role == 1) ws_strip<EPI, FAST, KS, SR, 1>(a, ro, w, As[cur], r0, col_base, g, t);
            else ws_strip<EPI, FAST, KS, SR, 2>(a, ro, w, As[cur], r0, col_base, g, t);
        }
        // the next strip into LDS, then this strip's stores: a wave's stores
        // and loads share one completion counter, so stores issued before the
        // wait for the staging loads would be waited for too
        if (more) store(cur ^ 1);
        if (wlive) {
            if (EPI != EPI_QKV || role == 0) ws_flush<EPI, NT, 0>(ro, t);
            else if (role == 1) ws_flush<EPI, NT, 1>(ro, t);
            else ws_flush<EPI, NT, 2>(ro, t);
        }
        __syncthreads();
        cur ^= 1;
    }
}

template <int EPI>
static void launch_epi(const GemmArgs& a, dim3 grid, hipStream_t s) {
    if (a.rq_fast)
        hipLaunchKernelGGL((k_gemm<EPI, true>), grid, dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL((k_gemm<EPI, false>), grid, dim3(256), 0, s, a);
}

template <int EPI, int KS>
static void launch_ws(const GemmArgs& a, hipStream_t s) {
    constexpr int SR = EPI == EPI_QKV ? 32 : 64;
    // two workgroups per CU (256 CUs), ncg column groups per row worker, the
    // workers a multiple of the 8 XCDs and no more than the strips
    const int ncg = (a.N + 255) / 256;
    const int nstrips = (a.M + SR - 1) / SR;
    int workers = std::max(NXCD, (512 / ncg) / NXCD * NXCD);
    // at least two strips per worker (a few thousand rows: fewer, fuller
    // workers load W fewer times; measured on the 4096-row decode QKV, 12.9 ->
    // 11 us per launch)
    workers = std::min(workers, std::max(NXCD, ((nstrips + 1) / 2 + NXCD - 1) / NXCD * NXCD));
    dim3 grid((unsigned)(workers * ncg));
    if (a.rq_fast)
        hipLaunchKernelGGL((k_gemm_ws<EPI, true, KS, SR>), grid, dim3(256), 0, s, a, ncg);
    else
        hipLaunchKernelGGL((k_gemm_ws<EPI, false, KS, SR>), grid, dim3(256), 0, s, a, ncg);
}

template <int EPI>
static bool try_ws(const GemmArgs& a, hipStream_t s) {
    if (a.tiled || a.N % 64 != 0 || (long long)a.N * a.K >= (1ll << 31) || a.M <= 0) return false;
    // 32-bit buffer offsets: the output rows, and the cache span of one strip
    if (64ll * a.ldo * (EPI == EPI_RAW ? 4 : 1) >= (1ll << 31)) return false;
    if (EPI == EPI_QKV && ((long long)a.KH * a.TP * 64 >= (1ll << 24) || a.T > a.TP)) return false;
    switch (a.K) {
        case 384: launch_ws<EPI, 6>(a, s); return true;
        case 512: launch_ws<EPI, 8>(a, s); return true;
        default: return false;
    }
}

void launch_gemm(const GemmArgs& a, int epi, hipStream_t s) {
    switch (epi) {
        case EPI_RAW: if (try_ws<EPI_RAW>(a, s)) return; break;
        case EPI_REQ: if (try_ws<EPI_REQ>(a, s)) return; break;
        case EPI_QKV: if (try_ws<EPI_QKV>(a, s)) return; break;
        default: if (try_ws<EPI_REGLU>(a, s)) return; break;
    }
    const int ntm = (a.M + BM - 1) / BM, ntn = (a.N + BN - 1) / BN;
    dim3 grid((unsigned)(((ntm + NXCD - 1) / NXCD) * NXCD * ntn));
    switch (epi) {
        case EPI_RAW: launch_epi<EPI_RAW>(a, grid, s); break;
        case EPI_REQ: launch_epi<EPI_REQ>(a, grid, s); break;
        case EPI_QKV: launch_epi<EPI_QKV>(a, grid, s); break;
        default: launch_epi<EPI_REGLU>(a, grid, s); break;
    }
}

// ---------------------------------------------------------------------------
// Row GEMM: a workgroup owns 64 rows and all d output columns, so the
// requantization, both RMSNorms and the residual add run in its epilogue and
// the projection output never leaves the chip.  NW waves split the columns
// (CT 16-wide tiles each, d = NW * CT * 16); the 64 x 64 A tile of each K step
// goes through double-buffered LDS, and each wave streams its own W columns
// straight into registers (no W element is used by two waves).
// ---------------------------------------------------------------------------
constexpr int RBM = 64;


// Epilogue of the row GEMM for rows m0 .. m0 + 16 RT - 1 (all d columns in
// the workgroup; RT = 4 row tiles in the 64-row kernels, 1 in the 16-row one):
// requantize, residual add, both RMSNorms (model.rs:424-468).
// Lane holds columns nb + 16 t + c4 .. +3 of rows m0 + 16 i + lr; w1r / w2r
// are its columns' norm weights.  Its residual inputs (int16 stream or the
// token's embedding row) are requested first so that their latency hides
// behind step 1 and the first reduction; mid() runs after that reduction,
// before the first store.
template <int NW, int CT, bool FAST, int RT, class Mid>
__device__ __forceinline__ void rn_epilogue(const RowGemmArgs& a, v4i (&acc)[RT][CT], int m0, const unsigned (&w1r)[CT],
                                            const unsigned (&w2r)[CT], unsigned (*red)[16 * RT], int* inv_s, Mid mid) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int nb = wave * CT * 16;
    const int lr = lane & 15, c4 = (lane >> 4) * 4;
    uint2 xr[RT][CT];
#pragma unroll
    for (int i = 0; i < RT; i++) {
        const int row = min(m0 + i * 16 + lr, a.M - 1);
        if (a.x_in) {
#pragma unroll
            for (int t = 0; t < CT; t++) xr[i][t] = *(const uint2*)(a.x_in + (size_t)row * a.d + nb + t * 16 + c4);
        } else {
            const int8_t* erow = a.embed + (size_t)a.tok[row] * a.d;
#pragma unroll
            for (int t = 0; t < CT; t++) xr[i][t] = make_uint2(*(const unsigned*)(erow + nb + t * 16 + c4), 0u);
        }
    }
    // 1. y = requant(acc); row sums of y^2
#pragma unroll
    for (int i = 0; i < RT; i++) {
        unsigned ss = 0;
#pragma unroll
        for (int t = 0; t < CT; t++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int y = rq<FAST>(acc[i][t][r], a.rq_scale, a.mult, a.shift);
                acc[i][t][r] = y;
                ss += (unsigned)__mul24(y, y);
            }
        ss += (unsigned)__shfl_xor((int)ss, 16, 64);
        ss += (unsigned)__shfl_xor((int)ss, 32, 64);
        if (lane < 16) red[wave][i * 16 + lane] = ss;
    }
    __syncthreads();
    auto row_inv = [&]() {
        if (wave == 0 && lane < 16 * RT) {
            unsigned s = 0;
#pragma unroll
            for (int w = 0; w < NW; w++) s += red[w][lane];
            int mean_sq = (int)(s / (unsigned)a.d) + 1;  // eps_scaled = 1 (rmsnorm.rs:80-83)
            inv_s[lane] = inv_rms_q15_fast(mean_sq);  // mean_sq <= 127^2 + 1
        }
        __syncthreads();
    };
    row_inv();
    mid();
    // 2. x = x_in + rmsnorm(y, w1); keep clamp(x); row sums of clamp(x)^2
#pragma unroll
    for (int i = 0; i < RT; i++) {
        const int row = m0 + i * 16 + lr;
        const bool live = row < a.M;
        const double inv = (double)inv_s[i * 16 + lr] * (1.0 / 32768.0);
        unsigned ss = 0;
#pragma unroll
        for (int t = 0; t < CT; t++) {
            const int n = nb + t * 16 + c4;
            int w1v[4], xo[4];
            unpack4s(w1r[t], w1v);
            if (a.x_in) {
                xo[0] = (int16_t)(xr[i][t].x & 0xFFFFu); xo[1] = (int16_t)(xr[i][t].x >> 16);
                xo[2] = (int16_t)(xr[i][t].y & 0xFFFFu); xo[3] = (int16_t)(xr[i][t].y >> 16);
            } else {
                unpack4s(xr[i][t].x, xo);
            }
            int xnw[4];
#pragma unroll
            for (int r = 0; r < 4; r++) {
                xnw[r] = xo[r] + rms_el(acc[i][t][r], w1v[r], inv);
                const int xc = clamp127(xnw[r]);
                acc[i][t][r] = xc;
                ss += (unsigned)__mul24(xc, xc);
            }
            if (a.x_out && live)
                *(uint2*)(a.x_out + (size_t)row * a.d + n) = make_uint2(((unsigned)xnw[0] & 0xFFFFu) | ((unsigned)xnw[1] << 16),
                                                                        ((unsigned)xnw[2] & 0xFFFFu) | ((unsigned)xnw[3] << 16));
        }
        ss += (unsigned)__shfl_xor((int)ss, 16, 64);
        ss += (unsigned)__shfl_xor((int)ss, 32, 64);
        if (lane < 16) red[wave][i * 16 + lane] = ss;
    }
    __syncthreads();
    row_inv();
    // 3. xn = rmsnorm(clamp(x), w2)
#pragma unroll
    for (int i = 0; i < RT; i++) {
        const int row = m0 + i * 16 + lr;
        if (row >= a.M) continue;
        const double inv = (double)inv_s[i * 16 + lr] * (1.0 / 32768.0);
#pragma unroll
        for (int t = 0; t < CT; t++) {
            const int n = nb + t * 16 + c4;
            int w2v[4];
            unpack4s(w2r[t], w2v);
            *(unsigned*)(a.xn + (size_t)row * a.d + n) =
                pack4i(rms_el(acc[i][t][0], w2v[0], inv), rms_el(acc[i][t][1], w2v[1], inv),
                       rms_el(acc[i][t][2], w2v[2], inv), rms_el(acc[i][t][3], w2v[3], inv));
        }
    }
}

template <int NW, int CT, bool FAST, bool FULL>
__global__ __launch_bounds__(64 * NW) void k_gemm_rn(RowGemmArgs a) {
    // FULL: the block's whole A (K <= 1024) staged at once, K steps without barriers
    __shared__ __attribute__((aligned(16))) int8_t As[FULL ? 16 : 2][RBM * 64];
    __shared__ unsigned red[NW][RBM];
    __shared__ int inv_s[RBM];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int m0 = blockIdx.x * RBM;
    const int nb = wave * CT * 16;  // first output column of this wave
    const int c4 = (lane >> 4) * 4;

    v4i acc[4][CT];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int t = 0; t < CT; t++) acc[i][t] = (v4i){0, 0, 0, 0};

    if constexpr (FULL) rowblock_mma_full<CT>(a.A, a.M, a.K, a.Wf, a.d, m0, nb, As, acc);
    else rowblock_mma<CT>(a.A, a.M, a.K, a.Wf, a.d, m0, nb, As, acc);
    unsigned w1r[CT], w2r[CT];
#pragma unroll
    for (int t = 0; t < CT; t++) {
        w1r[t] = *(const unsigned*)(a.w1 + nb + t * 16 + c4);
        w2r[t] = *(const unsigned*)(a.w2 + nb + t * 16 + c4);
    }
    rn_epilogue<NW, CT, FAST>(a, acc, m0, w1r, w2r, red, inv_s, [] {});
}

// ---------------------------------------------------------------------------
// Persistent W-stationary row GEMM for K = 64 KS: each wave keeps its CT
// column tiles of W for the whole K in registers (loaded once), one workgroup
// per CU walks 64-row strips, the next strip's A fetched into registers while
// the current one (double-buffered in LDS) is multiplied and written to LDS
// between the epilogue's first reduction and its first store.
// ---------------------------------------------------------------------------
template <int NW, int CT, int KS, bool FAST>
__global__ __launch_bounds__(64 * NW) void k_gemm_rn_ws(RowGemmArgs a) {
    constexpr int K = KS * 64, KPT = 4 * KS / NW;  // staging loads per thread
    static_assert(KPT * NW == 4 * KS, "a strip is 256 KS 16-byte chunks");
    __shared__ __attribute__((aligned(16))) int8_t As[2][KS * RBM * 64];
    __shared__ unsigned red[NW][RBM];
    __shared__ int inv_s[RBM];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, lr = lane & 15;
    const int nb = wave * CT * 16;
    const int c4 = (lane >> 4) * 4;
    const int nstrips = (a.M + RBM - 1) / RBM;
    if ((int)blockIdx.x >= nstrips) return;  // the whole workgroup

    v4i w[CT][KS];
    {
        const __amdgpu_buffer_rsrc_t rW = __builtin_amdgcn_make_buffer_rsrc((void*)a.W, (short)0, a.d * K, BUF_DWORD3);
        const int woff = (nb + lr) * K + (lane >> 4) * 16;
#pragma unroll
        for (int t = 0; t < CT; t++)
#pragma unroll
            for (int ks = 0; ks < KS; ks++) w[t][ks] = __builtin_amdgcn_raw_buffer_load_b128(rW, woff + t * 16 * K, ks * 64, 0);
    }
    unsigned w1r[CT], w2r[CT];
#pragma unroll
    for (int t = 0; t < CT; t++) {
        w1r[t] = *(const unsigned*)(a.w1 + nb + t * 16 + c4);
        w2r[t] = *(const unsigned*)(a.w2 + nb + t * 16 + c4);
    }
    // staging: chunk c = tid + 64 NW n -> row (c / 4) % 64, 16-byte chunk c % 4 of K step c / 256
    v4i st[KPT];
    auto fetch = [&](int s) {
        const int r0 = s * RBM;
        const int rows = min(a.M - r0, RBM);
        const __amdgpu_buffer_rsrc_t rA =
            __builtin_amdgcn_make_buffer_rsrc((void*)(a.A + (size_t)r0 * K), (short)0, rows * K, BUF_DWORD3);
#pragma unroll
        for (int n = 0; n < KPT; n++) {
            const int c = tid + 64 * NW * n;
            st[n] = __builtin_amdgcn_raw_buffer_load_b128(rA, ((c >> 2) & 63) * K + (c & 3) * 16 + (c >> 8) * 64, 0, 0);
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int n = 0; n < KPT; n++) {
            const int c = tid + 64 * NW * n;
            *(v4i*)(As[buf] + (c >> 8) * RBM * 64 + lds64((c >> 2) & 63, c & 3)) = st[n];
        }
    };
    fetch(blockIdx.x);
    store(0);
    __syncthreads();
    int cur = 0;
    for (int s = blockIdx.x; s < nstrips; s += gridDim.x) {
        const bool more = s + (int)gridDim.x < nstrips;
        if (more) fetch(s + gridDim.x);
        v4i acc[4][CT];
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int ks = 0; ks < KS; ks++) {
                const v4i af = *(const v4i*)(As[cur] + ks * RBM * 64 + lds64(i * 16 + lr, lane >> 4));
#pragma unroll
                for (int t = 0; t < CT; t++)
                    acc[i][t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(w[t][ks], af, ks == 0 ? (v4i){0, 0, 0, 0} : acc[i][t],
                                                                      0, 0, 0);
            }
        rn_epilogue<NW, CT, FAST>(a, acc, s * RBM, w1r, w2r, red, inv_s, [&] {
            if (more) store(cur ^ 1);
        });
        __syncthreads();
        cur ^= 1;
    }
}

// ---------------------------------------------------------------------------
// Row GEMM for a few thousand rows (decode steps of a few thousand streams):
// a workgroup owns 16 rows and all d columns, so M = 4096 rows fill the 256
// CUs with no split of K (and no partial sums through HBM).  The rows' whole
// A (16 x K bytes, K <= 4096) is staged in LDS at once; each wave streams its
// CT column tiles of W (fragment-major) straight into registers WP K steps
// ahead, every W operand used by one MFMA.  The epilogue is rn_epilogue over
// one row tile.
// ---------------------------------------------------------------------------
constexpr int RN16_KMAX = 4096;
constexpr int RN16_WP = 3;  // K steps of W in flight per wave

template <int NW, int CT, bool FAST>
__global__ __launch_bounds__(64 * NW) void k_gemm_rn16(RowGemmArgs a) {
    __shared__ __attribute__((aligned(16))) int8_t As[RN16_KMAX / 64][1024];  // K step kt: [16 rows][64], lds64 rows
    __shared__ unsigned red[NW][16];
    __shared__ int inv_s[16];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, lr = lane & 15;
    const int m0 = blockIdx.x * 16;
    const int nb = wave * CT * 16;
    const int c4 = (lane >> 4) * 4;
    const int nkt = a.K / 64;
    const int arows = min(a.M - m0, 16);
    const __amdgpu_buffer_rsrc_t rA =
        __builtin_amdgcn_make_buffer_rsrc((void*)(a.A + (size_t)m0 * a.K), (short)0, arows * a.K, BUF_DWORD3);
    const __amdgpu_buffer_rsrc_t rW = __builtin_amdgcn_make_buffer_rsrc((void*)a.Wf, (short)0, a.d * a.K, BUF_DWORD3);
    const int woff = (nb >> 4) * nkt * 1024 + lane * 16;
    v4i w[RN16_WP][CT];
    auto fetch_w = [&](v4i* wr, int kt) {
#pragma unroll
        for (int t = 0; t < CT; t++) wr[t] = __builtin_amdgcn_raw_buffer_load_b128(rW, woff + t * nkt * 1024, kt * 1024, 0);
    };
#pragma unroll
    for (int p = 0; p < RN16_WP - 1; p++)
        if (p < nkt) fetch_w(w[p], p);
    // chunk c: K step c / 64, row (c / 4) % 16, 16-byte piece c % 4 (rows past M read 0)
    for (int c = tid; c < nkt * 64; c += 64 * NW) {
        const int row = (c >> 2) & 15, pc = c & 3, kt = c >> 6;
        const v4i x = __builtin_amdgcn_raw_buffer_load_b128(rA, row * a.K + kt * 64 + pc * 16, 0, 0);
        *(v4i*)(As[kt] + lds64(row, pc)) = x;
    }
    unsigned w1r[CT], w2r[CT];
#pragma unroll
    for (int t = 0; t < CT; t++) {
        w1r[t] = *(const unsigned*)(a.w1 + nb + t * 16 + c4);
        w2r[t] = *(const unsigned*)(a.w2 + nb + t * 16 + c4);
    }
    __syncthreads();
    v4i acc[1][CT];
#pragma unroll
    for (int t = 0; t < CT; t++) acc[0][t] = (v4i){0, 0, 0, 0};
    // K step kt multiplies with w[kt % WP] after requesting step kt + WP - 1
    for (int k0 = 0; k0 < nkt; k0 += RN16_WP) {
#pragma unroll
        for (int u = 0; u < RN16_WP; u++) {
            const int kt = k0 + u;
            if (kt < nkt) {
                if (kt + RN16_WP - 1 < nkt) fetch_w(w[(u + RN16_WP - 1) % RN16_WP], kt + RN16_WP - 1);
                const v4i af = *(const v4i*)(As[kt] + lds64(lr, lane >> 4));
#pragma unroll
                for (int t = 0; t < CT; t++) acc[0][t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(w[u][t], af, acc[0][t], 0, 0, 0);
            }
        }
    }
    rn_epilogue<NW, CT, FAST>(a, acc, m0, w1r, w2r, red, inv_s, [] {});
}

// ---------------------------------------------------------------------------
// Split-K row GEMM for few rows (decode with a few thousand streams): the
// workgroup (row block, K slice) multiplies its K steps and stores the int32
// partial sums; k_rn_splitk_epi then sums the slices and runs the row GEMM's
// epilogue per row.  part: [splits][M][d].
// ---------------------------------------------------------------------------
template <int NW, int CT>
__global__ __launch_bounds__(64 * NW) void k_gemm_rn_part(RowGemmArgs a, int ks_per, int32_t* __restrict__ part) {
    __shared__ __attribute__((aligned(16))) int8_t As[2][RBM * 64];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int m0 = blockIdx.x * RBM, sp = blockIdx.y;
    const int nb = wave * CT * 16;
    const int lr = lane & 15, c4 = (lane >> 4) * 4;
    const int ks0 = sp * ks_per, nks = min(ks_per, a.K / 64 - ks0);
    v4i acc[4][CT];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int t = 0; t < CT; t++) acc[i][t] = (v4i){0, 0, 0, 0};
    rowblock_mma<CT>(a.A, a.M, a.K, a.Wf, a.d, m0, nb, As, acc, ks0, nks);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int row = m0 + i * 16 + lr;
        if (row < a.M) {
#pragma unroll
            for (int t = 0; t < CT; t++)
                *(int4*)(part + ((size_t)sp * a.M + row) * a.d + nb + t * 16 + c4) =
                    make_int4(acc[i][t][0], acc[i][t][1], acc[i][t][2], acc[i][t][3]);
        }
    }
}

constexpr int RN_MAX_SPLITS = 16;

// K slices for M rows: enough (row block, slice) workgroups for the 256 CUs, at
// least two K steps per slice; 1 = no split
static int rn_splits(int M, int K) {
    const int nblk = (M + RBM - 1) / RBM;
    if (nblk >= 96) return 1;
    return std::max(1, std::min(std::min(RN_MAX_SPLITS, K / 128), (384 + nblk - 1) / nblk));
}

size_t gemm_rn_ws_bytes(int M, int d) {
    return (size_t)RN_MAX_SPLITS * (size_t)M * (size_t)d * 4u * ((M + RBM - 1) / RBM < 96 ? 1u : 0u);
}

template <int NW, int CT>
static bool try_rn_splitk(const RowGemmArgs& a, hipStream_t s) {
    const int splits = rn_splits(a.M, a.K);
    if (splits < 2 || !a.ws || (size_t)splits * a.M * a.d * 4u > a.ws_bytes) return false;
    const int ks_per = (a.K / 64 + splits - 1) / splits;
    const int used = (a.K / 64 + ks_per - 1) / ks_per;  // slices that hold K steps
    dim3 grid((unsigned)((a.M + RBM - 1) / RBM), (unsigned)used);
    hipLaunchKernelGGL((k_gemm_rn_part<NW, CT>), grid, dim3(64 * NW), 0, s, a, ks_per, a.ws);
    launch_rn_splitk_epi(a, a.ws, used, s);
    return true;
}

bool gemm_rn_supported(int d) {
    const int h = d / 64;
    return d % 64 == 0 && ((h >= 4 && h <= 8) || h == 10 || h == 12 || h == 14 || h == 16);
}

template <int NW, int CT, int KS>
static void launch_rn_ws(const RowGemmArgs& a, hipStream_t s) {
    // one workgroup per CU
    const int nstrips = (a.M + RBM - 1) / RBM;
    dim3 grid((unsigned)std::min(nstrips, 256));
    if (a.rq_fast)
        hipLaunchKernelGGL((k_gemm_rn_ws<NW, CT, KS, true>), grid, dim3(64 * NW), 0, s, a);
    else
        hipLaunchKernelGGL((k_gemm_rn_ws<NW, CT, KS, false>), grid, dim3(64 * NW), 0, s, a);
}

// few 64-row blocks but at least RN16_MIN_BLOCKS blocks of 16 rows: one
// workgroup per 16 rows, K unsplit.  From 24 blocks it beats the split-K
// kernels (d768/L12 decode groups of 1,272 and 776 streams: O projection
// 1.70 vs 2.61 s, down projection 3.58 vs 4.14 s per 8 M-token job)
constexpr int RN16_MIN_BLOCKS = 24;
static bool use_rn16(const RowGemmArgs& a) {
    const int nblk = (a.M + RBM - 1) / RBM;
    return nblk < 96 && (a.M + 15) / 16 >= RN16_MIN_BLOCKS && a.K <= RN16_KMAX;
}

template <int NW, int CT>
static void launch_rn(const RowGemmArgs& a, hipStream_t s) {
    if (use_rn16(a)) {
        // 8 waves of d / 128 tiles where that divides (else the 64-row kernel's split)
        constexpr int TILES = NW * CT;
        constexpr int NW16 = TILES % 8 == 0 && TILES / 8 <= 8 ? 8 : NW, CT16 = TILES / NW16;
        static_assert(NW16 * CT16 == NW * CT, "the 16-row kernel splits the same d columns");
        const dim3 grid((unsigned)((a.M + 15) / 16));
        if (a.rq_fast) hipLaunchKernelGGL((k_gemm_rn16<NW16, CT16, true>), grid, dim3(64 * NW16), 0, s, a);
        else hipLaunchKernelGGL((k_gemm_rn16<NW16, CT16, false>), grid, dim3(64 * NW16), 0, s, a);
        return;
    }
    if (try_rn_splitk<NW, CT>(a, s)) return;
    dim3 grid((unsigned)((a.M + RBM - 1) / RBM));
    const bool full = a.K <= 1024;
    if (a.rq_fast) {
        if (full) hipLaunchKernelGGL((k_gemm_rn<NW, CT, true, true>), grid, dim3(64 * NW), 0, s, a);
        else hipLaunchKernelGGL((k_gemm_rn<NW, CT, true, false>), grid, dim3(64 * NW), 0, s, a);
    } else {
        if (full) hipLaunchKernelGGL((k_gemm_rn<NW, CT, false, true>), grid, dim3(64 * NW), 0, s, a);
        else hipLaunchKernelGGL((k_gemm_rn<NW, CT, false, false>), grid, dim3(64 * NW), 0, s, a);
    }
}

// d = 64 h columns over NW waves of CT 16-wide tiles: 8 waves where h is even
// (few accumulators per wave, many waves to hide the W stream's latency)
void launch_gemm_rn(const RowGemmArgs& a, hipStream_t s) {
    if (!a.tiled && a.d == 384 && a.M > 0 && (long long)a.M * a.K < (1ll << 40) && !use_rn16(a)) {
        if (a.K == 384) { launch_rn_ws<8, 3, 6>(a, s); return; }
        if (a.K == 512) { launch_rn_ws<8, 3, 8>(a, s); return; }
    }
    switch (a.d / 64) {
        case 4: launch_rn<8, 2>(a, s); break;
        case 5: launch_rn<4, 5>(a, s); break;
        case 6: launch_rn<8, 3>(a, s); break;
        case 7: launch_rn<4, 7>(a, s); break;
        case 8: launch_rn<8, 4>(a, s); break;
        case 10: launch_rn<8, 5>(a, s); break;
        case 12: launch_rn<8, 6>(a, s); break;
        case 14: launch_rn<8, 7>(a, s); break;
        default: launch_rn<16, 4>(a, s); break;
    }
}

}  // namespace czip
