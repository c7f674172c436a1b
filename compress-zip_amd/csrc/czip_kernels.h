// Kernel launchers of libczip_hip (device code lives in czip_kernels.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace czip {

enum GemmEpi : int {
    EPI_RAW = 0,    // int32 accumulators (LM head logits, model.rs:477)
    EPI_REQ = 1,    // requantize to int8 (model.rs:280-300)
    EPI_QKV = 2,    // requantize + RoPE(Q, two roundings) / RoPE(K) + KV scatter
    EPI_REGLU = 3,  // requantize gate/up pairs + ReGLU (reglu.rs:20-46)
};

struct GemmArgs {
    const int8_t* A;  // [M, K] row-major, or with a_rows a table of a_nrows rows
    const uint32_t* a_rows;  // nullptr, or row r of the product reads row a_rows[r] of A (< a_nrows)
    int a_nrows;
    const int8_t* W;  // [N, K] row-major (PyTorch "TN")
    int M, N, K;
    int32_t* out32;   // EPI_RAW  [M, ldo]
    int8_t* out8;     // EPI_REQ / EPI_REGLU / Q of EPI_QKV  [M, ldo]
    int ldo;
    int mult, shift;
    double rq_scale;  // mult * 2^-shift (mult when shift <= 0), used when rq_fast
    int rq_fast;      // 1: |acc * mult| < 2^53 and |acc * rq_scale| < 2^31: requant by one f64 FMA
    // EPI_QKV
    int d, T, kv_mode, G, KH;
    int TP;           // keys per V^T block: T rounded up to a multiple of 64
    int8_t* kc;       // [B, KH, T, 64]   rotated keys
    int8_t* vc;       // [B, KH, TP * 64] values, transposed in blocks of 2^vl keys (vt_off)
    int vl = 4;       // V^T block exponent: 4 for the prefill caches, 2 for the decode caches
    int pos;          // >= 0: every row is at this position and row = chunk (decode step)
    const int16_t* rcos;
    const int16_t* rsin;
    int tiled;        // 1: the tiled kernel only (no W-stationary one; a per-context test switch)
};

// The attention's exp table by table step t (exp_q16, lut.rs:213-235):
// E(t) = max(1, ((lut[t % 256] << 16 >> (t / 256)) + 2^15) >> 16) for
// t < 4096, and entry 4096 stands for every larger step (a shift by 16 or more
// leaves at most 1, which the clamp makes 1).  Entries hold E ^ 0x8080: the two
// bytes of E each offset by 128, i.e. the signed byte pair (hi, lo) of
// E - 32896 = 256 hi + lo that the PV products take.
constexpr int ETB_N = 4097;    // entries used
constexpr int ETB_PAD = 4104;  // entries allocated (whole 16-byte pieces)
inline void attn_etab_host(const uint16_t* lut, uint16_t* out) {
    for (int t = 0; t < ETB_PAD; t++) {
        unsigned e = 1;
        if (t < 4096) {
            const unsigned x = ((((unsigned)lut[t & 255]) << 16 >> (t >> 8)) + 0x8000u) >> 16;
            e = x < 1u ? 1u : x;
        }
        out[t] = (uint16_t)(e ^ 0x8080u);
    }
}

struct AttnArgs {
    const int8_t* q;          // [M, H*64]  rotated + NET_SHIFT-ed queries
    const int8_t* kc;         // [B, KH, T, 64]
    const int8_t* vc;         // [B, KH, TP * 64] values transposed in blocks of keys (vt_off): 16 keys
                              // for the prefill kernel, 4 for the decode kernel (caches a decode step appends to)
    int TP;
    const int32_t* lens;      // [B]
    const int32_t* score_mult;// [H]
    const int8_t* sink;       // [64] or nullptr
    const uint16_t* lut;      // [256]
    const uint16_t* etab;     // [ETB_PAD]: E(t) ^ 0x8080 by table step t (attn_etab_host)
    int8_t* out;              // [M, H*64]
    int M, T, H, G, KH, kv_mode;
    unsigned coef;
    int general;              // 1: scores may reach 2^30 or lut[0] != 65535 (wrapping score differences)
    int B;                    // chunks of the launch (set by launch_attention)
};

// GEMM over full rows (N = d) with the residual + RMSNorm epilogue
// (model.rs:424-439 after the output projection, 459-468 + 384-385 / 473-474
// after the down projection):
//   y = requant(A W^T); x = x_in + rmsnorm(y, w1); xn = rmsnorm(clamp(x), w2)
struct RowGemmArgs {
    const int8_t* A;      // [M, K]
    const int8_t* W;      // [d, K]
    const int8_t* Wf;     // the same, fragment-major (rowblock_mma)
    int M, K, d;
    int mult, shift;
    double rq_scale;
    int rq_fast;
    const int8_t* w1;      // norm of the projection output
    const int8_t* w2;      // norm of the clamped residual
    const int16_t* x_in;   // residual stream [M, d]; nullptr: the embedding rows of tok
    const uint32_t* tok;
    const int8_t* embed;
    int16_t* x_out;        // [M, d] or nullptr (not needed after the last layer)
    int8_t* xn;            // [M, d]
    int32_t* ws;           // optional workspace of ws_bytes for the split-K path (few rows)
    size_t ws_bytes;
    int tiled;             // 1: the tiled row kernel only (no W-stationary one; a per-context test switch)
};
bool gemm_rn_supported(int d);
// bytes of workspace the split-K row GEMM wants for M rows of width d (0: M is large enough without)
size_t gemm_rn_ws_bytes(int M, int d);
void launch_rn_splitk_epi(const RowGemmArgs& a, const int32_t* part, int splits, hipStream_t s);
void launch_gemm_rn(const RowGemmArgs& a, hipStream_t s);

// The FFN of one layer in one kernel (model.rs:438-468 from the pre-FFN norm's
// output): xn_out = rmsnorm(clamp(x), w2) with x = x_in + rmsnorm(requant(
// reglu(requant(xn W_up^T)) W_down^T), w1); the ReGLU output stays on chip.
struct FfnArgs {
    const int8_t* xn;       // [M, d] input rows (may alias xn_out: a strip is read before it is written)
    const int8_t* Wup;      // [2F, d] fragment-major, tile 2g = gate rows 16g.., tile 2g + 1 = the matching up rows
    const int8_t* Wdf;      // [d, F] fragment-major
    int M, d, F;
    int up_mult, up_shift, up_fast;
    double up_scale;
    int dn_mult, dn_shift, dn_fast;
    double dn_scale;
    const int8_t* w1;       // post-FFN norm
    const int8_t* w2;       // the next pre-norm (or the final norm)
    const int16_t* x_in;    // [M, d] residual stream
    int16_t* x_out;         // [M, d] or nullptr (after the last layer)
    int8_t* xn_out;         // [M, d]
};
bool ffn_supported(int d, int F);
void launch_ffn(const FfnArgs& a, hipStream_t s);

// LM head + logits -> (cum_lo, cum_hi) of each row's target (k_cdf mode 0)
// without the int32 logits leaving the chip; V = 1024.
struct HeadCdfArgs {
    const int8_t* A;           // [M, K] final-normalized rows
    const int8_t* W;           // [V, K] head weights, fragment-major (rowblock_mma)
    int M, K, V;
    const uint32_t* targets;   // [M]
    const int32_t* lens;       // [M / T]
    int T;
    const uint16_t* lut;       // [256]
    unsigned coef, total;
    int e0;                    // 1: lut[0] == 65535, so E at table step 0 is the max's E(0) (head_freqs)
    uint32_t* out;             // [., 2]
    long long out_row0;
};
bool head_cdf_supported(int V);
void launch_head_cdf(const HeadCdfArgs& a, hipStream_t s);

// Layer 0's Q/K/V from a per-token table: tab[v] = the requantized QKV
// projection of token v's normalized embedding (before RoPE); per row: RoPE
// on Q (two roundings) and K, scatter of K and V into the caches (the QKV
// GEMM's epilogue, attention.rs:29-83).
struct QkvTabArgs {
    const int8_t* tab;       // [vocab, qkv_n]: Q heads | K heads | V heads
    const uint32_t* tok;     // [M]
    int M, T, TP, pos;       // pos >= 0: every row at pos, row = stream (decode)
    int H, NG, KH, d, qkv_n; // NG = KV heads in the table
    const int16_t* rcos;
    const int16_t* rsin;
    int8_t* q8;              // [M, d]
    int8_t* kc;              // [B, KH, T, 64]
    int8_t* vc;              // [B, KH, TP * 64] values transposed in blocks of 2^vl keys (vt_off)
    int vl = 4;
    double inv_per_row = 0.0;  // 1 / (8 H + 24 NG), set by launch_qkv_table (the per-step kernel)
};
void launch_qkv_table(const QkvTabArgs& a, hipStream_t s);

void launch_prep_chunks(const uint32_t* toks, int64_t n_tokens, int64_t chunk0, int nb, int T,
                        uint32_t* inp, uint32_t* tgt, int32_t* lens, hipStream_t s);
// x may be nullptr (the residual stream is re-read from the embedding rows)
void launch_embed_norm(const uint32_t* inp, const int8_t* embed, const int8_t* w, int M, int d,
                       int16_t* x, int8_t* xn, hipStream_t s);
void launch_resid_norm(int16_t* x, const int8_t* y8, const int8_t* w1, const int8_t* w2, int M, int d,
                       int8_t* xn, hipStream_t s);
void launch_gemm(const GemmArgs& a, int epi, hipStream_t s);
void launch_attention(const AttnArgs& a, int B, hipStream_t s);
// mode 0: (lo, hi) of targets; mode 1: full inclusive cumfreqs; mode 2:
// targets are decoder values, out rows (sym, cum_lo, cum_hi).  Row r of the
// launch is written at output row out_row0 + r.
void launch_cdf(const int32_t* logits, int M, int V, const uint32_t* targets, const int32_t* lens, int T,
                const uint16_t* lut, unsigned coef, unsigned total, int mode, uint32_t* out, int64_t out_row0,
                hipStream_t s);
// [B, T] coder targets -> prefill inputs / targets, clamped lens, zeroed
// intervals, and *err = 1 if a live target is >= V (err cleared first)
void launch_prep_rows(const uint32_t* targets, const int32_t* lens_in, int B, int T, int V, uint32_t* inp,
                      uint32_t* tgt, int32_t* lens, uint32_t* out, int32_t* err, hipStream_t s);
// chunk c's lens[c] bytes from src + c * slot to dst + offs[c]
void launch_pack_chunks(const uint8_t* src, int64_t slot, const int32_t* lens, const int64_t* offs, int n,
                        uint8_t* dst, hipStream_t s);
void launch_encode(const uint32_t* lohi, const int32_t* lens, int nb, int T, unsigned total, uint8_t* out,
                   int64_t slot, int32_t* out_lens, int32_t* err, hipStream_t s);

// ---- batched decode (decompression) ----
struct DecState {        // one arithmetic decoder per stream (arith_coder.rs:139-164)
    uint32_t* low;
    uint32_t* high;
    uint32_t* code;
    int64_t* byte_pos;
    int32_t* bit_pos;
    uint32_t* pend_lo = nullptr;  // the last decoded symbol's interval [lo, hi) (fused head),
    uint32_t* pend_hi = nullptr;  // applied to the decoder by the next step's input kernel
};
struct DecStreams {      // per stream of the current group
    const uint8_t* data;      // all chunk bytes
    const int64_t* offs;      // [S] byte offset of the stream's chunk
    const int32_t* blen;      // [S] byte length
    const int32_t* ntok;      // [S] tokens to decode
    uint32_t* tokens;         // all decoded tokens
    const int64_t* tok_offs;  // [S] output offset of the stream's tokens
};
void launch_dec_init(DecState st, DecStreams ds, int S, hipStream_t s);
// inputs of step p: BOS at p = 0, else the token decoded at p - 1; rows past ntok get 0.
// upd: first apply the pending decoder step of step p - 1's symbol (the fused head's
// interval in st.pend_lo / pend_hi); total = the frequency total
void launch_dec_prep(DecStreams ds, DecState st, int S, int p, bool upd, unsigned total, uint32_t* inp, hipStream_t s);
// one query per (stream, head) at position p over cached keys 0..p
void launch_attn_decode(const AttnArgs& a, int S, int p, hipStream_t s);
// logits -> cumulative frequencies -> one arithmetic-decode step (arith_coder.rs:195-264)
void launch_cdf_decode(const int32_t* logits, int S, int V, const uint16_t* lut, unsigned coef, unsigned total,
                       int p, DecState st, DecStreams ds, hipStream_t s);
// LM head + frequency table + symbol search + decoder step of S streams in one
// kernel (head_cdf_supported(V)); A = the final-normalized rows [S, K]
struct HeadDecArgs {
    const int8_t* A;
    const int8_t* W;           // [V, K], fragment-major (rowblock_mma)
    int M, K, V;
    const uint16_t* lut;       // [256]
    unsigned coef, total;
    int e0;                    // as HeadCdfArgs::e0
    int p;                     // step
};
void launch_head_dec(const HeadDecArgs& a, DecState st, DecStreams ds, hipStream_t s);

}  // namespace czip
