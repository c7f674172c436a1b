/*
 * czip_oracle.h -- CPU oracle for the compress-zip integer transformer path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a plain-C restatement of the reference
 * Rust crate (the modules under rust/src), written loop-for-loop so that it can serve as
 * the parity checker for the HIP path and as the same-box CPU baseline.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it; the product library never links or calls it.
 *
 * Every function cites the reference file:line it restates.  Rust `--release`
 * semantics are reproduced exactly, including i32 wrap-around where the
 * reference relies on it (attention vacc, rust/src/attention.rs:208,274).
 */
#ifndef CZIP_ORACLE_H
#define CZIP_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- primitives (rust/src/primitives.rs) ---- */
int8_t   orc_clamp_i8(int32_t x);
int32_t  orc_sra_rne_s32(int32_t v, uint32_t sh);
int32_t  orc_sra_rne_s64_to_s32(int64_t v, uint32_t sh);
uint32_t orc_udiv_rne_u32(uint32_t n, uint32_t d);
int32_t  orc_div_rne_s32(int32_t num, int32_t denom);
int32_t  orc_div_rne_s32_by_u64(int32_t num, uint64_t denom);
uint32_t orc_isqrt32(uint32_t x);
size_t   orc_argmax(const int32_t* a, size_t n);

/* ---- LUT exp (rust/src/lut.rs, rust/src/softmax_cdf.rs) ---- */
int32_t  orc_exp_q16_from_neg_fixed(int32_t neg_x_q8, const uint16_t* lut);
uint16_t orc_exp_q16_coef(int32_t diff, const uint16_t* lut, uint32_t coef_q24);
uint32_t orc_attn_coef_q24(void);
uint32_t orc_cdf_coef_q24(void);
uint32_t orc_target_total(uint32_t vocab);
void     orc_gen_exp2_lut(uint16_t* out256);
void     orc_gen_rope_lut(double theta, int max_seq, int16_t* cos_out, int16_t* sin_out);

/* ---- ops (rmsnorm.rs, linear.rs, reglu.rs, model.rs, attention.rs) ---- */
int32_t  orc_inv_rms_q15(int32_t mean_sq);
void     orc_rmsnorm_i8_to_i8(const int8_t* x, const int8_t* w, int d, int32_t eps, int8_t* out);
void     orc_linear_i8_to_i32(const int8_t* x, const int8_t* w, int b, int in_dim, int out_dim, int32_t* out);
void     orc_requant(const int32_t* x, int n, int32_t mult, int8_t shift, int8_t* out);
void     orc_reglu(const int8_t* x, int d_ff, int8_t* out);
void     orc_rope_k(int8_t* x64, const int16_t* cos_row, const int16_t* sin_row);
void     orc_rope_q(int8_t* x64, const int16_t* cos_row, const int16_t* sin_row);

/* One query head's attention over keys 0..n_keys-1 (attention.rs:197-285):
 * q_rot already rotated, k/v [n_keys, 64] rows, ATTN_COEF_Q24 exp.  The final
 * i32 vacc and u64 S go to vacc_out/s_out when not NULL. */
void     orc_attend_head(const int8_t* q_rot, const int8_t* k, const int8_t* v, int n_keys, int32_t score_mult,
                         const int8_t* sink, const uint16_t* lut, int8_t* out, int32_t* vacc_out, uint64_t* s_out);
/* Count of vacc additions that wrapped the i32 range since the last reset
 * (instrumentation: every attention row of orc_forward and orc_attend_head). */
int64_t  orc_vacc_wraps(void);
void     orc_vacc_wraps_reset(void);

/* ---- softmax -> cumulative frequencies (softmax_cdf.rs:85-139) ---- */
void     orc_build_cumfreqs(const int32_t* logits, int v, const uint16_t* lut, uint32_t coef_q24,
                            uint32_t target_total, uint32_t* cum_out);

/* ---- model ---- */
enum { ORC_KV_RUST_COMPAT = 0, ORC_KV_GQA = 1 };

typedef struct {
    const int8_t*  attn_norm;
    const int8_t*  post_attn_norm;
    const int8_t*  ffn_norm;
    const int8_t*  post_ffn_norm;
    const int8_t*  qkv_w;     /* [d + 2*G*64, d] */
    const int8_t*  out_w;     /* [d, d] */
    const int8_t*  up_w;      /* [2F, d] */
    const int8_t*  down_w;    /* [d, F] */
    const int32_t* score_mult;/* [H] */
    const int8_t*  sink_key;  /* [64] or NULL */
    int32_t qkv_mult, out_mult, up_mult, down_mult;
    int32_t qkv_shift, out_shift, up_shift, down_shift;
} orc_layer;

typedef struct {
    int32_t vocab, n_layers, n_heads, n_kv_heads, d_model, d_ff, head_dim;
    int32_t max_seq_len, context_length, kv_mode;
    const int8_t*   embed;       /* [V, d] */
    const int8_t*   final_norm;  /* [d] */
    const int8_t*   head_w;      /* [V, d] */
    const uint16_t* exp2_lut;    /* [256] */
    const int16_t*  rope_cos;    /* [context_length, 32] */
    const int16_t*  rope_sin;
    uint32_t coef_q24, target_total;
    const orc_layer* layers;     /* [n_layers] */
} orc_model;

/* Per-sequence state: KV cache for every layer (rust/src/attention.rs:101-146). */
typedef struct orc_state orc_state;
orc_state* orc_state_new(const orc_model* m);
void       orc_state_free(orc_state* s);
void       orc_state_reset(orc_state* s);
/* Model::forward (model.rs:362-480).  Returns 0 on success, <0 on error
 * (position out of LUT/cache range, unsupported head count). */
int        orc_forward(orc_state* s, uint32_t token, int pos, int32_t* logits_out);
/* Validate the configuration the way the reference would (panics become codes). */
int        orc_model_check(const orc_model* m);

/* ---- arithmetic coder (arith_coder.rs) ---- */
typedef struct {
    uint64_t low, high;
    uint32_t underflow;
    uint8_t* out; size_t len, cap;
    uint8_t  cur; int32_t bit_pos;
} orc_encoder;
void orc_enc_init(orc_encoder* e);
void orc_enc_free(orc_encoder* e);
void orc_enc_encode(orc_encoder* e, const uint32_t* cum, int v, int sym);
void orc_enc_encode_range(orc_encoder* e, uint64_t lo, uint64_t hi, uint64_t total);
void orc_enc_finish(orc_encoder* e);

typedef struct {
    uint64_t low, high, code;
    const uint8_t* in; size_t len, byte_pos; int32_t bit_pos;
} orc_decoder;
void orc_dec_init(orc_decoder* d, const uint8_t* in, size_t len);
int  orc_dec_decode(orc_decoder* d, const uint32_t* cum, int v);

/* ---- chunk driver (main.rs:186-238, 371-396) ---- */
/* Compress one chunk: input tokens [n]; writes coded bytes (malloc'd) */
int orc_compress_chunk(const orc_model* m, const uint32_t* toks, int n, uint8_t** out, size_t* out_len);
int orc_decompress_chunk(const orc_model* m, const uint8_t* in, size_t len, int n, uint32_t* toks_out);
/* Many chunks on `threads` worker threads (rayon over chunks, main.rs:206-238).
 * Chunk c covers toks[c*chunk .. min((c+1)*chunk, n)).  out_buf has slot_bytes
 * per chunk; out_lens[c] receives the coded length.  clone_weights != 0 copies
 * the weights per chunk like Model::new(weights.clone()) (main.rs:215). */
int orc_compress_many(const orc_model* m, const uint32_t* toks, int64_t n, int chunk, int threads,
                      int clone_weights, uint8_t* out_buf, int64_t slot_bytes, int32_t* out_lens);
int orc_decompress_many(const orc_model* m, const uint8_t* bufs, const int64_t* offs,
                        const int32_t* lens, const int32_t* ntoks, int nchunks, int threads,
                        uint32_t* toks_out, const int64_t* tok_offs);

/* Per-token logits + cumfreqs of one chunk (test helper). */
int orc_chunk_trace(const orc_model* m, const uint32_t* inputs, int n, int32_t* logits_out,
                    uint32_t* cum_out);

#ifdef __cplusplus
}
#endif
#endif
