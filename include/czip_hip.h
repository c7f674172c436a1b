/*
 * czip_hip.h -- C-ABI of the MI355X (gfx950) integer-transformer path of
 * compress-zip: batched causal prefill -> quantized CDF -> arithmetic coding
 * (compress), and batched multi-stream decode (decompress).
 *
 * Plain C types only; no exceptions or aborts cross this boundary.  Every
 * entry point returns czip_status (0 = OK, negative = error class) and leaves
 * a message retrievable with czip_last_error().  A context owns one HIP
 * stream and all device memory it allocates; it is not thread-safe, but
 * several contexts may coexist (one per host thread / device).
 *
 * The reference has no FFI; each entry point names the Rust API it stands in
 * for (file:line in the reference crate, rust/src).
 */
#ifndef CZIP_HIP_H
#define CZIP_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef int32_t czip_status;
#define CZIP_OK            0
#define CZIP_E_ARG        -1  /* bad argument / null pointer / bad sizes        */
#define CZIP_E_CONFIG     -2  /* unsupported model shape (head_dim != 64, ...)  */
#define CZIP_E_HEADS      -3  /* n_heads not in {4,6,8} in rust-compat KV mode  */
                              /*   (the panic of rust/src/attention.rs:172)     */
#define CZIP_E_RANGE      -4  /* position past the RoPE LUT / KV cache          */
                              /*   (the index panics of lut.rs:169-177)         */
#define CZIP_E_TOKEN      -5  /* token id >= vocab                              */
#define CZIP_E_OVERFLOW   -6  /* coded chunk larger than its output slot        */
#define CZIP_E_HIP        -7  /* HIP runtime failure                            */
#define CZIP_E_IO         -8  /* file open/read/parse failure                   */
#define CZIP_E_MISSING    -9  /* required tensor absent (model.rs:152-154)      */
#define CZIP_E_NOMEM     -10  /* device or host allocation failed               */
#define CZIP_E_FORMAT    -11  /* malformed container / LUT size mismatch        */

/* KV-cache semantics.  RUST_COMPAT reproduces gqa_attention_mqa_i8
 * (rust/src/attention.rs:162-289): one cached head, K = the first kv head's
 * K slice and V = the next 64 values of the QKV row.  GQA is the extension
 * where query head h reads kv head floor(h*G/H) with its own K and V. */
#define CZIP_KV_RUST_COMPAT 0
#define CZIP_KV_GQA         1

/* Host pointers to one layer's tensors (rust/src/model.rs:52-83). */
typedef struct czip_layer_desc {
    const int8_t*  attn_norm;       /* [d]          */
    const int8_t*  post_attn_norm;  /* [d]          */
    const int8_t*  ffn_norm;        /* [d]          */
    const int8_t*  post_ffn_norm;   /* [d]          */
    const int8_t*  qkv_w;           /* [d+2*G*64,d] */
    const int8_t*  out_w;           /* [d,d]        */
    const int8_t*  up_w;            /* [2F,d] gate rows then up rows */
    const int8_t*  down_w;          /* [d,F]        */
    const int32_t* score_mult;      /* [H]          */
    const int8_t*  sink_key;        /* [64] or NULL */
    int32_t qkv_mult, out_mult, up_mult, down_mult;
    int32_t qkv_shift, out_shift, up_shift, down_shift;
} czip_layer_desc;

/* Host pointers + config of a whole model (rust/src/model.rs:19-48, 86-104). */
typedef struct czip_model_desc {
    int32_t vocab, n_layers, n_heads, n_kv_heads, d_model, d_ff, head_dim;
    int32_t max_seq_len, context_length, kv_mode;
    const int8_t*   embed;          /* [V,d]  */
    const int8_t*   final_norm;     /* [d]    */
    const int8_t*   head_w;         /* [V,d]  */
    const uint16_t* exp2_lut;       /* [256]  */
    const int16_t*  rope_cos;       /* [context_length,32] */
    const int16_t*  rope_sin;       /* [context_length,32] */
    uint32_t coef_q24, target_total;
    const czip_layer_desc* layers;  /* [n_layers] */
    int64_t exp2_len;               /* entries of exp2_lut (must be 256)            */
    int64_t rope_len;               /* entries of each RoPE table (context_length*32) */
} czip_model_desc;

typedef struct czip_model czip_model;   /* host-side loaded .czm file     */
typedef struct czip_ctx   czip_ctx;     /* device-side weights + stream   */
typedef struct czip_job   czip_job;     /* device buffers of one workload */

/* ---- host loader: replaces ModelWeights::load (rust/src/model.rs:108-274,
 *      rust/src/safetensors.rs:287-376).  Metadata defaults follow
 *      model.rs:113-145, scalar defaults model.rs:157-168. ---- */
czip_status czip_model_load(const char* path, int32_t kv_mode, czip_model** out);
const czip_model_desc* czip_model_desc_get(const czip_model* m);
/* Embedded tokenizer bytes (tensor "tokenizer.data"), NULL if absent. */
const uint8_t* czip_model_tokenizer(const czip_model* m, size_t* len, const char** codec);
void czip_model_free(czip_model* m);

/* ---- device context: replaces Model::new (rust/src/model.rs:315-351).
 *      Validates LUT sizes (model.rs:324-333) and head constraints
 *      (attention.rs:172).  Weights are copied; the caller keeps ownership. ---- */
czip_status czip_create(const czip_model_desc* w, int device, czip_ctx** out);
void        czip_destroy(czip_ctx* ctx);
const char* czip_last_error(const czip_ctx* ctx);   /* never NULL */
int         czip_device_count(void);

/* ---- debug / parity: logits of B chunks of T tokens (Model::forward,
 *      rust/src/model.rs:362-480, called at positions 0..lens[b]-1 with
 *      inputs[b*T + p]).  logits: host [B*T, V]; rows p >= lens[b] are 0. ---- */
czip_status czip_forward_logits(czip_ctx* ctx, const uint32_t* inputs, const int32_t* lens,
                                int32_t B, int32_t T, int32_t* logits);

/* ---- compress, per-token CDF only: for each chunk b and position p <
 *      lens[b], the coder interval of targets[b*T+p] under the CDF that
 *      Model::get_cumfreqs (model.rs:483-486, softmax_cdf.rs:85-139) builds
 *      from forward(prev, p) with prev = 1022 at p = 0 (main.rs:220-226).
 *      cum_lohi: host [B*T, 2] = (cum[tok-1] or 0, cum[tok]); the total is
 *      the model's target_total.  This is what a Rust caller binds when it
 *      keeps its own ArithEncoder (arith_coder.rs:80-98). ---- */
czip_status czip_prefill_cdf(czip_ctx* ctx, const uint32_t* targets, const int32_t* lens,
                             int32_t B, int32_t T, uint32_t* cum_lohi);

/* ---- czip_prefill_cdf without allocation.  No counterpart in the
 *      reference: this is for callers that cannot allocate device memory
 *      (tight serving loops, harnesses that forbid hipMalloc).  It runs
 *      eagerly and synchronizes, so it cannot itself be captured into a HIP
 *      graph.  The same (cum_lo, cum_hi) as czip_prefill_cdf, but
 *      targets [B*T], lens [B] and cum_lohi [B*T, 2] are DEVICE pointers on
 *      the context's device (4-, 4- and 8-byte aligned, as hipMalloc
 *      memory is), and every intermediate lives in one fixed
 *      device buffer of CZIP_NOALLOC_SCRATCH_BYTES per GPU (held from the
 *      library's load until the process ends): no hipMalloc / hipFree.
 *      B * T rows that need more than that give CZIP_E_RANGE (the shipped
 *      model needs ~3.5 KB per row: about 19K rows, e.g. 37 chunks of 512).
 *      lens are clamped to [0, T]; rows past a chunk's length come back 0; a
 *      target >= vocab in a live row gives CZIP_E_TOKEN.  Synchronous: the
 *      call first waits for all work queued on the device (its own stream
 *      does not wait for the caller's), so inputs written asynchronously on
 *      any stream before the call are complete when it reads them.  All
 *      calls on one GPU share its buffer, so calls that overlap in time on
 *      one GPU (several contexts or host threads) race. ---- */
#define CZIP_NOALLOC_SCRATCH_BYTES (64ull << 20)
czip_status czip_prefill_cdf_noalloc(czip_ctx* ctx, const uint32_t* d_targets, const int32_t* d_lens,
                                     int32_t B, int32_t T, uint32_t* d_cum_lohi);

/* Full cumulative tables (debug / parity), host [B*T, V]. */
czip_status czip_prefill_cumfreqs(czip_ctx* ctx, const uint32_t* inputs, const int32_t* lens,
                                  int32_t B, int32_t T, uint32_t* cumfreqs);

/* ---- compress end to end on the device: the rayon chunk loop of
 *      main.rs:206-238 (fresh model per chunk, BOS=1022, pos restarts at 0,
 *      encoder.finish per chunk) with forward, CDF and arithmetic coding all
 *      on the GPU.  Chunk c covers tokens[c*chunk .. min((c+1)*chunk, n)). ---- */
czip_status czip_compress_plan(czip_ctx* ctx, const uint32_t* tokens, int64_t n_tokens,
                               int32_t chunk, czip_job** job);
czip_status czip_job_run(czip_job* job);          /* device work only, synchronous */
int64_t     czip_job_chunks(const czip_job* job);
/* Coded bytes of every chunk into out[c*slot ..], lengths into lens[c]. */
czip_status czip_compress_fetch(czip_job* job, uint8_t* out, int64_t slot, int32_t* lens);
/* The coded bytes of every chunk back to back, chunk c at out[offs[c] ..
 * offs[c+1]) (nchunks + 1 offsets): the chunk data of the container, as
 * czip_container_pack takes it.  Only the coded bytes leave the device.
 * out == NULL fills offs only (offs[nchunks] = the bytes needed); a cap
 * below that gives CZIP_E_OVERFLOW.  (The same bytes as czip_compress_fetch,
 * which keeps the reference's one-Vec-per-chunk shape, main.rs:206-238.) */
czip_status czip_compress_fetch_packed(czip_job* job, uint8_t* out, int64_t cap, int64_t* offs);
void        czip_job_free(czip_job* job);
/* Upper bound of one chunk's coded size for `chunk` tokens. */
int64_t     czip_chunk_slot_bytes(int32_t chunk);

/* ---- decompress end to end on the device: the chunk loop of
 *      main.rs:377-396 (ArithDecoder per chunk, arith_coder.rs:153-264) run
 *      as batched autoregressive decode, one token per stream per step. ---- */
czip_status czip_decompress_plan(czip_ctx* ctx, const uint8_t* data, const int64_t* offs,
                                 const int32_t* lens, const int32_t* ntoks, int32_t nchunks,
                                 czip_job** job);
czip_status czip_decompress_fetch(czip_job* job, uint32_t* tokens_out, const int64_t* tok_offs);

/* ---- step-wise decode, for a caller that keeps its own ArithDecoder
 *      (arith_coder.rs:139-264): one call replaces, for S streams at once,
 *      the body of the per-token loop of main.rs:381-391,
 *        logits = model.forward(prev_token, pos);            (model.rs:362-480)
 *        cumfreqs = model.get_cumfreqs(&logits);             (model.rs:483-486)
 *        token = decoder.decode_symbol(&cumfreqs);           (arith_coder.rs:195-222)
 *      up to the decoder's own interval update and renormalisation.
 *      czip_decode_begin replaces Model::new + reset per stream (model.rs:315-357):
 *      it opens the context's decode session for S streams of at most T tokens
 *      (a KV cache per stream; an open session is replaced).
 *      czip_decode_step runs forward at position pos[s] on token tok_in[s] for
 *      every stream s (the BOS 1022 at position 0, main.rs:387).  Every active
 *      stream must be at the same position p (streams advance in lockstep; a new
 *      chunk restarts all of them at 0); pos[s] = -1 marks a stream with nothing
 *      to decode, whose output row is zero.
 *        value_or_null == NULL: out is [S, V], the inclusive cumulative
 *          frequencies get_cumfreqs returns (softmax_cdf.rs:85-139);
 *        else value_or_null[s] is the stream's decoder value
 *          ((code - low + 1) * total - 1) / range (arith_coder.rs:199-203) and
 *          out is [S, 3] = (symbol, cum_lo, cum_hi): the first symbol whose
 *          cumulative frequency exceeds the value, clamped to V - 1
 *          (bisect_cumfreqs, arith_coder.rs:225-241), cum_lo = cumfreqs[sym-1]
 *          (0 for sym 0) and cum_hi = cumfreqs[sym]; the caller then narrows and
 *          renormalises its decoder (arith_coder.rs:212-219) and feeds the
 *          symbol back as the next tok_in.
 *      czip_decode_end releases the session (czip_destroy does too). ---- */
czip_status czip_decode_begin(czip_ctx* ctx, int32_t S, int32_t T);
czip_status czip_decode_step(czip_ctx* ctx, const uint32_t* tok_in, const int32_t* pos,
                             const uint32_t* value_or_null, uint32_t* out);
void        czip_decode_end(czip_ctx* ctx);

/* ---- tokenizer (host): the BPE of the text configurations.
 *      czip_tokenizer_load replaces load_tiktoken_json_from_bytes
 *      (rust/src/tiktoken.rs:536-563); czip_tokenizer_from_model decompresses
 *      the model's embedded JSON like main.rs:88-109 (system libzstd /
 *      libbrotlidec).  czip_tokenize = encode_with_special_tokens
 *      (tiktoken.rs:215-269, 498-501) over UTF-8 text (CZIP_E_FORMAT if not
 *      valid UTF-8); `threads` > 1 splits the text at points where no pattern
 *      match can straddle, with identical output.  A text of `len` bytes never
 *      yields more than `len` tokens.  czip_detokenize = decode_bytes
 *      (tiktoken.rs:186-198).  *n_out receives the required count; a too small
 *      `cap` gives CZIP_E_OVERFLOW. ---- */
typedef struct czip_tokenizer czip_tokenizer;
czip_status czip_tokenizer_load(const char* json, size_t len, czip_tokenizer** out);
czip_status czip_tokenizer_from_model(const czip_model* m, czip_tokenizer** out);
void        czip_tokenizer_free(czip_tokenizer* t);
czip_status czip_tokenize(const czip_tokenizer* t, const char* text, size_t len, int32_t threads,
                          uint32_t* out, size_t cap, size_t* n_out);
czip_status czip_detokenize(const czip_tokenizer* t, const uint32_t* ids, size_t n, uint8_t* out,
                            size_t cap, size_t* n_out);

/* ---- CZIPv1 container (host): the .czip file of main.rs:241-279 / 339-361,
 *      laid out by rust/src/file_format.rs.  A file is the 16-byte outer header
 *      ("CZIPv1", flags, codec, uncompressed_len = input text bytes, header_len
 *      = inner header bytes), then the outer codec's stream of the payload:
 *      inner header (model_id_hash, chunk_count, last_chunk_tokens,
 *      tokenizer_id, context_length_log2, one u16 byte length per chunk) and
 *      the chunk bytes.  Codecs as main.rs: zstd level 22 or brotli quality 11,
 *      window 22 (system libzstd / libbrotlienc / libbrotlidec).
 *      czip_container_pack replaces CompressedFile::to_bytes_uncompressed plus
 *      the codec (file_format.rs:385-392, main.rs:255-279): chunks holds the
 *      chunk bytes back to back, chunk i at [offs[i], offs[i+1]) (chunk_count + 1
 *      offsets); a chunk over 65535 bytes gives CZIP_E_OVERFLOW (file_format.rs:311).
 *      czip_container_unpack replaces main.rs:332-361 + read_from_decompressed
 *      (file_format.rs:355-382): malformed input gives CZIP_E_FORMAT; *chunks and
 *      *offs are allocated by the library (release with czip_buffer_free).
 *      czip_model_id_hash = hash_model_path (main.rs:79-85): the first 8 hex
 *      digits of MD5(path). ---- */
#define CZIP_CODEC_ZSTD   0
#define CZIP_CODEC_BROTLI 1
typedef struct czip_container {
    uint8_t  flags;               /* bit 0: multifile (file_format.rs:69-73)  */
    uint8_t  codec;               /* CZIP_CODEC_ZSTD or CZIP_CODEC_BROTLI      */
    uint32_t uncompressed_len;    /* input text bytes                          */
    uint32_t model_id_hash;
    uint32_t chunk_count;
    uint16_t last_chunk_tokens;
    uint8_t  tokenizer_id;
    uint8_t  context_length_log2; /* tokens per chunk = 1 << log2 (0 reads as 6) */
} czip_container;
uint32_t    czip_model_id_hash(const char* path, size_t len);
czip_status czip_container_pack(const czip_container* info, const uint8_t* chunks, const int64_t* offs,
                                uint8_t** out, size_t* out_len);
czip_status czip_container_unpack(const uint8_t* data, size_t len, czip_container* info, uint8_t** chunks,
                                  int64_t** offs);
void        czip_buffer_free(void* p);

/* ---- instrumentation: per-kernel HIP-event timing on the context stream. ---- */
void        czip_set_profiling(czip_ctx* ctx, int32_t on);
/* Kernel names: "prep","embed_norm","gemm_qkv","attention","gemm_o_norm",
 * "gemm_up","gemm_down_norm","head_cdf","encode"; where a fused kernel has no
 * instance for the model shape: "gemm_o","gemm_down","row_norm","gemm_head",
 * "cdf"; decode: "dec_init","dec_prep","attn_decode","head_dec" (or, unfused,
 * "gemm_head","cdf_decode"). */
czip_status czip_kernel_stats(czip_ctx* ctx, const char* name, int64_t* launches, double* total_ms);
void        czip_reset_stats(czip_ctx* ctx);

#ifdef __cplusplus
}
#endif
#endif
