// C-ABI implementation of libczip_hip: model loading, device context,
// batched prefill / CDF / coding jobs.  See include/czip_hip.h.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cmath>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "czip_internal.h"
#include "czip_kernels.h"

using namespace czip;

namespace {

constexpr uint32_t BOS = 1022u;  // main.rs:222, 387
constexpr int FFN_MIN_ROWS = 1 << 19;  // rows from which a layer's FFN runs as one fused kernel
// device memory a job may use beyond its inputs and outputs (CZIP_SCRATCH_GB):
// a compress sub-batch, or a decode group's caches.  64 GB of the 288 GB holds
// the caches of 2,048 streams of 4,096 tokens of the d768/L12 GQA model (51.5
// GB) as one decode group (0.377 M tok/s, against 0.289 as the two groups of
// a 32 GB budget: each step's launches are twice as wide), and compresses the
// shipped model's 64 MiB text in 4 sub-batches (0.3% faster than 7 at 32 GB)
constexpr double SCRATCH_GB_DEFAULT = 64.0;
constexpr int DEC_LANES_MAX = 4;  // most HIP streams a decode group is split over
// V^T block exponent of the decode caches (vt_off): a step appends one key, whose 64 value
// bytes span 256 bytes with 4-key blocks (1 KB with the prefill caches' 16-key blocks); the
// decode attention reads this layout
constexpr int DEC_VL = 2;

struct DevLayer {
    int8_t *attn_norm = nullptr, *post_attn_norm = nullptr, *ffn_norm = nullptr, *post_ffn_norm = nullptr;
    int8_t *qkv_w = nullptr, *out_w = nullptr, *up_w = nullptr, *down_w = nullptr, *sink = nullptr;
    int8_t *out_wf = nullptr, *down_wf = nullptr;  // fragment-major copies (row GEMM)
    int8_t* up_wf16 = nullptr;  // fragment-major, gate and up tiles interleaved per 16 features (fused FFN)
    int32_t* score_mult = nullptr;
    int qkv_mult, out_mult, up_mult, down_mult, qkv_shift, out_shift, up_shift, down_shift;
    int qkv_n;  // QKV rows the attention reads
    int attn_general;  // attention must take its general path (see attention_needs_general)
};

// Requantization parameters of a GEMM launch (model.rs:280-300).  The fast
// path multiplies in f64, exact while |acc * mult| < 2^53: |acc| <= K * 127 * 128
// < 2^27 for K <= 8192, so |mult| < 2^26 suffices.
template <class G>
void set_requant(G& g, int mult, int shift) {
    g.mult = mult;
    g.shift = shift;
    // fast path: |acc * mult| < 2^53 (exact in f64) and |acc * mult * 2^-shift|
    // < 2^31 (the FMA rint's low word), with |acc| <= K * 127 * 128
    const long long am = mult < 0 ? -(long long)mult : (long long)mult;
    const double accmax = (double)g.K * 127.0 * 128.0;
    const double ymax = shift <= 0 ? accmax * (double)am : ldexp(accmax * (double)am, -shift);
    g.rq_fast = (am < (1ll << 26) && shift <= 62 && g.K <= 8192 && ymax < 2147483648.0) ? 1 : 0;
    g.rq_scale = shift <= 0 ? (double)mult : ldexp((double)mult, -shift);
}

// The prefill attention kernel's fast path assumes |score| < 2^30, so that
// score differences never wrap in i32, and exp2_lut[0] == 65535, so that a
// zero difference reads the table's first entry.  |score| <= 8 * |mult| + 1
// (|dot| <= 64 * 127 * 127, divided by 4 and by 2^15).
int attention_needs_general(const uint16_t* exp2_lut, const int32_t* score_mult, int n_heads) {
    if (exp2_lut[0] != 65535) return 1;
    for (int h = 0; h < n_heads; h++) {
        const long long m = score_mult[h];
        if (m >= (1ll << 27) || m <= -(1ll << 27)) return 1;
    }
    return 0;
}

struct Stat {
    int64_t launches = 0;
    double ms = 0;
};

}  // namespace

struct czip_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    hipStream_t lane_s[3] = {};  // a decode group's lanes after the first
    hipEvent_t lane_ev[4] = {};  // fork / join of the lanes
    czip_model_desc cfg{};
    int KH = 1;  // cached KV heads per layer
    bool rn_fused = false;  // residual + norms fused into the row GEMM (gemm_rn_supported(d_model))
    bool head_fused = false;  // LM head fused with the coder interval stage / decode step (head_cdf_supported(vocab))
    bool ffn_fused = false;   // up + ReGLU + down + norms in one kernel (ffn_supported(d_model, d_ff))
    int64_t ffn_min_rows = FFN_MIN_ROWS;  // rows from which it is used (CZIP_FFN_MIN_ROWS)
    // switches read from the environment once, at czip_create
    bool gemm_tiled = false;      // CZIP_GEMM_TILED: tiled GEMM kernels only
    bool qkv_gemm = false;        // CZIP_QKV_GEMM: layer 0's QKV by the GEMM, not the per-token table
    double scratch_gb = 0;        // CZIP_SCRATCH_GB: a job's scratch budget
    int64_t decode_streams = 0;   // CZIP_DECODE_STREAMS: most streams per decode group (0: no cap)
    int decode_lanes = 0;         // CZIP_DECODE_LANES: lanes per decode group (0: by group size)
    bool lut0_max = false;        // exp2_lut[0] == 65535: the heads' table step 0 is E(0) (HeadCdfArgs::e0)
    std::vector<void*> allocs;
    int8_t *embed = nullptr, *final_norm = nullptr, *head_w = nullptr, *head_wf = nullptr;
    int8_t* embed_xn = nullptr;  // rmsnorm(embed[v], layer 0's attn_norm) for every token v
    int8_t* qkv_tab = nullptr;   // layer 0's requantized QKV projection of embed_xn[v] (before RoPE)
    uint16_t* lut = nullptr;
    uint16_t* etab = nullptr;    // attention's exp table by step, weights as offset bytes (attn_etab_host)
    int16_t *rcos = nullptr, *rsin = nullptr;
    std::vector<DevLayer> layers;
    std::string err;
    bool profiling = false;
    std::map<std::string, Stat> stats;
    struct Pending {
        std::string name;
        hipEvent_t a, b;
    };
    std::vector<Pending> pending;
    std::vector<hipEvent_t> event_pool;
    czip_job* dec = nullptr;  // step-wise decode session (czip_decode_begin)
    uint8_t* noalloc = nullptr;  // this device's copy of `scratch` (czip_prefill_cdf_noalloc)
    std::string noalloc_err;
};

struct czip_job {
    czip_ctx* ctx = nullptr;
    int kind = 0;  // 0 compress
    int64_t n_tokens = 0, nchunks = 0;
    int T = 0, BC = 0;
    int64_t slot = 0;
    bool ran = false;  // the last czip_job_run succeeded: the outputs may be fetched
    std::vector<void*> allocs;
    uint32_t* tok = nullptr;
    uint8_t* out = nullptr;
    int32_t* out_lens = nullptr;
    int32_t* err = nullptr;
    // per sub-batch scratch
    uint32_t *inp = nullptr, *tgt = nullptr, *lohi = nullptr, *lohi_all = nullptr;
    int32_t* lens = nullptr;      // lengths of the chunks of the current sub-batch
    int32_t* lens_all = nullptr;  // lengths of every chunk of the job
    int16_t* x = nullptr;  // residual stream (|x| <= 127 * (2 * n_layers + 1) < 2^15)
    int8_t *xn = nullptr, *q8 = nullptr, *kc = nullptr, *vc = nullptr, *attn = nullptr, *y8 = nullptr, *r8 = nullptr;
    int32_t* logits = nullptr;
    int32_t* rn_ws = nullptr;  // split-K row GEMM workspace (decode with few streams)
    size_t rn_ws_bytes = 0;
    // decompress
    int S = 0;  // streams decoded together
    int64_t total_tokens = 0;
    std::vector<int32_t> h_ntok;
    uint8_t* d_data = nullptr;
    int64_t *d_offs = nullptr, *d_toff = nullptr, *st_bpos = nullptr;
    int32_t *d_blen = nullptr, *d_ntok = nullptr, *st_bit = nullptr;
    uint32_t *d_tokens = nullptr, *st_low = nullptr, *st_high = nullptr, *st_code = nullptr, *st_plo = nullptr, *st_phi = nullptr;
    // step-wise decode session
    uint32_t *d_val = nullptr, *d_out = nullptr;
    std::vector<int32_t> h_lens;
    std::vector<int32_t> h_done;  // per stream: the highest position whose K/V are cached since it last began at 0 (-1: none)
};

namespace {

czip_status fail(czip_ctx* c, czip_status rc, const std::string& msg) {
    if (c) c->err = msg;
    return rc;
}

#define HIPCHECK(ctx, call)                                                                   \
    do {                                                                                      \
        hipError_t e_ = (call);                                                               \
        if (e_ != hipSuccess)                                                                 \
            return fail((ctx), CZIP_E_HIP, std::string(#call) + ": " + hipGetErrorString(e_)); \
    } while (0)

template <typename T>
czip_status dalloc(czip_ctx* c, std::vector<void*>& owner, T** p, size_t count) {
    void* q = nullptr;
    size_t bytes = std::max<size_t>(count * sizeof(T), 256);
    bytes = (bytes + 255) & ~(size_t)255;
    hipError_t e = hipMalloc(&q, bytes);
    if (e != hipSuccess) return fail(c, CZIP_E_NOMEM, std::string("hipMalloc(") + std::to_string(bytes) + "): " + hipGetErrorString(e));
    owner.push_back(q);
    *p = (T*)q;
    return CZIP_OK;
}

template <typename T>
czip_status upload(czip_ctx* c, T** dst, const T* src, size_t count) {
    czip_status rc = dalloc(c, c->allocs, dst, count);
    if (rc) return rc;
    HIPCHECK(c, hipMemcpy(*dst, src, count * sizeof(T), hipMemcpyHostToDevice));
    return CZIP_OK;
}

// W [N, K] in the fragment-major order of rowblock_mma (N % 16 == 0, K % 64
// == 0): operand (tile t, K step s) at (t * K / 64 + s) * 1024, lane l's 16
// bytes at +16 l = W[16 t + l % 16, 64 s + 16 (l / 16) .. +16].
czip_status upload_frag_major(czip_ctx* c, int8_t** dst, const int8_t* W, size_t N, size_t K) {
    if (N % 16 != 0 || K % 64 != 0) return fail(c, CZIP_E_CONFIG, "weight shape not a multiple of 16 x 64");
    std::vector<int8_t> f(N * K);
    const size_t ns = K / 64;
    for (size_t t = 0; t < N / 16; t++)
        for (size_t s = 0; s < ns; s++)
            for (size_t l = 0; l < 64; l++)
                memcpy(&f[(t * ns + s) * 1024 + l * 16], W + (16 * t + l % 16) * K + 64 * s + 16 * (l / 16), 16);
    return upload(c, dst, f.data(), N * K);
}

// --- launch instrumentation ---
hipEvent_t take_event(czip_ctx* c) {
    if (!c->event_pool.empty()) {
        hipEvent_t e = c->event_pool.back();
        c->event_pool.pop_back();
        return e;
    }
    hipEvent_t e;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

struct Timed {
    czip_ctx* c;
    const char* name;
    hipEvent_t a = nullptr, b = nullptr;
    Timed(czip_ctx* c_, const char* n) : c(c_), name(n) {
        if (c->profiling) {
            a = take_event(c);
            b = take_event(c);
            if (a) hipEventRecord(a, c->stream);
        }
    }
    ~Timed() {
        if (c->profiling && a && b) {
            hipEventRecord(b, c->stream);
            c->pending.push_back({name, a, b});
        }
    }
};

void resolve_events(czip_ctx* c) {
    for (auto& p : c->pending) {
        float ms = 0;
        if (hipEventElapsedTime(&ms, p.a, p.b) == hipSuccess) {
            auto& s = c->stats[p.name];
            s.launches++;
            s.ms += ms;
        }
        c->event_pool.push_back(p.a);
        c->event_pool.push_back(p.b);
    }
    c->pending.clear();
}

// the GEMM launches with the context's kernel switch
void gemm(const czip_ctx* c, GemmArgs g, int epi, hipStream_t s) {
    g.tiled = c->gemm_tiled ? 1 : 0;
    launch_gemm(g, epi, s);
}
void gemm_rn(const czip_ctx* c, RowGemmArgs a, hipStream_t s) {
    a.tiled = c->gemm_tiled ? 1 : 0;
    launch_gemm_rn(a, s);
}

czip_status check_config(czip_ctx* c, const czip_model_desc& w) {
    if (w.head_dim != 64) return fail(c, CZIP_E_CONFIG, "head_dim must be 64 (attention.rs:9)");
    if (w.n_heads < 1 || w.d_model != w.n_heads * 64) return fail(c, CZIP_E_CONFIG, "d_model must equal n_heads*64");
    if (w.d_model > 1024) return fail(c, CZIP_E_CONFIG, "d_model > 1024 unsupported");
    if (w.d_ff < 32 || w.d_ff % 32 != 0) return fail(c, CZIP_E_CONFIG, "d_ff must be a multiple of 32");
    if (w.d_ff % 64 != 0) return fail(c, CZIP_E_CONFIG, "d_ff must be a multiple of 64");
    if (w.vocab < 2 || w.vocab > 8192 || w.vocab % 64 != 0) return fail(c, CZIP_E_CONFIG, "vocab must be a multiple of 64 in [64, 8192]");
    if (w.n_layers < 1 || w.n_layers > 128)
        return fail(c, CZIP_E_CONFIG, "n_layers must be in [1, 128] (the residual stream is held in int16)");
    if (w.n_kv_heads < 1) return fail(c, CZIP_E_CONFIG, "n_kv_heads must be >= 1");
    if (w.kv_mode == CZIP_KV_RUST_COMPAT) {
        if (!(w.n_heads == 4 || w.n_heads == 6 || w.n_heads == 8))
            return fail(c, CZIP_E_HEADS, "n_heads must be 4, 6 or 8 in rust-compat KV mode (attention.rs:172)");
        int len = w.d_model + 2 * w.n_kv_heads * 64;
        if (len / (w.d_model + 128) != 1) return fail(c, CZIP_E_HEADS, "QKV row splits into more than one MQA row (attention.rs:176)");
    } else if (w.kv_mode == CZIP_KV_GQA) {
        if (w.n_heads % w.n_kv_heads != 0) return fail(c, CZIP_E_CONFIG, "n_heads must be a multiple of n_kv_heads");
    } else {
        return fail(c, CZIP_E_ARG, "unknown kv_mode");
    }
    if (w.exp2_len != 256) return fail(c, CZIP_E_FORMAT, "Exp2 LUT must have exactly 256 entries (lut.rs:57-64)");
    if (w.context_length < 1 || w.rope_len != (int64_t)w.context_length * 32)
        return fail(c, CZIP_E_FORMAT, "RoPE LUT arrays size mismatch with max_seq_len * half_dim (lut.rs:148-165)");
    if (w.context_length > 65535)
        return fail(c, CZIP_E_CONFIG, "context_length > 65535 unsupported (the attention sum S is held in 32 bits)");
    if ((uint64_t)w.target_total <= (uint64_t)w.vocab) return fail(c, CZIP_E_CONFIG, "target_total must exceed vocab");
    return CZIP_OK;
}

}  // namespace

// ===========================================================================
// Model loader
// ===========================================================================
extern "C" czip_status czip_model_load(const char* path, int32_t kv_mode, czip_model** out) {
    if (!path || !out) return CZIP_E_ARG;
    auto m = std::make_unique<czip_model>();
    std::string err;
    czip_status rc = load_czm(path, kv_mode, m->hm, err);
    if (rc) {
        fprintf(stderr, "czip_model_load: %s\n", err.c_str());
        return rc;
    }
    *out = m.release();
    return CZIP_OK;
}

extern "C" const czip_model_desc* czip_model_desc_get(const czip_model* m) { return m ? &m->hm.desc : nullptr; }

extern "C" const uint8_t* czip_model_tokenizer(const czip_model* m, size_t* len, const char** codec) {
    if (!m) return nullptr;
    if (len) *len = m->hm.tokenizer_len;
    if (codec) *codec = m->hm.tokenizer_codec.c_str();
    return m->hm.tokenizer;
}

extern "C" void czip_model_free(czip_model* m) { delete m; }

// ===========================================================================
// Context
// ===========================================================================
extern "C" int czip_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

extern "C" const char* czip_last_error(const czip_ctx* c) { return c ? c->err.c_str() : "null context"; }

// ---------------------------------------------------------------------------
// The one fixed device buffer of czip_prefill_cdf_noalloc: a file-scope
// device array that the code object loader places on every GPU the library
// runs on, held until the process ends.  In host code `scratch` names a
// host-side stand-in, never the device memory: its device address is looked
// up once per device (hipGetSymbolAddress, with that device current) and only
// that address is handed to kernels.
// ---------------------------------------------------------------------------
constexpr size_t NOALLOC_SCRATCH_BYTES = CZIP_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[NOALLOC_SCRATCH_BYTES];

namespace {
std::mutex g_scratch_mu;
std::map<int, uint8_t*> g_scratch_addr;  // device -> address of that device's `scratch`

// device must be current
hipError_t scratch_address(int device, uint8_t** out) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    auto it = g_scratch_addr.find(device);
    if (it != g_scratch_addr.end()) {
        *out = it->second;
        return hipSuccess;
    }
    void* p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) return e != hipSuccess ? e : hipErrorInvalidSymbol;
    g_scratch_addr[device] = (uint8_t*)p;
    *out = (uint8_t*)p;
    return hipSuccess;
}
}  // namespace

extern "C" czip_status czip_create(const czip_model_desc* w, int device, czip_ctx** out) {
    if (!w || !out) return CZIP_E_ARG;
    *out = nullptr;
    auto c = std::make_unique<czip_ctx>();
    czip_status rc = check_config(c.get(), *w);
    if (rc) {
        fprintf(stderr, "czip_create: %s\n", c->err.c_str());
        return rc;
    }
    c->cfg = *w;
    c->cfg.layers = nullptr;
    c->device = device;
    if (hipSetDevice(device) != hipSuccess) return CZIP_E_HIP;
    if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) return CZIP_E_HIP;
    const size_t d = (size_t)w->d_model, F = (size_t)w->d_ff, V = (size_t)w->vocab, G = (size_t)w->n_kv_heads;
    c->KH = w->kv_mode == CZIP_KV_GQA ? w->n_kv_heads : 1;
    c->rn_fused = gemm_rn_supported(w->d_model) && getenv("CZIP_UNFUSED_NORM") == nullptr;
    c->head_fused = head_cdf_supported(w->vocab) && w->coef_q24 < (1u << 23) && getenv("CZIP_UNFUSED_HEAD") == nullptr;
    c->ffn_fused = c->rn_fused && ffn_supported(w->d_model, w->d_ff) && getenv("CZIP_UNFUSED_FFN") == nullptr;
    if (const char* e = getenv("CZIP_FFN_MIN_ROWS")) c->ffn_min_rows = std::max(1ll, atoll(e));
    c->gemm_tiled = getenv("CZIP_GEMM_TILED") != nullptr;
    c->qkv_gemm = getenv("CZIP_QKV_GEMM") != nullptr;
    c->scratch_gb = SCRATCH_GB_DEFAULT;
    if (const char* e = getenv("CZIP_SCRATCH_GB")) c->scratch_gb = atof(e);
    if (const char* e = getenv("CZIP_DECODE_STREAMS")) c->decode_streams = std::max(1ll, atoll(e));
    if (const char* e = getenv("CZIP_DECODE_LANES")) {
        const int n = atoi(e);
        if (n >= 1 && n <= DEC_LANES_MAX) c->decode_lanes = n;
    }
    czip_ctx* C = c.get();
#define UP(dst, src, n) if ((rc = upload(C, &dst, src, n))) return rc;
    UP(c->embed, w->embed, V * d)
    UP(c->final_norm, w->final_norm, d)
    UP(c->head_w, w->head_w, V * d)
    if ((rc = upload_frag_major(C, &c->head_wf, w->head_w, V, d))) return rc;
    UP(c->lut, w->exp2_lut, 256)
    c->lut0_max = w->exp2_lut[0] == 65535;
    {
        std::vector<uint16_t> et(ETB_PAD);
        attn_etab_host(w->exp2_lut, et.data());
        UP(c->etab, et.data(), et.size())
    }
    UP(c->rcos, w->rope_cos, (size_t)w->rope_len)
    UP(c->rsin, w->rope_sin, (size_t)w->rope_len)
    c->layers.resize((size_t)w->n_layers);
    std::vector<int8_t> perm(2 * F * d);
    for (int l = 0; l < w->n_layers; l++) {
        const czip_layer_desc& L = w->layers[l];
        DevLayer& D = c->layers[(size_t)l];
        if (!L.attn_norm || !L.post_attn_norm || !L.ffn_norm || !L.post_ffn_norm || !L.qkv_w || !L.out_w || !L.up_w ||
            !L.down_w || !L.score_mult)
            return fail(C, CZIP_E_ARG, "layer tensor pointer is NULL");
        D.qkv_n = w->kv_mode == CZIP_KV_GQA ? (int)(d + 2 * G * 64) : (int)(d + 128);
        UP(D.attn_norm, L.attn_norm, d)
        UP(D.post_attn_norm, L.post_attn_norm, d)
        UP(D.ffn_norm, L.ffn_norm, d)
        UP(D.post_ffn_norm, L.post_ffn_norm, d)
        UP(D.qkv_w, L.qkv_w, (size_t)D.qkv_n * d)
        UP(D.out_w, L.out_w, d * d)
        if ((rc = upload_frag_major(C, &D.out_wf, L.out_w, d, d))) return rc;
        // gate/up interleave in groups of 32 rows so one 64-wide GEMM tile holds matching pairs
        for (size_t grp = 0; grp < F / 32; grp++) {
            memcpy(&perm[(grp * 64) * d], L.up_w + (grp * 32) * d, 32 * d);
            memcpy(&perm[(grp * 64 + 32) * d], L.up_w + (F + grp * 32) * d, 32 * d);
        }
        UP(D.up_w, perm.data(), 2 * F * d)
        UP(D.down_w, L.down_w, d * F)
        if ((rc = upload_frag_major(C, &D.down_wf, L.down_w, d, F))) return rc;
        if (c->ffn_fused) {
            // rows 32 g .. +16 = gate rows 16 g .., rows 32 g + 16 .. = the matching up rows
            for (size_t g = 0; g < F / 16; g++) {
                memcpy(&perm[(g * 32) * d], L.up_w + (g * 16) * d, 16 * d);
                memcpy(&perm[(g * 32 + 16) * d], L.up_w + (F + g * 16) * d, 16 * d);
            }
            if ((rc = upload_frag_major(C, &D.up_wf16, perm.data(), 2 * F, d))) return rc;
        }
        UP(D.score_mult, L.score_mult, (size_t)w->n_heads)
        if (L.sink_key) { UP(D.sink, L.sink_key, 64) }
        D.attn_general = attention_needs_general(w->exp2_lut, L.score_mult, w->n_heads);
        D.qkv_mult = L.qkv_mult; D.out_mult = L.out_mult; D.up_mult = L.up_mult; D.down_mult = L.down_mult;
        D.qkv_shift = L.qkv_shift; D.out_shift = L.out_shift; D.up_shift = L.up_shift; D.down_shift = L.down_shift;
    }
#undef UP
    {
        // layer 0's normalized input, and so its QKV projection before RoPE,
        // depend on the token alone: normalize every vocabulary row once with
        // the prefill's own kernel and project the table with the QKV GEMM's
        // requantization; per row only RoPE and the cache scatter remain
        std::vector<uint32_t> iota(V);
        for (size_t v = 0; v < V; v++) iota[v] = (uint32_t)v;
        uint32_t* d_iota = nullptr;
        if ((rc = upload(C, &d_iota, iota.data(), V))) return rc;
        if ((rc = dalloc(C, C->allocs, &c->embed_xn, V * d))) return rc;
        launch_embed_norm(d_iota, c->embed, c->layers[0].attn_norm, (int)V, (int)d, nullptr, c->embed_xn, c->stream);
        const DevLayer& L0 = c->layers[0];
        if ((rc = dalloc(C, C->allocs, &c->qkv_tab, V * (size_t)L0.qkv_n))) return rc;
        GemmArgs g{};
        g.A = c->embed_xn; g.W = L0.qkv_w; g.M = (int)V; g.N = L0.qkv_n; g.K = (int)d;
        g.out8 = c->qkv_tab; g.ldo = L0.qkv_n; set_requant(g, L0.qkv_mult, L0.qkv_shift);
        gemm(C, g, EPI_REQ, c->stream);
        HIPCHECK(C, hipGetLastError());
        HIPCHECK(C, hipStreamSynchronize(c->stream));
    }
    {
        // the no-alloc entry point's buffer on this device (its failure only
        // disables that entry point)
        hipError_t e = scratch_address(device, &c->noalloc);
        if (e != hipSuccess) {
            c->noalloc = nullptr;
            c->noalloc_err = std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e);
        }
    }
    *out = c.release();
    return CZIP_OK;
}

static void free_decode_session(czip_ctx* c);

extern "C" void czip_destroy(czip_ctx* c) {
    if (!c) return;
    hipSetDevice(c->device);
    if (c->stream) hipStreamSynchronize(c->stream);
    free_decode_session(c);
    for (auto& p : c->pending) { hipEventDestroy(p.a); hipEventDestroy(p.b); }
    for (auto e : c->event_pool) hipEventDestroy(e);
    for (void* p : c->allocs) hipFree(p);
    for (auto e : c->lane_ev) if (e) hipEventDestroy(e);
    for (auto q : c->lane_s) if (q) hipStreamDestroy(q);
    if (c->stream) hipStreamDestroy(c->stream);
    delete c;
}

extern "C" void czip_set_profiling(czip_ctx* c, int32_t on) {
    if (c) c->profiling = on != 0;
}

extern "C" czip_status czip_kernel_stats(czip_ctx* c, const char* name, int64_t* launches, double* total_ms) {
    if (!c || !name) return CZIP_E_ARG;
    auto it = c->stats.find(name);
    if (launches) *launches = it == c->stats.end() ? 0 : it->second.launches;
    if (total_ms) *total_ms = it == c->stats.end() ? 0.0 : it->second.ms;
    return CZIP_OK;
}

extern "C" void czip_reset_stats(czip_ctx* c) {
    if (c) c->stats.clear();
}

// ===========================================================================
// Forward pass over a batch of chunks (shared by every entry point)
// ===========================================================================
namespace {

int pad64(int T) { return (T + 63) & ~63; }

// device bytes per token row of a forward batch (logits: the int32 logits are
// materialized, i.e. the head is not fused with the coder interval stage)
size_t row_bytes(const czip_ctx* c, bool logits = true) {
    const size_t d = (size_t)c->cfg.d_model, F = (size_t)c->cfg.d_ff, V = (size_t)c->cfg.vocab;
    return 2 * d /*x*/ + 5 * d /*xn q8 attn y8*/ + F /*r8*/ + (logits ? 4 * V : 0) + 8 /*lohi*/ + 8 /*inp tgt*/ +
           2 * (size_t)c->KH * 64 /*kv*/ + 64;
}

czip_status alloc_scratch(czip_ctx* c, czip_job* j, int BC, int T, bool logits = true) {
    const size_t M = (size_t)BC * T;
    const size_t d = (size_t)c->cfg.d_model, F = (size_t)c->cfg.d_ff, V = (size_t)c->cfg.vocab;
    czip_status rc;
    if ((rc = dalloc(c, j->allocs, &j->inp, M))) return rc;
    if ((rc = dalloc(c, j->allocs, &j->tgt, M))) return rc;
    if ((rc = dalloc(c, j->allocs, &j->x, M * d))) return rc;
    if ((rc = dalloc(c, j->allocs, &j->xn, M * d))) return rc;
    if ((rc = dalloc(c, j->allocs, &j->q8, M * d))) return rc;
    if ((rc = dalloc(c, j->allocs, &j->attn, M * d))) return rc;
    if ((rc = dalloc(c, j->allocs, &j->y8, M * d))) return rc;
    if ((rc = dalloc(c, j->allocs, &j->r8, M * F))) return rc;
    if ((rc = dalloc(c, j->allocs, &j->kc, M * (size_t)c->KH * 64))) return rc;
    if ((rc = dalloc(c, j->allocs, &j->vc, (size_t)BC * pad64(T) * (size_t)c->KH * 64))) return rc;
    if (logits && (rc = dalloc(c, j->allocs, &j->logits, M * V))) return rc;
    return CZIP_OK;
}

int pick_batch_chunks(const czip_ctx* c, int64_t nchunks, int T, bool logits = true) {
    const double gb = c->scratch_gb;
    double per_chunk = (double)row_bytes(c, logits) * T;
    int64_t bc = (int64_t)(gb * 1e9 / per_chunk);
    bc = std::max<int64_t>(1, std::min<int64_t>(bc, nchunks));
    return (int)bc;
}

// Output projection, residual + norms and FFN of layer l on M rows whose
// attention output is j->attn (model.rs:423-468); leaves the next layer's (or
// the final) normalized input in j->xn and the residual stream in j->x.  With
// the row GEMM the projection outputs stay on chip; layer 0 re-reads its
// residual input from the embedding rows of j->inp.
// A job's per-row buffers, or the rows of one decode lane (a contiguous range
// of its streams) with its share of the split-K workspace
struct RowBufs {
    uint32_t* inp;
    int16_t* x;
    int8_t *xn, *q8, *attn, *y8, *r8;
    int32_t* rn_ws;
    size_t rn_ws_bytes;
};

RowBufs row_bufs(const czip_ctx* c, const czip_job* j, int64_t r0 = 0, int ws_parts = 1, int ws_part = 0) {
    const size_t d = (size_t)c->cfg.d_model, F = (size_t)c->cfg.d_ff, r = (size_t)r0;
    const size_t wb = j->rn_ws_bytes / (size_t)ws_parts / 16 * 16;
    return RowBufs{j->inp + r, j->x + r * d, j->xn + r * d, j->q8 + r * d, j->attn + r * d,
                   j->y8 ? j->y8 + r * d : nullptr, j->r8 ? j->r8 + r * F : nullptr,
                   j->rn_ws ? j->rn_ws + wb / 4 * (size_t)ws_part : nullptr, wb};
}

void post_attention(czip_ctx* c, const RowBufs& r, int l, int M, hipStream_t s, bool beside_lanes = false) {
    const int d = c->cfg.d_model, F = c->cfg.d_ff;
    const DevLayer& L = c->layers[(size_t)l];
    const bool last = l + 1 == c->cfg.n_layers;
    const int8_t* next = last ? c->final_norm : c->layers[(size_t)l + 1].attn_norm;
    if (c->rn_fused) {
        RowGemmArgs o{};
        o.A = r.attn; o.W = L.out_w; o.Wf = L.out_wf; o.M = M; o.K = d; o.d = d;
        set_requant(o, L.out_mult, L.out_shift);
        o.w1 = L.ffn_norm; o.w2 = L.post_attn_norm;
        o.x_in = l == 0 ? nullptr : r.x; o.tok = r.inp; o.embed = c->embed;
        o.x_out = r.x; o.xn = r.xn; o.ws = r.rn_ws; o.ws_bytes = r.rn_ws_bytes;
        { Timed t(c, "gemm_o_norm"); gemm_rn(c, o, s); }
    } else {
        GemmArgs o{};
        o.A = r.attn; o.W = L.out_w; o.M = M; o.N = d; o.K = d; o.out8 = r.y8; o.ldo = d;
        set_requant(o, L.out_mult, L.out_shift);
        { Timed t(c, "gemm_o"); gemm(c, o, EPI_REQ, s); }
        { Timed t(c, "row_norm"); launch_resid_norm(r.x, r.y8, L.ffn_norm, L.post_attn_norm, M, d, r.xn, s); }
    }
    // the fused FFN walks 128-row strips with one workgroup per CU: it pays
    // off for prefill sub-batches, while a decode step's rows alone balance
    // better over the separate kernels' 64-row blocks; beside other decode
    // lanes (which fill its last round of strips) its one launch per layer
    // instead of two is the faster choice again
    if (c->ffn_fused && (M >= c->ffn_min_rows || beside_lanes)) {
        GemmArgs u{}, dn{};  // requantization parameters of the two products
        u.K = d; set_requant(u, L.up_mult, L.up_shift);
        dn.K = F; set_requant(dn, L.down_mult, L.down_shift);
        FfnArgs f{};
        f.xn = r.xn; f.Wup = L.up_wf16; f.Wdf = L.down_wf; f.M = M; f.d = d; f.F = F;
        f.up_mult = u.mult; f.up_shift = u.shift; f.up_fast = u.rq_fast; f.up_scale = u.rq_scale;
        f.dn_mult = dn.mult; f.dn_shift = dn.shift; f.dn_fast = dn.rq_fast; f.dn_scale = dn.rq_scale;
        f.w1 = L.post_ffn_norm; f.w2 = next; f.x_in = r.x; f.x_out = last ? nullptr : r.x; f.xn_out = r.xn;
        Timed t(c, "ffn");
        launch_ffn(f, s);
        return;
    }
    GemmArgs u{};
    u.A = r.xn; u.W = L.up_w; u.M = M; u.N = 2 * F; u.K = d; u.out8 = r.r8; u.ldo = F;
    set_requant(u, L.up_mult, L.up_shift);
    { Timed t(c, "gemm_up"); gemm(c, u, EPI_REGLU, s); }
    if (c->rn_fused) {
        RowGemmArgs dn{};
        dn.A = r.r8; dn.W = L.down_w; dn.Wf = L.down_wf; dn.M = M; dn.K = F; dn.d = d;
        set_requant(dn, L.down_mult, L.down_shift);
        dn.w1 = L.post_ffn_norm; dn.w2 = next;
        dn.x_in = r.x; dn.x_out = last ? nullptr : r.x; dn.xn = r.xn; dn.ws = r.rn_ws; dn.ws_bytes = r.rn_ws_bytes;
        { Timed t(c, "gemm_down_norm"); gemm_rn(c, dn, s); }
    } else {
        GemmArgs dn{};
        dn.A = r.r8; dn.W = L.down_w; dn.M = M; dn.N = d; dn.K = F; dn.out8 = r.y8; dn.ldo = d;
        set_requant(dn, L.down_mult, L.down_shift);
        { Timed t(c, "gemm_down"); gemm(c, dn, EPI_REQ, s); }
        { Timed t(c, "row_norm"); launch_resid_norm(r.x, r.y8, L.post_ffn_norm, next, M, d, r.xn, s); }
    }
}

// Layer 0's QKV: from the per-token table (RoPE + scatter), or the GEMM over
// the gathered normalized embedding rows (CZIP_QKV_GEMM=1, or a launch too
// large for the table kernel's 32-bit item index).
void layer0_qkv(czip_ctx* c, GemmArgs& g, const uint32_t* tok, hipStream_t s) {
    const DevLayer& L = c->layers[0];
    const int NG = c->cfg.kv_mode == CZIP_KV_GQA ? c->cfg.n_kv_heads : 1;
    const long long items = (long long)g.M * (8 * c->cfg.n_heads + 24 * NG);
    if (!c->qkv_gemm && items < (1ll << 31)) {
        QkvTabArgs q{};
        q.tab = c->qkv_tab; q.tok = tok; q.M = g.M; q.T = g.T; q.TP = g.TP; q.pos = g.pos; q.vl = g.vl;
        q.H = c->cfg.n_heads; q.NG = NG; q.KH = c->KH; q.d = c->cfg.d_model; q.qkv_n = L.qkv_n;
        q.rcos = c->rcos; q.rsin = c->rsin; q.q8 = g.out8; q.kc = g.kc; q.vc = g.vc;
        Timed t(c, "qkv_table");
        launch_qkv_table(q, s);
        return;
    }
    g.A = c->embed_xn; g.a_rows = tok; g.a_nrows = c->cfg.vocab;
    Timed t(c, "gemm_qkv");
    gemm(c, g, EPI_QKV, s);
}

// Run every layer on rows [0, nb*T) whose inputs are j->inp / j->lens; leaves
// logits in j->logits (head), else the final-normalized rows in j->xn.
// (model.rs:362-480 as batched launches)
czip_status forward_batch(czip_ctx* c, czip_job* j, int nb, int T, bool head = true) {
    const int M = nb * T;
    const int d = c->cfg.d_model, F = c->cfg.d_ff, V = c->cfg.vocab, H = c->cfg.n_heads;
    hipStream_t s = c->stream;
    if (!c->rn_fused) {
        Timed t(c, "embed_norm");
        launch_embed_norm(j->inp, c->embed, c->layers[0].attn_norm, M, d, j->x, j->xn, s);
    }
    for (int l = 0; l < c->cfg.n_layers; l++) {
        const DevLayer& L = c->layers[(size_t)l];
        GemmArgs g{};
        g.A = j->xn; g.W = L.qkv_w; g.M = M; g.N = L.qkv_n; g.K = d;
        g.out8 = j->q8; g.ldo = d; set_requant(g, L.qkv_mult, L.qkv_shift);
        g.d = d; g.T = T; g.TP = pad64(T); g.pos = -1; g.kv_mode = c->cfg.kv_mode; g.G = c->cfg.n_kv_heads; g.KH = c->KH;
        g.kc = j->kc; g.vc = j->vc; g.rcos = c->rcos; g.rsin = c->rsin;
        if (l == 0) {
            layer0_qkv(c, g, j->inp, s);
        } else {
            Timed t(c, "gemm_qkv");
            gemm(c, g, EPI_QKV, s);
        }
        AttnArgs a{};
        a.q = j->q8; a.kc = j->kc; a.vc = j->vc; a.TP = pad64(T); a.lens = j->lens; a.score_mult = L.score_mult;
        a.sink = L.sink; a.lut = c->lut; a.etab = c->etab; a.out = j->attn; a.M = M; a.T = T; a.H = H; a.G = c->cfg.n_kv_heads;
        a.KH = c->KH; a.kv_mode = c->cfg.kv_mode; a.coef = 378194u;  // ATTN_COEF_Q24 (attention.rs:17-19)
        a.general = L.attn_general;
        { Timed t(c, "attention"); launch_attention(a, nb, s); }
        post_attention(c, row_bufs(c, j), l, M, s);
    }
    if (head) {
        GemmArgs h{};
        h.A = j->xn; h.W = c->head_w; h.M = M; h.N = V; h.K = d; h.out32 = j->logits; h.ldo = V;
        Timed t(c, "gemm_head");
        gemm(c, h, EPI_RAW, s);
    }
    return CZIP_OK;
}

czip_status check_lens(czip_ctx* c, const int32_t* lens, int B, int T) {
    if (T < 1) return fail(c, CZIP_E_ARG, "T must be >= 1");
    if (T > c->cfg.context_length || T > c->cfg.max_seq_len)
        return fail(c, CZIP_E_RANGE, "chunk length exceeds the RoPE LUT / KV cache (lut.rs:169-177)");
    for (int b = 0; b < B; b++)
        if (lens[b] < 0 || lens[b] > T) return fail(c, CZIP_E_ARG, "lens[b] out of [0, T]");
    return CZIP_OK;
}

czip_status check_tokens(czip_ctx* c, const uint32_t* t, int64_t n) {
    for (int64_t i = 0; i < n; i++)
        if (t[i] >= (uint32_t)c->cfg.vocab) return fail(c, CZIP_E_TOKEN, "token id >= vocab at index " + std::to_string(i));
    return CZIP_OK;
}

void free_job_mem(czip_job* j) {
    for (void* p : j->allocs) hipFree(p);
    j->allocs.clear();
}

// Debug paths (forward_logits / prefill_cdf / prefill_cumfreqs): one job
// over caller-given input rows, processed in sub-batches.
czip_status run_rows(czip_ctx* c, const uint32_t* rows_in, const uint32_t* rows_tgt, const int32_t* lens, int B, int T,
                     int mode, void* host_out) {
    czip_status rc = check_lens(c, lens, B, T);
    if (rc) return rc;
    if ((rc = check_tokens(c, rows_in, (int64_t)B * T))) return rc;
    if (rows_tgt && (rc = check_tokens(c, rows_tgt, (int64_t)B * T))) return rc;
    HIPCHECK(c, hipSetDevice(c->device));
    czip_job j;
    j.ctx = c;
    const int BC = pick_batch_chunks(c, B, T);
    if ((rc = alloc_scratch(c, &j, BC, T))) { free_job_mem(&j); return rc; }
    const int V = c->cfg.vocab;
    uint32_t* dcum = nullptr;
    if (mode == 2 && (rc = dalloc(c, j.allocs, &dcum, (size_t)BC * T * V))) { free_job_mem(&j); return rc; }
    if ((rc = dalloc(c, j.allocs, &j.lohi, (size_t)BC * T * 2))) { free_job_mem(&j); return rc; }
    if ((rc = dalloc(c, j.allocs, &j.lens, (size_t)BC))) { free_job_mem(&j); return rc; }
    for (int b0 = 0; b0 < B && rc == 0; b0 += BC) {
        const int nb = std::min(BC, B - b0);
        const size_t M = (size_t)nb * T;
        hipError_t e = hipMemcpyAsync(j.inp, rows_in + (size_t)b0 * T, M * 4, hipMemcpyHostToDevice, c->stream);
        if (e == hipSuccess && rows_tgt)
            e = hipMemcpyAsync(j.tgt, rows_tgt + (size_t)b0 * T, M * 4, hipMemcpyHostToDevice, c->stream);
        if (e == hipSuccess) e = hipMemcpyAsync(j.lens, lens + b0, (size_t)nb * 4, hipMemcpyHostToDevice, c->stream);
        if (e != hipSuccess) { rc = fail(c, CZIP_E_HIP, hipGetErrorString(e)); break; }
        if ((rc = forward_batch(c, &j, nb, T))) break;
        if (mode == 0) {
            e = hipMemcpyAsync((int32_t*)host_out + (size_t)b0 * T * V, j.logits, M * V * 4, hipMemcpyDeviceToHost, c->stream);
        } else if (mode == 1) {
            { Timed t(c, "cdf"); launch_cdf(j.logits, (int)M, V, j.tgt, j.lens, T, c->lut, c->cfg.coef_q24, c->cfg.target_total, 0, j.lohi, 0, c->stream); }
            e = hipMemcpyAsync((uint32_t*)host_out + (size_t)b0 * T * 2, j.lohi, M * 8, hipMemcpyDeviceToHost, c->stream);
        } else {
            { Timed t(c, "cdf"); launch_cdf(j.logits, (int)M, V, nullptr, j.lens, T, c->lut, c->cfg.coef_q24, c->cfg.target_total, 1, dcum, 0, c->stream); }
            e = hipMemcpyAsync((uint32_t*)host_out + (size_t)b0 * T * V, dcum, M * V * 4, hipMemcpyDeviceToHost, c->stream);
        }
        if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
        if (e != hipSuccess) { rc = fail(c, CZIP_E_HIP, hipGetErrorString(e)); break; }
    }
    resolve_events(c);
    free_job_mem(&j);
    if (rc) return rc;
    // rows past each chunk's length are not computed: report zeros
    for (int b = 0; b < B; b++)
        for (int p = lens[b]; p < T; p++) {
            size_t r = (size_t)b * T + p;
            if (mode == 0) memset((int32_t*)host_out + r * V, 0, (size_t)V * 4);
            else if (mode == 1) memset((uint32_t*)host_out + r * 2, 0, 8);
            else memset((uint32_t*)host_out + r * V, 0, (size_t)V * 4);
        }
    return CZIP_OK;
}

}  // namespace

extern "C" czip_status czip_forward_logits(czip_ctx* c, const uint32_t* inputs, const int32_t* lens, int32_t B,
                                           int32_t T, int32_t* logits) {
    if (!c || !inputs || !lens || !logits || B < 0) return c ? fail(c, CZIP_E_ARG, "null argument") : CZIP_E_ARG;
    if (B == 0) return CZIP_OK;
    return run_rows(c, inputs, nullptr, lens, B, T, 0, logits);
}

static czip_status inputs_from_targets(czip_ctx* c, const uint32_t* targets, const int32_t* lens, int B, int T,
                                       std::vector<uint32_t>& inp) {
    inp.assign((size_t)B * T, 0u);
    for (int b = 0; b < B; b++)
        for (int p = 0; p < lens[b] && p < T; p++) inp[(size_t)b * T + p] = p == 0 ? BOS : targets[(size_t)b * T + p - 1];
    (void)c;
    return CZIP_OK;
}

extern "C" czip_status czip_prefill_cdf(czip_ctx* c, const uint32_t* targets, const int32_t* lens, int32_t B,
                                        int32_t T, uint32_t* cum_lohi) {
    if (!c || !targets || !lens || !cum_lohi || B < 0) return c ? fail(c, CZIP_E_ARG, "null argument") : CZIP_E_ARG;
    if (B == 0) return CZIP_OK;
    czip_status rc = check_lens(c, lens, B, T);
    if (rc) return rc;
    std::vector<uint32_t> inp, tgt((size_t)B * T, 0u);
    for (int b = 0; b < B; b++)
        for (int p = 0; p < lens[b]; p++) tgt[(size_t)b * T + p] = targets[(size_t)b * T + p];
    inputs_from_targets(c, tgt.data(), lens, B, T, inp);
    return run_rows(c, inp.data(), tgt.data(), lens, B, T, 1, cum_lohi);
}

extern "C" czip_status czip_prefill_cumfreqs(czip_ctx* c, const uint32_t* inputs, const int32_t* lens, int32_t B,
                                             int32_t T, uint32_t* cumfreqs) {
    if (!c || !inputs || !lens || !cumfreqs || B < 0) return c ? fail(c, CZIP_E_ARG, "null argument") : CZIP_E_ARG;
    if (B == 0) return CZIP_OK;
    return run_rows(c, inputs, nullptr, lens, B, T, 2, cumfreqs);
}

// ===========================================================================
// Compress job
// ===========================================================================
extern "C" int64_t czip_chunk_slot_bytes(int32_t chunk) {
    // at most 32 coded bits per token (a frequency >= 1 of a total < 2^30,
    // plus the renormalisation bit), the terminating bit and a partial byte
    return (int64_t)chunk * 4 + 16;
}

extern "C" czip_status czip_compress_plan(czip_ctx* c, const uint32_t* tokens, int64_t n, int32_t chunk, czip_job** out) {
    if (!c || !out || (n > 0 && !tokens) || n < 0) return c ? fail(c, CZIP_E_ARG, "bad argument") : CZIP_E_ARG;
    *out = nullptr;
    if (chunk < 1) return fail(c, CZIP_E_ARG, "chunk must be >= 1");
    if (chunk > c->cfg.context_length || chunk > c->cfg.max_seq_len)
        return fail(c, CZIP_E_RANGE, "chunk length exceeds the RoPE LUT / KV cache (lut.rs:169-177)");
    if ((uint32_t)c->cfg.vocab <= BOS) return fail(c, CZIP_E_TOKEN, "BOS token 1022 is outside the vocabulary");
    czip_status rc = check_tokens(c, tokens, n);
    if (rc) return rc;
    HIPCHECK(c, hipSetDevice(c->device));
    auto j = std::make_unique<czip_job>();
    j->ctx = c;
    j->kind = 0;
    j->n_tokens = n;
    j->T = chunk;
    j->nchunks = (n + chunk - 1) / chunk;
    j->slot = czip_chunk_slot_bytes(chunk);
    const int64_t nch = std::max<int64_t>(j->nchunks, 1);
    j->BC = pick_batch_chunks(c, nch, chunk, !c->head_fused);
    if ((rc = dalloc(c, j->allocs, &j->tok, (size_t)std::max<int64_t>(n, 1)))) { free_job_mem(j.get()); return rc; }
    if ((rc = dalloc(c, j->allocs, &j->out, (size_t)(nch * j->slot)))) { free_job_mem(j.get()); return rc; }
    if ((rc = dalloc(c, j->allocs, &j->out_lens, (size_t)nch))) { free_job_mem(j.get()); return rc; }
    if (nch > 0 && hipMemset(j->out_lens, 0, (size_t)nch * 4) != hipSuccess) {
        free_job_mem(j.get());
        return fail(c, CZIP_E_HIP, "hipMemset of the chunk lengths");
    }
    if ((rc = dalloc(c, j->allocs, &j->err, 1))) { free_job_mem(j.get()); return rc; }
    // coder intervals and lengths of every chunk, so one encoder launch covers all chunks
    if ((rc = dalloc(c, j->allocs, &j->lohi_all, (size_t)(nch * chunk * 2)))) { free_job_mem(j.get()); return rc; }
    if ((rc = dalloc(c, j->allocs, &j->lens_all, (size_t)nch))) { free_job_mem(j.get()); return rc; }
    if ((rc = alloc_scratch(c, j.get(), j->BC, chunk, !c->head_fused))) { free_job_mem(j.get()); return rc; }
    if (n > 0) {
        hipError_t e = hipMemcpy(j->tok, tokens, (size_t)n * 4, hipMemcpyHostToDevice);
        if (e != hipSuccess) { free_job_mem(j.get()); return fail(c, CZIP_E_HIP, hipGetErrorString(e)); }
    }
    *out = j.release();
    return CZIP_OK;
}

extern "C" int64_t czip_job_chunks(const czip_job* j) { return j ? j->nchunks : 0; }

static czip_status run_compress(czip_job* j) {
    czip_ctx* c = j->ctx;
    hipStream_t s = c->stream;
    const int T = j->T, V = c->cfg.vocab;
    HIPCHECK(c, hipMemsetAsync(j->err, 0, 4, s));
    for (int64_t c0 = 0; c0 < j->nchunks; c0 += j->BC) {
        const int nb = (int)std::min<int64_t>(j->BC, j->nchunks - c0);
        const int M = nb * T;
        j->lens = j->lens_all + c0;
        { Timed t(c, "prep"); launch_prep_chunks(j->tok, j->n_tokens, c0, nb, T, j->inp, j->tgt, j->lens, s); }
        czip_status rc = forward_batch(c, j, nb, T, !c->head_fused);
        if (rc) return rc;
        if (c->head_fused) {
            HeadCdfArgs h{};
            h.A = j->xn; h.W = c->head_wf; h.M = M; h.K = c->cfg.d_model; h.V = V; h.targets = j->tgt; h.lens = j->lens;
            h.T = T; h.lut = c->lut; h.coef = c->cfg.coef_q24; h.total = c->cfg.target_total; h.e0 = c->lut0_max;
            h.out = j->lohi_all; h.out_row0 = c0 * T;
            Timed t(c, "head_cdf");
            launch_head_cdf(h, s);
        } else {
            Timed t(c, "cdf");
            launch_cdf(j->logits, M, V, j->tgt, j->lens, T, c->lut, c->cfg.coef_q24, c->cfg.target_total, 0, j->lohi_all, c0 * T, s);
        }
    }
    if (j->nchunks > 0) {
        Timed t(c, "encode");
        launch_encode(j->lohi_all, j->lens_all, (int)j->nchunks, T, c->cfg.target_total, j->out, j->slot, j->out_lens,
                      j->err, s);
    }
    HIPCHECK(c, hipGetLastError());
    HIPCHECK(c, hipStreamSynchronize(s));
    resolve_events(c);
    int32_t err = 0;
    HIPCHECK(c, hipMemcpy(&err, j->err, 4, hipMemcpyDeviceToHost));
    if (err) return fail(c, CZIP_E_OVERFLOW, "coded chunk exceeded its slot");
    return CZIP_OK;
}

static czip_status run_decompress(czip_job* j);

extern "C" czip_status czip_job_run(czip_job* j) {
    if (!j) return CZIP_E_ARG;
    j->ran = false;
    HIPCHECK(j->ctx, hipSetDevice(j->ctx->device));
    czip_status rc;
    if (j->kind == 0) rc = run_compress(j);
    else if (j->kind == 1) rc = run_decompress(j);
    else return fail(j->ctx, CZIP_E_ARG, "unknown job kind");
    j->ran = rc == CZIP_OK;
    return rc;
}

extern "C" czip_status czip_compress_fetch(czip_job* j, uint8_t* out, int64_t slot, int32_t* lens) {
    if (!j || j->kind != 0 || !lens || (j->nchunks > 0 && !out)) return CZIP_E_ARG;
    czip_ctx* c = j->ctx;
    if (j->nchunks == 0) return CZIP_OK;
    if (!j->ran) return fail(c, CZIP_E_ARG, "fetch before a successful czip_job_run");
    HIPCHECK(c, hipSetDevice(c->device));
    HIPCHECK(c, hipMemcpy(lens, j->out_lens, (size_t)j->nchunks * 4, hipMemcpyDeviceToHost));
    for (int64_t i = 0; i < j->nchunks; i++) {
        if (lens[i] < 0 || lens[i] > j->slot) return fail(c, CZIP_E_OVERFLOW, "coded chunk length outside its slot");
        if (lens[i] > slot) return fail(c, CZIP_E_OVERFLOW, "caller slot smaller than a coded chunk");
    }
    if (slot == j->slot) {
        HIPCHECK(c, hipMemcpy(out, j->out, (size_t)(j->nchunks * j->slot), hipMemcpyDeviceToHost));
    } else {
        HIPCHECK(c, hipMemcpy2D(out, (size_t)slot, j->out, (size_t)j->slot, (size_t)std::min(slot, j->slot),
                                (size_t)j->nchunks, hipMemcpyDeviceToHost));
    }
    return CZIP_OK;
}

extern "C" czip_status czip_compress_fetch_packed(czip_job* j, uint8_t* out, int64_t cap, int64_t* offs) {
    if (!j || j->kind != 0 || !offs) return CZIP_E_ARG;
    czip_ctx* c = j->ctx;
    offs[0] = 0;
    if (j->nchunks == 0) return CZIP_OK;
    if (!j->ran) return fail(c, CZIP_E_ARG, "fetch before a successful czip_job_run");
    const size_t n = (size_t)j->nchunks;
    std::vector<int32_t> lens(n);
    HIPCHECK(c, hipSetDevice(c->device));
    HIPCHECK(c, hipMemcpy(lens.data(), j->out_lens, n * 4, hipMemcpyDeviceToHost));
    // the packing kernel reads lens[i] bytes of slot i: every length must lie
    // in its slot before it is launched
    for (size_t i = 0; i < n; i++) {
        if (lens[i] < 0 || lens[i] > j->slot) return fail(c, CZIP_E_OVERFLOW, "coded chunk length outside its slot");
        offs[i + 1] = offs[i] + lens[i];
    }
    if (!out) return CZIP_OK;
    if (offs[n] > cap) return fail(c, CZIP_E_OVERFLOW, "output smaller than the coded bytes");
    std::vector<void*> tmp;
    int64_t* d_offs = nullptr;
    uint8_t* d_packed = nullptr;
    czip_status rc;
    if ((rc = dalloc(c, tmp, &d_offs, n)) || (rc = dalloc(c, tmp, &d_packed, (size_t)std::max<int64_t>(offs[n], 1)))) {
        for (void* p : tmp) hipFree(p);
        return rc;
    }
    hipError_t e = hipMemcpyAsync(d_offs, offs, n * 8, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) {
        launch_pack_chunks(j->out, j->slot, j->out_lens, d_offs, (int)n, d_packed, c->stream);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipMemcpyAsync(out, d_packed, (size_t)offs[n], hipMemcpyDeviceToHost, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    for (void* p : tmp) hipFree(p);
    if (e != hipSuccess) return fail(c, CZIP_E_HIP, hipGetErrorString(e));
    return CZIP_OK;
}

// ===========================================================================
// Decompress job: streams of S chunks decode in lockstep, one token per
// stream per step, through the same layer kernels as the prefill (M = S rows)
// plus the decode attention and the fused CDF + arithmetic-decode kernel.
// ===========================================================================
extern "C" czip_status czip_decompress_plan(czip_ctx* c, const uint8_t* data, const int64_t* offs, const int32_t* lens,
                                            const int32_t* ntoks, int32_t nchunks, czip_job** out) {
    if (!c || !out || nchunks < 0 || (nchunks > 0 && (!offs || !lens || !ntoks)))
        return c ? fail(c, CZIP_E_ARG, "bad argument") : CZIP_E_ARG;
    *out = nullptr;
    if ((uint32_t)c->cfg.vocab <= BOS) return fail(c, CZIP_E_TOKEN, "BOS token 1022 is outside the vocabulary");
    const int cap = std::min(c->cfg.context_length, c->cfg.max_seq_len);
    int64_t total_bytes = 0, total_tokens = 0;
    int Tcap = 1;
    for (int i = 0; i < nchunks; i++) {
        if (lens[i] < 0 || offs[i] < 0 || ntoks[i] < 0) return fail(c, CZIP_E_ARG, "negative chunk length/offset");
        if (ntoks[i] > cap) return fail(c, CZIP_E_RANGE, "chunk token count exceeds the RoPE LUT / KV cache");
        total_bytes = std::max<int64_t>(total_bytes, offs[i] + lens[i]);
        total_tokens += ntoks[i];
        Tcap = std::max(Tcap, (int)ntoks[i]);
    }
    if (total_bytes > 0 && !data) return fail(c, CZIP_E_ARG, "null data");
    HIPCHECK(c, hipSetDevice(c->device));
    auto j = std::make_unique<czip_job>();
    j->ctx = c;
    j->kind = 1;
    j->nchunks = nchunks;
    j->T = Tcap;
    j->total_tokens = total_tokens;
    j->h_ntok.assign(ntoks, ntoks + nchunks);
    const size_t d = (size_t)c->cfg.d_model, L = (size_t)c->cfg.n_layers;
    const double gb = c->scratch_gb;
    const double per_stream = (double)row_bytes(c, !c->head_fused) + 2.0 * L * (double)c->KH * pad64(Tcap) * 64 + 64;
    int64_t S = (int64_t)(gb * 1e9 / per_stream);
    if (c->decode_streams > 0) S = std::min<int64_t>(S, c->decode_streams);
    S = std::min<int64_t>(S, INT32_MAX / (int64_t)d);  // decode row offsets are 32-bit
    S = std::max<int64_t>(1, std::min<int64_t>(S, std::max(nchunks, 1)));
    j->S = (int)S;
    std::vector<int64_t> toff((size_t)std::max(nchunks, 1), 0);
    for (int i = 1; i < nchunks; i++) toff[(size_t)i] = toff[(size_t)i - 1] + ntoks[i - 1];
    czip_status rc = CZIP_OK;
    auto& A = j->allocs;
    const size_t nc = (size_t)std::max(nchunks, 1);
    if ((rc = dalloc(c, A, &j->d_data, (size_t)std::max<int64_t>(total_bytes, 1) + 16)) ||  // the decoder's word reads
        (rc = dalloc(c, A, &j->d_offs, nc)) || (rc = dalloc(c, A, &j->d_blen, nc)) ||
        (rc = dalloc(c, A, &j->d_ntok, nc)) || (rc = dalloc(c, A, &j->d_toff, nc)) ||
        (rc = dalloc(c, A, &j->d_tokens, (size_t)std::max<int64_t>(total_tokens, 1))) ||
        (rc = dalloc(c, A, &j->st_low, (size_t)S)) || (rc = dalloc(c, A, &j->st_high, (size_t)S)) ||
        (rc = dalloc(c, A, &j->st_plo, (size_t)S)) || (rc = dalloc(c, A, &j->st_phi, (size_t)S)) ||
        (rc = dalloc(c, A, &j->st_code, (size_t)S)) || (rc = dalloc(c, A, &j->st_bpos, (size_t)S)) ||
        (rc = dalloc(c, A, &j->st_bit, (size_t)S)) || (rc = dalloc(c, A, &j->inp, (size_t)S)) ||
        (rc = dalloc(c, A, &j->x, (size_t)S * d)) || (rc = dalloc(c, A, &j->xn, (size_t)S * d)) ||
        (rc = dalloc(c, A, &j->q8, (size_t)S * d)) || (rc = dalloc(c, A, &j->attn, (size_t)S * d)) ||
        (rc = dalloc(c, A, &j->y8, (size_t)S * d)) || (rc = dalloc(c, A, &j->r8, (size_t)S * c->cfg.d_ff)) ||
        (rc = dalloc(c, A, &j->logits, c->head_fused ? 1 : (size_t)S * c->cfg.vocab)) ||
        (rc = dalloc(c, A, &j->rn_ws, std::max<size_t>(gemm_rn_ws_bytes((int)S, (int)d) / 4, 1))) ||
        (rc = dalloc(c, A, &j->kc, L * (size_t)S * c->KH * pad64(Tcap) * 64)) ||
        (rc = dalloc(c, A, &j->vc, L * (size_t)S * c->KH * pad64(Tcap) * 64))) {
        free_job_mem(j.get());
        return rc;
    }
    j->rn_ws_bytes = gemm_rn_ws_bytes((int)S, (int)d);
    hipError_t e = hipSuccess;
    if (total_bytes > 0) e = hipMemcpy(j->d_data, data, (size_t)total_bytes, hipMemcpyHostToDevice);
    if (e == hipSuccess && nchunks > 0) e = hipMemcpy(j->d_offs, offs, (size_t)nchunks * 8, hipMemcpyHostToDevice);
    if (e == hipSuccess && nchunks > 0) e = hipMemcpy(j->d_blen, lens, (size_t)nchunks * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess && nchunks > 0) e = hipMemcpy(j->d_ntok, ntoks, (size_t)nchunks * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess && nchunks > 0) e = hipMemcpy(j->d_toff, toff.data(), (size_t)nchunks * 8, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        free_job_mem(j.get());
        return fail(c, CZIP_E_HIP, hipGetErrorString(e));
    }
    *out = j.release();
    return CZIP_OK;
}

// Streams of a group decoded as independent lanes (contiguous ranges of the
// group, each on its own HIP stream): one lane's kernels fill the others'
// partly empty last rounds of workgroups.  Two lanes measured best (three and
// four lose to their smaller launches).  Not while per-kernel events are
// recorded (they time one stream), nor for groups whose lanes would be small;
// CZIP_DECODE_LANES=n (1..4) sets the number for every group.
constexpr int DEC_LANE_MIN_STREAMS = 16384;
constexpr int DEC_LANES_DEFAULT = 2;

static int decode_lanes(const czip_ctx* c, int S) {
    if (c->profiling) return 1;
    if (c->decode_lanes > 0) return std::min(c->decode_lanes, S);
    return std::max(1, std::min(DEC_LANES_DEFAULT, S / DEC_LANE_MIN_STREAMS));
}

static czip_status run_decompress(czip_job* j) {
    czip_ctx* c = j->ctx;
    const int d = c->cfg.d_model, V = c->cfg.vocab, H = c->cfg.n_heads;
    const int Tc = j->T;
    // KV caches per layer: K and V [S][KH][TP][64] (key-major); TP = the
    // longest stream rounded up to whole 64-key tiles
    const int TP = pad64(Tc);
    const size_t layer_kv = (size_t)j->S * c->KH * TP * 64, stream_kv = (size_t)c->KH * TP * 64;
    for (int64_t g0 = 0; g0 < j->nchunks; g0 += j->S) {
        const int S = (int)std::min<int64_t>(j->S, j->nchunks - g0);
        const int nl = decode_lanes(c, S);
        for (int ln = 1; ln < nl; ln++) {
            if (c->lane_s[ln - 1]) continue;
            if (hipStreamCreateWithFlags(&c->lane_s[ln - 1], hipStreamNonBlocking) != hipSuccess) {
                c->lane_s[ln - 1] = nullptr;
                return fail(c, CZIP_E_HIP, "hipStreamCreateWithFlags");
            }
        }
        for (int e = 0; e < (nl > 1 ? nl : 0); e++) {
            if (c->lane_ev[e]) continue;
            if (hipEventCreateWithFlags(&c->lane_ev[e], hipEventDisableTiming) != hipSuccess) {
                c->lane_ev[e] = nullptr;
                return fail(c, CZIP_E_HIP, "hipEventCreateWithFlags");
            }
        }
        struct Lane {
            int r0, S;
            hipStream_t s;
            RowBufs r;
            DecState st;
            DecStreams ds;
        };
        Lane lanes[DEC_LANES_MAX];
        for (int ln = 0; ln < nl; ln++) {
            Lane& L = lanes[ln];
            L.r0 = (int)((int64_t)S * ln / nl);
            L.S = (int)((int64_t)S * (ln + 1) / nl) - L.r0;
            L.s = ln == 0 ? c->stream : c->lane_s[ln - 1];
            L.r = row_bufs(c, j, L.r0, nl, ln);
            const size_t r0 = (size_t)L.r0;
            L.st = DecState{j->st_low + r0, j->st_high + r0, j->st_code + r0, j->st_bpos + r0, j->st_bit + r0,
                            j->st_plo + r0, j->st_phi + r0};
            L.ds = DecStreams{j->d_data, j->d_offs + g0 + L.r0, j->d_blen + g0 + L.r0, j->d_ntok + g0 + L.r0,
                              j->d_tokens, j->d_toff + g0 + L.r0};
        }
        int steps = 0;
        for (int i = 0; i < S; i++) steps = std::max(steps, j->h_ntok[(size_t)(g0 + i)]);
        if (nl > 1) {  // the other lanes start after what the context's stream holds
            HIPCHECK(c, hipEventRecord(c->lane_ev[0], c->stream));
            for (int ln = 1; ln < nl; ln++) HIPCHECK(c, hipStreamWaitEvent(lanes[ln].s, c->lane_ev[0], 0));
        }
        for (int ln = 0; ln < nl; ln++) {
            Timed t(c, "dec_init");
            launch_dec_init(lanes[ln].st, lanes[ln].ds, lanes[ln].S, lanes[ln].s);
        }
        for (int p = 0; p < steps; p++) {
            for (int ln = 0; ln < nl; ln++) {
                const Lane& Ln = lanes[ln];
                const hipStream_t s = Ln.s;
                const int M = Ln.S;
                {
                    Timed t(c, "dec_prep");
                    launch_dec_prep(Ln.ds, Ln.st, M, p, c->head_fused && p > 0, c->cfg.target_total, Ln.r.inp, s);
                }
                if (!c->rn_fused) {
                    Timed t(c, "embed_norm");
                    launch_embed_norm(Ln.r.inp, c->embed, c->layers[0].attn_norm, M, d, Ln.r.x, Ln.r.xn, s);
                }
                for (int l = 0; l < c->cfg.n_layers; l++) {
                    const DevLayer& L = c->layers[(size_t)l];
                    int8_t* kc = j->kc + (size_t)l * layer_kv + (size_t)Ln.r0 * stream_kv;
                    int8_t* vc = j->vc + (size_t)l * layer_kv + (size_t)Ln.r0 * stream_kv;
                    GemmArgs g{};
                    g.A = Ln.r.xn; g.W = L.qkv_w; g.M = M; g.N = L.qkv_n; g.K = d;
                    g.out8 = Ln.r.q8; g.ldo = d; set_requant(g, L.qkv_mult, L.qkv_shift);
                    g.d = d; g.T = TP; g.TP = TP; g.pos = p; g.vl = DEC_VL; g.kv_mode = c->cfg.kv_mode; g.G = c->cfg.n_kv_heads;
                    g.KH = c->KH; g.kc = kc; g.vc = vc; g.rcos = c->rcos; g.rsin = c->rsin;
                    if (l == 0) {
                        layer0_qkv(c, g, Ln.r.inp, s);
                    } else {
                        Timed t(c, "gemm_qkv");
                        gemm(c, g, EPI_QKV, s);
                    }
                    AttnArgs a{};
                    a.q = Ln.r.q8; a.kc = kc; a.vc = vc; a.TP = TP; a.lens = Ln.ds.ntok; a.score_mult = L.score_mult;
                    a.sink = L.sink; a.lut = c->lut; a.etab = c->etab; a.out = Ln.r.attn; a.M = M; a.T = TP; a.H = H;
                    a.G = c->cfg.n_kv_heads; a.KH = c->KH; a.kv_mode = c->cfg.kv_mode; a.coef = 378194u;
                    a.general = L.attn_general;
                    { Timed t(c, "attn_decode"); launch_attn_decode(a, M, p, s); }
                    post_attention(c, Ln.r, l, M, s, nl > 1);
                }
                if (c->head_fused) {
                    HeadDecArgs h{};
                    h.A = Ln.r.xn; h.W = c->head_wf; h.M = M; h.K = d; h.V = V;
                    h.lut = c->lut; h.coef = c->cfg.coef_q24; h.total = c->cfg.target_total; h.e0 = c->lut0_max; h.p = p;
                    Timed t(c, "head_dec");
                    launch_head_dec(h, Ln.st, Ln.ds, s);
                } else {
                    GemmArgs hd{};
                    hd.A = Ln.r.xn; hd.W = c->head_w; hd.M = M; hd.N = V; hd.K = d;
                    hd.out32 = j->logits + (size_t)Ln.r0 * V; hd.ldo = V;
                    { Timed t(c, "gemm_head"); gemm(c, hd, EPI_RAW, s); }
                    {
                        Timed t(c, "cdf_decode");
                        launch_cdf_decode(hd.out32, M, V, c->lut, c->cfg.coef_q24, c->cfg.target_total, p, Ln.st, Ln.ds, s);
                    }
                }
            }
        }
        for (int ln = 1; ln < nl; ln++) {  // the next group (and the caller) see every lane done
            HIPCHECK(c, hipEventRecord(c->lane_ev[ln], lanes[ln].s));
            HIPCHECK(c, hipStreamWaitEvent(c->stream, c->lane_ev[ln], 0));
        }
    }
    HIPCHECK(c, hipGetLastError());
    HIPCHECK(c, hipStreamSynchronize(c->stream));
    resolve_events(c);
    return CZIP_OK;
}

extern "C" czip_status czip_decompress_fetch(czip_job* j, uint32_t* tokens_out, const int64_t* tok_offs) {
    if (!j || j->kind != 1 || (j->total_tokens > 0 && !tokens_out)) return CZIP_E_ARG;
    czip_ctx* c = j->ctx;
    if (j->total_tokens == 0) return CZIP_OK;
    if (!j->ran) return fail(c, CZIP_E_ARG, "fetch before a successful czip_job_run");
    HIPCHECK(c, hipSetDevice(c->device));
    if (!tok_offs) {
        HIPCHECK(c, hipMemcpy(tokens_out, j->d_tokens, (size_t)j->total_tokens * 4, hipMemcpyDeviceToHost));
        return CZIP_OK;
    }
    std::vector<uint32_t> all((size_t)j->total_tokens);
    HIPCHECK(c, hipMemcpy(all.data(), j->d_tokens, all.size() * 4, hipMemcpyDeviceToHost));
    int64_t src = 0;
    for (int64_t i = 0; i < j->nchunks; i++) {
        memcpy(tokens_out + tok_offs[i], all.data() + src, (size_t)j->h_ntok[(size_t)i] * 4);
        src += j->h_ntok[(size_t)i];
    }
    return CZIP_OK;
}

extern "C" void czip_job_free(czip_job* j) {
    if (!j) return;
    hipSetDevice(j->ctx->device);
    hipStreamSynchronize(j->ctx->stream);
    free_job_mem(j);
    delete j;
}

// ===========================================================================
// Step-wise decode: the caller keeps its own arithmetic decoder and drives
// the per-token loop of main.rs:381-391 for S streams at a time.
// ===========================================================================
static void free_decode_session(czip_ctx* c) {
    if (!c || !c->dec) return;
    free_job_mem(c->dec);
    delete c->dec;
    c->dec = nullptr;
}

extern "C" czip_status czip_decode_begin(czip_ctx* c, int32_t S, int32_t T) {
    if (!c) return CZIP_E_ARG;
    if (S < 1 || T < 1) return fail(c, CZIP_E_ARG, "S and T must be >= 1");
    if ((int64_t)S * c->cfg.d_model > INT32_MAX)
        return fail(c, CZIP_E_RANGE, "S * d_model must stay below 2^31 (decode row offsets are 32-bit)");
    if (T > c->cfg.context_length || T > c->cfg.max_seq_len)
        return fail(c, CZIP_E_RANGE, "T exceeds the RoPE LUT / KV cache (lut.rs:169-177)");
    HIPCHECK(c, hipSetDevice(c->device));
    HIPCHECK(c, hipStreamSynchronize(c->stream));
    free_decode_session(c);
    auto j = std::make_unique<czip_job>();
    j->ctx = c;
    j->kind = 2;
    j->S = S;
    j->T = T;
    const size_t d = (size_t)c->cfg.d_model, L = (size_t)c->cfg.n_layers, V = (size_t)c->cfg.vocab;
    const size_t kv = L * (size_t)S * c->KH * pad64(T) * 64;
    auto& A = j->allocs;
    czip_status rc;
    if ((rc = dalloc(c, A, &j->inp, (size_t)S)) || (rc = dalloc(c, A, &j->d_ntok, (size_t)S)) ||
        (rc = dalloc(c, A, &j->d_val, (size_t)S)) || (rc = dalloc(c, A, &j->d_out, (size_t)S * std::max<size_t>(V, 3))) ||
        (rc = dalloc(c, A, &j->x, (size_t)S * d)) || (rc = dalloc(c, A, &j->xn, (size_t)S * d)) ||
        (rc = dalloc(c, A, &j->q8, (size_t)S * d)) || (rc = dalloc(c, A, &j->attn, (size_t)S * d)) ||
        (rc = dalloc(c, A, &j->y8, (size_t)S * d)) || (rc = dalloc(c, A, &j->r8, (size_t)S * c->cfg.d_ff)) ||
        (rc = dalloc(c, A, &j->logits, (size_t)S * V)) ||
        (rc = dalloc(c, A, &j->rn_ws, std::max<size_t>(gemm_rn_ws_bytes(S, (int)d) / 4, 1))) ||
        (rc = dalloc(c, A, &j->kc, kv)) || (rc = dalloc(c, A, &j->vc, kv))) {
        free_job_mem(j.get());
        return rc;
    }
    j->rn_ws_bytes = gemm_rn_ws_bytes(S, (int)d);
    j->h_lens.assign((size_t)S, -1);
    j->h_done.assign((size_t)S, -1);
    c->dec = j.release();
    return CZIP_OK;
}

extern "C" czip_status czip_decode_step(czip_ctx* c, const uint32_t* tok_in, const int32_t* pos,
                                        const uint32_t* value_or_null, uint32_t* out) {
    if (!c) return CZIP_E_ARG;
    czip_job* j = c->dec;
    if (!j) return fail(c, CZIP_E_ARG, "no decode session (czip_decode_begin)");
    if (!tok_in || !pos || !out) return fail(c, CZIP_E_ARG, "null argument");
    const int S = j->S, V = c->cfg.vocab, d = c->cfg.d_model;
    const size_t orow = value_or_null ? 3 : (size_t)V;
    int p = -1;
    for (int i = 0; i < S; i++) {
        if (pos[i] < -1) return fail(c, CZIP_E_ARG, "pos[s] must be a position or -1");
        if (pos[i] >= 0 && p >= 0 && pos[i] != p)
            return fail(c, CZIP_E_ARG, "every active stream must be at the same position");
        if (pos[i] >= 0) p = pos[i];
    }
    if (p < 0) {
        memset(out, 0, (size_t)S * orow * 4);
        return CZIP_OK;
    }
    if (p >= j->T) return fail(c, CZIP_E_RANGE, "position past the session's T (lut.rs:169-177)");
    for (int i = 0; i < S; i++) {
        if (pos[i] < 0) continue;
        if (tok_in[i] >= (uint32_t)V) return fail(c, CZIP_E_TOKEN, "token id >= vocab at stream " + std::to_string(i));
        // attention at p reads the stream's cached keys 0..p-1
        if (p > 0 && j->h_done[(size_t)i] < p - 1)
            return fail(c, CZIP_E_ARG, "stream " + std::to_string(i) + " is active at position " + std::to_string(p) +
                                           " but its positions before it were never decoded");
    }
    for (int i = 0; i < S; i++)
        if (pos[i] >= 0) j->h_done[(size_t)i] = p == 0 ? 0 : std::max(j->h_done[(size_t)i], p);
    HIPCHECK(c, hipSetDevice(c->device));
    hipStream_t s = c->stream;
    // inactive streams (pos -1) attend to nothing and read token 0; their rows are zeroed below
    std::vector<uint32_t> tin((size_t)S);
    bool lens_changed = false;
    for (int i = 0; i < S; i++) {
        tin[(size_t)i] = pos[i] >= 0 ? tok_in[i] : 0u;
        const int32_t l = pos[i] >= 0 ? j->T : 0;
        lens_changed |= j->h_lens[(size_t)i] != l;
        j->h_lens[(size_t)i] = l;
    }
    HIPCHECK(c, hipMemcpyAsync(j->inp, tin.data(), (size_t)S * 4, hipMemcpyHostToDevice, s));
    if (lens_changed) HIPCHECK(c, hipMemcpyAsync(j->d_ntok, j->h_lens.data(), (size_t)S * 4, hipMemcpyHostToDevice, s));
    if (value_or_null) HIPCHECK(c, hipMemcpyAsync(j->d_val, value_or_null, (size_t)S * 4, hipMemcpyHostToDevice, s));
    const int TP = pad64(j->T);
    const size_t layer_kv = (size_t)S * c->KH * TP * 64;
    if (!c->rn_fused) { Timed t(c, "embed_norm"); launch_embed_norm(j->inp, c->embed, c->layers[0].attn_norm, S, d, j->x, j->xn, s); }
    for (int l = 0; l < c->cfg.n_layers; l++) {
        const DevLayer& L = c->layers[(size_t)l];
        int8_t* kc = j->kc + (size_t)l * layer_kv;
        int8_t* vc = j->vc + (size_t)l * layer_kv;
        GemmArgs g{};
        g.A = j->xn; g.W = L.qkv_w; g.M = S; g.N = L.qkv_n; g.K = d;
        g.out8 = j->q8; g.ldo = d; set_requant(g, L.qkv_mult, L.qkv_shift);
        g.d = d; g.T = TP; g.TP = TP; g.pos = p; g.vl = DEC_VL; g.kv_mode = c->cfg.kv_mode; g.G = c->cfg.n_kv_heads;
        g.KH = c->KH; g.kc = kc; g.vc = vc; g.rcos = c->rcos; g.rsin = c->rsin;
        if (l == 0) {
            layer0_qkv(c, g, j->inp, s);
        } else {
            Timed t(c, "gemm_qkv");
            gemm(c, g, EPI_QKV, s);
        }
        AttnArgs a{};
        a.q = j->q8; a.kc = kc; a.vc = vc; a.TP = TP; a.lens = j->d_ntok; a.score_mult = L.score_mult;
        a.sink = L.sink; a.lut = c->lut; a.etab = c->etab; a.out = j->attn; a.M = S; a.T = TP; a.H = c->cfg.n_heads; a.G = c->cfg.n_kv_heads;
        a.KH = c->KH; a.kv_mode = c->cfg.kv_mode; a.coef = 378194u;  // ATTN_COEF_Q24 (attention.rs:17-19)
        a.general = L.attn_general;
        { Timed t(c, "attn_decode"); launch_attn_decode(a, S, p, s); }
        post_attention(c, row_bufs(c, j), l, S, s);
    }
    {
        GemmArgs hd{};
        hd.A = j->xn; hd.W = c->head_w; hd.M = S; hd.N = V; hd.K = d; hd.out32 = j->logits; hd.ldo = V;
        { Timed t(c, "gemm_head"); gemm(c, hd, EPI_RAW, s); }
        Timed t(c, "cdf");
        launch_cdf(j->logits, S, V, value_or_null ? j->d_val : nullptr, nullptr, 1, c->lut, c->cfg.coef_q24,
                   c->cfg.target_total, value_or_null ? 2 : 1, j->d_out, 0, s);
    }
    HIPCHECK(c, hipGetLastError());
    HIPCHECK(c, hipMemcpyAsync(out, j->d_out, (size_t)S * orow * 4, hipMemcpyDeviceToHost, s));
    HIPCHECK(c, hipStreamSynchronize(s));
    resolve_events(c);
    for (int i = 0; i < S; i++)
        if (pos[i] < 0) memset(out + (size_t)i * orow, 0, orow * 4);
    return CZIP_OK;
}

extern "C" void czip_decode_end(czip_ctx* c) {
    if (!c) return;
    hipSetDevice(c->device);
    hipStreamSynchronize(c->stream);
    free_decode_session(c);
}

// ===========================================================================
// czip_prefill_cdf without allocation: the same intervals, with every
// intermediate in the device's fixed `scratch` buffer
// ===========================================================================
namespace {

// Bump allocator over a fixed buffer (base == nullptr: size only).
struct Carve {
    uint8_t* base;
    size_t off = 0;
    template <typename T>
    T* take(size_t count) {
        T* p = base ? (T*)(base + off) : nullptr;
        off += (std::max<size_t>(count * sizeof(T), 1) + 255) & ~(size_t)255;
        return p;
    }
};

// the forward's buffers for B chunks of T rows (alloc_scratch's set, less
// what the fused kernels never touch) plus the row prep's
int32_t* carve_prefill(czip_ctx* c, czip_job* j, Carve& cv, int B, int T) {
    const size_t M = (size_t)B * T, d = (size_t)c->cfg.d_model, F = (size_t)c->cfg.d_ff, V = (size_t)c->cfg.vocab;
    int32_t* err = cv.take<int32_t>(1);
    j->inp = cv.take<uint32_t>(M);
    j->tgt = cv.take<uint32_t>(M);
    j->lens = cv.take<int32_t>((size_t)B);
    j->x = cv.take<int16_t>(M * d);
    j->xn = cv.take<int8_t>(M * d);
    j->q8 = cv.take<int8_t>(M * d);
    j->attn = cv.take<int8_t>(M * d);
    j->y8 = c->rn_fused ? nullptr : cv.take<int8_t>(M * d);
    j->r8 = cv.take<int8_t>(M * F);
    j->kc = cv.take<int8_t>(M * (size_t)c->KH * 64);
    j->vc = cv.take<int8_t>((size_t)B * pad64(T) * (size_t)c->KH * 64);
    j->logits = c->head_fused ? nullptr : cv.take<int32_t>(M * V);
    return err;
}

}  // namespace

extern "C" czip_status czip_prefill_cdf_noalloc(czip_ctx* c, const uint32_t* d_targets, const int32_t* d_lens,
                                                int32_t B, int32_t T, uint32_t* d_cum_lohi) {
    if (!c) return CZIP_E_ARG;
    if (!d_targets || !d_lens || !d_cum_lohi || B < 0) return fail(c, CZIP_E_ARG, "null argument");
    if (((uintptr_t)d_targets & 3) || ((uintptr_t)d_lens & 3) || ((uintptr_t)d_cum_lohi & 7))
        return fail(c, CZIP_E_ARG, "targets / lens must be 4-byte and cum_lohi 8-byte aligned");
    if (B == 0) return CZIP_OK;
    if (T < 1) return fail(c, CZIP_E_ARG, "T must be >= 1");
    if (T > c->cfg.context_length || T > c->cfg.max_seq_len)
        return fail(c, CZIP_E_RANGE, "chunk length exceeds the RoPE LUT / KV cache (lut.rs:169-177)");
    if ((uint32_t)c->cfg.vocab <= BOS) return fail(c, CZIP_E_TOKEN, "BOS token 1022 is outside the vocabulary");
    if (!c->noalloc) return fail(c, CZIP_E_HIP, "no scratch buffer on this device: " + c->noalloc_err);
    czip_job j;
    j.ctx = c;
    Carve size{nullptr};
    carve_prefill(c, &j, size, B, T);
    if (size.off > NOALLOC_SCRATCH_BYTES)
        return fail(c, CZIP_E_RANGE,
                    "B * T = " + std::to_string((long long)B * T) + " rows need " + std::to_string(size.off) +
                        " bytes of scratch; the no-alloc entry point holds " + std::to_string(NOALLOC_SCRATCH_BYTES));
    HIPCHECK(c, hipSetDevice(c->device));
    // the context's stream does not wait for the caller's streams (it is a
    // non-blocking stream): finish everything queued on the device, so inputs
    // that the caller produced asynchronously have landed before they are read
    HIPCHECK(c, hipDeviceSynchronize());
    hipStream_t s = c->stream;
    Carve cv{c->noalloc};
    int32_t* err = carve_prefill(c, &j, cv, B, T);
    const int M = B * T, V = c->cfg.vocab;
    launch_prep_rows(d_targets, d_lens, B, T, V, j.inp, j.tgt, j.lens, d_cum_lohi, err, s);
    czip_status rc = forward_batch(c, &j, B, T, !c->head_fused);
    if (rc) return rc;
    if (c->head_fused) {
        HeadCdfArgs h{};
        h.A = j.xn; h.W = c->head_wf; h.M = M; h.K = c->cfg.d_model; h.V = V; h.targets = j.tgt; h.lens = j.lens;
        h.T = T; h.lut = c->lut; h.coef = c->cfg.coef_q24; h.total = c->cfg.target_total; h.e0 = c->lut0_max;
        h.out = d_cum_lohi; h.out_row0 = 0;
        Timed t(c, "head_cdf");
        launch_head_cdf(h, s);
    } else {
        Timed t(c, "cdf");
        launch_cdf(j.logits, M, V, j.tgt, j.lens, T, c->lut, c->cfg.coef_q24, c->cfg.target_total, 0, d_cum_lohi, 0, s);
    }
    HIPCHECK(c, hipGetLastError());
    int32_t h_err = 0;
    HIPCHECK(c, hipMemcpyAsync(&h_err, err, 4, hipMemcpyDeviceToHost, s));
    HIPCHECK(c, hipStreamSynchronize(s));
    resolve_events(c);
    if (h_err) return fail(c, CZIP_E_TOKEN, "a target id >= vocab in a live row");
    return CZIP_OK;
}
