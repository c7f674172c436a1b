/*
 * czip_oracle.c -- CPU oracle (test infrastructure only; see czip_oracle.h).
 *
 * A literal restatement of the reference Rust crate.  Signed-overflow is
 * avoided by doing wrapping arithmetic in unsigned types, which reproduces
 * Rust's `--release` wrap-around (rust/Cargo.toml:29-31 enables no overflow
 * checks) without C undefined behaviour.
 */
#include "czip_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#define HEAD_DIM 64
#define HALF_DIM 32

static inline int32_t wsub32(int32_t a, int32_t b) { return (int32_t)((uint32_t)a - (uint32_t)b); }
static inline int32_t wadd32(int32_t a, int32_t b) { return (int32_t)((uint32_t)a + (uint32_t)b); }
static inline int32_t wmul32(int32_t a, int32_t b) { return (int32_t)((uint32_t)a * (uint32_t)b); }

/* primitives.rs:9-11 */
int8_t orc_clamp_i8(int32_t x) { return (int8_t)(x < -127 ? -127 : (x > 127 ? 127 : x)); }

/* primitives.rs:18-42 */
int32_t orc_sra_rne_s32(int32_t v, uint32_t sh) {
    if (sh == 0) return v;
    int32_t sign = v >> 31;
    uint32_t av = (uint32_t)wsub32(v ^ sign, sign);
    uint32_t mask = (1u << sh) - 1u;
    uint32_t r = av & mask;
    uint32_t q = av >> sh;
    uint32_t half = 1u << (sh - 1);
    if (r > half) q += 1;
    else if (r == half) q += q & 1u;
    int32_t out = (int32_t)q;
    return wsub32(out ^ sign, sign);
}

/* primitives.rs:49-73 */
int32_t orc_sra_rne_s64_to_s32(int64_t v, uint32_t sh) {
    if (sh == 0) return (int32_t)(v < INT32_MIN ? INT32_MIN : (v > INT32_MAX ? INT32_MAX : v));
    int64_t sign = v >> 63;
    uint64_t av = (uint64_t)((uint64_t)(v ^ sign) - (uint64_t)sign);
    uint64_t mask = (1ull << sh) - 1ull;
    uint64_t r = av & mask;
    uint64_t q = av >> sh;
    uint64_t half = 1ull << (sh - 1);
    if (r > half) q += 1;
    else if (r == half) q += q & 1ull;
    int64_t out = (int64_t)q;
    int64_t so = (int64_t)((uint64_t)(out ^ sign) - (uint64_t)sign);
    return (int32_t)(so < INT32_MIN ? INT32_MIN : (so > INT32_MAX ? INT32_MAX : so));
}

/* primitives.rs:80-97 */
uint32_t orc_udiv_rne_u32(uint32_t n, uint32_t d) {
    if (d == 0) return 0;
    uint32_t q = n / d;
    uint32_t r = n - q * d;
    uint32_t tr = r << 1;
    if (tr > d) return q + 1;
    if (tr == d) return q + (q & 1u);
    return q;
}

/* primitives.rs:103-125 */
int32_t orc_div_rne_s32(int32_t num, int32_t denom) {
    if (denom == 0) return 0;
    int32_t sign = ((num < 0) != (denom < 0)) ? -1 : 1;
    uint32_t an = num < 0 ? 0u - (uint32_t)num : (uint32_t)num;
    uint32_t ad = denom < 0 ? 0u - (uint32_t)denom : (uint32_t)denom;
    uint32_t q = an / ad;
    uint32_t r = an - q * ad;
    uint32_t tr = r << 1;
    uint32_t rq = tr > ad ? q + 1 : (tr == ad ? q + (q & 1u) : q);
    return wmul32((int32_t)rq, sign);
}

/* primitives.rs:163-185 */
int32_t orc_div_rne_s32_by_u64(int32_t num, uint64_t denom) {
    if (denom == 0) return 0;
    int32_t sign = num < 0 ? -1 : 1;
    uint64_t an = (uint64_t)(num < 0 ? 0u - (uint32_t)num : (uint32_t)num);
    uint64_t q = an / denom;
    uint64_t r = an - q * denom;
    uint64_t tr = r << 1;
    uint64_t rq = tr > denom ? q + 1 : (tr == denom ? q + (q & 1ull) : q);
    return wmul32((int32_t)(uint32_t)rq, sign);
}

/* primitives.rs:192-213 */
uint32_t orc_isqrt32(uint32_t x) {
    uint32_t op = x, res = 0, one = 1u << 30;
    while (one > op) one >>= 2;
    while (one != 0) {
        if (op >= res + one) { op -= res + one; res = (res >> 1) + one; }
        else res >>= 1;
        one >>= 2;
    }
    return res;
}

/* primitives.rs:278-295 */
size_t orc_argmax(const int32_t* a, size_t n) {
    if (n == 0) return 0;
    size_t mi = 0; int32_t mv = a[0];
    for (size_t i = 1; i < n; i++) if (a[i] > mv) { mv = a[i]; mi = i; }
    return mi;
}

/* lut.rs:192-209 (off the hot path; kept for the reference KATs) */
int32_t orc_exp_q16_from_neg_fixed(int32_t neg_x_q8, const uint16_t* lut) {
    uint32_t nx = neg_x_q8 < 0 ? 0u : (uint32_t)neg_x_q8;
    uint32_t ip = nx >> 8;
    uint32_t fr = nx & 255u;
    if (ip >= 16) return 0;
    return (int32_t)lut[fr] >> ip;
}

/* lut.rs:213-235 and softmax_cdf.rs:55-77 (identical bodies) */
uint16_t orc_exp_q16_coef(int32_t diff, const uint16_t* lut, uint32_t coef_q24) {
    if (diff >= 0) return 65535;
    uint32_t neg = 0u - (uint32_t)diff;
    uint32_t t256 = (uint32_t)(((uint64_t)neg * (uint64_t)coef_q24 + (1ull << 23)) >> 24);
    uint32_t ip = t256 >> 8;
    uint32_t fr = t256 & 255u;
    if (ip >= 31) return 1;
    uint32_t base = (1u << 16) >> ip;
    uint32_t out = (base * (uint32_t)lut[fr] + 0x8000u) >> 16;
    if (out < 1) out = 1;
    if (out > 65535) out = 65535;
    return (uint16_t)out;
}

/* attention.rs:17-19: ATTN_COEF_Q24 = (LOG2E/64 * 2^24 + 0.5) as u32 */
uint32_t orc_attn_coef_q24(void) {
    const double log2e = 1.4426950408889634;
    return (uint32_t)((log2e / 64.0) * (double)(1ull << 24) + 0.5);
}

/* softmax_cdf.rs:23-28 (f64::round rounds half away from zero) */
uint32_t orc_cdf_coef_q24(void) {
    const double log2e = 1.4426950408889634;
    double c = (0.1 * log2e) / 64.0 * (double)(1u << 24);
    uint32_t r = (uint32_t)round(c);
    return r < 1 ? 1 : r;
}

/* softmax_cdf.rs:39-46 */
uint32_t orc_target_total(uint32_t vocab) {
    uint32_t q = 1u << 30;
    uint32_t t = q > vocab ? q - vocab : 0;
    t = t > 1024 ? t - 1024 : 0;
    return t > vocab + 1 ? t : vocab + 1;
}

/* primitives.rs:260-275 (host-side rounding used by the LUT generators) */
static int64_t round_tte_host(double x) {
    double rounded = round(x);
    double fl = floor(x);
    double diff = x - fl;
    if (fabs(diff - 0.5) < 2.220446049250313e-16) {
        return (((int64_t)fl) & 1) == 0 ? (int64_t)fl : (int64_t)ceil(x);
    }
    return (int64_t)rounded;
}

/* lut.rs:40-52 */
void orc_gen_exp2_lut(uint16_t* out) {
    for (int i = 0; i < 256; i++) {
        double v = pow(2.0, -((double)i / 256.0)) * 65536.0;
        int64_t q = round_tte_host(v);
        out[i] = (uint16_t)(q < 1 ? 1 : (q > 65535 ? 65535 : q));
    }
}

/* lut.rs:97-136 */
void orc_gen_rope_lut(double theta, int max_seq, int16_t* cs, int16_t* sn) {
    for (int p = 0; p < max_seq; p++)
        for (int i = 0; i < HALF_DIM; i++) {
            double freq = 1.0 / pow(theta, (double)(2 * i) / 64.0);
            double ang = (double)p * freq;
            int64_t c = round_tte_host(cos(ang) * 32768.0);
            int64_t s = round_tte_host(sin(ang) * 32768.0);
            cs[p * HALF_DIM + i] = (int16_t)(c < -32768 ? -32768 : (c > 32767 ? 32767 : c));
            sn[p * HALF_DIM + i] = (int16_t)(s < -32768 ? -32768 : (s > 32767 ? 32767 : s));
        }
}

/* rmsnorm.rs:14-30 */
int32_t orc_inv_rms_q15(int32_t mean_sq) {
    uint32_t ms = mean_sq > 0 ? (uint32_t)mean_sq : 1u;
    uint32_t xs = ms << 16;
    uint32_t s = orc_isqrt32(xs);
    uint32_t inv = orc_udiv_rne_u32(8388608u, s);
    if (inv < 1) inv = 1;
    if (inv > 32768) inv = 32768;
    return (int32_t)inv;
}

/* rmsnorm.rs:40-75 (single row) */
void orc_rmsnorm_i8_to_i8(const int8_t* x, const int8_t* w, int d, int32_t eps, int8_t* out) {
    uint32_t ss = 0;
    for (int i = 0; i < d; i++) ss += (uint32_t)((int32_t)x[i] * (int32_t)x[i]);
    int32_t mean_sq = wadd32((int32_t)(ss / (uint32_t)d), eps);
    if (mean_sq < 1) mean_sq = 1;
    int32_t inv = orc_inv_rms_q15(mean_sq);
    for (int i = 0; i < d; i++) {
        int32_t tmp = wmul32((int32_t)x[i] * (int32_t)w[i], inv);
        out[i] = orc_clamp_i8(orc_sra_rne_s32(tmp, 15));
    }
}

/* linear.rs:12-31 */
void orc_linear_i8_to_i32(const int8_t* x, const int8_t* w, int b, int in_dim, int out_dim, int32_t* out) {
    for (int bb = 0; bb < b; bb++) {
        const int8_t* xr = x + (size_t)bb * in_dim;
        for (int o = 0; o < out_dim; o++) {
            const int8_t* wr = w + (size_t)o * in_dim;
            int32_t acc = 0;
            for (int i = 0; i < in_dim; i++) acc += (int32_t)xr[i] * (int32_t)wr[i];
            out[(size_t)bb * out_dim + o] = acc;
        }
    }
}

/* model.rs:280-300 */
void orc_requant(const int32_t* x, int n, int32_t mult, int8_t shift, int8_t* out) {
    for (int i = 0; i < n; i++) {
        int64_t p = (int64_t)x[i] * (int64_t)mult;
        int64_t r;
        if (shift <= 0) r = p;
        else r = orc_sra_rne_s64_to_s32(p, (uint32_t)shift);
        out[i] = (int8_t)(r < -127 ? -127 : (r > 127 ? 127 : r));
    }
}

/* reglu.rs:20-46 (single row) */
void orc_reglu(const int8_t* x, int d_ff, int8_t* out) {
    for (int i = 0; i < d_ff; i++) {
        int32_t g = x[i], u = x[d_ff + i];
        int32_t gr = g > 0 ? g : 0;
        out[i] = orc_clamp_i8(orc_sra_rne_s32(gr * u, 7));
    }
}

/* attention.rs:29-50 */
void orc_rope_k(int8_t* x, const int16_t* c, const int16_t* s) {
    for (int i = 0; i < HALF_DIM; i++) {
        int32_t xv = x[i], yv = x[i + HALF_DIM];
        int32_t ci = c[i], si = s[i];
        int32_t xr = wsub32(xv * ci, yv * si);
        int32_t yr = wadd32(xv * si, yv * ci);
        x[i] = orc_clamp_i8(orc_sra_rne_s32(xr, 15));
        x[i + HALF_DIM] = orc_clamp_i8(orc_sra_rne_s32(yr, 15));
    }
}

/* attention.rs:53-83 (NET_SHIFT = SQRT_HEAD_DIM_SHIFT - Q_SHIFT = 1) */
void orc_rope_q(int8_t* x, const int16_t* c, const int16_t* s) {
    for (int i = 0; i < HALF_DIM; i++) {
        int32_t xv = x[i], yv = x[i + HALF_DIM];
        int32_t ci = c[i], si = s[i];
        int32_t xr = orc_sra_rne_s32(wsub32(xv * ci, yv * si), 15);
        int32_t yr = orc_sra_rne_s32(wadd32(xv * si, yv * ci), 15);
        xr = orc_sra_rne_s32(xr, 1);
        yr = orc_sra_rne_s32(yr, 1);
        x[i] = orc_clamp_i8(xr);
        x[i + HALF_DIM] = orc_clamp_i8(yr);
    }
}

/* attention.rs:88-97 */
static int32_t qk_dot(const int8_t* q, const int8_t* k) {
    int32_t dot = 0;
    for (int i = 0; i < HEAD_DIM; i++) dot += (int32_t)q[i] * (int32_t)k[i];
    return dot;
}

/* softmax_cdf.rs:85-139 */
void orc_build_cumfreqs(const int32_t* logits, int v, const uint16_t* lut, uint32_t coef,
                        uint32_t target_total, uint32_t* cum) {
    int32_t mx = logits[0];
    for (int i = 1; i < v; i++) if (logits[i] > mx) mx = logits[i];
    size_t am = orc_argmax(logits, (size_t)v);
    uint16_t* e = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)v);
    uint64_t sum = 0;
    for (int i = 0; i < v; i++) {
        e[i] = orc_exp_q16_coef(wsub32(logits[i], mx), lut, coef);
        sum += e[i];
    }
    uint64_t rem_tot = (uint64_t)target_total - (uint64_t)v;
    uint64_t fsum = 0;
    uint32_t* f = cum; /* build freqs in place, then prefix-sum */
    for (int i = 0; i < v; i++) {
        uint64_t extra = ((uint64_t)e[i] * rem_tot) / sum;
        f[i] = 1u + (uint32_t)extra;
        fsum += f[i];
    }
    uint64_t rem = (uint64_t)target_total - fsum;
    f[am] += (uint32_t)rem;
    uint32_t run = 0;
    for (int i = 0; i < v; i++) { run += f[i]; cum[i] = run; }
    free(e);
}

/* ------------------------------------------------------------------ */
/* Model                                                              */
/* ------------------------------------------------------------------ */

struct orc_state {
    const orc_model* m;
    int kv_heads;        /* heads stored in the cache per layer */
    int8_t* k;           /* [L][max_seq][kv_heads*64] */
    int8_t* v;
    int32_t* x; int8_t* xi8; int8_t* nrm; int32_t* qkv32; int8_t* qkv8;
    int8_t* attn; int32_t* o32; int8_t* o8; int32_t* up32; int8_t* up8; int8_t* r8;
    int32_t* dn32; int8_t* dn8;
};

static int kv_heads_of(const orc_model* m) { return m->kv_mode == ORC_KV_GQA ? m->n_kv_heads : 1; }

int orc_model_check(const orc_model* m) {
    if (m->head_dim != HEAD_DIM) return -2;
    if (m->d_model != m->n_heads * HEAD_DIM) return -2;
    if (m->kv_mode == ORC_KV_RUST_COMPAT) {
        /* attention.rs:172 */
        if (!(m->n_heads == 4 || m->n_heads == 6 || m->n_heads == 8)) return -3;
        /* attention.rs:176: b = len / (d + 128) must be exactly one row */
        int len = m->d_model + 2 * m->n_kv_heads * HEAD_DIM;
        if (len / (m->d_model + 2 * HEAD_DIM) != 1) return -3;
    } else {
        if (m->n_kv_heads < 1 || m->n_heads % m->n_kv_heads != 0) return -3;
    }
    return 0;
}

orc_state* orc_state_new(const orc_model* m) {
    orc_state* s = (orc_state*)calloc(1, sizeof(orc_state));
    s->m = m;
    s->kv_heads = kv_heads_of(m);
    size_t kvsz = (size_t)m->n_layers * (size_t)m->max_seq_len * (size_t)s->kv_heads * HEAD_DIM;
    s->k = (int8_t*)calloc(kvsz, 1);
    s->v = (int8_t*)calloc(kvsz, 1);
    int d = m->d_model, F = m->d_ff, G = m->n_kv_heads;
    int qkvn = d + 2 * G * HEAD_DIM;
    s->x = (int32_t*)calloc((size_t)d, 4);
    s->xi8 = (int8_t*)calloc((size_t)d, 1);
    s->nrm = (int8_t*)calloc((size_t)d, 1);
    s->qkv32 = (int32_t*)calloc((size_t)qkvn, 4);
    s->qkv8 = (int8_t*)calloc((size_t)qkvn, 1);
    s->attn = (int8_t*)calloc((size_t)d, 1);
    s->o32 = (int32_t*)calloc((size_t)d, 4);
    s->o8 = (int8_t*)calloc((size_t)d, 1);
    s->up32 = (int32_t*)calloc((size_t)2 * F, 4);
    s->up8 = (int8_t*)calloc((size_t)2 * F, 1);
    s->r8 = (int8_t*)calloc((size_t)F, 1);
    s->dn32 = (int32_t*)calloc((size_t)d, 4);
    s->dn8 = (int8_t*)calloc((size_t)d, 1);
    return s;
}

void orc_state_reset(orc_state* s) {
    const orc_model* m = s->m;
    size_t kvsz = (size_t)m->n_layers * (size_t)m->max_seq_len * (size_t)s->kv_heads * HEAD_DIM;
    memset(s->k, 0, kvsz);
    memset(s->v, 0, kvsz);
}

void orc_state_free(orc_state* s) {
    if (!s) return;
    free(s->k); free(s->v); free(s->x); free(s->xi8); free(s->nrm); free(s->qkv32); free(s->qkv8);
    free(s->attn); free(s->o32); free(s->o8); free(s->up32); free(s->up8); free(s->r8);
    free(s->dn32); free(s->dn8); free(s);
}

/* Number of vacc additions whose exact sum left the i32 range (and so
 * wrapped, as a Rust --release build does), over every attend_head call of
 * the process.  Instrumentation for the tests; not part of the algorithm. */
static int64_t g_vacc_wraps = 0;
int64_t orc_vacc_wraps(void) { return __atomic_load_n(&g_vacc_wraps, __ATOMIC_RELAXED); }
void orc_vacc_wraps_reset(void) { __atomic_store_n(&g_vacc_wraps, 0, __ATOMIC_RELAXED); }

/* Online-softmax attention of one query head over cache rows 0..=step
 * (attention.rs:197-285).  q is already rotated. */
static void attend_head(const int8_t* q_rot, const int8_t* kc, const int8_t* vc, int stride,
                        int step, int32_t mult, const int8_t* sink, const uint16_t* lut,
                        uint32_t coef, int8_t* out, int32_t* vacc_out, uint64_t* s_out) {
    int64_t wraps = 0;
    int32_t m = INT32_MIN;
    uint64_t S = 0;
    int32_t vacc[HEAD_DIM];
    memset(vacc, 0, sizeof(vacc));
    if (sink) {                                   /* attention.rs:211-224 */
        int32_t dot = qk_dot(q_rot, sink);
        int32_t du = orc_sra_rne_s32(dot, 2);
        int32_t sc = orc_sra_rne_s64_to_s32((int64_t)du * (int64_t)mult, 15);
        m = sc;
        S = orc_exp_q16_coef(0, lut, coef);
    }
    for (int t = 0; t <= step; t++) {
        const int8_t* k = kc + (size_t)t * stride;
        int32_t dot = qk_dot(q_rot, k);
        int32_t du = orc_sra_rne_s32(dot, 2);
        int32_t score = orc_sra_rne_s64_to_s32((int64_t)du * (int64_t)mult, 15);
        if (score > m) {
            if (m != INT32_MIN) {
                uint16_t so = orc_exp_q16_coef(wsub32(m, score), lut, coef);
                S = (S * (uint64_t)so + 0x8000ull) >> 16;
                for (int i = 0; i < HEAD_DIM; i++) {
                    int64_t p = (int64_t)vacc[i] * (int64_t)so;
                    int64_t adj = p >= 0 ? p + (1ll << 15) : p - (1ll << 15);
                    vacc[i] = (int32_t)(adj >> 16);
                }
            }
            m = score;
        }
        uint16_t w = orc_exp_q16_coef(wsub32(score, m), lut, coef);
        S += w;
        const int8_t* v = vc + (size_t)t * stride;
        for (int i = 0; i < HEAD_DIM; i++) {
            int64_t exact = (int64_t)vacc[i] + (int64_t)w * (int64_t)v[i];
            vacc[i] = wadd32(vacc[i], (int32_t)w * (int32_t)v[i]);
            wraps += exact != (int64_t)vacc[i];
        }
    }
    uint64_t den = S == 0 ? 1 : S;
    for (int i = 0; i < HEAD_DIM; i++) out[i] = orc_clamp_i8(orc_div_rne_s32_by_u64(vacc[i], den));
    if (vacc_out) memcpy(vacc_out, vacc, sizeof(vacc));
    if (s_out) *s_out = S;
    if (wraps) __atomic_add_fetch(&g_vacc_wraps, wraps, __ATOMIC_RELAXED);
}

void orc_attend_head(const int8_t* q_rot, const int8_t* k, const int8_t* v, int n_keys, int32_t score_mult,
                     const int8_t* sink, const uint16_t* lut, int8_t* out, int32_t* vacc_out, uint64_t* s_out) {
    attend_head(q_rot, k, v, HEAD_DIM, n_keys - 1, score_mult, sink, lut, orc_attn_coef_q24(), out, vacc_out, s_out);
}

int orc_forward(orc_state* s, uint32_t token, int pos, int32_t* logits) {
    const orc_model* m = s->m;
    int rc = orc_model_check(m);
    if (rc) return rc;
    if (pos < 0 || pos >= m->context_length || pos >= m->max_seq_len) return -4;
    if ((int)token >= m->vocab) return -5;
    const int d = m->d_model, F = m->d_ff, H = m->n_heads, G = m->n_kv_heads;
    const int kvdim = G * HEAD_DIM;
    const int qkvn = d + 2 * kvdim;
    const int32_t eps = 1; /* compute_eps_scaled(1e-5), rmsnorm.rs:80-83 */
    const uint32_t acoef = orc_attn_coef_q24();
    const int16_t* cs = m->rope_cos + (size_t)pos * HALF_DIM;
    const int16_t* sn = m->rope_sin + (size_t)pos * HALF_DIM;
    const int KH = s->kv_heads;
    const int kstride = KH * HEAD_DIM;

    for (int i = 0; i < d; i++) s->x[i] = m->embed[(size_t)token * d + i];   /* model.rs:372-374 */
    for (int l = 0; l < m->n_layers; l++) {
        const orc_layer* L = &m->layers[l];
        for (int i = 0; i < d; i++) s->xi8[i] = orc_clamp_i8(s->x[i]);          /* model.rs:384 */
        orc_rmsnorm_i8_to_i8(s->xi8, L->attn_norm, d, eps, s->nrm);
        orc_linear_i8_to_i32(s->nrm, L->qkv_w, 1, d, qkvn, s->qkv32);          /* model.rs:389 */
        orc_requant(s->qkv32, qkvn, L->qkv_mult, (int8_t)L->qkv_shift, s->qkv8); /* model.rs:397-399 */

        int8_t* kc = s->k + (size_t)l * m->max_seq_len * kstride;
        int8_t* vc = s->v + (size_t)l * m->max_seq_len * kstride;
        /* K rotate + store, V store (attention.rs:186-194) */
        for (int g = 0; g < KH; g++) {
            int8_t kr[HEAD_DIM];
            const int8_t* ksrc; const int8_t* vsrc;
            if (m->kv_mode == ORC_KV_GQA) {
                ksrc = s->qkv8 + d + g * HEAD_DIM;
                vsrc = s->qkv8 + d + kvdim + g * HEAD_DIM;
            } else {  /* MQA slicing of the concatenated [q | k | v] (attention.rs:182-194) */
                ksrc = s->qkv8 + d;
                vsrc = s->qkv8 + d + HEAD_DIM;
            }
            memcpy(kr, ksrc, HEAD_DIM);
            orc_rope_k(kr, cs, sn);
            memcpy(kc + (size_t)pos * kstride + g * HEAD_DIM, kr, HEAD_DIM);
            memcpy(vc + (size_t)pos * kstride + g * HEAD_DIM, vsrc, HEAD_DIM);
        }
        for (int h = 0; h < H; h++) {
            int8_t qr[HEAD_DIM];
            memcpy(qr, s->qkv8 + h * HEAD_DIM, HEAD_DIM);
            orc_rope_q(qr, cs, sn);
            int g = (m->kv_mode == ORC_KV_GQA) ? (h * G) / H : 0;
            attend_head(qr, kc + g * HEAD_DIM, vc + g * HEAD_DIM, kstride, pos, L->score_mult[h],
                        L->sink_key, m->exp2_lut, acoef, s->attn + h * HEAD_DIM, NULL, NULL);
        }
        orc_linear_i8_to_i32(s->attn, L->out_w, 1, d, d, s->o32);             /* model.rs:424-425 */
        orc_requant(s->o32, d, L->out_mult, (int8_t)L->out_shift, s->o8);
        orc_rmsnorm_i8_to_i8(s->o8, L->ffn_norm, d, eps, s->nrm);              /* model.rs:429 */
        for (int i = 0; i < d; i++) s->x[i] = wadd32(s->x[i], s->nrm[i]);
        for (int i = 0; i < d; i++) s->xi8[i] = orc_clamp_i8(s->x[i]);          /* model.rs:438-439 */
        orc_rmsnorm_i8_to_i8(s->xi8, L->post_attn_norm, d, eps, s->nrm);
        orc_linear_i8_to_i32(s->nrm, L->up_w, 1, d, 2 * F, s->up32);           /* model.rs:443-450 */
        orc_requant(s->up32, 2 * F, L->up_mult, (int8_t)L->up_shift, s->up8);
        orc_reglu(s->up8, F, s->r8);                                            /* model.rs:453-456 */
        orc_linear_i8_to_i32(s->r8, L->down_w, 1, F, d, s->dn32);              /* model.rs:459-460 */
        orc_requant(s->dn32, d, L->down_mult, (int8_t)L->down_shift, s->dn8);
        orc_rmsnorm_i8_to_i8(s->dn8, L->post_ffn_norm, d, eps, s->nrm);         /* model.rs:463-468 */
        for (int i = 0; i < d; i++) s->x[i] = wadd32(s->x[i], s->nrm[i]);
    }
    for (int i = 0; i < d; i++) s->xi8[i] = orc_clamp_i8(s->x[i]);              /* model.rs:473-477 */
    orc_rmsnorm_i8_to_i8(s->xi8, m->final_norm, d, eps, s->nrm);
    orc_linear_i8_to_i32(s->nrm, m->head_w, 1, d, m->vocab, logits);
    return 0;
}

/* ------------------------------------------------------------------ */
/* Arithmetic coder (arith_coder.rs)                                  */
/* ------------------------------------------------------------------ */
#define STATE_MASK 0xFFFFFFFFull
#define HALF_R (1ull << 31)
#define QUARTER_R (1ull << 30)

void orc_enc_init(orc_encoder* e) {
    e->low = 0; e->high = STATE_MASK; e->underflow = 0;
    e->cap = 256; e->len = 0; e->out = (uint8_t*)malloc(e->cap);
    e->cur = 0; e->bit_pos = 7;
}
void orc_enc_free(orc_encoder* e) { free(e->out); e->out = NULL; }

static void push_byte(orc_encoder* e, uint8_t b) {
    if (e->len == e->cap) { e->cap *= 2; e->out = (uint8_t*)realloc(e->out, e->cap); }
    e->out[e->len++] = b;
}
/* arith_coder.rs:51-62 */
static void emit_bit(orc_encoder* e, int bit) {
    if (bit) e->cur |= (uint8_t)(1u << e->bit_pos);
    e->bit_pos -= 1;
    if (e->bit_pos < 0) { push_byte(e, e->cur); e->cur = 0; e->bit_pos = 7; }
}
/* arith_coder.rs:66-73 */
static void emit_bit_uf(orc_encoder* e, int bit) {
    emit_bit(e, bit);
    for (uint32_t i = 0; i < e->underflow; i++) emit_bit(e, bit ^ 1);
    e->underflow = 0;
}
/* arith_coder.rs:101-119 */
static void enc_renorm(orc_encoder* e) {
    for (;;) {
        if (((e->low ^ e->high) & HALF_R) == 0) {
            emit_bit_uf(e, (int)((e->low >> 31) & 1));
            e->low = (e->low << 1) & STATE_MASK;
            e->high = ((e->high << 1) & STATE_MASK) | 1;
        } else if ((e->low & ~e->high & QUARTER_R) != 0) {
            e->underflow += 1;
            e->low = ((e->low << 1) ^ HALF_R) & STATE_MASK;
            e->high = (((e->high ^ HALF_R) << 1) | HALF_R | 1) & STATE_MASK;
        } else break;
    }
}
/* arith_coder.rs:80-98 (cumulative range form) */
void orc_enc_encode_range(orc_encoder* e, uint64_t lo, uint64_t hi, uint64_t total) {
    uint64_t range = e->high - e->low + 1;
    e->high = e->low + (hi * range / total) - 1;
    e->low = e->low + (lo * range / total);
    enc_renorm(e);
}
void orc_enc_encode(orc_encoder* e, const uint32_t* cum, int v, int sym) {
    uint64_t total = cum[v - 1];
    uint64_t hi = cum[sym];
    uint64_t lo = sym > 0 ? cum[sym - 1] : 0;
    orc_enc_encode_range(e, lo, hi, total);
}
/* arith_coder.rs:122-130 */
void orc_enc_finish(orc_encoder* e) {
    emit_bit(e, 1);
    if (e->bit_pos < 7) push_byte(e, e->cur);
}

/* arith_coder.rs:176-190 */
static int read_bit(orc_decoder* d) {
    if (d->byte_pos >= d->len) return 0;
    int bit = (d->in[d->byte_pos] >> d->bit_pos) & 1;
    d->bit_pos -= 1;
    if (d->bit_pos < 0) { d->byte_pos += 1; d->bit_pos = 7; }
    return bit;
}
/* arith_coder.rs:153-172 */
void orc_dec_init(orc_decoder* d, const uint8_t* in, size_t len) {
    d->low = 0; d->high = STATE_MASK; d->code = 0;
    d->in = in; d->len = len; d->byte_pos = 0; d->bit_pos = 7;
    for (int i = 0; i < 32; i++) d->code = (d->code << 1) | (uint64_t)read_bit(d);
}
/* arith_coder.rs:195-264 */
int orc_dec_decode(orc_decoder* d, const uint32_t* cum, int v) {
    uint64_t total = cum[v - 1];
    uint64_t range = d->high - d->low + 1;
    uint64_t off = d->code - d->low;
    uint64_t value = ((off + 1) * total - 1) / range;
    uint32_t val32 = (uint32_t)value;
    int lo = 0, hi = v;
    while (lo < hi) {
        int mid = (lo + hi) / 2;
        if (val32 < cum[mid]) hi = mid; else lo = mid + 1;
    }
    int sym = lo < v - 1 ? lo : v - 1;
    uint64_t sh = cum[sym];
    uint64_t sl = sym > 0 ? cum[sym - 1] : 0;
    d->high = d->low + (sh * range / total) - 1;
    d->low = d->low + (sl * range / total);
    for (;;) {
        if (((d->low ^ d->high) & HALF_R) == 0) {
            d->low = (d->low << 1) & STATE_MASK;
            d->high = ((d->high << 1) & STATE_MASK) | 1;
            d->code = ((d->code << 1) & STATE_MASK) | (uint64_t)read_bit(d);
        } else if ((d->low & ~d->high & QUARTER_R) != 0) {
            d->low = ((d->low << 1) ^ HALF_R) & STATE_MASK;
            d->high = (((d->high ^ HALF_R) << 1) | HALF_R | 1) & STATE_MASK;
            uint64_t hb = d->code & HALF_R;
            uint64_t shf = (d->code << 1) & (STATE_MASK >> 1);
            d->code = hb | shf | (uint64_t)read_bit(d);
        } else break;
    }
    return sym;
}

/* ------------------------------------------------------------------ */
/* Chunk driver (main.rs:206-238, 377-396)                            */
/* ------------------------------------------------------------------ */
#define BOS_TOKEN 1022u

int orc_compress_chunk(const orc_model* m, const uint32_t* toks, int n, uint8_t** out, size_t* out_len) {
    orc_state* s = orc_state_new(m);
    int32_t* logits = (int32_t*)malloc(sizeof(int32_t) * (size_t)m->vocab);
    uint32_t* cum = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)m->vocab);
    orc_encoder e;
    orc_enc_init(&e);
    int rc = 0;
    for (int i = 0; i < n && rc == 0; i++) {
        uint32_t prev = i == 0 ? BOS_TOKEN : toks[i - 1];
        rc = orc_forward(s, prev, i, logits);
        if (rc) break;
        orc_build_cumfreqs(logits, m->vocab, m->exp2_lut, m->coef_q24, m->target_total, cum);
        if ((int)toks[i] >= m->vocab) { rc = -5; break; }
        orc_enc_encode(&e, cum, m->vocab, (int)toks[i]);
    }
    orc_enc_finish(&e);
    *out = e.out; *out_len = e.len;
    free(logits); free(cum); orc_state_free(s);
    return rc;
}

int orc_decompress_chunk(const orc_model* m, const uint8_t* in, size_t len, int n, uint32_t* toks) {
    orc_state* s = orc_state_new(m);
    int32_t* logits = (int32_t*)malloc(sizeof(int32_t) * (size_t)m->vocab);
    uint32_t* cum = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)m->vocab);
    orc_decoder d;
    orc_dec_init(&d, in, len);
    int rc = 0;
    for (int i = 0; i < n; i++) {
        uint32_t prev = i == 0 ? BOS_TOKEN : toks[i - 1];
        rc = orc_forward(s, prev, i, logits);
        if (rc) break;
        orc_build_cumfreqs(logits, m->vocab, m->exp2_lut, m->coef_q24, m->target_total, cum);
        toks[i] = (uint32_t)orc_dec_decode(&d, cum, m->vocab);
    }
    free(logits); free(cum); orc_state_free(s);
    return rc;
}

int orc_chunk_trace(const orc_model* m, const uint32_t* inputs, int n, int32_t* logits_out, uint32_t* cum_out) {
    orc_state* s = orc_state_new(m);
    int rc = 0;
    for (int i = 0; i < n; i++) {
        int32_t* lg = logits_out + (size_t)i * m->vocab;
        rc = orc_forward(s, inputs[i], i, lg);
        if (rc) break;
        if (cum_out)
            orc_build_cumfreqs(lg, m->vocab, m->exp2_lut, m->coef_q24, m->target_total,
                               cum_out + (size_t)i * m->vocab);
    }
    orc_state_free(s);
    return rc;
}

/* Deep copy of the weights, the per-chunk `(*weights).clone()` of main.rs:215. */
typedef struct { orc_model m; orc_layer* layers; void* blob; } model_clone;

static size_t mclone_size(const orc_model* m) {
    size_t d = m->d_model, F = m->d_ff, V = m->vocab, G = m->n_kv_heads, H = m->n_heads;
    size_t per_layer = 4 * d + (d + 2 * G * 64) * d + d * d + 2 * F * d + d * F + 4 * H + 64;
    return 2 * V * d + d + 512 + 4 * (size_t)m->context_length * 32 + (size_t)m->n_layers * per_layer + 16 * (16 + 12 * (size_t)m->n_layers);
}
static void* blob_copy(uint8_t** p, const void* src, size_t n) {
    void* dst = *p;
    memcpy(dst, src, n);
    *p += (n + 15) & ~(size_t)15;
    return dst;
}
static void mclone_make(const orc_model* src, model_clone* c) {
    size_t d = src->d_model, F = src->d_ff, V = src->vocab, G = src->n_kv_heads, H = src->n_heads;
    c->m = *src;
    c->layers = (orc_layer*)malloc(sizeof(orc_layer) * (size_t)src->n_layers);
    c->blob = malloc(mclone_size(src));
    uint8_t* p = (uint8_t*)c->blob;
    c->m.embed = (const int8_t*)blob_copy(&p, src->embed, V * d);
    c->m.head_w = (const int8_t*)blob_copy(&p, src->head_w, V * d);
    c->m.final_norm = (const int8_t*)blob_copy(&p, src->final_norm, d);
    c->m.exp2_lut = (const uint16_t*)blob_copy(&p, src->exp2_lut, 512);
    c->m.rope_cos = (const int16_t*)blob_copy(&p, src->rope_cos, 2 * (size_t)src->context_length * 32);
    c->m.rope_sin = (const int16_t*)blob_copy(&p, src->rope_sin, 2 * (size_t)src->context_length * 32);
    for (int l = 0; l < src->n_layers; l++) {
        const orc_layer* a = &src->layers[l];
        orc_layer* b = &c->layers[l];
        *b = *a;
        b->attn_norm = (const int8_t*)blob_copy(&p, a->attn_norm, d);
        b->post_attn_norm = (const int8_t*)blob_copy(&p, a->post_attn_norm, d);
        b->ffn_norm = (const int8_t*)blob_copy(&p, a->ffn_norm, d);
        b->post_ffn_norm = (const int8_t*)blob_copy(&p, a->post_ffn_norm, d);
        b->qkv_w = (const int8_t*)blob_copy(&p, a->qkv_w, (d + 2 * G * 64) * d);
        b->out_w = (const int8_t*)blob_copy(&p, a->out_w, d * d);
        b->up_w = (const int8_t*)blob_copy(&p, a->up_w, 2 * F * d);
        b->down_w = (const int8_t*)blob_copy(&p, a->down_w, d * F);
        b->score_mult = (const int32_t*)blob_copy(&p, a->score_mult, 4 * H);
        if (a->sink_key) b->sink_key = (const int8_t*)blob_copy(&p, a->sink_key, 64);
    }
    c->m.layers = c->layers;
}
static void mclone_free(model_clone* c) { free(c->layers); free(c->blob); }

typedef struct {
    const orc_model* m; const uint32_t* toks; int64_t n; int chunk; int clone;
    uint8_t* out_buf; int64_t slot; int32_t* out_lens;
    int64_t nchunks; int64_t next; pthread_mutex_t mu; int rc;
    /* decompress */
    const uint8_t* bufs; const int64_t* offs; const int32_t* lens; const int32_t* ntoks;
    uint32_t* toks_out; const int64_t* tok_offs;
} pool_job;

static int64_t take(pool_job* j) {
    pthread_mutex_lock(&j->mu);
    int64_t c = j->next < j->nchunks ? j->next++ : -1;
    pthread_mutex_unlock(&j->mu);
    return c;
}

static void* comp_worker(void* arg) {
    pool_job* j = (pool_job*)arg;
    for (;;) {
        int64_t c = take(j);
        if (c < 0) break;
        int64_t s0 = c * j->chunk;
        int64_t e0 = s0 + j->chunk < j->n ? s0 + j->chunk : j->n;
        model_clone mc; const orc_model* mm = j->m;
        if (j->clone) { mclone_make(j->m, &mc); mm = &mc.m; }
        uint8_t* bytes = NULL; size_t blen = 0;
        int rc = orc_compress_chunk(mm, j->toks + s0, (int)(e0 - s0), &bytes, &blen);
        if (j->clone) mclone_free(&mc);
        if (rc == 0 && (int64_t)blen > j->slot) rc = -6;
        if (rc == 0) { memcpy(j->out_buf + c * j->slot, bytes, blen); j->out_lens[c] = (int32_t)blen; }
        else { pthread_mutex_lock(&j->mu); j->rc = rc; pthread_mutex_unlock(&j->mu); }
        free(bytes);
    }
    return NULL;
}

int orc_compress_many(const orc_model* m, const uint32_t* toks, int64_t n, int chunk, int threads,
                      int clone, uint8_t* out_buf, int64_t slot, int32_t* out_lens) {
    pool_job j;
    memset(&j, 0, sizeof(j));
    j.m = m; j.toks = toks; j.n = n; j.chunk = chunk; j.clone = clone;
    j.out_buf = out_buf; j.slot = slot; j.out_lens = out_lens;
    j.nchunks = (n + chunk - 1) / chunk; j.next = 0; j.rc = 0;
    pthread_mutex_init(&j.mu, NULL);
    if (threads < 1) threads = 1;
    pthread_t* th = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)threads);
    for (int i = 0; i < threads; i++) pthread_create(&th[i], NULL, comp_worker, &j);
    for (int i = 0; i < threads; i++) pthread_join(th[i], NULL);
    free(th);
    pthread_mutex_destroy(&j.mu);
    return j.rc;
}

static void* decomp_worker(void* arg) {
    pool_job* j = (pool_job*)arg;
    for (;;) {
        int64_t c = take(j);
        if (c < 0) break;
        int rc = orc_decompress_chunk(j->m, j->bufs + j->offs[c], (size_t)j->lens[c], j->ntoks[c],
                                      j->toks_out + j->tok_offs[c]);
        if (rc) { pthread_mutex_lock(&j->mu); j->rc = rc; pthread_mutex_unlock(&j->mu); }
    }
    return NULL;
}

int orc_decompress_many(const orc_model* m, const uint8_t* bufs, const int64_t* offs,
                        const int32_t* lens, const int32_t* ntoks, int nchunks, int threads,
                        uint32_t* toks_out, const int64_t* tok_offs) {
    pool_job j;
    memset(&j, 0, sizeof(j));
    j.m = m; j.bufs = bufs; j.offs = offs; j.lens = lens; j.ntoks = ntoks;
    j.nchunks = nchunks; j.toks_out = toks_out; j.tok_offs = tok_offs;
    pthread_mutex_init(&j.mu, NULL);
    if (threads < 1) threads = 1;
    pthread_t* th = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)threads);
    for (int i = 0; i < threads; i++) pthread_create(&th[i], NULL, decomp_worker, &j);
    for (int i = 0; i < threads; i++) pthread_join(th[i], NULL);
    free(th);
    pthread_mutex_destroy(&j.mu);
    return j.rc;
}
