// .czm (safetensors) reader: the host model loader behind czip_model_load.
//
// Layout (rust/src/safetensors.rs:287-376): u64 LE header length, a JSON
// object {name: {dtype, shape, data_offsets}, "__metadata__": {k: v}}, then
// the tensor bytes.  Config keys and defaults follow rust/src/model.rs:113-145
// and the per-scalar defaults model.rs:157-168.
#include <cstdio>
#include <cstdlib>
#include <cstdint>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "czip_internal.h"
#include "czip_json.h"

namespace czip {
namespace {

size_t dtype_size(const std::string& dt, bool& ok) {
    ok = true;
    // rust/src/safetensors.rs:226-243 (BOOL is mapped to a 4-byte Int32 there)
    if (dt == "I8" || dt == "U8") return 1;
    if (dt == "I16" || dt == "U16" || dt == "F16" || dt == "BF16") return 2;
    if (dt == "I32" || dt == "U32" || dt == "F32" || dt == "BOOL") return 4;
    if (dt == "I64") return 8;
    ok = false;
    return 0;
}

bool parse_usize(const std::map<std::string, std::string>& md, const char* k, long long& out) {
    auto it = md.find(k);
    if (it == md.end() || it->second.empty()) return false;
    // str::parse::<usize> accepts only ASCII digits (an optional '+')
    const std::string& s = it->second;
    size_t i = (s[0] == '+') ? 1 : 0;
    if (i >= s.size()) return false;
    long long v = 0;
    for (; i < s.size(); i++) {
        if (s[i] < '0' || s[i] > '9') return false;
        v = v * 10 + (s[i] - '0');
        if (v > (1ll << 40)) return false;
    }
    out = v;
    return true;
}

}  // namespace

czip_status load_czm(const char* path, int32_t kv_mode, HostModel& hm, std::string& err) {
    FILE* f = fopen(path, "rb");
    if (!f) { err = std::string("cannot open ") + path; return CZIP_E_IO; }
    fseek(f, 0, SEEK_END);
    long sz = ftell(f);
    fseek(f, 0, SEEK_SET);
    if (sz < 8) { fclose(f); err = "file too short"; return CZIP_E_IO; }
    hm.blob.resize((size_t)sz);
    if (fread(hm.blob.data(), 1, (size_t)sz, f) != (size_t)sz) { fclose(f); err = "read failed"; return CZIP_E_IO; }
    fclose(f);
    uint64_t hlen = 0;
    memcpy(&hlen, hm.blob.data(), 8);
    if (8 + hlen > (uint64_t)sz) { err = "Invalid header size"; return CZIP_E_IO; }
    JParser jp{(const char*)hm.blob.data() + 8, (const char*)hm.blob.data() + 8 + hlen};
    JVal root;
    if (!jp.val(root, 0) || root.kind != JVal::OBJ) { err = "header is not a JSON object"; return CZIP_E_IO; }
    const size_t base = 8 + (size_t)hlen;
    for (auto& kv : root.obj) {
        if (kv.first == "__metadata__") {
            for (auto& m : kv.second.obj)
                if (m.second.kind == JVal::STR) hm.meta[m.first] = m.second.str;
            continue;
        }
        const JVal* dt = kv.second.get("dtype");
        const JVal* sh = kv.second.get("shape");
        const JVal* off = kv.second.get("data_offsets");
        if (!dt || dt->kind != JVal::STR || !sh || sh->kind != JVal::ARR || !off || off->kind != JVal::ARR ||
            off->arr.size() != 2) {
            err = "bad tensor entry " + kv.first;
            return CZIP_E_IO;
        }
        bool ok;
        size_t es = dtype_size(dt->str, ok);
        if (!ok) { err = "Unknown dtype: " + dt->str; return CZIP_E_IO; }
        HostTensor t;
        t.dtype = dt->str;
        // shapes and offsets are usize in the reference's header type
        // (safetensors.rs:287-376): non-negative integers, checked without wrap
        auto is_usize = [](const JVal& j) { return j.kind == JVal::NUM && j.isint && j.inum >= 0; };
        size_t numel = 1;
        for (auto& d : sh->arr) {
            if (!is_usize(d)) { err = "bad shape for " + kv.first; return CZIP_E_IO; }
            t.shape.push_back(d.inum);
            if (d.inum != 0 && numel > SIZE_MAX / (size_t)d.inum) { err = "shape overflow for " + kv.first; return CZIP_E_IO; }
            numel *= (size_t)d.inum;
        }
        if (!is_usize(off->arr[0]) || !is_usize(off->arr[1])) { err = "bad data_offsets for " + kv.first; return CZIP_E_IO; }
        const size_t a = (size_t)off->arr[0].inum, b = (size_t)off->arr[1].inum, blob = (size_t)sz - base;
        if (numel > SIZE_MAX / es || b < a || b > blob || b - a != numel * es) {
            err = "bad data_offsets for " + kv.first;
            return CZIP_E_IO;
        }
        t.data = hm.blob.data() + base + a;
        t.bytes = b - a;
        t.numel = numel;
        hm.tensors[kv.first] = t;
    }

    // ---- config (model.rs:113-145) ----
    long long v;
    auto pu = [&](const char* k, long long dflt) { long long x; return parse_usize(hm.meta, k, x) ? x : dflt; };
    long long ctx;
    if (parse_usize(hm.meta, "context_length", v)) ctx = v;
    else if (parse_usize(hm.meta, "context_length_log2", v)) ctx = 1ll << v;
    else ctx = pu("max_seq_len", 64);
    czip_model_desc& d = hm.desc;
    memset(&d, 0, sizeof(d));
    d.vocab = (int32_t)pu("vocab_size", 1024);
    d.n_layers = (int32_t)pu("n_layers", 1);
    d.n_heads = (int32_t)pu("n_heads", 6);
    d.n_kv_heads = (int32_t)pu("n_kv_heads", 1);
    d.d_model = (int32_t)pu("d_model", 384);
    d.d_ff = (int32_t)pu("d_ff", 1024);
    d.head_dim = (int32_t)pu("head_dim", 64);
    d.max_seq_len = (int32_t)pu("max_seq_len", 64);
    d.context_length = (int32_t)ctx;
    d.kv_mode = kv_mode;
    auto cod = hm.meta.find("tokenizer_codec");
    hm.tokenizer_codec = cod == hm.meta.end() ? "zstd" : cod->second;

    auto need = [&](const std::string& name, const char* dtype, size_t numel, const void** out) -> czip_status {
        auto it = hm.tensors.find(name);
        if (it == hm.tensors.end()) { err = "Missing tensor: " + name; return CZIP_E_MISSING; }
        if (it->second.dtype != dtype && !(std::string(dtype) == "I32" && it->second.dtype == "BOOL")) {
            err = "unexpected dtype for " + name + ": " + it->second.dtype;
            return CZIP_E_FORMAT;
        }
        if (numel && it->second.numel != numel) { err = "unexpected size for " + name; return CZIP_E_FORMAT; }
        *out = it->second.data;
        return CZIP_OK;
    };
    auto scalar_i32 = [&](const std::string& name, int32_t dflt) -> int32_t {
        auto it = hm.tensors.find(name);
        if (it == hm.tensors.end() || it->second.numel < 1) return dflt;
        int32_t x;
        memcpy(&x, it->second.data, 4);
        return x;
    };
    auto scalar_i8 = [&](const std::string& name, int32_t dflt) -> int32_t {
        auto it = hm.tensors.find(name);
        if (it == hm.tensors.end() || it->second.numel < 1) return dflt;
        return (int32_t)(int8_t)it->second.data[0];
    };
    auto scalar_u32 = [&](const std::string& name, bool& present) -> uint32_t {
        auto it = hm.tensors.find(name);
        present = it != hm.tensors.end() && it->second.numel >= 1;
        uint32_t x = 0;
        if (present) memcpy(&x, it->second.data, 4);
        return x;
    };
    const size_t D = (size_t)d.d_model, F = (size_t)d.d_ff, V = (size_t)d.vocab, G = (size_t)d.n_kv_heads;
    czip_status rc;
    const void* p;
    if ((rc = need("embed.weight", "I8", V * D, &p))) return rc;
    d.embed = (const int8_t*)p;
    hm.layers.resize((size_t)d.n_layers);
    for (int l = 0; l < d.n_layers; l++) {
        std::string pre = "layers." + std::to_string(l);
        czip_layer_desc& L = hm.layers[(size_t)l];
        memset(&L, 0, sizeof(L));
#define NEED(field, name, dt, n, ty) \
        if ((rc = need(pre + name, dt, n, &p))) return rc; L.field = (const ty*)p;
        NEED(attn_norm, ".attn_norm.weight", "I8", D, int8_t)
        NEED(post_attn_norm, ".post_attn_norm.weight", "I8", D, int8_t)
        NEED(ffn_norm, ".ffn_norm.weight", "I8", D, int8_t)
        NEED(post_ffn_norm, ".post_ffn_norm.weight", "I8", D, int8_t)
        NEED(qkv_w, ".attn.qkv.weight", "I8", (D + 2 * G * 64) * D, int8_t)
        NEED(out_w, ".attn.out.weight", "I8", D * D, int8_t)
        NEED(up_w, ".ffn.up.weight", "I8", 2 * F * D, int8_t)
        NEED(down_w, ".ffn.down.weight", "I8", D * F, int8_t)
        NEED(score_mult, ".attn.score_mult", "I32", (size_t)d.n_heads, int32_t)
#undef NEED
        auto sk = hm.tensors.find(pre + ".attn.sink_key");
        L.sink_key = (sk != hm.tensors.end() && sk->second.numel == 64) ? (const int8_t*)sk->second.data : nullptr;
        L.qkv_mult = scalar_i32(pre + ".attn.qkv.mult", 1);
        L.out_mult = scalar_i32(pre + ".attn.out.mult", 1);
        L.up_mult = scalar_i32(pre + ".ffn.up.mult", 1);
        L.down_mult = scalar_i32(pre + ".ffn.down.mult", 1);
        L.qkv_shift = scalar_i8(pre + ".attn.qkv.shift", 0);
        L.out_shift = scalar_i8(pre + ".attn.out.shift", 0);
        L.up_shift = scalar_i8(pre + ".ffn.up.shift", 0);
        L.down_shift = scalar_i8(pre + ".ffn.down.shift", 0);
    }
    d.layers = hm.layers.data();
    if ((rc = need("norm.weight", "I8", D, &p))) return rc;
    d.final_norm = (const int8_t*)p;
    if ((rc = need("head.weight", "I8", V * D, &p))) return rc;
    d.head_w = (const int8_t*)p;
    // LUT sizes are validated at context creation (model.rs:324-333)
    if ((rc = need("lut.exp2", "U16", 0, &p))) return rc;
    d.exp2_lut = (const uint16_t*)p;
    hm.exp2_numel = hm.tensors["lut.exp2"].numel;
    if ((rc = need("lut.rope_cos", "I16", 0, &p))) return rc;
    d.rope_cos = (const int16_t*)p;
    if ((rc = need("lut.rope_sin", "I16", 0, &p))) return rc;
    d.rope_sin = (const int16_t*)p;
    hm.rope_numel = std::min(hm.tensors["lut.rope_cos"].numel, hm.tensors["lut.rope_sin"].numel);
    d.exp2_len = (int64_t)hm.exp2_numel;
    d.rope_len = (int64_t)hm.rope_numel;
    bool has;
    uint32_t c = scalar_u32("softmax.coef_q24", has);
    d.coef_q24 = has ? c : default_cdf_coef_q24();
    uint32_t tt = scalar_u32("softmax.target_total", has);
    d.target_total = has ? tt : default_target_total((uint32_t)d.vocab);
    auto tok = hm.tensors.find("tokenizer.data");
    if (tok != hm.tensors.end()) { hm.tokenizer = tok->second.data; hm.tokenizer_len = tok->second.bytes; }
    return CZIP_OK;
}

// softmax_cdf.rs:23-28 (f64::round is half-away-from-zero)
uint32_t default_cdf_coef_q24() {
    const double log2e = 1.4426950408889634;
    double c = (0.1 * log2e) / 64.0 * (double)(1u << 24);
    double r = c < 0 ? -__builtin_floor(-c + 0.5) : __builtin_floor(c + 0.5);
    uint32_t u = (uint32_t)r;
    return u < 1 ? 1 : u;
}

// softmax_cdf.rs:39-46
uint32_t default_target_total(uint32_t vocab) {
    uint32_t q = 1u << 30;
    uint32_t t = q > vocab ? q - vocab : 0;
    t = t > 1024 ? t - 1024 : 0;
    return t > vocab + 1 ? t : vocab + 1;
}

}  // namespace czip
