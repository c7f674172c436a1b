// CZIPv1 container (rust/src/file_format.rs; main.rs:79-85, 241-279, 339-361):
// a 16-byte outer header, then the outer codec's stream of the payload
// (inner header || chunk bytes).  Host code; the outer codecs come from the
// system libzstd / libbrotlienc / libbrotlidec, loaded at first use.
#include <dlfcn.h>

#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "czip_hip.h"

namespace {

// ---------------------------------------------------------------------------
// MD5 (RFC 1321), for the model id hash of main.rs:79-85.
// ---------------------------------------------------------------------------
struct Md5 {
    uint32_t h[4] = {0x67452301u, 0xefcdab89u, 0x98badcfeu, 0x10325476u};

    static uint32_t rotl(uint32_t x, int c) { return (x << c) | (x >> (32 - c)); }

    void block(const uint8_t* p) {
        // per-round shift amounts and T[i] = floor(2^32 * |sin(i + 1)|) (RFC 1321, 3.4),
        // the latter evaluated once in long double (checked by the RFC test vectors)
        static const int S[64] = {7, 12, 17, 22, 7, 12, 17, 22, 7, 12, 17, 22, 7, 12, 17, 22,
                                  5, 9,  14, 20, 5, 9,  14, 20, 5, 9,  14, 20, 5, 9,  14, 20,
                                  4, 11, 16, 23, 4, 11, 16, 23, 4, 11, 16, 23, 4, 11, 16, 23,
                                  6, 10, 15, 21, 6, 10, 15, 21, 6, 10, 15, 21, 6, 10, 15, 21};
        struct Table {
            uint32_t t[64];
            Table() {
                for (int i = 0; i < 64; i++)
                    t[i] = (uint32_t)(unsigned long long)(__builtin_fabsl(__builtin_sinl((long double)(i + 1))) *
                                                          4294967296.0L);
            }
        };
        static const Table tab;  // thread-safe one-time initialization
        const uint32_t* T = tab.t;
        uint32_t X[16];
        for (int i = 0; i < 16; i++)
            X[i] = (uint32_t)p[4 * i] | ((uint32_t)p[4 * i + 1] << 8) | ((uint32_t)p[4 * i + 2] << 16) |
                   ((uint32_t)p[4 * i + 3] << 24);
        uint32_t a = h[0], b = h[1], c = h[2], d = h[3];
        for (int i = 0; i < 64; i++) {
            uint32_t f;
            int g;
            if (i < 16) { f = (b & c) | (~b & d); g = i; }
            else if (i < 32) { f = (d & b) | (~d & c); g = (5 * i + 1) & 15; }
            else if (i < 48) { f = b ^ c ^ d; g = (3 * i + 5) & 15; }
            else { f = c ^ (b | ~d); g = (7 * i) & 15; }
            const uint32_t t = d;
            d = c;
            c = b;
            b = b + rotl(a + f + T[i] + X[g], S[i]);
            a = t;
        }
        h[0] += a; h[1] += b; h[2] += c; h[3] += d;
    }

    void digest(const uint8_t* msg, size_t len, uint8_t out[16]) {
        size_t i = 0;
        for (; i + 64 <= len; i += 64) block(msg + i);
        uint8_t tail[128] = {0};
        const size_t rem = len - i;
        memcpy(tail, msg + i, rem);
        tail[rem] = 0x80;
        const size_t tl = rem + 1 + 8 <= 64 ? 64 : 128;
        const unsigned long long bits = (unsigned long long)len * 8ull;
        for (int k = 0; k < 8; k++) tail[tl - 8 + k] = (uint8_t)(bits >> (8 * k));
        block(tail);
        if (tl == 128) block(tail + 64);
        for (int k = 0; k < 4; k++)
            for (int j = 0; j < 4; j++) out[4 * k + j] = (uint8_t)(h[k] >> (8 * j));
    }
};

// ---------------------------------------------------------------------------
// Outer codecs (main.rs:261-275, 348-359): zstd level 22 / brotli quality 11,
// window 22, through the system libraries.
// ---------------------------------------------------------------------------
void* lib(const char* name) {
    void* h = dlopen(name, RTLD_NOW | RTLD_LOCAL);
    return h;
}

czip_status zstd_pack(const uint8_t* in, size_t n, std::vector<uint8_t>& out) {
    void* h = lib("libzstd.so.1");
    if (!h) return CZIP_E_IO;
    auto bound = (size_t (*)(size_t))dlsym(h, "ZSTD_compressBound");
    auto comp = (size_t (*)(void*, size_t, const void*, size_t, int))dlsym(h, "ZSTD_compress");
    auto is_err = (unsigned (*)(size_t))dlsym(h, "ZSTD_isError");
    if (!bound || !comp || !is_err) return CZIP_E_IO;
    out.resize(bound(n));
    const size_t r = comp(out.data(), out.size(), in, n, 22);
    if (is_err(r)) return CZIP_E_FORMAT;
    out.resize(r);
    return CZIP_OK;
}

czip_status zstd_unpack(const uint8_t* in, size_t n, std::vector<uint8_t>& out) {
    void* h = lib("libzstd.so.1");
    if (!h) return CZIP_E_IO;
    struct InB { const void* src; size_t size; size_t pos; };
    struct OutB { void* dst; size_t size; size_t pos; };
    auto create = (void* (*)())dlsym(h, "ZSTD_createDStream");
    auto init = (size_t (*)(void*))dlsym(h, "ZSTD_initDStream");
    auto step = (size_t (*)(void*, OutB*, InB*))dlsym(h, "ZSTD_decompressStream");
    auto destroy = (size_t (*)(void*))dlsym(h, "ZSTD_freeDStream");
    auto is_err = (unsigned (*)(size_t))dlsym(h, "ZSTD_isError");
    if (!create || !init || !step || !destroy || !is_err) return CZIP_E_IO;
    void* ds = create();
    if (!ds) return CZIP_E_NOMEM;
    init(ds);
    InB ib{in, n, 0};
    out.clear();
    std::vector<uint8_t> buf(1 << 20);
    czip_status rc = CZIP_OK;
    size_t last = 1;
    while (ib.pos < ib.size || last != 0) {
        OutB ob{buf.data(), buf.size(), 0};
        last = step(ds, &ob, &ib);
        if (is_err(last)) { rc = CZIP_E_FORMAT; break; }
        out.insert(out.end(), buf.data(), buf.data() + ob.pos);
        if (ib.pos >= ib.size && ob.pos == 0 && last != 0) { rc = CZIP_E_FORMAT; break; }  // truncated frame
    }
    destroy(ds);
    return rc;
}

czip_status brotli_pack(const uint8_t* in, size_t n, std::vector<uint8_t>& out) {
    void* h = lib("libbrotlienc.so.1");
    if (!h) return CZIP_E_IO;
    auto maxsz = (size_t (*)(size_t))dlsym(h, "BrotliEncoderMaxCompressedSize");
    auto comp = (int (*)(int, int, int, size_t, const uint8_t*, size_t*, uint8_t*))dlsym(h, "BrotliEncoderCompress");
    if (!maxsz || !comp) return CZIP_E_IO;
    size_t cap = maxsz(n);
    if (cap == 0) cap = n + (n >> 2) + 1024;
    out.resize(cap);
    size_t outl = cap;
    // quality 11, lgwin 22, BROTLI_MODE_GENERIC (0)
    if (comp(11, 22, 0, n, in, &outl, out.data()) != 1) return CZIP_E_FORMAT;
    out.resize(outl);
    return CZIP_OK;
}

czip_status brotli_unpack(const uint8_t* in, size_t n, std::vector<uint8_t>& out) {
    void* h = lib("libbrotlidec.so.1");
    if (!h) return CZIP_E_IO;
    auto create = (void* (*)(void*, void*, void*))dlsym(h, "BrotliDecoderCreateInstance");
    auto step = (int (*)(void*, size_t*, const uint8_t**, size_t*, uint8_t**, size_t*))dlsym(
        h, "BrotliDecoderDecompressStream");
    auto destroy = (void (*)(void*))dlsym(h, "BrotliDecoderDestroyInstance");
    if (!create || !step || !destroy) return CZIP_E_IO;
    void* st = create(nullptr, nullptr, nullptr);
    if (!st) return CZIP_E_NOMEM;
    out.clear();
    std::vector<uint8_t> buf(1 << 20);
    size_t avail_in = n;
    const uint8_t* next_in = in;
    czip_status rc = CZIP_OK;
    for (;;) {
        size_t avail_out = buf.size();
        uint8_t* next_out = buf.data();
        // BROTLI_DECODER_RESULT_ERROR 0, SUCCESS 1, NEEDS_MORE_INPUT 2, NEEDS_MORE_OUTPUT 3
        const int r = step(st, &avail_in, &next_in, &avail_out, &next_out, nullptr);
        out.insert(out.end(), buf.data(), next_out);
        if (r == 1) break;
        if (r == 3) continue;
        rc = CZIP_E_FORMAT;  // error or truncated stream
        break;
    }
    destroy(st);
    return rc;
}

void put32(std::vector<uint8_t>& v, uint32_t x) {
    for (int k = 0; k < 4; k++) v.push_back((uint8_t)(x >> (8 * k)));
}
void put16(std::vector<uint8_t>& v, uint16_t x) {
    v.push_back((uint8_t)x);
    v.push_back((uint8_t)(x >> 8));
}
uint32_t get32(const uint8_t* p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}
uint16_t get16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

}  // namespace

extern "C" uint32_t czip_model_id_hash(const char* path, size_t len) {
    // main.rs:79-85: the first 8 hex digits of MD5(path) as a u32, i.e. the
    // first 4 digest bytes read big-endian
    uint8_t d[16];
    Md5().digest((const uint8_t*)path, path ? len : 0, d);
    return ((uint32_t)d[0] << 24) | ((uint32_t)d[1] << 16) | ((uint32_t)d[2] << 8) | (uint32_t)d[3];
}

extern "C" czip_status czip_container_pack(const czip_container* info, const uint8_t* chunks, const int64_t* offs,
                                           uint8_t** out, size_t* out_len) {
    if (!info || !out || !out_len || (info->chunk_count && (!chunks || !offs))) return CZIP_E_ARG;
    if (info->codec != CZIP_CODEC_ZSTD && info->codec != CZIP_CODEC_BROTLI) return CZIP_E_ARG;
    const uint32_t nch = info->chunk_count;
    // inner header (file_format.rs:245-256): hash, chunk count, last chunk
    // tokens, tokenizer id, log2 context length, one u16 byte length per chunk
    std::vector<uint8_t> payload;
    put32(payload, info->model_id_hash);
    put32(payload, nch);
    put16(payload, info->last_chunk_tokens);
    payload.push_back(info->tokenizer_id);
    payload.push_back(info->context_length_log2);
    for (uint32_t i = 0; i < nch; i++) {
        const int64_t l = offs[i + 1] - offs[i];
        if (l < 0 || l > 65535) return CZIP_E_OVERFLOW;  // "Chunk too large" (file_format.rs:311)
        put16(payload, (uint16_t)l);
    }
    const uint32_t header_len = 12u + 2u * nch;
    if (nch) payload.insert(payload.end(), chunks + offs[0], chunks + offs[nch]);
    std::vector<uint8_t> packed;
    czip_status rc = info->codec == CZIP_CODEC_ZSTD ? zstd_pack(payload.data(), payload.size(), packed)
                                                    : brotli_pack(payload.data(), payload.size(), packed);
    if (rc) return rc;
    // outer header (file_format.rs:145-153)
    std::vector<uint8_t> file;
    const char magic[6] = {'C', 'Z', 'I', 'P', 'v', '1'};
    file.insert(file.end(), magic, magic + 6);
    file.push_back(info->flags);
    file.push_back(info->codec);
    put32(file, info->uncompressed_len);
    put32(file, header_len);
    file.insert(file.end(), packed.begin(), packed.end());
    uint8_t* buf = (uint8_t*)malloc(file.size());
    if (!buf) return CZIP_E_NOMEM;
    memcpy(buf, file.data(), file.size());
    *out = buf;
    *out_len = file.size();
    return CZIP_OK;
}

extern "C" czip_status czip_container_unpack(const uint8_t* data, size_t len, czip_container* info, uint8_t** chunks,
                                             int64_t** offs) {
    if (!data || !info || !chunks || !offs) return CZIP_E_ARG;
    *chunks = nullptr;
    *offs = nullptr;
    // outer header (file_format.rs:112-142)
    if (len < 16) return CZIP_E_FORMAT;                    // "Outer header too short"
    if (memcmp(data, "CZIPv1", 6) != 0) return CZIP_E_FORMAT;  // "Invalid magic bytes"
    info->flags = data[6];
    info->codec = data[7];
    if (info->codec != CZIP_CODEC_ZSTD && info->codec != CZIP_CODEC_BROTLI) return CZIP_E_FORMAT;  // "Unknown codec"
    info->uncompressed_len = get32(data + 8);
    std::vector<uint8_t> payload;
    czip_status rc = info->codec == CZIP_CODEC_ZSTD ? zstd_unpack(data + 16, len - 16, payload)
                                                    : brotli_unpack(data + 16, len - 16, payload);
    if (rc) return rc;
    // inner header (file_format.rs:199-242); log2 0 reads as the default 6
    if (payload.size() < 12) return CZIP_E_FORMAT;  // "Inner header too short"
    info->model_id_hash = get32(payload.data());
    info->chunk_count = get32(payload.data() + 4);
    info->last_chunk_tokens = get16(payload.data() + 8);
    info->tokenizer_id = payload[10];
    info->context_length_log2 = payload[11] == 0 ? 6 : payload[11];
    const uint64_t nch = info->chunk_count;
    if (payload.size() < 12 + 2 * nch) return CZIP_E_FORMAT;  // "Inner header too short for N chunks"
    int64_t* o = (int64_t*)malloc((nch + 1) * sizeof(int64_t));
    if (!o) return CZIP_E_NOMEM;
    o[0] = 0;
    for (uint64_t i = 0; i < nch; i++) o[i + 1] = o[i] + get16(payload.data() + 12 + 2 * i);
    const size_t body = 12 + 2 * nch;
    if (payload.size() < body + (size_t)o[nch]) {  // "Chunk data truncated"
        free(o);
        return CZIP_E_FORMAT;
    }
    uint8_t* c = (uint8_t*)malloc(o[nch] ? (size_t)o[nch] : 1);
    if (!c) {
        free(o);
        return CZIP_E_NOMEM;
    }
    memcpy(c, payload.data() + body, (size_t)o[nch]);
    *chunks = c;
    *offs = o;
    return CZIP_OK;
}

extern "C" void czip_buffer_free(void* p) { free(p); }
