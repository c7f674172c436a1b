// BPE tokenizer of the czip models (host side of the text configurations).
//
// Loads the tiktoken-style JSON embedded in a .czm file
// (rust/src/tiktoken.rs:504-563, main.rs:87-109) and implements
// encode_with_special_tokens (tiktoken.rs:215-269, 498-501) and decode_bytes
// (tiktoken.rs:186-198).  The pre-split regex of the model,
//
//   '(?i:[sdmt]|ll|ve|re)|[^\r\n\p{L}\p{N}]?+\p{L}++|\p{N}{1,3}+|
//    ?[^\s\p{L}\p{N}]++[\r\n]*+|\s++$|\s*[\r\n]|\s+(?!\S)|\s
//
// is executed by a hand-written scanner that tries the alternatives in order
// at each position with the same possessive / backtracking semantics, so no
// regex engine is needed.  The merges give the ids _byte_pair_merge
// (tiktoken.rs:26-82) gives, by a heap of candidate pairs.
#include <dlfcn.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <queue>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include "czip_internal.h"
#include "czip_json.h"
#include "czip_unicode_tables.h"

namespace czip {
namespace {

const char* kPattern =
    "'(?i:[sdmt]|ll|ve|re)|[^\\r\\n\\p{L}\\p{N}]?+\\p{L}++|\\p{N}{1,3}+| ?[^\\s\\p{L}\\p{N}]++[\\r\\n]*+|\\s++$|"
    "\\s*[\\r\\n]|\\s+(?!\\S)|\\s";

bool in_ranges(uint32_t c, const uint32_t (*r)[2], int n) {
    int lo = 0, hi = n - 1;
    while (lo <= hi) {
        int mid = (lo + hi) >> 1;
        if (c < r[mid][0]) hi = mid - 1;
        else if (c > r[mid][1]) lo = mid + 1;
        else return true;
    }
    return false;
}

inline bool is_letter(uint32_t c) {
    if (c < 128) return (c | 32) - 'a' < 26u;
    return in_ranges(c, kLetterRanges, kLetterRangesCount);
}
inline bool is_number(uint32_t c) {
    if (c < 128) return c - '0' < 10u;
    return in_ranges(c, kNumberRanges, kNumberRangesCount);
}
// Unicode White_Space (the \s of Rust's regex)
inline bool is_space(uint32_t c) {
    if (c < 128) return c == ' ' || (c >= 9 && c <= 13);
    return c == 0x85 || c == 0xA0 || c == 0x1680 || (c >= 0x2000 && c <= 0x200A) || c == 0x2028 || c == 0x2029 ||
           c == 0x202F || c == 0x205F || c == 0x3000;
}

// decode one UTF-8 code point at s[i] (input already validated)
inline uint32_t cp_at(const uint8_t* s, size_t n, size_t i, size_t& len) {
    if (i >= n) { len = 0; return 0xFFFFFFFFu; }
    uint8_t b = s[i];
    if (b < 0x80) { len = 1; return b; }
    if (b < 0xE0) { len = 2; return ((b & 0x1Fu) << 6) | (s[i + 1] & 0x3Fu); }
    if (b < 0xF0) { len = 3; return ((b & 0x0Fu) << 12) | ((s[i + 1] & 0x3Fu) << 6) | (s[i + 2] & 0x3Fu); }
    len = 4;
    return ((b & 0x07u) << 18) | ((s[i + 1] & 0x3Fu) << 12) | ((s[i + 2] & 0x3Fu) << 6) | (s[i + 3] & 0x3Fu);
}

bool valid_utf8(const uint8_t* s, size_t n) {
    size_t i = 0;
    while (i < n) {
        uint8_t b = s[i];
        size_t k;
        uint32_t c;
        if (b < 0x80) { i++; continue; }
        if (b >= 0xC2 && b < 0xE0) { k = 1; c = b & 0x1Fu; }
        else if (b >= 0xE0 && b < 0xF0) { k = 2; c = b & 0x0Fu; }
        else if (b >= 0xF0 && b < 0xF5) { k = 3; c = b & 0x07u; }
        else return false;
        for (size_t j = 1; j <= k; j++) {
            if (i + j >= n || (s[i + j] & 0xC0) != 0x80) return false;
            c = (c << 6) | (s[i + j] & 0x3Fu);
        }
        if ((k == 2 && (c < 0x800 || (c >= 0xD800 && c <= 0xDFFF))) || (k == 3 && (c < 0x10000 || c > 0x10FFFF)))
            return false;
        i += k + 1;
    }
    return true;
}

inline bool is_crlf(uint32_t c) { return c == '\r' || c == '\n'; }
inline uint32_t fold(uint32_t c) { return c < 128 ? (c | 32) : (c == 0x17F ? 's' : c); }  // (?i) for [sdmt] / ll / ve / re

// End (byte offset) of the pattern's match starting at byte i; `n` is the
// full text length ($ is the end of the text).
size_t match_end(const uint8_t* s, size_t n, size_t i) {
    size_t l0, l1, l2;
    const uint32_t c0 = cp_at(s, n, i, l0);
    // 1. '(?i:[sdmt]|ll|ve|re)
    if (c0 == '\'') {
        const uint32_t c1 = fold(cp_at(s, n, i + 1, l1));
        if (l1 && (c1 == 's' || c1 == 'd' || c1 == 'm' || c1 == 't')) return i + 1 + l1;
        if (l1) {
            const uint32_t c2 = fold(cp_at(s, n, i + 1 + l1, l2));
            if (l2 && ((c1 == 'l' && c2 == 'l') || (c1 == 'v' && c2 == 'e') || (c1 == 'r' && c2 == 'e')))
                return i + 1 + l1 + l2;
        }
    }
    // 2. [^\r\n\p{L}\p{N}]?+\p{L}++
    {
        size_t j = i;
        bool ok = false;
        if (is_letter(c0)) ok = true;
        else if (!is_crlf(c0) && !is_number(c0)) {
            size_t l;
            if (is_letter(cp_at(s, n, i + l0, l))) { j = i + l0; ok = true; }
        }
        if (ok) {
            size_t l;
            while (j < n && is_letter(cp_at(s, n, j, l))) j += l;
            return j;
        }
    }
    // 3. \p{N}{1,3}+
    if (is_number(c0)) {
        size_t j = i + l0, l;
        for (int k = 1; k < 3 && j < n && is_number(cp_at(s, n, j, l)); k++) j += l;
        return j;
    }
    // 4.  ?[^\s\p{L}\p{N}]++[\r\n]*+
    {
        auto punct = [](uint32_t c) { return !is_space(c) && !is_letter(c) && !is_number(c); };
        size_t j = (c0 == ' ') ? i + 1 : i, l;
        size_t k = j;
        while (k < n) {
            uint32_t c = cp_at(s, n, k, l);
            if (!punct(c)) break;
            k += l;
        }
        if (k > j) {
            while (k < n && (s[k] == '\r' || s[k] == '\n')) k++;
            return k;
        }
        // a leading space that is not followed by punctuation leaves nothing for the class
    }
    if (is_space(c0)) {
        size_t k = i, l, last_crlf = (size_t)-1, last_start = i;
        int count = 0;
        while (k < n) {
            uint32_t c = cp_at(s, n, k, l);
            if (!is_space(c)) break;
            if (is_crlf(c)) last_crlf = k;
            last_start = k;
            count++;
            k += l;
        }
        // 5. \s++$
        if (k == n) return n;
        // 6. \s*[\r\n]
        if (last_crlf != (size_t)-1) return last_crlf + 1;
        // 7. \s+(?!\S): the run less its last character (needs two or more)
        if (count >= 2) return last_start;
        // 8. \s
        return i + l0;
    }
    // not reached for valid text: every code point matches one alternative
    return i + (l0 ? l0 : 1);
}

using Rank = uint32_t;
constexpr Rank RANK_MAX = 0xFFFFFFFFu;

}  // namespace
}  // namespace czip

struct czip_tokenizer {
    std::unordered_map<std::string, czip::Rank> enc;
    std::unordered_map<czip::Rank, std::string> dec;
    std::vector<std::pair<std::string, czip::Rank>> specials;
};

namespace czip {
namespace {

Rank rank_of(const czip_tokenizer* t, const uint8_t* p, size_t len) {
    auto it = t->enc.find(std::string((const char*)p, len));
    return it == t->enc.end() ? RANK_MAX : it->second;
}

// Byte-pair encoding of one pre-split piece, to the result tiktoken.rs:26-107
// defines: from single bytes, merge the adjacent pair of parts whose
// concatenation has the lowest rank (the leftmost such pair on a tie) until no
// adjacent concatenation is a token; the ids are the parts' ranks.  Parts are
// a linked list over their start offsets; every pair formed goes into a
// min-heap ordered by (rank, start), and a popped pair whose span no longer
// matches the current parts (one of them has since merged) is dropped, so a
// piece of n bytes costs O(n log n) rank lookups.
bool byte_pair_encode(const czip_tokenizer* t, const uint8_t* piece, size_t len, std::vector<Rank>& out) {
    if (len == 0) return true;
    if (len > UINT32_MAX - 1) return false;
    const uint32_t n = (uint32_t)len, none = UINT32_MAX;
    std::vector<uint32_t> nxt(n), prv(n);  // start of the next / previous part (n after the last, none before the first)
    std::vector<uint8_t> alive(n, 1);
    for (uint32_t s = 0; s < n; s++) {
        nxt[s] = s + 1;
        prv[s] = s ? s - 1 : none;
    }
    struct Pair {
        Rank r;
        uint32_t s, e;  // bytes [s, e): the part at s and the one after it
    };
    auto later = [](const Pair& a, const Pair& b) { return a.r != b.r ? a.r > b.r : a.s > b.s; };
    std::priority_queue<Pair, std::vector<Pair>, decltype(later)> heap(later);
    auto offer = [&](uint32_t s) {  // the pair starting at part s, if it is a token
        const uint32_t m = nxt[s];
        if (m >= n) return;
        const Rank r = rank_of(t, piece + s, nxt[m] - s);
        if (r != RANK_MAX) heap.push({r, s, nxt[m]});
    };
    for (uint32_t s = 0; s + 1 < n; s++) offer(s);
    while (!heap.empty()) {
        const Pair p = heap.top();
        heap.pop();
        if (!alive[p.s] || nxt[p.s] >= n || nxt[nxt[p.s]] != p.e) continue;  // stale
        alive[nxt[p.s]] = 0;
        nxt[p.s] = p.e;
        if (p.e < n) prv[p.e] = p.s;
        if (prv[p.s] != none) offer(prv[p.s]);
        offer(p.s);
    }
    for (uint32_t s = 0; s < n; s = nxt[s]) {
        const Rank r = rank_of(t, piece + s, nxt[s] - s);
        if (r == RANK_MAX) return false;
        out.push_back(r);
    }
    return true;
}

// encode_ordinary over s[begin, end) (tiktoken.rs:200-213, 240-251), with a piece cache
bool encode_plain(const czip_tokenizer* t, const uint8_t* s, size_t n, size_t begin, size_t end,
                  std::vector<Rank>& out, std::unordered_map<std::string, std::vector<Rank>>& cache) {
    size_t i = begin;
    while (i < end) {
        size_t j = match_end(s, n, i);
        if (j > end) j = end;  // split points are chosen so that this never cuts a match
        std::string piece((const char*)s + i, j - i);
        auto it = t->enc.find(piece);
        if (it != t->enc.end()) {
            out.push_back(it->second);
        } else {
            auto ct = cache.find(piece);
            if (ct == cache.end()) {
                std::vector<Rank> toks;
                if (!byte_pair_encode(t, s + i, j - i, toks)) return false;
                ct = cache.emplace(std::move(piece), std::move(toks)).first;
            }
            out.insert(out.end(), ct->second.begin(), ct->second.end());
        }
        i = j;
    }
    return true;
}

// encode_with_special_tokens (tiktoken.rs:215-269): split on special tokens
bool encode_range(const czip_tokenizer* t, const uint8_t* s, size_t n, size_t begin, size_t end,
                  std::vector<Rank>& out) {
    std::unordered_map<std::string, std::vector<Rank>> cache;
    size_t start = begin;
    for (;;) {
        size_t best = end, best_len = 0;
        Rank best_rank = 0;
        for (auto& sp : t->specials) {
            if (sp.first.empty()) continue;
            const void* f = memmem(s + start, end - start, sp.first.data(), sp.first.size());
            if (f) {
                size_t pos = (size_t)((const uint8_t*)f - s);
                if (pos < best) { best = pos; best_len = sp.first.size(); best_rank = sp.second; }
            }
        }
        if (!encode_plain(t, s, n, start, best, out, cache)) return false;
        if (best == end) break;
        out.push_back(best_rank);
        start = best + best_len;
    }
    return true;
}

}  // namespace

czip_status tokenizer_from_json(const char* json, size_t len, czip_tokenizer** out, std::string& err) {
    JParser jp{json, json + len};
    JVal root;
    if (!jp.val(root, 0) || root.kind != JVal::OBJ) { err = "tokenizer JSON is not an object"; return CZIP_E_FORMAT; }
    const JVal* pat = root.get("pat_str");
    const JVal* mr = root.get("mergeable_ranks");
    const JVal* st = root.get("special_tokens");
    if (!pat || pat->kind != JVal::STR || !mr || mr->kind != JVal::OBJ || !st || st->kind != JVal::OBJ) {
        err = "tokenizer JSON lacks pat_str / mergeable_ranks / special_tokens";
        return CZIP_E_FORMAT;
    }
    if (pat->str != kPattern) { err = "unsupported pre-tokenizer pattern"; return CZIP_E_FORMAT; }
    auto t = new czip_tokenizer();
    for (auto& kv : mr->obj) {
        // token_str_to_bytes (tiktoken.rs:517-525): every char is one byte 0..255
        std::string bytes;
        const uint8_t* p = (const uint8_t*)kv.first.data();
        size_t n = kv.first.size(), i = 0, l;
        while (i < n) {
            uint32_t c = cp_at(p, n, i, l);
            if (c > 255) { delete t; err = "token char outside byte range"; return CZIP_E_FORMAT; }
            bytes.push_back((char)c);
            i += l;
        }
        Rank r = (Rank)kv.second.inum;
        t->enc[bytes] = r;
        t->dec[r] = bytes;
    }
    if (t->dec.size() != t->enc.size()) { delete t; err = "duplicate token ranks"; return CZIP_E_FORMAT; }
    for (auto& kv : st->obj) {
        Rank r = (Rank)kv.second.inum;
        t->specials.push_back({kv.first, r});
        t->dec.emplace(r, kv.first);
    }
    const JVal* nv = root.get("explicit_n_vocab");
    if (nv && nv->kind == JVal::NUM && (size_t)nv->inum != t->enc.size() + t->specials.size()) {
        delete t;
        err = "explicit_n_vocab != computed size";
        return CZIP_E_FORMAT;
    }
    *out = t;
    return CZIP_OK;
}

}  // namespace czip

using namespace czip;

extern "C" czip_status czip_tokenizer_load(const char* json, size_t len, czip_tokenizer** out) {
    if (!json || !out) return CZIP_E_ARG;
    std::string err;
    czip_status rc = tokenizer_from_json(json, len, out, err);
    if (rc) fprintf(stderr, "czip_tokenizer_load: %s\n", err.c_str());
    return rc;
}

extern "C" czip_status czip_tokenizer_from_model(const czip_model* m, czip_tokenizer** out) {
    if (!m || !out) return CZIP_E_ARG;
    size_t len = 0;
    const char* codec = nullptr;
    const uint8_t* data = czip_model_tokenizer(m, &len, &codec);
    if (!data) return CZIP_E_MISSING;
    std::vector<char> json;
    // main.rs:88-109: zstd or brotli, from the system libraries
    if (std::string(codec) == "zstd") {
        void* h = dlopen("libzstd.so.1", RTLD_NOW | RTLD_LOCAL);
        if (!h) return CZIP_E_IO;
        auto get_size = (unsigned long long (*)(const void*, size_t))dlsym(h, "ZSTD_getFrameContentSize");
        auto decomp = (size_t (*)(void*, size_t, const void*, size_t))dlsym(h, "ZSTD_decompress");
        auto is_err = (unsigned (*)(size_t))dlsym(h, "ZSTD_isError");
        if (!get_size || !decomp || !is_err) return CZIP_E_IO;
        unsigned long long sz = get_size(data, len);
        if (sz > (1ull << 30)) return CZIP_E_FORMAT;
        json.resize((size_t)sz);
        size_t r = decomp(json.data(), json.size(), data, len);
        if (is_err(r)) return CZIP_E_FORMAT;
        json.resize(r);
    } else if (std::string(codec) == "brotli") {
        void* h = dlopen("libbrotlidec.so.1", RTLD_NOW | RTLD_LOCAL);
        if (!h) return CZIP_E_IO;
        auto decomp = (int (*)(size_t, const uint8_t*, size_t*, uint8_t*))dlsym(h, "BrotliDecoderDecompress");
        if (!decomp) return CZIP_E_IO;
        size_t cap = 1 << 20;
        for (;;) {
            json.resize(cap);
            size_t outl = cap;
            if (decomp(len, data, &outl, (uint8_t*)json.data()) == 1) { json.resize(outl); break; }
            if (cap > (1u << 30)) return CZIP_E_FORMAT;
            cap *= 4;
        }
    } else {
        return CZIP_E_FORMAT;  // "Unknown tokenizer codec" (main.rs:104-107)
    }
    return czip_tokenizer_load(json.data(), json.size(), out);
}

extern "C" void czip_tokenizer_free(czip_tokenizer* t) { delete t; }

extern "C" czip_status czip_tokenize(const czip_tokenizer* t, const char* text, size_t len, int32_t threads,
                                     uint32_t* out, size_t cap, size_t* n_out) {
    if (!t || (!text && len) || !n_out) return CZIP_E_ARG;
    const uint8_t* s = (const uint8_t*)text;
    if (!valid_utf8(s, len)) return CZIP_E_FORMAT;  // the reference reads the input as &str
    // Split points: just after a '\n' whose next character is an ASCII letter.
    // No match of the pattern contains both characters (a letter run never
    // starts with CR/LF, and the other alternatives never end in a letter
    // after a CR/LF), so the pieces are identical to one sequential pass.
    int nt = threads < 1 ? 1 : threads;
    std::vector<size_t> cuts{0};
    if (nt > 1 && len > ((size_t)1 << 20)) {
        size_t longest = 0;
        for (auto& sp : t->specials) longest = std::max(longest, sp.first.size());
        for (int k = 1; k < nt; k++) {
            size_t p = len * (size_t)k / (size_t)nt;
            while (p + 1 < len && !(s[p] == '\n' && is_letter(s[p + 1]))) p++;
            if (p + 1 >= len) break;
            size_t cut = p + 1;
            // never cut through a special token
            bool inside = false;
            for (auto& sp : t->specials) {
                size_t lo = cut >= sp.first.size() ? cut - sp.first.size() + 1 : 0;
                for (size_t q = lo; q < cut && q + sp.first.size() <= len; q++)
                    if (memcmp(s + q, sp.first.data(), sp.first.size()) == 0 && q + sp.first.size() > cut) inside = true;
            }
            if (!inside && cut > cuts.back()) cuts.push_back(cut);
        }
    }
    cuts.push_back(len);
    const size_t nseg = cuts.size() - 1;
    std::vector<std::vector<Rank>> parts(nseg);
    std::vector<int> ok(nseg, 1);
    if (nseg == 1) {
        ok[0] = encode_range(t, s, len, 0, len, parts[0]);
    } else {
        std::vector<std::thread> th;
        for (size_t k = 0; k < nseg; k++)
            th.emplace_back([&, k] { ok[k] = encode_range(t, s, len, cuts[k], cuts[k + 1], parts[k]); });
        for (auto& x : th) x.join();
    }
    size_t total = 0;
    for (size_t k = 0; k < nseg; k++) {
        if (!ok[k]) return CZIP_E_FORMAT;  // unknown byte / merged piece (tiktoken.rs:90, 100-103)
        total += parts[k].size();
    }
    *n_out = total;
    if (total > cap || (total && !out)) return CZIP_E_OVERFLOW;
    size_t o = 0;
    for (auto& p : parts) {
        memcpy(out + o, p.data(), p.size() * sizeof(Rank));
        o += p.size();
    }
    return CZIP_OK;
}

extern "C" czip_status czip_detokenize(const czip_tokenizer* t, const uint32_t* ids, size_t n, uint8_t* out,
                                       size_t cap, size_t* n_out) {
    if (!t || (!ids && n) || !n_out) return CZIP_E_ARG;
    size_t total = 0;
    for (size_t i = 0; i < n; i++) {
        auto it = t->dec.find(ids[i]);
        if (it == t->dec.end()) return CZIP_E_TOKEN;  // DecodeKeyError (tiktoken.rs:186-198)
        total += it->second.size();
    }
    *n_out = total;
    if (total > cap || (total && !out)) return CZIP_E_OVERFLOW;
    size_t o = 0;
    for (size_t i = 0; i < n; i++) {
        const std::string& b = t->dec.find(ids[i])->second;
        memcpy(out + o, b.data(), b.size());
        o += b.size();
    }
    return CZIP_OK;
}
