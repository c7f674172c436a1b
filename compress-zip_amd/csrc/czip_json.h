// Minimal JSON reader shared by the .czm loader and the tokenizer loader.
#pragma once

#include <cstdlib>
#include <cstring>
#include <string>
#include <utility>
#include <vector>

namespace czip {

struct JVal {
    enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
    double num = 0;
    long long inum = 0;
    bool isint = false;
    std::string str;
    std::vector<JVal> arr;
    std::vector<std::pair<std::string, JVal>> obj;
    const JVal* get(const std::string& k) const {
        for (auto& kv : obj)
            if (kv.first == k) return &kv.second;
        return nullptr;
    }
};

struct JParser {
    const char* p;
    const char* e;
    bool ok = true;
    void ws() {
        while (p < e && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) p++;
    }
    bool lit(const char* s) {
        size_t n = strlen(s);
        if ((size_t)(e - p) >= n && memcmp(p, s, n) == 0) { p += n; return true; }
        return false;
    }
    static void put_utf8(std::string& o, unsigned cp) {
        if (cp < 0x80) o += (char)cp;
        else if (cp < 0x800) { o += (char)(0xC0 | (cp >> 6)); o += (char)(0x80 | (cp & 63)); }
        else if (cp < 0x10000) {
            o += (char)(0xE0 | (cp >> 12)); o += (char)(0x80 | ((cp >> 6) & 63)); o += (char)(0x80 | (cp & 63));
        } else {
            o += (char)(0xF0 | (cp >> 18)); o += (char)(0x80 | ((cp >> 12) & 63));
            o += (char)(0x80 | ((cp >> 6) & 63)); o += (char)(0x80 | (cp & 63));
        }
    }
    unsigned hex4() {
        if (e - p < 4) { ok = false; return 0; }
        unsigned v = 0;
        for (int i = 0; i < 4; i++) {
            char c = *p++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= (unsigned)(c - '0');
            else if (c >= 'a' && c <= 'f') v |= (unsigned)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= (unsigned)(c - 'A' + 10);
            else ok = false;
        }
        return v;
    }
    bool str(std::string& o) {
        if (p >= e || *p != '"') return false;
        p++;
        while (p < e && *p != '"') {
            char c = *p++;
            if (c != '\\') { o += c; continue; }
            if (p >= e) return false;
            char x = *p++;
            switch (x) {
                case '"': o += '"'; break;
                case '\\': o += '\\'; break;
                case '/': o += '/'; break;
                case 'b': o += '\b'; break;
                case 'f': o += '\f'; break;
                case 'n': o += '\n'; break;
                case 'r': o += '\r'; break;
                case 't': o += '\t'; break;
                case 'u': {
                    unsigned cp = hex4();
                    if (cp >= 0xD800 && cp < 0xDC00 && e - p >= 6 && p[0] == '\\' && p[1] == 'u') {
                        p += 2;
                        unsigned lo = hex4();
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    }
                    put_utf8(o, cp);
                    break;
                }
                default: return false;
            }
        }
        if (p >= e) return false;
        p++;
        return ok;
    }
    bool val(JVal& v, int depth) {
        if (depth > 64) return false;
        ws();
        if (p >= e) return false;
        if (*p == '{') {
            p++;
            v.kind = JVal::OBJ;
            ws();
            if (p < e && *p == '}') { p++; return true; }
            for (;;) {
                ws();
                std::string k;
                if (!str(k)) return false;
                ws();
                if (p >= e || *p != ':') return false;
                p++;
                JVal c;
                if (!val(c, depth + 1)) return false;
                v.obj.emplace_back(std::move(k), std::move(c));
                ws();
                if (p < e && *p == ',') { p++; continue; }
                if (p < e && *p == '}') { p++; return true; }
                return false;
            }
        }
        if (*p == '[') {
            p++;
            v.kind = JVal::ARR;
            ws();
            if (p < e && *p == ']') { p++; return true; }
            for (;;) {
                JVal c;
                if (!val(c, depth + 1)) return false;
                v.arr.push_back(std::move(c));
                ws();
                if (p < e && *p == ',') { p++; continue; }
                if (p < e && *p == ']') { p++; return true; }
                return false;
            }
        }
        if (*p == '"') { v.kind = JVal::STR; return str(v.str); }
        if (lit("true")) { v.kind = JVal::BOOL; v.num = 1; return true; }
        if (lit("false")) { v.kind = JVal::BOOL; return true; }
        if (lit("null")) { v.kind = JVal::NUL; return true; }
        const char* s = p;
        bool isint = true;
        if (p < e && (*p == '-' || *p == '+')) p++;
        while (p < e && ((*p >= '0' && *p <= '9') || *p == '.' || *p == 'e' || *p == 'E' || *p == '-' || *p == '+')) {
            if (*p == '.' || *p == 'e' || *p == 'E') isint = false;
            p++;
        }
        if (p == s) return false;
        std::string t(s, p);
        v.kind = JVal::NUM;
        v.isint = isint;
        v.num = strtod(t.c_str(), nullptr);
        v.inum = isint ? strtoll(t.c_str(), nullptr, 10) : (long long)v.num;
        return true;
    }
};

}  // namespace czip
