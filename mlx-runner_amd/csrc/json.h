// Minimal JSON reader/writer for config.json and safetensors headers (untrusted input: depth and
// size limited, every accessor checks the type).
#pragma once
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace mlxr {

struct Json {
    enum Type { Null, Bool, Num, Str, Arr, Obj } t = Null;
    double num = 0;
    std::string str;
    std::vector<Json> arr;
    std::vector<std::pair<std::string, Json>> obj;

    const Json* get(const char* k) const {
        if (t != Obj) return nullptr;
        for (auto& kv : obj) if (kv.first == k) return &kv.second;
        return nullptr;
    }
    bool isNum() const { return t == Num; }
    double numOr(const char* k, double d) const { const Json* v = get(k); return v && (v->t == Num || v->t == Bool) ? v->num : d; }
    bool boolOr(const char* k, bool d) const { const Json* v = get(k); return v && v->t == Bool ? v->num != 0 : d; }
    std::string strOr(const char* k, const std::string& d) const { const Json* v = get(k); return v && v->t == Str ? v->str : d; }

    static bool parse(const char* text, size_t len, Json& out, std::string& err) {
        const char* p = text; const char* end = text + len;
        if (!value(p, end, out, 0, err)) return false;
        ws(p, end);
        if (p != end) { err = "trailing characters"; return false; }
        return true;
    }

private:
    static void ws(const char*& p, const char* e) { while (p < e && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) p++; }
    static bool string(const char*& p, const char* e, std::string& s, std::string& err) {
        if (p >= e || *p != '"') { err = "expected string"; return false; }
        p++;
        while (p < e && *p != '"') {
            char c = *p++;
            if (c == '\\') {
                if (p >= e) break;
                c = *p++;
                switch (c) {
                    case 'n': c = '\n'; break; case 't': c = '\t'; break; case 'r': c = '\r'; break;
                    case 'b': c = '\b'; break; case 'f': c = '\f'; break;
                    case 'u': { if (e - p < 4) { err = "bad escape"; return false; } p += 4; c = '?'; break; }
                    default: break;
                }
            }
            s.push_back(c);
        }
        if (p >= e) { err = "unterminated string"; return false; }
        p++;
        return true;
    }
    static bool value(const char*& p, const char* e, Json& v, int depth, std::string& err) {
        if (depth > 64) { err = "nesting too deep"; return false; }
        ws(p, e);
        if (p >= e) { err = "unexpected end"; return false; }
        if (*p == '{') {
            v.t = Obj; p++; ws(p, e);
            if (p < e && *p == '}') { p++; return true; }
            for (;;) {
                std::string k;
                ws(p, e);
                if (!string(p, e, k, err)) return false;
                ws(p, e);
                if (p >= e || *p != ':') { err = "expected ':'"; return false; }
                p++;
                Json child;
                if (!value(p, e, child, depth + 1, err)) return false;
                v.obj.emplace_back(std::move(k), std::move(child));
                ws(p, e);
                if (p < e && *p == ',') { p++; continue; }
                if (p < e && *p == '}') { p++; return true; }
                err = "expected ',' or '}'"; return false;
            }
        }
        if (*p == '[') {
            v.t = Arr; p++; ws(p, e);
            if (p < e && *p == ']') { p++; return true; }
            for (;;) {
                Json child;
                if (!value(p, e, child, depth + 1, err)) return false;
                v.arr.push_back(std::move(child));
                ws(p, e);
                if (p < e && *p == ',') { p++; continue; }
                if (p < e && *p == ']') { p++; return true; }
                err = "expected ',' or ']'"; return false;
            }
        }
        if (*p == '"') { v.t = Str; return string(p, e, v.str, err); }
        if (e - p >= 4 && !strncmp(p, "true", 4)) { v.t = Bool; v.num = 1; p += 4; return true; }
        if (e - p >= 5 && !strncmp(p, "false", 5)) { v.t = Bool; v.num = 0; p += 5; return true; }
        if (e - p >= 4 && !strncmp(p, "null", 4)) { v.t = Null; p += 4; return true; }
        char buf[64]; size_t n = 0;
        while (p < e && n < 63 && (strchr("+-0123456789.eE", *p))) buf[n++] = *p++;
        buf[n] = 0;
        if (!n) { err = "unexpected character"; return false; }
        char* endp; v.num = strtod(buf, &endp);
        if (endp == buf) { err = "bad number"; return false; }
        v.t = Num;
        return true;
    }
};

}  // namespace mlxr
