// ibh_json.h -- minimal JSON reader for the IBF headers (host code).
#pragma once

#include <stdlib.h>
#include <string.h>

#include <string>
#include <utility>
#include <vector>

namespace ibh {

// The IBF v1 and v5 headers are plain JSON (ibf_loader.c:124-221,
// pq_decode.c:685-721).
struct JVal {
    enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
    double num = 0;
    bool b = false;
    std::string str;
    std::vector<JVal> arr;
    std::vector<std::pair<std::string, JVal>> obj;
    const JVal* get(const char* k) const {
        if (kind != OBJ) return nullptr;
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
        const size_t n = strlen(s);
        if ((size_t)(e - p) >= n && !memcmp(p, s, n)) {
            p += n;
            return true;
        }
        return false;
    }
    std::string string() {
        std::string s;
        p++;   // opening quote
        while (p < e && *p != '"') {
            if (*p == '\\' && p + 1 < e) {
                p++;
                const char c = *p;
                if (c == 'n') s += '\n';
                else if (c == 't') s += '\t';
                else if (c == 'r') s += '\r';
                else if (c == 'b') s += '\b';
                else if (c == 'f') s += '\f';
                else if (c == 'u') { s += '?'; p += (e - p > 4) ? 4 : 0; }
                else s += c;
                p++;
            } else {
                s += *p++;
            }
        }
        if (p >= e) ok = false;
        else p++;
        return s;
    }
    JVal value(int depth) {
        JVal v;
        ws();
        if (p >= e || depth > 64) { ok = false; return v; }
        if (*p == '{') {
            v.kind = JVal::OBJ;
            p++;
            ws();
            if (p < e && *p == '}') { p++; return v; }
            while (ok) {
                ws();
                if (p >= e || *p != '"') { ok = false; break; }
                std::string k = string();
                ws();
                if (p >= e || *p != ':') { ok = false; break; }
                p++;
                v.obj.emplace_back(std::move(k), value(depth + 1));
                ws();
                if (p < e && *p == ',') { p++; continue; }
                if (p < e && *p == '}') { p++; break; }
                ok = false;
            }
        } else if (*p == '[') {
            v.kind = JVal::ARR;
            p++;
            ws();
            if (p < e && *p == ']') { p++; return v; }
            while (ok) {
                v.arr.push_back(value(depth + 1));
                ws();
                if (p < e && *p == ',') { p++; continue; }
                if (p < e && *p == ']') { p++; break; }
                ok = false;
            }
        } else if (*p == '"') {
            v.kind = JVal::STR;
            v.str = string();
        } else if (lit("true")) {
            v.kind = JVal::BOOL; v.b = true;
        } else if (lit("false")) {
            v.kind = JVal::BOOL;
        } else if (lit("null")) {
        } else {
            std::string num;
            while (p < e && (strchr("+-.eE", *p) || (*p >= '0' && *p <= '9'))) num += *p++;
            if (num.empty()) { ok = false; return v; }
            v.kind = JVal::NUM;
            v.num = strtod(num.c_str(), nullptr);
        }
        return v;
    }
};

// cJSON's valueint saturates the double to int (ibf_loader.c:41-45 reads it).
inline int jint(const JVal* o, const char* k, int def) {
    const JVal* v = o ? o->get(k) : nullptr;
    if (!v || v->kind != JVal::NUM) return def;
    if (v->num >= 2147483647.0) return 2147483647;
    if (v->num <= -2147483648.0) return (-2147483647 - 1);
    return (int)v->num;
}
inline double jdbl(const JVal* o, const char* k, double def) {
    const JVal* v = o ? o->get(k) : nullptr;
    return v && v->kind == JVal::NUM ? v->num : def;
}
inline size_t jsize(const JVal* o, const char* k, size_t def) {
    const JVal* v = o ? o->get(k) : nullptr;
    return v && v->kind == JVal::NUM ? (size_t)v->num : def;
}


}  // namespace ibh
