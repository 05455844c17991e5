// A small JSON reader (the config, the `.lsq` header, the tokenizer's files): objects keep their
// key order, numbers are doubles; errors are LS_E_FORMAT.
#pragma once

#include <cctype>
#include <cstring>
#include <string>
#include <utility>
#include <vector>

#include "common.hpp"

namespace ls {

struct Json {
    enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
    bool b = false;
    double num = 0;
    std::string str;
    std::vector<Json> arr;
    std::vector<std::pair<std::string, Json>> obj;

    const Json* get(const std::string& k) const {
        if (kind != Obj) return nullptr;
        for (auto& kv : obj)
            if (kv.first == k) return &kv.second;
        return nullptr;
    }
};

struct JsonParser {
    const std::string& s;
    size_t i = 0;
    explicit JsonParser(const std::string& t) : s(t) {}

    [[noreturn]] void err(const char* what) { fail(std::string("json: ") + what + " at byte " + std::to_string(i), LS_E_FORMAT); }
    void ws() {
        while (i < s.size() && (s[i] == ' ' || s[i] == '\n' || s[i] == '\r' || s[i] == '\t')) i++;
    }
    bool lit(const char* w) {
        size_t n = std::strlen(w);
        if (s.compare(i, n, w) == 0) {
            i += n;
            return true;
        }
        return false;
    }
    static void put_utf8(std::string& o, uint32_t cp) {
        if (cp < 0x80) {
            o += char(cp);
        } else if (cp < 0x800) {
            o += char(0xC0 | (cp >> 6));
            o += char(0x80 | (cp & 0x3F));
        } else if (cp < 0x10000) {
            o += char(0xE0 | (cp >> 12));
            o += char(0x80 | ((cp >> 6) & 0x3F));
            o += char(0x80 | (cp & 0x3F));
        } else {
            o += char(0xF0 | (cp >> 18));
            o += char(0x80 | ((cp >> 12) & 0x3F));
            o += char(0x80 | ((cp >> 6) & 0x3F));
            o += char(0x80 | (cp & 0x3F));
        }
    }
    uint32_t hex4() {
        if (i + 4 > s.size()) err("short \\u escape");
        uint32_t v = 0;
        for (int k = 0; k < 4; k++) {
            char c = s[i++];
            v <<= 4;
            if (c >= '0' && c <= '9') v |= c - '0';
            else if (c >= 'a' && c <= 'f') v |= c - 'a' + 10;
            else if (c >= 'A' && c <= 'F') v |= c - 'A' + 10;
            else err("bad \\u escape");
        }
        return v;
    }
    std::string string() {
        if (s[i] != '"') err("expected a string");
        i++;
        std::string o;
        while (true) {
            if (i >= s.size()) err("unterminated string");
            char c = s[i++];
            if (c == '"') break;
            if (c != '\\') {
                o += c;
                continue;
            }
            if (i >= s.size()) err("unterminated escape");
            char e = s[i++];
            switch (e) {
                case '"': o += '"'; break;
                case '\\': o += '\\'; break;
                case '/': o += '/'; break;
                case 'b': o += '\b'; break;
                case 'f': o += '\f'; break;
                case 'n': o += '\n'; break;
                case 'r': o += '\r'; break;
                case 't': o += '\t'; break;
                case 'u': {
                    uint32_t cp = hex4();
                    if (cp >= 0xD800 && cp < 0xDC00 && i + 6 <= s.size() && s[i] == '\\' && s[i + 1] == 'u') {
                        i += 2;
                        uint32_t lo = hex4();
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    }
                    put_utf8(o, cp);
                    break;
                }
                default: err("bad escape");
            }
        }
        return o;
    }
    Json value(int depth = 0) {
        if (depth > 64) err("nesting too deep");
        ws();
        if (i >= s.size()) err("unexpected end");
        Json j;
        char c = s[i];
        if (c == '{') {
            j.kind = Json::Obj;
            i++;
            ws();
            if (i < s.size() && s[i] == '}') {
                i++;
                return j;
            }
            while (true) {
                ws();
                std::string k = string();
                ws();
                if (i >= s.size() || s[i] != ':') err("expected ':'");
                i++;
                j.obj.emplace_back(k, value(depth + 1));
                ws();
                if (i < s.size() && s[i] == ',') {
                    i++;
                    continue;
                }
                if (i < s.size() && s[i] == '}') {
                    i++;
                    break;
                }
                err("expected ',' or '}'");
            }
        } else if (c == '[') {
            j.kind = Json::Arr;
            i++;
            ws();
            if (i < s.size() && s[i] == ']') {
                i++;
                return j;
            }
            while (true) {
                j.arr.push_back(value(depth + 1));
                ws();
                if (i < s.size() && s[i] == ',') {
                    i++;
                    continue;
                }
                if (i < s.size() && s[i] == ']') {
                    i++;
                    break;
                }
                err("expected ',' or ']'");
            }
        } else if (c == '"') {
            j.kind = Json::Str;
            j.str = string();
        } else if (lit("true")) {
            j.kind = Json::Bool;
            j.b = true;
        } else if (lit("false")) {
            j.kind = Json::Bool;
        } else if (lit("null")) {
            j.kind = Json::Null;
        } else {
            size_t st = i;
            if (s[i] == '-') i++;
            while (i < s.size() && (isdigit((unsigned char)s[i]) || s[i] == '.' || s[i] == 'e' || s[i] == 'E' || s[i] == '+' || s[i] == '-')) i++;
            if (st == i) err("unexpected character");
            j.kind = Json::Num;
            try {
                j.num = std::stod(s.substr(st, i - st));
            } catch (...) {
                err("bad number");
            }
        }
        return j;
    }
    Json parse() {
        Json j = value();
        ws();
        if (i != s.size()) err("trailing characters");
        return j;
    }
};


}  // namespace ls
