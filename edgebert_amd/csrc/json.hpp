// json.hpp -- a small JSON reader for the safetensors header and tokenizer.json.
#pragma once
#include <cstdlib>
#include <cstring>
#include <map>
#include <string>
#include <vector>

namespace ebh {
namespace json {

struct JVal {
    enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
    double num = 0;
    std::string str;
    std::vector<JVal> arr;
    std::map<std::string, JVal> obj;
};

struct Parser {
    const char* p;
    const char* end;
    std::string err;

    void ws() {
        while (p < end && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) ++p;
    }
    bool expect(char c) {
        ws();
        if (p < end && *p == c) { ++p; return true; }
        err = std::string("expected '") + c + "'";
        return false;
    }
    static bool hex4(const char* q, unsigned& v) {
        v = 0;
        for (int i = 0; i < 4; ++i) {
            const char h = q[i];
            v <<= 4;
            if (h >= '0' && h <= '9') v |= h - '0';
            else if (h >= 'a' && h <= 'f') v |= h - 'a' + 10;
            else if (h >= 'A' && h <= 'F') v |= h - 'A' + 10;
            else return false;
        }
        return true;
    }
    static void put_utf8(std::string& out, unsigned cp) {
        if (cp < 0x80) {
            out += (char)cp;
        } else if (cp < 0x800) {
            out += (char)(0xC0 | (cp >> 6));
            out += (char)(0x80 | (cp & 0x3F));
        } else if (cp < 0x10000) {
            out += (char)(0xE0 | (cp >> 12));
            out += (char)(0x80 | ((cp >> 6) & 0x3F));
            out += (char)(0x80 | (cp & 0x3F));
        } else {
            out += (char)(0xF0 | (cp >> 18));
            out += (char)(0x80 | ((cp >> 12) & 0x3F));
            out += (char)(0x80 | ((cp >> 6) & 0x3F));
            out += (char)(0x80 | (cp & 0x3F));
        }
    }
    bool parse_string(std::string& out) {
        if (!expect('"')) return false;
        while (p < end && *p != '"') {
            char c = *p++;
            if (c == '\\') {
                if (p >= end) break;
                char e = *p++;
                switch (e) {
                    case '"': out += '"'; break;
                    case '\\': out += '\\'; break;
                    case '/': out += '/'; break;
                    case 'b': out += '\b'; break;
                    case 'f': out += '\f'; break;
                    case 'n': out += '\n'; break;
                    case 'r': out += '\r'; break;
                    case 't': out += '\t'; break;
                    case 'u': {
                        unsigned cp = 0;
                        if (end - p < 4 || !hex4(p, cp)) { err = "bad \\u escape"; return false; }
                        p += 4;
                        if (cp >= 0xD800 && cp < 0xDC00) {  // high surrogate: a low one must follow
                            unsigned lo = 0;
                            if (end - p < 6 || p[0] != '\\' || p[1] != 'u' || !hex4(p + 2, lo) || lo < 0xDC00 ||
                                lo > 0xDFFF) {
                                err = "unpaired surrogate in \\u escape";
                                return false;
                            }
                            p += 6;
                            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                        } else if (cp >= 0xDC00 && cp <= 0xDFFF) {
                            err = "unpaired surrogate in \\u escape";
                            return false;
                        }
                        put_utf8(out, cp);
                        break;
                    }
                    default: err = "bad escape"; return false;
                }
            } else {
                out += c;
            }
        }
        if (p >= end) { err = "unterminated string"; return false; }
        ++p;
        return true;
    }
    bool parse(JVal& v, int depth = 0) {
        if (depth > 64) { err = "nesting too deep"; return false; }
        ws();
        if (p >= end) { err = "unexpected end"; return false; }
        char c = *p;
        if (c == '{') {
            ++p;
            v.kind = JVal::OBJ;
            ws();
            if (p < end && *p == '}') { ++p; return true; }
            while (true) {
                std::string key;
                if (!parse_string(key)) return false;
                if (!expect(':')) return false;
                JVal child;
                if (!parse(child, depth + 1)) return false;
                v.obj[key] = std::move(child);
                ws();
                if (p < end && *p == ',') { ++p; continue; }
                return expect('}');
            }
        }
        if (c == '[') {
            ++p;
            v.kind = JVal::ARR;
            ws();
            if (p < end && *p == ']') { ++p; return true; }
            while (true) {
                JVal child;
                if (!parse(child, depth + 1)) return false;
                v.arr.push_back(std::move(child));
                ws();
                if (p < end && *p == ',') { ++p; continue; }
                return expect(']');
            }
        }
        if (c == '"') { v.kind = JVal::STR; return parse_string(v.str); }
        if (c == 't' && end - p >= 4 && !strncmp(p, "true", 4)) { p += 4; v.kind = JVal::BOOL; v.num = 1; return true; }
        if (c == 'f' && end - p >= 5 && !strncmp(p, "false", 5)) { p += 5; v.kind = JVal::BOOL; return true; }
        if (c == 'n' && end - p >= 4 && !strncmp(p, "null", 4)) { p += 4; v.kind = JVal::NUL; return true; }
        if (c == '-' || (c >= '0' && c <= '9')) {
            const char* q = p;
            while (q < end && (strchr("+-.eE", *q) || (*q >= '0' && *q <= '9'))) ++q;
            v.kind = JVal::NUM;
            v.num = strtod(std::string(p, q).c_str(), nullptr);
            p = q;
            return true;
        }
        err = "unexpected character";
        return false;
    }
};

// Member `key` of an object, or nullptr.
inline const JVal* get(const JVal& v, const char* key) {
    if (v.kind != JVal::OBJ) return nullptr;
    auto it = v.obj.find(key);
    return it == v.obj.end() ? nullptr : &it->second;
}

}  // namespace json
}  // namespace ebh
