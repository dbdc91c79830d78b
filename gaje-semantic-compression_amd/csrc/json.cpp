// Minimal recursive-descent JSON parser (RFC 8259 subset sufficient for the
// .gaje.flat metadata and directory).
#include "json.h"

#include <cerrno>
#include <cstdlib>
#include <cstring>

namespace gaje {

const JsonValue *JsonValue::get(const char *key) const {
    for (const auto &m : members)
        if (m.first == key) return &m.second;
    return nullptr;
}

int JsonValue::count(const char *key) const {
    int c = 0;
    for (const auto &m : members)
        if (m.first == key) ++c;
    return c;
}

namespace {

struct Parser {
    const char *p, *end;
    std::string err;
    int depth = 0;

    bool fail(const char *msg) {
        if (err.empty()) err = msg;
        return false;
    }
    void ws() {
        while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
    }
    bool lit(const char *s) {
        size_t n = strlen(s);
        if ((size_t)(end - p) < n || memcmp(p, s, n) != 0) return fail("invalid literal");
        p += n;
        return true;
    }
    static void put_utf8(std::string &o, uint32_t cp) {
        if (cp < 0x80) {
            o += (char)cp;
        } else if (cp < 0x800) {
            o += (char)(0xC0 | (cp >> 6));
            o += (char)(0x80 | (cp & 0x3F));
        } else if (cp < 0x10000) {
            o += (char)(0xE0 | (cp >> 12));
            o += (char)(0x80 | ((cp >> 6) & 0x3F));
            o += (char)(0x80 | (cp & 0x3F));
        } else {
            o += (char)(0xF0 | (cp >> 18));
            o += (char)(0x80 | ((cp >> 12) & 0x3F));
            o += (char)(0x80 | ((cp >> 6) & 0x3F));
            o += (char)(0x80 | (cp & 0x3F));
        }
    }
    bool hex4(uint32_t &v) {
        if (end - p < 4) return fail("truncated \\u escape");
        v = 0;
        for (int i = 0; i < 4; ++i) {
            char c = *p++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= c - '0';
            else if (c >= 'a' && c <= 'f') v |= c - 'a' + 10;
            else if (c >= 'A' && c <= 'F') v |= c - 'A' + 10;
            else return fail("bad \\u escape");
        }
        return true;
    }
    bool string(std::string &o) {
        if (p >= end || *p != '"') return fail("expected string");
        ++p;
        while (true) {
            if (p >= end) return fail("unterminated string");
            unsigned char c = (unsigned char)*p++;
            if (c == '"') return true;
            if (c < 0x20) return fail("control character in string");
            if (c != '\\') {
                o += (char)c;
                continue;
            }
            if (p >= end) return fail("truncated escape");
            char e = *p++;
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
                    uint32_t cp;
                    if (!hex4(cp)) return false;
                    if (cp >= 0xD800 && cp < 0xDC00) {
                        uint32_t lo;
                        if (end - p < 6 || p[0] != '\\' || p[1] != 'u') return fail("lone surrogate");
                        p += 2;
                        if (!hex4(lo) || lo < 0xDC00 || lo >= 0xE000) return fail("bad surrogate pair");
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    } else if (cp >= 0xDC00 && cp < 0xE000) {
                        return fail("lone surrogate");
                    }
                    put_utf8(o, cp);
                    break;
                }
                default: return fail("invalid escape");
            }
        }
    }
    bool number(JsonValue &v) {
        const char *s = p;
        bool neg = false, integer = true;
        if (p < end && *p == '-') { neg = true; ++p; }
        if (p >= end || !(*p >= '0' && *p <= '9')) return fail("invalid number");
        if (*p == '0') ++p;
        else while (p < end && *p >= '0' && *p <= '9') ++p;
        if (p < end && *p == '.') {
            integer = false;
            ++p;
            if (p >= end || !(*p >= '0' && *p <= '9')) return fail("invalid number");
            while (p < end && *p >= '0' && *p <= '9') ++p;
        }
        if (p < end && (*p == 'e' || *p == 'E')) {
            integer = false;
            ++p;
            if (p < end && (*p == '+' || *p == '-')) ++p;
            if (p >= end || !(*p >= '0' && *p <= '9')) return fail("invalid number");
            while (p < end && *p >= '0' && *p <= '9') ++p;
        }
        std::string text(s, p - s);
        v.type = JsonValue::Number;
        v.number = strtod(text.c_str(), nullptr);
        v.is_integer = integer;
        v.negative = neg;
        if (integer && !neg) {
            errno = 0;
            unsigned long long u = strtoull(text.c_str(), nullptr, 10);
            if (errno == ERANGE) v.is_integer = false;  // beyond u64: not a usize
            v.uinteger = u;
        }
        return true;
    }
    bool value(JsonValue &v) {
        if (++depth > 128) return fail("nesting too deep");
        ws();
        if (p >= end) return fail("unexpected end of input");
        bool ok;
        char c = *p;
        if (c == '{') ok = object(v);
        else if (c == '[') ok = array(v);
        else if (c == '"') { v.type = JsonValue::String; ok = string(v.str); }
        else if (c == 't') { v.type = JsonValue::Bool; v.boolean = true; ok = lit("true"); }
        else if (c == 'f') { v.type = JsonValue::Bool; v.boolean = false; ok = lit("false"); }
        else if (c == 'n') { v.type = JsonValue::Null; ok = lit("null"); }
        else ok = number(v);
        --depth;
        return ok;
    }
    bool array(JsonValue &v) {
        v.type = JsonValue::Array;
        ++p;
        ws();
        if (p < end && *p == ']') { ++p; return true; }
        while (true) {
            v.items.emplace_back();
            if (!value(v.items.back())) return false;
            ws();
            if (p >= end) return fail("unterminated array");
            if (*p == ',') { ++p; continue; }
            if (*p == ']') { ++p; return true; }
            return fail("expected ',' or ']'");
        }
    }
    bool object(JsonValue &v) {
        v.type = JsonValue::Object;
        ++p;
        ws();
        if (p < end && *p == '}') { ++p; return true; }
        while (true) {
            ws();
            std::string key;
            if (!string(key)) return false;
            ws();
            if (p >= end || *p != ':') return fail("expected ':'");
            ++p;
            v.members.emplace_back(std::move(key), JsonValue());
            if (!value(v.members.back().second)) return false;
            ws();
            if (p >= end) return fail("unterminated object");
            if (*p == ',') { ++p; continue; }
            if (*p == '}') { ++p; return true; }
            return fail("expected ',' or '}'");
        }
    }
};

}  // namespace

bool json_parse(const char *data, size_t len, JsonValue &out, std::string &err) {
    Parser ps{data, data + len, {}, 0};
    out = JsonValue();
    if (!ps.value(out)) {
        err = ps.err;
        return false;
    }
    ps.ws();
    if (ps.p != ps.end) {
        err = "trailing characters";
        return false;
    }
    return true;
}

bool utf8_valid(const unsigned char *s, size_t n) {
    size_t i = 0;
    while (i < n) {
        unsigned char c = s[i];
        if (c < 0x80) { ++i; continue; }
        int len;
        uint32_t cp;
        if ((c & 0xE0) == 0xC0) { len = 2; cp = c & 0x1F; }
        else if ((c & 0xF0) == 0xE0) { len = 3; cp = c & 0x0F; }
        else if ((c & 0xF8) == 0xF0) { len = 4; cp = c & 0x07; }
        else return false;
        if (i + len > n) return false;
        for (int k = 1; k < len; ++k) {
            if ((s[i + k] & 0xC0) != 0x80) return false;
            cp = (cp << 6) | (s[i + k] & 0x3F);
        }
        if ((len == 2 && cp < 0x80) || (len == 3 && cp < 0x800) || (len == 4 && cp < 0x10000))
            return false;  // overlong
        if (cp > 0x10FFFF || (cp >= 0xD800 && cp < 0xE000)) return false;
        i += len;
    }
    return true;
}

}  // namespace gaje
