#include "json.hpp"

#include <cerrno>
#include <cstdlib>
#include <cstring>

namespace tmg {

const JsonValue *JsonValue::get(const std::string &key) const {
    if (kind != Object) return nullptr;
    for (const auto &kv : obj)
        if (kv.first == key) return &kv.second;
    return nullptr;
}

bool JsonValue::as_u64(unsigned long long *out) const {
    if (kind != Number || !is_u64) return false;
    *out = u64;
    return true;
}

bool JsonValue::as_f64(double *out) const {
    if (kind != Number) return false;
    *out = num;
    return true;
}

namespace {

struct Parser {
    const char *p, *end;
    std::string err;
    int depth = 0;

    void ws() {
        while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) p++;
    }
    bool fail(const char *msg) {
        if (err.empty()) err = msg;
        return false;
    }
    bool lit(const char *s) {
        size_t n = strlen(s);
        if ((size_t)(end - p) < n || memcmp(p, s, n) != 0) return false;
        p += n;
        return true;
    }
    static void utf8(std::string &o, unsigned cp) {
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
    bool hex4(unsigned *cp) {
        if (end - p < 4) return fail("truncated \\u escape");
        unsigned v = 0;
        for (int i = 0; i < 4; i++) {
            char c = *p++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= (unsigned)(c - '0');
            else if (c >= 'a' && c <= 'f') v |= (unsigned)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= (unsigned)(c - 'A' + 10);
            else return fail("bad \\u escape");
        }
        *cp = v;
        return true;
    }
    bool string(std::string &o) {
        if (p >= end || *p != '"') return fail("expected string");
        p++;
        while (p < end && *p != '"') {
            char c = *p++;
            if ((unsigned char)c < 0x20) return fail("control character in string");
            if (c != '\\') {
                o += c;
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
                    unsigned cp;
                    if (!hex4(&cp)) return false;
                    if (cp >= 0xD800 && cp < 0xDC00) {
                        unsigned lo;
                        if (!(lit("\\u") && hex4(&lo)) || lo < 0xDC00 || lo > 0xDFFF)
                            return fail("bad surrogate pair");
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    }
                    utf8(o, cp);
                    break;
                }
                default: return fail("bad escape");
            }
        }
        if (p >= end) return fail("unterminated string");
        p++;
        return true;
    }
    bool number(JsonValue &v) {
        const char *s = p;
        bool neg = false, integral = true;
        if (p < end && *p == '-') {
            neg = true;
            p++;
        }
        if (p >= end || !(*p >= '0' && *p <= '9')) return fail("bad number");
        if (*p == '0') p++;
        else
            while (p < end && *p >= '0' && *p <= '9') p++;
        if (p < end && *p == '.') {
            integral = false;
            p++;
            if (p >= end || !(*p >= '0' && *p <= '9')) return fail("bad number");
            while (p < end && *p >= '0' && *p <= '9') p++;
        }
        if (p < end && (*p == 'e' || *p == 'E')) {
            integral = false;
            p++;
            if (p < end && (*p == '+' || *p == '-')) p++;
            if (p >= end || !(*p >= '0' && *p <= '9')) return fail("bad number");
            while (p < end && *p >= '0' && *p <= '9') p++;
        }
        std::string lit_s(s, (size_t)(p - s));
        v.kind = JsonValue::Number;
        v.num = strtod(lit_s.c_str(), nullptr);
        if (integral && !neg) {
            errno = 0;
            unsigned long long u = strtoull(lit_s.c_str(), nullptr, 10);
            if (errno == 0) {
                v.is_u64 = true;
                v.u64 = u;
            }
        }
        return true;
    }
    bool value(JsonValue &v) {
        if (++depth > 256) return fail("nesting too deep");
        ws();
        if (p >= end) return fail("unexpected end of input");
        bool ok = true;
        char c = *p;
        if (c == '{') {
            p++;
            v.kind = JsonValue::Object;
            ws();
            if (p < end && *p == '}') {
                p++;
            } else {
                for (;;) {
                    ws();
                    std::string k;
                    if (!string(k)) return false;
                    ws();
                    if (p >= end || *p != ':') return fail("expected ':'");
                    p++;
                    JsonValue child;
                    if (!value(child)) return false;
                    v.obj.emplace_back(std::move(k), std::move(child));
                    ws();
                    if (p < end && *p == ',') {
                        p++;
                        continue;
                    }
                    if (p < end && *p == '}') {
                        p++;
                        break;
                    }
                    return fail("expected ',' or '}'");
                }
            }
        } else if (c == '[') {
            p++;
            v.kind = JsonValue::Array;
            ws();
            if (p < end && *p == ']') {
                p++;
            } else {
                for (;;) {
                    JsonValue child;
                    if (!value(child)) return false;
                    v.arr.push_back(std::move(child));
                    ws();
                    if (p < end && *p == ',') {
                        p++;
                        continue;
                    }
                    if (p < end && *p == ']') {
                        p++;
                        break;
                    }
                    return fail("expected ',' or ']'");
                }
            }
        } else if (c == '"') {
            v.kind = JsonValue::String;
            ok = string(v.str);
        } else if (c == 't') {
            if (!lit("true")) return fail("bad literal");
            v.kind = JsonValue::Bool;
            v.b = true;
        } else if (c == 'f') {
            if (!lit("false")) return fail("bad literal");
            v.kind = JsonValue::Bool;
        } else if (c == 'n') {
            if (!lit("null")) return fail("bad literal");
            v.kind = JsonValue::Null;
        } else {
            ok = number(v);
        }
        depth--;
        return ok;
    }
};

}  // namespace

bool json_parse(const char *text, size_t len, JsonValue *out, std::string *err) {
    Parser ps{text, text + len, {}};
    JsonValue v;
    if (!ps.value(v)) {
        if (err) *err = ps.err;
        return false;
    }
    ps.ws();
    if (ps.p != ps.end) {
        if (err) *err = "trailing characters after JSON value";
        return false;
    }
    *out = std::move(v);
    return true;
}

}  // namespace tmg
