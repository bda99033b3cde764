// Minimal JSON reader for the checkpoint metadata (safetensors headers, config.json,
// model.safetensors.index.json). Builds a small DOM; objects keep member order and
// duplicate keys (safetensors rejects duplicate tensor names, so the reader must see them).
// Accepts RFC 8259 JSON: no comments, no trailing commas, nesting up to 64 levels (the
// depth limit of System.Text.Json's JsonDocument, which the reference parses with,
// SafeTensors.cs:23 and Qwen36Weights.cs:27). Host code only.
#pragma once
#include <stdint.h>

#include <cmath>
#include <cstdlib>
#include <string>
#include <utility>
#include <vector>

namespace dih {
namespace json {

struct Value {
    enum Type { Null, Bool, Number, String, Array, Object };
    Type type = Null;
    bool boolean = false;
    double number = 0.0;
    bool integral = false;  // number written without fraction/exponent and within int64
    int64_t integer = 0;
    std::string text;
    std::vector<Value> items;
    std::vector<std::pair<std::string, Value>> members;

    // first member named `key`, or nullptr
    const Value *find(const std::string &key) const {
        if (type != Object) return nullptr;
        for (const auto &m : members)
            if (m.first == key) return &m.second;
        return nullptr;
    }
    bool is_int32() const { return type == Number && integral && integer >= INT32_MIN && integer <= INT32_MAX; }
};

class Parser {
  public:
    Parser(const char *p, size_t n) : p_(p), end_(p + n) {}

    bool parse(Value &out, std::string &err) {
        skip_ws();
        if (!value(out, 0)) {
            err = err_.empty() ? "Invalid JSON" : err_;
            return false;
        }
        skip_ws();
        if (p_ != end_) {
            err = "Invalid JSON: trailing characters";
            return false;
        }
        return true;
    }

  private:
    const char *p_, *end_;
    std::string err_;

    bool fail(const char *msg) {
        if (err_.empty()) err_ = std::string("Invalid JSON: ") + msg;
        return false;
    }
    void skip_ws() {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
    }
    bool literal(const char *word) {
        const char *q = p_;
        for (; *word; ++word, ++q)
            if (q >= end_ || *q != *word) return fail("bad literal");
        p_ = q;
        return true;
    }
    bool value(Value &v, int depth) {
        if (depth > 64) return fail("nesting too deep");
        if (p_ >= end_) return fail("unexpected end");
        switch (*p_) {
            case '{': return object(v, depth);
            case '[': return array(v, depth);
            case '"': v.type = Value::String; return string(v.text);
            case 't': v.type = Value::Bool; v.boolean = true; return literal("true");
            case 'f': v.type = Value::Bool; v.boolean = false; return literal("false");
            case 'n': v.type = Value::Null; return literal("null");
            default: return number(v);
        }
    }
    bool object(Value &v, int depth) {
        v.type = Value::Object;
        ++p_;
        skip_ws();
        if (p_ < end_ && *p_ == '}') { ++p_; return true; }
        for (;;) {
            skip_ws();
            if (p_ >= end_ || *p_ != '"') return fail("expected member name");
            std::string key;
            if (!string(key)) return false;
            skip_ws();
            if (p_ >= end_ || *p_ != ':') return fail("expected ':'");
            ++p_;
            skip_ws();
            v.members.emplace_back(std::move(key), Value());
            if (!value(v.members.back().second, depth + 1)) return false;
            skip_ws();
            if (p_ < end_ && *p_ == ',') { ++p_; continue; }
            if (p_ < end_ && *p_ == '}') { ++p_; return true; }
            return fail("expected ',' or '}'");
        }
    }
    bool array(Value &v, int depth) {
        v.type = Value::Array;
        ++p_;
        skip_ws();
        if (p_ < end_ && *p_ == ']') { ++p_; return true; }
        for (;;) {
            skip_ws();
            v.items.emplace_back();
            if (!value(v.items.back(), depth + 1)) return false;
            skip_ws();
            if (p_ < end_ && *p_ == ',') { ++p_; continue; }
            if (p_ < end_ && *p_ == ']') { ++p_; return true; }
            return fail("expected ',' or ']'");
        }
    }
    static void put_utf8(std::string &s, uint32_t cp) {
        if (cp < 0x80) {
            s += (char)cp;
        } else if (cp < 0x800) {
            s += (char)(0xc0 | (cp >> 6));
            s += (char)(0x80 | (cp & 0x3f));
        } else if (cp < 0x10000) {
            s += (char)(0xe0 | (cp >> 12));
            s += (char)(0x80 | ((cp >> 6) & 0x3f));
            s += (char)(0x80 | (cp & 0x3f));
        } else {
            s += (char)(0xf0 | (cp >> 18));
            s += (char)(0x80 | ((cp >> 12) & 0x3f));
            s += (char)(0x80 | ((cp >> 6) & 0x3f));
            s += (char)(0x80 | (cp & 0x3f));
        }
    }
    bool hex4(uint32_t &cp) {
        if (end_ - p_ < 4) return fail("short \\u escape");
        cp = 0;
        for (int i = 0; i < 4; i++, ++p_) {
            const char c = *p_;
            cp <<= 4;
            if (c >= '0' && c <= '9') cp |= (uint32_t)(c - '0');
            else if (c >= 'a' && c <= 'f') cp |= (uint32_t)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') cp |= (uint32_t)(c - 'A' + 10);
            else return fail("bad \\u escape");
        }
        return true;
    }
    // a UTF-8 sequence starting at p_ (lead byte >= 0x80), copied through after validation
    bool utf8(std::string &s) {
        const unsigned char c = (unsigned char)*p_;
        int n;
        uint32_t cp;
        if (c >= 0xc2 && c <= 0xdf) { n = 1; cp = c & 0x1f; }
        else if (c >= 0xe0 && c <= 0xef) { n = 2; cp = c & 0x0f; }
        else if (c >= 0xf0 && c <= 0xf4) { n = 3; cp = c & 0x07; }
        else return fail("invalid UTF-8");
        if (end_ - p_ < n + 1) return fail("invalid UTF-8");
        for (int i = 1; i <= n; i++) {
            const unsigned char d = (unsigned char)p_[i];
            if ((d & 0xc0) != 0x80) return fail("invalid UTF-8");
            cp = (cp << 6) | (d & 0x3f);
        }
        if ((n == 2 && cp < 0x800) || (n == 3 && (cp < 0x10000 || cp > 0x10ffff)) || (cp >= 0xd800 && cp <= 0xdfff))
            return fail("invalid UTF-8");
        s.append(p_, (size_t)n + 1);
        p_ += n + 1;
        return true;
    }
    bool string(std::string &s) {
        ++p_;  // opening quote
        for (;;) {
            if (p_ >= end_) return fail("unterminated string");
            const unsigned char c = (unsigned char)*p_;
            if (c == '"') { ++p_; return true; }
            if (c < 0x20) return fail("control character in string");
            if (c >= 0x80) {
                if (!utf8(s)) return false;
                continue;
            }
            if (c != '\\') { s += (char)c; ++p_; continue; }
            ++p_;
            if (p_ >= end_) return fail("unterminated escape");
            const char e = *p_++;
            switch (e) {
                case '"': s += '"'; break;
                case '\\': s += '\\'; break;
                case '/': s += '/'; break;
                case 'b': s += '\b'; break;
                case 'f': s += '\f'; break;
                case 'n': s += '\n'; break;
                case 'r': s += '\r'; break;
                case 't': s += '\t'; break;
                case 'u': {
                    uint32_t cp;
                    if (!hex4(cp)) return false;
                    if (cp >= 0xd800 && cp <= 0xdbff) {  // high surrogate: a low one must follow
                        uint32_t lo;
                        if (end_ - p_ < 2 || p_[0] != '\\' || p_[1] != 'u') return fail("lone surrogate");
                        p_ += 2;
                        if (!hex4(lo) || lo < 0xdc00 || lo > 0xdfff) return fail("lone surrogate");
                        cp = 0x10000 + ((cp - 0xd800) << 10) + (lo - 0xdc00);
                    } else if (cp >= 0xdc00 && cp <= 0xdfff) {
                        return fail("lone surrogate");
                    }
                    put_utf8(s, cp);
                    break;
                }
                default: return fail("bad escape");
            }
        }
    }
    bool number(Value &v) {
        const char *s = p_;
        bool frac = false;
        if (p_ < end_ && *p_ == '-') ++p_;
        if (p_ >= end_) return fail("bad number");
        if (*p_ == '0') {
            ++p_;
        } else if (*p_ >= '1' && *p_ <= '9') {
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        } else {
            return fail("unexpected character");
        }
        if (p_ < end_ && *p_ == '.') {
            frac = true;
            ++p_;
            if (p_ >= end_ || *p_ < '0' || *p_ > '9') return fail("bad number");
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        if (p_ < end_ && (*p_ == 'e' || *p_ == 'E')) {
            frac = true;
            ++p_;
            if (p_ < end_ && (*p_ == '+' || *p_ == '-')) ++p_;
            if (p_ >= end_ || *p_ < '0' || *p_ > '9') return fail("bad number");
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        const std::string tok(s, p_);
        v.type = Value::Number;
        v.number = std::strtod(tok.c_str(), nullptr);
        v.integral = false;
        if (!frac) {
            // exact int64 or not integral at all
            const bool neg = tok[0] == '-';
            uint64_t mag = 0;
            bool ok = true;
            for (size_t i = neg ? 1 : 0; i < tok.size(); i++) {
                const uint64_t d = (uint64_t)(tok[i] - '0');
                if (mag > (UINT64_MAX - d) / 10) { ok = false; break; }
                mag = mag * 10 + d;
            }
            if (ok && (neg ? mag <= (uint64_t)INT64_MAX + 1 : mag <= (uint64_t)INT64_MAX)) {
                v.integral = true;
                v.integer = neg ? (int64_t)(0 - mag) : (int64_t)mag;
            }
        }
        return true;
    }
};

inline bool parse(const char *p, size_t n, Value &out, std::string &err) {
    Parser ps(p, n);
    return ps.parse(out, err);
}

}  // namespace json
}  // namespace dih
