// hk_json.h -- a small JSON reader for the container headers and catalog
// manifests the loader parses (RFC 8259: objects, arrays, strings with
// escapes, numbers, true/false/null).  Integers are kept exactly when the
// literal has no fraction or exponent, so "integer" fields follow the
// reference's serde_json as_u64 / as_i64 rules: 5 is an integer, 5.0 and 5e0
// are not.  Duplicate keys: the last one wins (serde_json's map behaviour).
#pragma once

#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <string>
#include <utility>
#include <vector>

namespace hk {
namespace json {

struct Value {
    enum Type { Null, Bool, Number, String, Array, Object } type = Null;
    bool b = false;
    double num = 0.0;
    bool is_int = false;  // an integer literal that fits u64 (non-negative) or i64 (negative)
    bool neg = false;
    uint64_t mag = 0;     // |value| of an integer literal
    std::string s;
    std::vector<Value> arr;
    std::vector<std::pair<std::string, Value>> obj;

    const Value* get(const std::string& key) const {
        if (type != Object) return nullptr;
        for (size_t i = obj.size(); i-- > 0;)
            if (obj[i].first == key) return &obj[i].second;
        return nullptr;
    }
    const std::string* str() const { return type == String ? &s : nullptr; }
    // as_u64: a non-negative integer literal
    bool u64(uint64_t* out) const {
        if (type != Number || !is_int || neg) return false;
        *out = mag;
        return true;
    }
    bool negative_int() const { return type == Number && is_int && neg; }
    bool f64(double* out) const {
        if (type != Number) return false;
        *out = num;
        return true;
    }
};

class Parser {
public:
    Parser(const char* p, size_t n) : p_(p), e_(p + n) {}

    bool parse(Value* out, std::string* err) {
        ws();
        if (!value(out, 0)) {
            *err = err_.empty() ? "invalid JSON" : err_;
            return false;
        }
        ws();
        if (p_ != e_) {
            *err = "trailing characters after the JSON value";
            return false;
        }
        return true;
    }

private:
    const char* p_;
    const char* e_;
    std::string err_;

    void ws() {
        while (p_ < e_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
    }
    bool fail(const char* m) {
        if (err_.empty()) err_ = m;
        return false;
    }
    bool lit(const char* w) {
        const char* q = p_;
        for (; *w; ++w, ++q)
            if (q >= e_ || *q != *w) return false;
        p_ = q;
        return true;
    }

    bool value(Value* v, int depth) {
        if (depth > 64) return fail("JSON nested too deeply");
        if (p_ >= e_) return fail("unexpected end of JSON");
        switch (*p_) {
        case '{': return object(v, depth);
        case '[': return array(v, depth);
        case '"': v->type = Value::String; return string(&v->s);
        case 't': v->type = Value::Bool; v->b = true; return lit("true") || fail("invalid literal");
        case 'f': v->type = Value::Bool; v->b = false; return lit("false") || fail("invalid literal");
        case 'n': v->type = Value::Null; return lit("null") || fail("invalid literal");
        default: return number(v);
        }
    }

    bool object(Value* v, int depth) {
        v->type = Value::Object;
        ++p_;
        ws();
        if (p_ < e_ && *p_ == '}') {
            ++p_;
            return true;
        }
        for (;;) {
            ws();
            if (p_ >= e_ || *p_ != '"') return fail("expected an object key");
            std::string key;
            if (!string(&key)) return false;
            ws();
            if (p_ >= e_ || *p_ != ':') return fail("expected ':' after an object key");
            ++p_;
            ws();
            Value child;
            if (!value(&child, depth + 1)) return false;
            v->obj.emplace_back(std::move(key), std::move(child));
            ws();
            if (p_ < e_ && *p_ == ',') {
                ++p_;
                continue;
            }
            if (p_ < e_ && *p_ == '}') {
                ++p_;
                return true;
            }
            return fail("expected ',' or '}' in an object");
        }
    }

    bool array(Value* v, int depth) {
        v->type = Value::Array;
        ++p_;
        ws();
        if (p_ < e_ && *p_ == ']') {
            ++p_;
            return true;
        }
        for (;;) {
            ws();
            Value child;
            if (!value(&child, depth + 1)) return false;
            v->arr.push_back(std::move(child));
            ws();
            if (p_ < e_ && *p_ == ',') {
                ++p_;
                continue;
            }
            if (p_ < e_ && *p_ == ']') {
                ++p_;
                return true;
            }
            return fail("expected ',' or ']' in an array");
        }
    }

    static void utf8(uint32_t cp, std::string* out) {
        if (cp < 0x80) {
            out->push_back((char)cp);
        } else if (cp < 0x800) {
            out->push_back((char)(0xC0 | (cp >> 6)));
            out->push_back((char)(0x80 | (cp & 0x3F)));
        } else if (cp < 0x10000) {
            out->push_back((char)(0xE0 | (cp >> 12)));
            out->push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
            out->push_back((char)(0x80 | (cp & 0x3F)));
        } else {
            out->push_back((char)(0xF0 | (cp >> 18)));
            out->push_back((char)(0x80 | ((cp >> 12) & 0x3F)));
            out->push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
            out->push_back((char)(0x80 | (cp & 0x3F)));
        }
    }

    bool hex4(uint32_t* out) {
        uint32_t v = 0;
        for (int i = 0; i < 4; ++i, ++p_) {
            if (p_ >= e_) return fail("truncated \\u escape");
            const char c = *p_;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
            else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
            else return fail("invalid \\u escape");
        }
        *out = v;
        return true;
    }

    bool string(std::string* out) {
        ++p_;  // opening quote
        for (;;) {
            if (p_ >= e_) return fail("unterminated string");
            const unsigned char c = (unsigned char)*p_++;
            if (c == '"') return true;
            if (c < 0x20) return fail("control character in a string");
            if (c != '\\') {
                out->push_back((char)c);
                continue;
            }
            if (p_ >= e_) return fail("unterminated escape");
            const char esc = *p_++;
            switch (esc) {
            case '"': out->push_back('"'); break;
            case '\\': out->push_back('\\'); break;
            case '/': out->push_back('/'); break;
            case 'b': out->push_back('\b'); break;
            case 'f': out->push_back('\f'); break;
            case 'n': out->push_back('\n'); break;
            case 'r': out->push_back('\r'); break;
            case 't': out->push_back('\t'); break;
            case 'u': {
                uint32_t cp;
                if (!hex4(&cp)) return false;
                if (cp >= 0xD800 && cp < 0xDC00) {  // a surrogate pair
                    uint32_t lo;
                    if (!(p_ + 1 < e_ && p_[0] == '\\' && p_[1] == 'u')) return fail("unpaired surrogate");
                    p_ += 2;
                    if (!hex4(&lo) || lo < 0xDC00 || lo > 0xDFFF) return fail("invalid surrogate pair");
                    cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                } else if (cp >= 0xDC00 && cp < 0xE000) {
                    return fail("unpaired surrogate");
                }
                utf8(cp, out);
                break;
            }
            default: return fail("invalid escape");
            }
        }
    }

    bool number(Value* v) {
        v->type = Value::Number;
        const char* s = p_;
        bool neg = false;
        if (p_ < e_ && *p_ == '-') {
            neg = true;
            ++p_;
        }
        if (p_ >= e_ || *p_ < '0' || *p_ > '9') return fail("invalid number");
        if (*p_ == '0' && p_ + 1 < e_ && p_[1] >= '0' && p_[1] <= '9') return fail("leading zero in a number");
        uint64_t mag = 0;
        bool fits = true;
        while (p_ < e_ && *p_ >= '0' && *p_ <= '9') {
            const uint64_t d = (uint64_t)(*p_ - '0');
            if (mag > (UINT64_MAX - d) / 10) fits = false;
            else mag = mag * 10 + d;
            ++p_;
        }
        bool frac = false;
        if (p_ < e_ && *p_ == '.') {
            frac = true;
            ++p_;
            if (p_ >= e_ || *p_ < '0' || *p_ > '9') return fail("invalid fraction");
            while (p_ < e_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        if (p_ < e_ && (*p_ == 'e' || *p_ == 'E')) {
            frac = true;
            ++p_;
            if (p_ < e_ && (*p_ == '+' || *p_ == '-')) ++p_;
            if (p_ >= e_ || *p_ < '0' || *p_ > '9') return fail("invalid exponent");
            while (p_ < e_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        const std::string text(s, (size_t)(p_ - s));
        v->num = std::strtod(text.c_str(), nullptr);
        v->neg = neg && !(mag == 0 && !frac);  // -0 is the integer 0
        v->mag = mag;
        // integers: u64 when non-negative, i64 when negative (serde_json's two integer forms)
        v->is_int = !frac && fits && (!neg || mag <= (uint64_t)INT64_MAX + 1u);
        return true;
    }
};

inline bool parse(const uint8_t* p, size_t n, Value* out, std::string* err) {
    return Parser(reinterpret_cast<const char*>(p), n).parse(out, err);
}

}  // namespace json
}  // namespace hk
