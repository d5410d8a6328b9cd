// json.hpp — a small JSON reader for the checkpoint metadata (layout.json).
// Objects, arrays, strings (with \uXXXX escapes, UTF-8 out), numbers,
// true/false/null. Integers are kept exactly (up to 2^64-1 unsigned, and
// negative 64-bit); a number with a fraction or exponent is kept as a double
// and counts as an integer only when it is integral (as NSNumber bridging
// to Int does in the reference's reader).
#pragma once

#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace tfq {
namespace json {

struct Value {
    enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
    bool b = false;
    bool is_int = false;        // integral number
    bool neg = false;           // integral and negative
    uint64_t u = 0;             // magnitude when is_int
    double d = 0.0;
    std::string s;
    std::vector<Value> a;
    std::map<std::string, Value> o;

    const Value* get(const std::string& key) const {
        if (kind != Object) return nullptr;
        auto it = o.find(key);
        return it == o.end() ? nullptr : &it->second;
    }
    // Non-negative integer that fits `max`.
    bool as_uint(uint64_t& out, uint64_t max = UINT64_MAX) const {
        if (kind != Number || !is_int || neg || u > max) return false;
        out = u;
        return true;
    }
    // Signed integer (Swift `as? Int`).
    bool as_int(int64_t& out) const {
        if (kind != Number || !is_int) return false;
        if (neg) {
            if (u > (uint64_t)INT64_MAX + 1) return false;
            out = (int64_t)(0 - u);
        } else {
            if (u > (uint64_t)INT64_MAX) return false;
            out = (int64_t)u;
        }
        return true;
    }
};

class Parser {
public:
    Parser(const char* p, size_t n) : p_(p), end_(p + n) {}

    // Parses one document; false (with error()) on malformed input.
    bool parse(Value& out) {
        ws();
        if (!value(out, 0)) return false;
        ws();
        if (p_ != end_) return bad("trailing characters");
        return true;
    }
    const std::string& error() const { return err_; }

private:
    const char* p_;
    const char* end_;
    std::string err_;

    bool bad(const char* what) {
        err_ = what;
        return false;
    }
    void ws() {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
    }
    bool lit(const char* w) {
        size_t n = 0;
        while (w[n]) ++n;
        if ((size_t)(end_ - p_) < n) return false;
        for (size_t i = 0; i < n; ++i)
            if (p_[i] != w[i]) return false;
        p_ += n;
        return true;
    }
    bool value(Value& v, int depth) {
        if (depth > 64) return bad("nesting too deep");
        if (p_ >= end_) return bad("unexpected end");
        const char c = *p_;
        if (c == '{') return object(v, depth);
        if (c == '[') return array(v, depth);
        if (c == '"') {
            v.kind = Value::String;
            return string(v.s);
        }
        if (c == 't') {
            if (!lit("true")) return bad("bad literal");
            v.kind = Value::Bool;
            v.b = true;
            return true;
        }
        if (c == 'f') {
            if (!lit("false")) return bad("bad literal");
            v.kind = Value::Bool;
            return true;
        }
        if (c == 'n') {
            if (!lit("null")) return bad("bad literal");
            v.kind = Value::Null;
            return true;
        }
        return number(v);
    }
    bool object(Value& v, int depth) {
        v.kind = Value::Object;
        ++p_;
        ws();
        if (p_ < end_ && *p_ == '}') {
            ++p_;
            return true;
        }
        for (;;) {
            ws();
            std::string key;
            if (p_ >= end_ || *p_ != '"' || !string(key)) return bad("bad object key");
            ws();
            if (p_ >= end_ || *p_ != ':') return bad("missing ':'");
            ++p_;
            ws();
            Value item;
            if (!value(item, depth + 1)) return false;
            v.o[key] = std::move(item);
            ws();
            if (p_ < end_ && *p_ == ',') {
                ++p_;
                continue;
            }
            if (p_ < end_ && *p_ == '}') {
                ++p_;
                return true;
            }
            return bad("bad object");
        }
    }
    bool array(Value& v, int depth) {
        v.kind = Value::Array;
        ++p_;
        ws();
        if (p_ < end_ && *p_ == ']') {
            ++p_;
            return true;
        }
        for (;;) {
            ws();
            Value item;
            if (!value(item, depth + 1)) return false;
            v.a.push_back(std::move(item));
            ws();
            if (p_ < end_ && *p_ == ',') {
                ++p_;
                continue;
            }
            if (p_ < end_ && *p_ == ']') {
                ++p_;
                return true;
            }
            return bad("bad array");
        }
    }
    static void utf8(std::string& s, uint32_t cp) {
        if (cp < 0x80) {
            s += (char)cp;
        } else if (cp < 0x800) {
            s += (char)(0xC0 | (cp >> 6));
            s += (char)(0x80 | (cp & 0x3F));
        } else if (cp < 0x10000) {
            s += (char)(0xE0 | (cp >> 12));
            s += (char)(0x80 | ((cp >> 6) & 0x3F));
            s += (char)(0x80 | (cp & 0x3F));
        } else {
            s += (char)(0xF0 | (cp >> 18));
            s += (char)(0x80 | ((cp >> 12) & 0x3F));
            s += (char)(0x80 | ((cp >> 6) & 0x3F));
            s += (char)(0x80 | (cp & 0x3F));
        }
    }
    bool hex4(uint32_t& out) {
        if (end_ - p_ < 4) return false;
        out = 0;
        for (int i = 0; i < 4; ++i) {
            const char c = *p_++;
            out <<= 4;
            if (c >= '0' && c <= '9') out |= (uint32_t)(c - '0');
            else if (c >= 'a' && c <= 'f') out |= (uint32_t)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') out |= (uint32_t)(c - 'A' + 10);
            else return false;
        }
        return true;
    }
    bool string(std::string& s) {
        ++p_;                                            // opening quote
        while (p_ < end_) {
            const char c = *p_++;
            if (c == '"') return true;
            if ((unsigned char)c < 0x20) return bad("control character in string");
            if (c != '\\') {
                s += c;
                continue;
            }
            if (p_ >= end_) break;
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
                    if (!hex4(cp)) return bad("bad \\u escape");
                    if (cp >= 0xD800 && cp < 0xDC00) {           // surrogate pair
                        uint32_t lo;
                        if (end_ - p_ < 6 || p_[0] != '\\' || p_[1] != 'u') return bad("bad surrogate");
                        p_ += 2;
                        if (!hex4(lo) || lo < 0xDC00 || lo >= 0xE000) return bad("bad surrogate");
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    }
                    utf8(s, cp);
                    break;
                }
                default: return bad("bad escape");
            }
        }
        return bad("unterminated string");
    }
    bool number(Value& v) {
        const char* start = p_;
        bool neg = false;
        if (p_ < end_ && *p_ == '-') {
            neg = true;
            ++p_;
        }
        if (p_ >= end_ || *p_ < '0' || *p_ > '9') return bad("bad value");
        if (*p_ == '0' && p_ + 1 < end_ && p_[1] >= '0' && p_[1] <= '9') return bad("leading zero");
        uint64_t u = 0;
        bool overflow = false;
        while (p_ < end_ && *p_ >= '0' && *p_ <= '9') {
            const uint64_t dgt = (uint64_t)(*p_ - '0');
            if (u > (UINT64_MAX - dgt) / 10) overflow = true;
            else u = u * 10 + dgt;
            ++p_;
        }
        bool frac = false;
        if (p_ < end_ && *p_ == '.') {
            frac = true;
            ++p_;
            if (p_ >= end_ || *p_ < '0' || *p_ > '9') return bad("bad fraction");
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        if (p_ < end_ && (*p_ == 'e' || *p_ == 'E')) {
            frac = true;
            ++p_;
            if (p_ < end_ && (*p_ == '+' || *p_ == '-')) ++p_;
            if (p_ >= end_ || *p_ < '0' || *p_ > '9') return bad("bad exponent");
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        v.kind = Value::Number;
        v.d = std::strtod(std::string(start, p_).c_str(), nullptr);
        if (!frac && !overflow) {
            v.is_int = true;
            v.neg = neg && u != 0;
            v.u = u;
        } else if (std::isfinite(v.d) && v.d == std::floor(v.d) && std::fabs(v.d) < 9.2e18) {
            v.is_int = true;
            v.neg = v.d < 0;
            v.u = (uint64_t)std::fabs(v.d);
        }
        return true;
    }
};

}  // namespace json
}  // namespace tfq
