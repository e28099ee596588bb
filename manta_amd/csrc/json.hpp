// json.hpp -- the small JSON reader/writer the artifact codec needs.
//
// Reading follows RFC 8259 with the error wording of Go's encoding/json
// scanner (the reference decodes artifacts with json.Unmarshal,
// artifact/manta/module.go:494-505): "unexpected end of JSON input",
// "invalid character 'x' looking for beginning of value", ... .  Objects keep
// their keys in document order (a repeated key: the last one wins on lookup,
// as Unmarshal's last assignment does).  Numbers keep their source text.
//
// Writing reproduces json.MarshalIndent(v, "", "  ") formatting: two-space
// indent, "key": value, empty containers as {} / [], map keys sorted by the
// caller, and Go's HTML-safe string escaping (<, >, & and U+2028/U+2029 as
// \u escapes).
#pragma once

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <memory>
#include <string>
#include <utility>
#include <vector>

namespace mjson {

enum class Kind { Null, Bool, Number, String, Array, Object };

struct Value {
    Kind kind = Kind::Null;
    bool b = false;
    std::string text;  // String: decoded UTF-8; Number: source text
    std::vector<Value> items;
    std::vector<std::pair<std::string, Value>> members;

    // The last member, in document order, whose name is `key` or equals it
    // under ASCII case folding, else null: Unmarshal maps every such key to
    // the same struct field and each one overwrites it, so the last wins.
    const Value* get(const char* key) const {
        const Value* last = nullptr;
        for (const auto& m : members)
            if (m.first == key || fold_equal(m.first, key)) last = &m.second;
        return last;
    }
    static bool fold_equal(const std::string& a, const char* b) {
        size_t n = strlen(b);
        if (a.size() != n) return false;
        for (size_t i = 0; i < n; i++) {
            char x = a[i], y = b[i];
            if (x >= 'A' && x <= 'Z') x = (char)(x - 'A' + 'a');
            if (y >= 'A' && y <= 'Z') y = (char)(y - 'A' + 'a');
            if (x != y) return false;
        }
        return true;
    }
    const char* kind_name() const {
        switch (kind) {
            case Kind::Null: return "null";
            case Kind::Bool: return "bool";
            case Kind::Number: return "number";
            case Kind::String: return "string";
            case Kind::Array: return "array";
            default: return "object";
        }
    }
};

class Parser {
public:
    Parser(const char* p, size_t n) : p_(p), n_(n) {}

    // Parse one value covering the whole input; false with err set on failure.
    bool parse(Value* out, std::string* err) {
        skip_ws();
        if (!value(out, 0)) {
            *err = err_;
            return false;
        }
        skip_ws();
        if (i_ < n_) {
            *err = invalid("after top-level value");
            return false;
        }
        return true;
    }

private:
    const char* p_;
    size_t n_;
    size_t i_ = 0;
    std::string err_;

    static constexpr int kMaxDepth = 10000;

    void skip_ws() {
        while (i_ < n_ && (p_[i_] == ' ' || p_[i_] == '\t' || p_[i_] == '\n' || p_[i_] == '\r')) i_++;
    }
    std::string quote_char(unsigned char c) const {
        char buf[16];
        if (c == '\'') return "'\\''";
        if (c == '"') return "'\"'";
        if (c < 0x20 || c >= 0x7f) {
            snprintf(buf, sizeof buf, "'\\x%02x'", c);
            return buf;
        }
        snprintf(buf, sizeof buf, "'%c'", c);
        return buf;
    }
    std::string invalid(const char* context) const {
        if (i_ >= n_) return "unexpected end of JSON input";
        return "invalid character " + quote_char((unsigned char)p_[i_]) + " " + context;
    }
    bool fail(const char* context) {
        err_ = invalid(context);
        return false;
    }
    bool literal(const char* word, Value* out, Kind k, bool bv) {
        size_t len = strlen(word);
        for (size_t j = 0; j < len; j++) {
            if (i_ + j >= n_) {
                i_ = n_;
                err_ = "unexpected end of JSON input";
                return false;
            }
            if (p_[i_ + j] != word[j]) {
                i_ += j;
                char ctx[64];
                snprintf(ctx, sizeof ctx, "in literal %s (expecting '%c')", word, word[j]);
                return fail(ctx);
            }
        }
        i_ += len;
        out->kind = k;
        out->b = bv;
        return true;
    }
    bool value(Value* out, int depth) {
        if (depth > kMaxDepth) {
            err_ = "exceeded max depth";
            return false;
        }
        if (i_ >= n_) return fail("looking for beginning of value");
        const char c = p_[i_];
        if (c == '{') return object(out, depth);
        if (c == '[') return array(out, depth);
        if (c == '"') {
            out->kind = Kind::String;
            return string(&out->text);
        }
        if (c == 't') return literal("true", out, Kind::Bool, true);
        if (c == 'f') return literal("false", out, Kind::Bool, false);
        if (c == 'n') return literal("null", out, Kind::Null, false);
        if (c == '-' || (c >= '0' && c <= '9')) return number(out);
        return fail("looking for beginning of value");
    }
    bool digits() {
        size_t s = i_;
        while (i_ < n_ && p_[i_] >= '0' && p_[i_] <= '9') i_++;
        return i_ > s;
    }
    bool number(Value* out) {
        const size_t s = i_;
        if (p_[i_] == '-') {
            i_++;
            if (i_ >= n_ || p_[i_] < '0' || p_[i_] > '9') return fail("in numeric literal");
        }
        if (p_[i_] == '0') i_++;
        else digits();
        if (i_ < n_ && p_[i_] == '.') {
            i_++;
            if (!digits()) return fail("after decimal point in numeric literal");
        }
        if (i_ < n_ && (p_[i_] == 'e' || p_[i_] == 'E')) {
            i_++;
            if (i_ < n_ && (p_[i_] == '+' || p_[i_] == '-')) i_++;
            if (!digits()) return fail("in exponent of numeric literal");
        }
        out->kind = Kind::Number;
        out->text.assign(p_ + s, i_ - s);
        return true;
    }
    static void put_utf8(std::string* s, uint32_t cp) {
        if (cp < 0x80) {
            s->push_back((char)cp);
        } else if (cp < 0x800) {
            s->push_back((char)(0xC0 | (cp >> 6)));
            s->push_back((char)(0x80 | (cp & 0x3F)));
        } else if (cp < 0x10000) {
            s->push_back((char)(0xE0 | (cp >> 12)));
            s->push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
            s->push_back((char)(0x80 | (cp & 0x3F)));
        } else {
            s->push_back((char)(0xF0 | (cp >> 18)));
            s->push_back((char)(0x80 | ((cp >> 12) & 0x3F)));
            s->push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
            s->push_back((char)(0x80 | (cp & 0x3F)));
        }
    }
    bool hex4(uint32_t* v) {
        *v = 0;
        for (int j = 0; j < 4; j++) {
            if (i_ >= n_) return fail("in \\u hexadecimal character escape");
            char h = p_[i_];
            int d = h >= '0' && h <= '9' ? h - '0' : h >= 'a' && h <= 'f' ? h - 'a' + 10 : h >= 'A' && h <= 'F' ? h - 'A' + 10 : -1;
            if (d < 0) return fail("in \\u hexadecimal character escape");
            *v = *v * 16 + (uint32_t)d;
            i_++;
        }
        return true;
    }
    bool string(std::string* out) {
        i_++;  // opening quote
        out->clear();
        for (;;) {
            if (i_ >= n_) {
                err_ = "unexpected end of JSON input";
                return false;
            }
            const unsigned char c = (unsigned char)p_[i_];
            if (c == '"') {
                i_++;
                return true;
            }
            if (c < 0x20) return fail("in string literal");
            if (c != '\\') {
                out->push_back((char)c);
                i_++;
                continue;
            }
            i_++;
            if (i_ >= n_) {
                err_ = "unexpected end of JSON input";
                return false;
            }
            const char e = p_[i_];
            switch (e) {
                case '"': out->push_back('"'); i_++; break;
                case '\\': out->push_back('\\'); i_++; break;
                case '/': out->push_back('/'); i_++; break;
                case 'b': out->push_back('\b'); i_++; break;
                case 'f': out->push_back('\f'); i_++; break;
                case 'n': out->push_back('\n'); i_++; break;
                case 'r': out->push_back('\r'); i_++; break;
                case 't': out->push_back('\t'); i_++; break;
                case 'u': {
                    i_++;
                    uint32_t cp;
                    if (!hex4(&cp)) return false;
                    if (cp >= 0xD800 && cp < 0xDC00) {
                        // a high surrogate pairs with a following \uDC00-\uDFFF
                        if (i_ + 1 < n_ && p_[i_] == '\\' && p_[i_ + 1] == 'u') {
                            const size_t save = i_;
                            i_ += 2;
                            uint32_t lo;
                            if (!hex4(&lo)) return false;
                            if (lo >= 0xDC00 && lo < 0xE000) {
                                cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                            } else {
                                cp = 0xFFFD;
                                i_ = save;
                            }
                        } else {
                            cp = 0xFFFD;
                        }
                    } else if (cp >= 0xDC00 && cp < 0xE000) {
                        cp = 0xFFFD;
                    }
                    put_utf8(out, cp);
                    break;
                }
                default: return fail("in string escape code");
            }
        }
    }
    bool array(Value* out, int depth) {
        out->kind = Kind::Array;
        i_++;
        skip_ws();
        if (i_ < n_ && p_[i_] == ']') {
            i_++;
            return true;
        }
        for (;;) {
            skip_ws();
            out->items.emplace_back();
            if (!value(&out->items.back(), depth + 1)) return false;
            skip_ws();
            if (i_ >= n_) {
                err_ = "unexpected end of JSON input";
                return false;
            }
            if (p_[i_] == ',') {
                i_++;
                continue;
            }
            if (p_[i_] == ']') {
                i_++;
                return true;
            }
            return fail("after array element");
        }
    }
    bool object(Value* out, int depth) {
        out->kind = Kind::Object;
        i_++;
        skip_ws();
        if (i_ < n_ && p_[i_] == '}') {
            i_++;
            return true;
        }
        for (;;) {
            skip_ws();
            if (i_ >= n_) {
                err_ = "unexpected end of JSON input";
                return false;
            }
            if (p_[i_] != '"') return fail("looking for beginning of object key string");
            std::string key;
            if (!string(&key)) return false;
            skip_ws();
            if (i_ >= n_) {
                err_ = "unexpected end of JSON input";
                return false;
            }
            if (p_[i_] != ':') return fail("after object key");
            i_++;
            skip_ws();
            out->members.emplace_back(std::move(key), Value());
            if (!value(&out->members.back().second, depth + 1)) return false;
            skip_ws();
            if (i_ >= n_) {
                err_ = "unexpected end of JSON input";
                return false;
            }
            if (p_[i_] == ',') {
                i_++;
                continue;
            }
            if (p_[i_] == '}') {
                i_++;
                return true;
            }
            return fail("after object key:value pair");
        }
    }
};

// ---------------------------------------------------------------- writer

// Go's HTML-safe string encoding (encoding/json encodeState.string).
inline void put_string(std::string* o, const std::string& s) {
    static const char* hex = "0123456789abcdef";
    o->push_back('"');
    for (size_t i = 0; i < s.size(); i++) {
        const unsigned char c = (unsigned char)s[i];
        switch (c) {
            case '"': *o += "\\\""; continue;
            case '\\': *o += "\\\\"; continue;
            case '\n': *o += "\\n"; continue;
            case '\r': *o += "\\r"; continue;
            case '\t': *o += "\\t"; continue;
            case '\b': *o += "\\b"; continue;
            case '\f': *o += "\\f"; continue;
            default: break;
        }
        if (c < 0x20 || c == '<' || c == '>' || c == '&') {
            *o += "\\u00";
            o->push_back(hex[c >> 4]);
            o->push_back(hex[c & 15]);
            continue;
        }
        // U+2028 / U+2029 (E2 80 A8 / E2 80 A9)
        if (c == 0xE2 && i + 2 < s.size() && (unsigned char)s[i + 1] == 0x80 &&
            ((unsigned char)s[i + 2] == 0xA8 || (unsigned char)s[i + 2] == 0xA9)) {
            *o += (unsigned char)s[i + 2] == 0xA8 ? "\\u2028" : "\\u2029";
            i += 2;
            continue;
        }
        o->push_back((char)c);
    }
    o->push_back('"');
}

// Streaming writer for MarshalIndent(v, "", "  ") output.
class Writer {
public:
    std::string out;

    void begin_object() { open('{'); }
    void end_object() { close('}'); }
    void begin_array() { open('['); }
    void end_array() { close(']'); }
    void key(const char* k) {
        item();
        put_string(&out, k);
        out += ": ";
        after_key_ = true;
    }
    void str(const std::string& s) {
        item();
        put_string(&out, s);
    }
    void raw(const std::string& s) {
        item();
        out += s;
    }
    void num(long long v) { raw(std::to_string(v)); }
    void boolean(bool v) { raw(v ? "true" : "false"); }
    void null() { raw("null"); }

private:
    struct Frame {
        char close;
        int count;
    };
    std::vector<Frame> stack_;
    bool after_key_ = false;

    void newline() {
        out.push_back('\n');
        for (size_t i = 0; i < stack_.size(); i++) out += "  ";
    }
    void item() {
        if (after_key_) {
            after_key_ = false;
            return;
        }
        if (stack_.empty()) return;
        if (stack_.back().count++ > 0) out.push_back(',');
        newline();
    }
    void open(char c) {
        item();
        out.push_back(c);
        stack_.push_back({c == '{' ? '}' : ']', 0});
    }
    void close(char c) {
        const int n = stack_.back().count;
        stack_.pop_back();
        if (n > 0) newline();
        out.push_back(c);
    }
};

// Re-emit a parsed value (used for free-form metadata), object keys sorted
// as Go's encoder sorts map keys.
inline void write_value(Writer* w, const Value& v) {
    switch (v.kind) {
        case Kind::Null: w->null(); break;
        case Kind::Bool: w->boolean(v.b); break;
        case Kind::Number: w->raw(v.text); break;
        case Kind::String: w->str(v.text); break;
        case Kind::Array:
            w->begin_array();
            for (const auto& it : v.items) write_value(w, it);
            w->end_array();
            break;
        case Kind::Object: {
            // last occurrence of each key, in sorted order
            std::vector<std::pair<std::string, const Value*>> m;
            for (const auto& kv : v.members) {
                bool found = false;
                for (auto& e : m)
                    if (e.first == kv.first) {
                        e.second = &kv.second;
                        found = true;
                    }
                if (!found) m.emplace_back(kv.first, &kv.second);
            }
            std::sort(m.begin(), m.end(), [](const auto& a, const auto& b) { return a.first < b.first; });
            w->begin_object();
            for (const auto& e : m) {
                w->key(e.first.c_str());
                write_value(w, *e.second);
            }
            w->end_object();
            break;
        }
    }
}

}  // namespace mjson
