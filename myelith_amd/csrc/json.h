// json.h -- a small JSON reader for the artifact manifests (RFC 8259 text:
// objects, arrays, strings with escapes, numbers, true/false/null).
// Numbers keep their text so that integers are read exactly.
#pragma once

#include <cerrno>
#include <cstdint>
#include <cstdlib>
#include <memory>
#include <string>
#include <utility>
#include <vector>

namespace myl {

struct Json {
    enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
    bool b = false;
    std::string s;                                  // String, or the text of a Number
    std::vector<Json> items;                        // Array
    std::vector<std::pair<std::string, Json>> members;  // Object, in file order

    bool is_object() const { return kind == Object; }
    bool is_array() const { return kind == Array; }
    bool is_string() const { return kind == String; }
    bool is_number() const { return kind == Number; }
    bool is_bool() const { return kind == Bool; }

    // The member named `key` (the last one when a key repeats), or nullptr.
    const Json* get(const std::string& key) const {
        if (kind != Object) return nullptr;
        for (size_t i = members.size(); i-- > 0;)
            if (members[i].first == key) return &members[i].second;
        return nullptr;
    }

    // An integral Number that fits int64 (no fraction or exponent).
    bool as_i64(int64_t* out) const {
        if (kind != Number || s.empty()) return false;
        for (size_t i = (s[0] == '-'); i < s.size(); ++i)
            if (s[i] < '0' || s[i] > '9') return false;
        errno = 0;
        char* end = nullptr;
        const long long v = std::strtoll(s.c_str(), &end, 10);
        if (errno || !end || *end) return false;
        *out = v;
        return true;
    }

    bool as_f64(double* out) const {
        if (kind != Number) return false;
        char* end = nullptr;
        *out = std::strtod(s.c_str(), &end);
        return end && !*end;
    }
};

class JsonParser {
public:
    // Parses `text` into *out; on failure returns false and sets `error`.
    static bool parse(const std::string& text, Json* out, std::string* error) {
        JsonParser p(text);
        p.ws();
        if (!p.value(out, 0)) {
            *error = p.err_ + " at byte " + std::to_string(p.i_);
            return false;
        }
        p.ws();
        if (p.i_ != text.size()) {
            *error = "trailing characters at byte " + std::to_string(p.i_);
            return false;
        }
        return true;
    }

private:
    explicit JsonParser(const std::string& t) : t_(t) {}

    bool fail(const char* what) {
        if (err_.empty()) err_ = what;
        return false;
    }
    void ws() {
        while (i_ < t_.size() && (t_[i_] == ' ' || t_[i_] == '\t' || t_[i_] == '\n' || t_[i_] == '\r')) ++i_;
    }
    bool lit(const char* word) {
        size_t n = 0;
        while (word[n]) ++n;
        if (t_.compare(i_, n, word) != 0) return fail("invalid literal");
        i_ += n;
        return true;
    }

    bool value(Json* v, int depth) {
        if (depth > 64) return fail("nesting too deep");
        if (i_ >= t_.size()) return fail("unexpected end of input");
        const char c = t_[i_];
        if (c == '{') return object(v, depth);
        if (c == '[') return array(v, depth);
        if (c == '"') {
            v->kind = Json::String;
            return string(&v->s);
        }
        if (c == 't') { v->kind = Json::Bool; v->b = true; return lit("true"); }
        if (c == 'f') { v->kind = Json::Bool; v->b = false; return lit("false"); }
        if (c == 'n') { v->kind = Json::Null; return lit("null"); }
        if (c == '-' || (c >= '0' && c <= '9')) return number(v);
        return fail("unexpected character");
    }

    bool object(Json* v, int depth) {
        v->kind = Json::Object;
        ++i_;
        ws();
        if (i_ < t_.size() && t_[i_] == '}') { ++i_; return true; }
        for (;;) {
            ws();
            if (i_ >= t_.size() || t_[i_] != '"') return fail("expected a member name");
            std::string key;
            if (!string(&key)) return false;
            ws();
            if (i_ >= t_.size() || t_[i_] != ':') return fail("expected ':'");
            ++i_;
            ws();
            v->members.emplace_back(std::move(key), Json());
            if (!value(&v->members.back().second, depth + 1)) return false;
            ws();
            if (i_ < t_.size() && t_[i_] == ',') { ++i_; continue; }
            if (i_ < t_.size() && t_[i_] == '}') { ++i_; return true; }
            return fail("expected ',' or '}'");
        }
    }

    bool array(Json* v, int depth) {
        v->kind = Json::Array;
        ++i_;
        ws();
        if (i_ < t_.size() && t_[i_] == ']') { ++i_; return true; }
        for (;;) {
            ws();
            v->items.emplace_back();
            if (!value(&v->items.back(), depth + 1)) return false;
            ws();
            if (i_ < t_.size() && t_[i_] == ',') { ++i_; continue; }
            if (i_ < t_.size() && t_[i_] == ']') { ++i_; return true; }
            return fail("expected ',' or ']'");
        }
    }

    bool number(Json* v) {
        const size_t start = i_;
        if (t_[i_] == '-') ++i_;
        auto digits = [&]() {
            const size_t d0 = i_;
            while (i_ < t_.size() && t_[i_] >= '0' && t_[i_] <= '9') ++i_;
            return i_ > d0;
        };
        if (i_ < t_.size() && t_[i_] == '0') ++i_;
        else if (!digits()) return fail("invalid number");
        if (i_ < t_.size() && t_[i_] == '.') {
            ++i_;
            if (!digits()) return fail("invalid number");
        }
        if (i_ < t_.size() && (t_[i_] == 'e' || t_[i_] == 'E')) {
            ++i_;
            if (i_ < t_.size() && (t_[i_] == '+' || t_[i_] == '-')) ++i_;
            if (!digits()) return fail("invalid number");
        }
        v->kind = Json::Number;
        v->s = t_.substr(start, i_ - start);
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

    bool hex4(uint32_t* out) {
        if (i_ + 4 > t_.size()) return fail("truncated \\u escape");
        uint32_t v = 0;
        for (int k = 0; k < 4; ++k) {
            const char c = t_[i_++];
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
        ++i_;  // opening quote
        for (;;) {
            if (i_ >= t_.size()) return fail("unterminated string");
            const char c = t_[i_++];
            if (c == '"') return true;
            if ((unsigned char)c < 0x20) return fail("control character in string");
            if (c != '\\') {
                out->push_back(c);
                continue;
            }
            if (i_ >= t_.size()) return fail("unterminated escape");
            const char e = t_[i_++];
            switch (e) {
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
                    if (cp >= 0xD800 && cp < 0xDC00) {
                        uint32_t lo;
                        if (i_ + 2 > t_.size() || t_[i_] != '\\' || t_[i_ + 1] != 'u') return fail("lone surrogate");
                        i_ += 2;
                        if (!hex4(&lo)) return false;
                        if (lo < 0xDC00 || lo >= 0xE000) return fail("lone surrogate");
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    } else if (cp >= 0xDC00 && cp < 0xE000) {
                        return fail("lone surrogate");
                    }
                    put_utf8(out, cp);
                    break;
                }
                default: return fail("invalid escape");
            }
        }
    }

    const std::string& t_;
    size_t i_ = 0;
    std::string err_;
};

}  // namespace myl
