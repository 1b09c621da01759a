#pragma once

// Minimal JSON reader for pack manifests and model configs: objects, arrays,
// strings (common escapes, \uXXXX to UTF-8), numbers, booleans, null.
// Host-only C++17 (same role as the reference's include/runtime/json.cuh).

#include <cstdint>
#include <cstdlib>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace opworks::json {

class Value {
  public:
    enum class Kind { null, boolean, number, string, array, object };
    using Array = std::vector<Value>;
    using Object = std::map<std::string, Value>;

    Value() = default;
    static Value make_bool(bool b) {
        Value v;
        v.kind_ = Kind::boolean;
        v.b_ = b;
        return v;
    }
    static Value make_number(double d) {
        Value v;
        v.kind_ = Kind::number;
        v.num_ = d;
        return v;
    }
    static Value make_string(std::string s) {
        Value v;
        v.kind_ = Kind::string;
        v.str_ = std::move(s);
        return v;
    }
    static Value make_array(Array a) {
        Value v;
        v.kind_ = Kind::array;
        v.arr_ = std::make_shared<Array>(std::move(a));
        return v;
    }
    static Value make_object(Object o) {
        Value v;
        v.kind_ = Kind::object;
        v.obj_ = std::make_shared<Object>(std::move(o));
        return v;
    }

    Kind kind() const { return kind_; }
    bool is_null() const { return kind_ == Kind::null; }
    bool is_number() const { return kind_ == Kind::number; }
    bool is_string() const { return kind_ == Kind::string; }
    bool is_array() const { return kind_ == Kind::array; }
    bool is_object() const { return kind_ == Kind::object; }

    double as_number() const {
        if (kind_ != Kind::number)
            throw std::runtime_error("json: expected a number");
        return num_;
    }
    // Integral numbers within +-2^53 (exact in a double); anything else,
    // including inf / nan from overflowing literals, is rejected before the
    // conversion, which would be undefined outside int64's range.
    int64_t as_int() const {
        const double d = as_number();
        constexpr double kExact = 9007199254740992.0; // 2^53
        if (!(d >= -kExact && d <= kExact) || d != static_cast<double>(static_cast<int64_t>(d)))
            throw std::runtime_error("json: expected an integer");
        return static_cast<int64_t>(d);
    }
    bool as_bool() const {
        if (kind_ != Kind::boolean)
            throw std::runtime_error("json: expected a boolean");
        return b_;
    }
    const std::string &as_string() const {
        if (kind_ != Kind::string)
            throw std::runtime_error("json: expected a string");
        return str_;
    }
    const Array &as_array() const {
        if (kind_ != Kind::array)
            throw std::runtime_error("json: expected an array");
        return *arr_;
    }
    const Object &as_object() const {
        if (kind_ != Kind::object)
            throw std::runtime_error("json: expected an object");
        return *obj_;
    }
    const Value *find(const std::string &key) const {
        if (kind_ != Kind::object)
            return nullptr;
        auto it = obj_->find(key);
        return it == obj_->end() ? nullptr : &it->second;
    }
    const Value &at(const std::string &key) const {
        const Value *v = find(key);
        if (!v)
            throw std::runtime_error("json: missing key '" + key + "'");
        return *v;
    }

  private:
    Kind kind_ = Kind::null;
    bool b_ = false;
    double num_ = 0;
    std::string str_;
    std::shared_ptr<Array> arr_;
    std::shared_ptr<Object> obj_;
};

namespace detail {

class Parser {
  public:
    explicit Parser(const std::string &text) : s_(text) {}

    Value document() {
        Value v = value(0);
        skip_ws();
        if (pos_ != s_.size())
            fail("trailing characters");
        return v;
    }

  private:
    static constexpr int kMaxDepth = 256;
    const std::string &s_;
    size_t pos_ = 0;

    [[noreturn]] void fail(const char *what) const {
        throw std::runtime_error(std::string("json: ") + what + " at offset " + std::to_string(pos_));
    }
    void skip_ws() {
        while (pos_ < s_.size() && (s_[pos_] == ' ' || s_[pos_] == '\n' || s_[pos_] == '\t' || s_[pos_] == '\r'))
            ++pos_;
    }
    char peek() {
        skip_ws();
        if (pos_ >= s_.size())
            fail("unexpected end of input");
        return s_[pos_];
    }
    void expect(char c) {
        if (peek() != c)
            fail("unexpected character");
        ++pos_;
    }
    bool literal(const char *word) {
        size_t n = 0;
        while (word[n])
            ++n;
        if (s_.compare(pos_, n, word) == 0) {
            pos_ += n;
            return true;
        }
        return false;
    }

    Value value(int depth) {
        if (depth > kMaxDepth)
            fail("nesting too deep");
        const char c = peek();
        if (c == '{')
            return object(depth);
        if (c == '[')
            return array(depth);
        if (c == '"')
            return Value::make_string(string());
        if (literal("true"))
            return Value::make_bool(true);
        if (literal("false"))
            return Value::make_bool(false);
        if (literal("null"))
            return Value();
        if (c == '-' || (c >= '0' && c <= '9'))
            return number();
        fail("invalid value");
    }

    Value object(int depth) {
        expect('{');
        Value::Object o;
        if (peek() == '}') {
            ++pos_;
            return Value::make_object(std::move(o));
        }
        while (true) {
            if (peek() != '"')
                fail("expected a key");
            std::string key = string();
            expect(':');
            o[key] = value(depth + 1);
            const char c = peek();
            ++pos_;
            if (c == '}')
                break;
            if (c != ',')
                fail("expected ',' or '}'");
        }
        return Value::make_object(std::move(o));
    }

    Value array(int depth) {
        expect('[');
        Value::Array a;
        if (peek() == ']') {
            ++pos_;
            return Value::make_array(std::move(a));
        }
        while (true) {
            a.push_back(value(depth + 1));
            const char c = peek();
            ++pos_;
            if (c == ']')
                break;
            if (c != ',')
                fail("expected ',' or ']'");
        }
        return Value::make_array(std::move(a));
    }

    static void put_utf8(std::string &out, uint32_t cp) {
        if (cp < 0x80) {
            out += static_cast<char>(cp);
        } else if (cp < 0x800) {
            out += static_cast<char>(0xC0 | (cp >> 6));
            out += static_cast<char>(0x80 | (cp & 0x3F));
        } else if (cp < 0x10000) {
            out += static_cast<char>(0xE0 | (cp >> 12));
            out += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
            out += static_cast<char>(0x80 | (cp & 0x3F));
        } else {
            out += static_cast<char>(0xF0 | (cp >> 18));
            out += static_cast<char>(0x80 | ((cp >> 12) & 0x3F));
            out += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
            out += static_cast<char>(0x80 | (cp & 0x3F));
        }
    }

    uint32_t hex4() {
        if (pos_ + 4 > s_.size())
            fail("truncated \\u escape");
        uint32_t v = 0;
        for (int i = 0; i < 4; ++i) {
            const char c = s_[pos_++];
            v <<= 4;
            if (c >= '0' && c <= '9')
                v |= c - '0';
            else if (c >= 'a' && c <= 'f')
                v |= c - 'a' + 10;
            else if (c >= 'A' && c <= 'F')
                v |= c - 'A' + 10;
            else
                fail("bad hex digit");
        }
        return v;
    }

    std::string string() {
        expect('"');
        std::string out;
        while (true) {
            if (pos_ >= s_.size())
                fail("unterminated string");
            const char c = s_[pos_++];
            if (c == '"')
                break;
            if (static_cast<unsigned char>(c) < 0x20)
                fail("control character in string");
            if (c != '\\') {
                out += c;
                continue;
            }
            if (pos_ >= s_.size())
                fail("unterminated escape");
            const char e = s_[pos_++];
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
                uint32_t cp = hex4();
                if (cp >= 0xD800 && cp < 0xDC00 && s_.compare(pos_, 2, "\\u") == 0) {
                    pos_ += 2;
                    const uint32_t lo = hex4();
                    if (lo >= 0xDC00 && lo < 0xE000)
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    else
                        fail("bad surrogate pair");
                }
                put_utf8(out, cp);
                break;
            }
            default: fail("unknown escape");
            }
        }
        return out;
    }

    Value number() {
        const size_t start = pos_;
        if (s_[pos_] == '-')
            ++pos_;
        while (pos_ < s_.size() && ((s_[pos_] >= '0' && s_[pos_] <= '9') || s_[pos_] == '.' || s_[pos_] == 'e' ||
                                    s_[pos_] == 'E' || s_[pos_] == '+' || s_[pos_] == '-'))
            ++pos_;
        const std::string tok = s_.substr(start, pos_ - start);
        char *end = nullptr;
        const double d = std::strtod(tok.c_str(), &end);
        if (end == tok.c_str() || *end != '\0')
            fail("malformed number");
        return Value::make_number(d);
    }
};

} // namespace detail

inline Value parse(const std::string &text) { return detail::Parser(text).document(); }

} // namespace opworks::json
