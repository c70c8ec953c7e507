#include "json.hpp"

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <sstream>

namespace edge_fm {

class JsonParser {
public:
    explicit JsonParser(const std::string& s) : s_(s) {}

    Json parse_document() {
        Json v = value();
        ws();
        if (i_ != s_.size()) fail("trailing characters");
        return v;
    }

private:
    const std::string& s_;
    size_t i_ = 0;

    [[noreturn]] void fail(const std::string& what) const {
        throw std::runtime_error("JSON parse error at offset " + std::to_string(i_) + ": " + what);
    }
    void ws() {
        while (i_ < s_.size() && (s_[i_] == ' ' || s_[i_] == '\n' || s_[i_] == '\r' || s_[i_] == '\t')) ++i_;
    }
    char peek() {
        ws();
        if (i_ >= s_.size()) fail("unexpected end");
        return s_[i_];
    }
    void expect(char c) {
        if (peek() != c) fail(std::string("expected '") + c + "'");
        ++i_;
    }
    bool literal(const char* lit) {
        size_t n = std::char_traits<char>::length(lit);
        if (s_.compare(i_, n, lit) == 0) {
            i_ += n;
            return true;
        }
        return false;
    }

    Json value() {
        char c = peek();
        if (c == '{') return object();
        if (c == '[') return array();
        if (c == '"') return Json(string());
        if (literal("true")) return Json(true);
        if (literal("false")) return Json(false);
        if (literal("null")) return Json();
        return number();
    }

    Json object() {
        expect('{');
        Json o = Json::object();
        if (peek() == '}') {
            ++i_;
            return o;
        }
        while (true) {
            if (peek() != '"') fail("expected key");
            std::string k = string();
            expect(':');
            o.o_[k] = value();
            char c = peek();
            ++i_;
            if (c == '}') break;
            if (c != ',') fail("expected ',' or '}'");
        }
        return o;
    }

    Json array() {
        expect('[');
        Json a = Json::array();
        if (peek() == ']') {
            ++i_;
            return a;
        }
        while (true) {
            a.a_.push_back(value());
            char c = peek();
            ++i_;
            if (c == ']') break;
            if (c != ',') fail("expected ',' or ']'");
        }
        return a;
    }

    static void put_utf8(std::string& out, uint32_t cp) {
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

    uint32_t hex4() {
        if (i_ + 4 > s_.size()) fail("bad \\u escape");
        uint32_t v = 0;
        for (int k = 0; k < 4; ++k) {
            char c = s_[i_++];
            v <<= 4;
            if (c >= '0' && c <= '9') v |= c - '0';
            else if (c >= 'a' && c <= 'f') v |= c - 'a' + 10;
            else if (c >= 'A' && c <= 'F') v |= c - 'A' + 10;
            else fail("bad hex digit");
        }
        return v;
    }

    std::string string() {
        expect('"');
        std::string out;
        while (true) {
            if (i_ >= s_.size()) fail("unterminated string");
            char c = s_[i_++];
            if (c == '"') break;
            if (c != '\\') {
                out += c;
                continue;
            }
            if (i_ >= s_.size()) fail("bad escape");
            char e = s_[i_++];
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
                    if (cp >= 0xD800 && cp < 0xDC00 && i_ + 1 < s_.size() && s_[i_] == '\\' && s_[i_ + 1] == 'u') {
                        i_ += 2;
                        uint32_t lo = hex4();
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    }
                    put_utf8(out, cp);
                    break;
                }
                default: fail("bad escape");
            }
        }
        return out;
    }

    Json number() {
        ws();
        size_t start = i_;
        if (i_ < s_.size() && (s_[i_] == '-' || s_[i_] == '+')) ++i_;
        bool is_int = true;
        while (i_ < s_.size()) {
            char c = s_[i_];
            if (c >= '0' && c <= '9') {
                ++i_;
            } else if (c == '.' || c == 'e' || c == 'E' || c == '-' || c == '+') {
                is_int = false;
                ++i_;
            } else {
                break;
            }
        }
        if (start == i_) fail("unexpected character");
        const std::string tok = s_.substr(start, i_ - start);
        char* end = nullptr;
        double v = std::strtod(tok.c_str(), &end);
        if (end == tok.c_str()) fail("bad number");
        if (is_int) {
            Json j((int64_t)std::strtoll(tok.c_str(), nullptr, 10));
            return j;
        }
        return Json(v);
    }
};

Json Json::parse(const std::string& text) { return JsonParser(text).parse_document(); }

Json Json::parse_file(const std::string& path) {
    std::ifstream f(path);
    if (!f) throw std::runtime_error("cannot open JSON file: " + path);
    std::stringstream ss;
    ss << f.rdbuf();
    return parse(ss.str());
}

bool Json::as_bool() const {
    if (type_ == Type::Bool) return b_;
    if (type_ == Type::Number) return n_ != 0.0;
    throw std::runtime_error("JSON value is not a bool");
}
double Json::as_double() const {
    if (type_ != Type::Number) throw std::runtime_error("JSON value is not a number");
    return n_;
}
int64_t Json::as_int() const {
    if (type_ != Type::Number) throw std::runtime_error("JSON value is not a number");
    return (int64_t)std::llround(n_);
}
const std::string& Json::as_string() const {
    if (type_ != Type::String) throw std::runtime_error("JSON value is not a string");
    return s_;
}
const std::vector<Json>& Json::as_array() const {
    if (type_ != Type::Array) throw std::runtime_error("JSON value is not an array");
    return a_;
}
std::vector<Json>& Json::as_array() {
    if (type_ != Type::Array) throw std::runtime_error("JSON value is not an array");
    return a_;
}
const std::map<std::string, Json>& Json::as_object() const {
    if (type_ != Type::Object) throw std::runtime_error("JSON value is not an object");
    return o_;
}
bool Json::contains(const std::string& key) const { return type_ == Type::Object && o_.count(key) > 0; }
const Json& Json::at(const std::string& key) const {
    if (type_ != Type::Object) throw std::runtime_error("JSON value is not an object (key '" + key + "')");
    auto it = o_.find(key);
    if (it == o_.end()) throw std::runtime_error("JSON key not found: " + key);
    return it->second;
}
Json& Json::operator[](const std::string& key) {
    if (type_ == Type::Null) type_ = Type::Object;
    if (type_ != Type::Object) throw std::runtime_error("JSON value is not an object");
    return o_[key];
}
const Json& Json::operator[](size_t i) const { return as_array().at(i); }
size_t Json::size() const {
    if (type_ == Type::Array) return a_.size();
    if (type_ == Type::Object) return o_.size();
    return 0;
}
void Json::push_back(Json v) {
    if (type_ == Type::Null) type_ = Type::Array;
    as_array().push_back(std::move(v));
}

std::string Json::get_string(const std::string& key, const std::string& def) const {
    if (!contains(key) || o_.at(key).is_null()) return def;
    return o_.at(key).as_string();
}
double Json::get_double(const std::string& key, double def) const {
    if (!contains(key) || o_.at(key).is_null()) return def;
    return o_.at(key).as_double();
}
int64_t Json::get_int(const std::string& key, int64_t def) const {
    if (!contains(key) || o_.at(key).is_null()) return def;
    return o_.at(key).as_int();
}
bool Json::get_bool(const std::string& key, bool def) const {
    if (!contains(key) || o_.at(key).is_null()) return def;
    return o_.at(key).as_bool();
}

void Json::update(const Json& other) {
    if (!is_object() || !other.is_object()) {
        *this = other;
        return;
    }
    for (const auto& kv : other.o_) {
        auto it = o_.find(kv.first);
        if (it != o_.end() && it->second.is_object() && kv.second.is_object()) {
            it->second.update(kv.second);
        } else {
            o_[kv.first] = kv.second;
        }
    }
}

static void dump_string(std::string& out, const std::string& s) {
    out += '"';
    for (char c : s) {
        switch (c) {
            case '"': out += "\\\""; break;
            case '\\': out += "\\\\"; break;
            case '\n': out += "\\n"; break;
            case '\r': out += "\\r"; break;
            case '\t': out += "\\t"; break;
            default:
                if ((unsigned char)c < 0x20) {
                    char buf[8];
                    std::snprintf(buf, sizeof(buf), "\\u%04x", (unsigned)c);
                    out += buf;
                } else {
                    out += c;
                }
        }
    }
    out += '"';
}

void Json::dump_to(std::string& out) const {
    switch (type_) {
        case Type::Null: out += "null"; break;
        case Type::Bool: out += b_ ? "true" : "false"; break;
        case Type::Number: {
            char buf[64];
            if (is_int_ || (std::floor(n_) == n_ && std::fabs(n_) < 9e15)) std::snprintf(buf, sizeof(buf), "%lld", (long long)n_);
            else std::snprintf(buf, sizeof(buf), "%.17g", n_);
            out += buf;
            break;
        }
        case Type::String: dump_string(out, s_); break;
        case Type::Array: {
            out += '[';
            for (size_t i = 0; i < a_.size(); ++i) {
                if (i) out += ',';
                a_[i].dump_to(out);
            }
            out += ']';
            break;
        }
        case Type::Object: {
            out += '{';
            bool first = true;
            for (const auto& kv : o_) {
                if (!first) out += ',';
                first = false;
                dump_string(out, kv.first);
                out += ':';
                kv.second.dump_to(out);
            }
            out += '}';
            break;
        }
    }
}

std::string Json::dump() const {
    std::string out;
    dump_to(out);
    return out;
}

}  // namespace edge_fm
