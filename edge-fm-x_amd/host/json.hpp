// Minimal JSON value, parser and serializer for the engine configuration, the
// operator implementation table and safetensors headers (the reference uses
// nlohmann/json, which is not available here). Supports the full JSON grammar;
// numbers are kept as double plus an "is integer" flag.
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace edge_fm {

class Json {
public:
    enum class Type { Null, Bool, Number, String, Array, Object };

    Json() = default;
    Json(std::nullptr_t) {}
    Json(bool b) : type_(Type::Bool), b_(b) {}
    Json(int v) : type_(Type::Number), n_(v), is_int_(true) {}
    Json(int64_t v) : type_(Type::Number), n_((double)v), is_int_(true) {}
    Json(double v) : type_(Type::Number), n_(v) {}
    Json(const char* s) : type_(Type::String), s_(s) {}
    Json(std::string s) : type_(Type::String), s_(std::move(s)) {}

    static Json array() { Json j; j.type_ = Type::Array; return j; }
    static Json object() { Json j; j.type_ = Type::Object; return j; }
    static Json parse(const std::string& text);
    static Json parse_file(const std::string& path);

    Type type() const { return type_; }
    bool is_null() const { return type_ == Type::Null; }
    bool is_bool() const { return type_ == Type::Bool; }
    bool is_number() const { return type_ == Type::Number; }
    bool is_integer() const { return type_ == Type::Number && is_int_; }
    bool is_string() const { return type_ == Type::String; }
    bool is_array() const { return type_ == Type::Array; }
    bool is_object() const { return type_ == Type::Object; }

    bool as_bool() const;
    double as_double() const;
    int64_t as_int() const;
    const std::string& as_string() const;
    const std::vector<Json>& as_array() const;
    std::vector<Json>& as_array();
    const std::map<std::string, Json>& as_object() const;

    bool contains(const std::string& key) const;
    const Json& at(const std::string& key) const;   // throws if missing
    Json& operator[](const std::string& key);       // creates (object) entries
    const Json& operator[](size_t i) const;
    size_t size() const;
    void push_back(Json v);

    // Typed lookups with defaults (null or missing -> default).
    std::string get_string(const std::string& key, const std::string& def = "") const;
    double get_double(const std::string& key, double def) const;
    int64_t get_int(const std::string& key, int64_t def) const;
    bool get_bool(const std::string& key, bool def) const;

    // Recursive merge: object members of `other` override / extend this object
    // (EngineConfig default-merge semantics, src/engine/engine.cpp:207-212).
    void update(const Json& other);

    std::string dump() const;

private:
    Type type_ = Type::Null;
    bool b_ = false;
    double n_ = 0.0;
    bool is_int_ = false;
    std::string s_;
    std::vector<Json> a_;
    std::map<std::string, Json> o_;

    void dump_to(std::string& out) const;
    friend class JsonParser;
};

}  // namespace edge_fm
