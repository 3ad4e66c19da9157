// Minimal JSON reader for config.json and safetensors headers.
// Numbers keep two views, like serde_json: an exact u64 when the literal is a
// non-negative integer (as_u64), and a double (as_f64).
#pragma once

#include <map>
#include <memory>
#include <string>
#include <vector>

namespace tmg {

struct JsonValue {
    enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
    bool b = false;
    double num = 0.0;
    bool is_u64 = false;
    unsigned long long u64 = 0;
    std::string str;
    std::vector<JsonValue> arr;
    std::vector<std::pair<std::string, JsonValue>> obj;

    const JsonValue *get(const std::string &key) const;
    bool as_u64(unsigned long long *out) const;
    bool as_f64(double *out) const;
};

// Parses `text`; on failure returns false and sets *err.
bool json_parse(const char *text, size_t len, JsonValue *out, std::string *err);

}  // namespace tmg
