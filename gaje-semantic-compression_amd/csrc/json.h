// Minimal JSON reader for the .gaje.flat metadata and tensor directory.
// Only what serde_json needs to decide for ModelConfig / FlatTensorEntry:
// objects, arrays, strings (with \u escapes), numbers, booleans and null.
#pragma once

#include <cstdint>
#include <string>
#include <utility>
#include <vector>

namespace gaje {

struct JsonValue {
    enum Type { Null, Bool, Number, String, Array, Object } type = Null;
    bool boolean = false;
    double number = 0.0;
    bool is_integer = false;   // lexically an integer (no '.', 'e' or 'E')
    bool negative = false;
    uint64_t uinteger = 0;     // exact value when is_integer && !negative
    std::string str;
    std::vector<JsonValue> items;
    std::vector<std::pair<std::string, JsonValue>> members;

    // First member with this key, or nullptr.
    const JsonValue *get(const char *key) const;
    // Number of members with this key (serde rejects duplicate struct fields).
    int count(const char *key) const;
};

// Parses the whole buffer as one JSON value (trailing whitespace allowed).
// Returns false and fills `err` on malformed input.
bool json_parse(const char *data, size_t len, JsonValue &out, std::string &err);

// True if the buffer is well-formed UTF-8 (std::str::from_utf8).
bool utf8_valid(const unsigned char *data, size_t len);

}  // namespace gaje
