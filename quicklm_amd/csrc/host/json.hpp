// Minimal JSON reader for config.json and safetensors headers.
// Plays the role of the reference's JsonParser (src/io/json_parser.hpp:61-73):
// objects, arrays, strings (with \uXXXX escapes kept as UTF-8), numbers as
// double, true/false/null. Throws std::runtime_error on malformed input.
#pragma once

#include <cstdint>
#include <cstdlib>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <string_view>
#include <vector>

namespace qlm {

struct Json {
    enum class Kind { Null, Bool, Number, String, Array, Object };
    Kind kind = Kind::Null;
    bool b = false;
    double num = 0.0;
    std::string str;
    std::vector<Json> arr;
    std::map<std::string, Json> obj;

    bool is_object() const { return kind == Kind::Object; }
    bool is_array() const { return kind == Kind::Array; }
    bool has(const std::string& k) const { return kind == Kind::Object && obj.count(k) != 0; }
    const Json& at(const std::string& k) const {
        auto it = obj.find(k);
        if (kind != Kind::Object || it == obj.end()) throw std::runtime_error("json: missing key '" + k + "'");
        return it->second;
    }
    double number() const {
        if (kind != Kind::Number) throw std::runtime_error("json: not a number");
        return num;
    }
    const std::string& string() const {
        if (kind != Kind::String) throw std::runtime_error("json: not a string");
        return str;
    }
    double get(const std::string& k, double dflt) const { return has(k) ? at(k).number() : dflt; }

    static Json parse(std::string_view text) {
        size_t i = 0;
        Json v = value(text, i);
        ws(text, i);
        if (i != text.size()) throw std::runtime_error("json: trailing characters");
        return v;
    }

   private:
    static void ws(std::string_view t, size_t& i) {
        while (i < t.size() && (t[i] == ' ' || t[i] == '\n' || t[i] == '\r' || t[i] == '\t')) ++i;
    }
    static void expect(std::string_view t, size_t& i, char c) {
        ws(t, i);
        if (i >= t.size() || t[i] != c) throw std::runtime_error(std::string("json: expected '") + c + "'");
        ++i;
    }
    static Json value(std::string_view t, size_t& i) {
        ws(t, i);
        if (i >= t.size()) throw std::runtime_error("json: unexpected end");
        const char c = t[i];
        Json v;
        if (c == '{') {
            v.kind = Kind::Object;
            ++i;
            ws(t, i);
            if (i < t.size() && t[i] == '}') { ++i; return v; }
            for (;;) {
                ws(t, i);
                Json k = string_value(t, i);
                expect(t, i, ':');
                v.obj[k.str] = value(t, i);
                ws(t, i);
                if (i < t.size() && t[i] == ',') { ++i; continue; }
                expect(t, i, '}');
                return v;
            }
        }
        if (c == '[') {
            v.kind = Kind::Array;
            ++i;
            ws(t, i);
            if (i < t.size() && t[i] == ']') { ++i; return v; }
            for (;;) {
                v.arr.push_back(value(t, i));
                ws(t, i);
                if (i < t.size() && t[i] == ',') { ++i; continue; }
                expect(t, i, ']');
                return v;
            }
        }
        if (c == '"') return string_value(t, i);
        if (t.substr(i, 4) == "true") { i += 4; v.kind = Kind::Bool; v.b = true; return v; }
        if (t.substr(i, 5) == "false") { i += 5; v.kind = Kind::Bool; return v; }
        if (t.substr(i, 4) == "null") { i += 4; return v; }
        // number
        size_t j = i;
        while (j < t.size() && (std::isdigit((unsigned char)t[j]) || t[j] == '-' || t[j] == '+' ||
                                t[j] == '.' || t[j] == 'e' || t[j] == 'E'))
            ++j;
        if (j == i) throw std::runtime_error("json: bad token");
        v.kind = Kind::Number;
        v.num = std::strtod(std::string(t.substr(i, j - i)).c_str(), nullptr);
        i = j;
        return v;
    }
    static void put_utf8(std::string& s, uint32_t cp) {
        if (cp < 0x80) s += (char)cp;
        else if (cp < 0x800) { s += (char)(0xC0 | (cp >> 6)); s += (char)(0x80 | (cp & 0x3F)); }
        else if (cp < 0x10000) {
            s += (char)(0xE0 | (cp >> 12)); s += (char)(0x80 | ((cp >> 6) & 0x3F));
            s += (char)(0x80 | (cp & 0x3F));
        } else {
            s += (char)(0xF0 | (cp >> 18)); s += (char)(0x80 | ((cp >> 12) & 0x3F));
            s += (char)(0x80 | ((cp >> 6) & 0x3F)); s += (char)(0x80 | (cp & 0x3F));
        }
    }
    static Json string_value(std::string_view t, size_t& i) {
        ws(t, i);
        if (i >= t.size() || t[i] != '"') throw std::runtime_error("json: expected string");
        ++i;
        Json v;
        v.kind = Kind::String;
        while (i < t.size() && t[i] != '"') {
            char c = t[i++];
            if (c != '\\') { v.str += c; continue; }
            if (i >= t.size()) break;
            char e = t[i++];
            switch (e) {
                case 'n': v.str += '\n'; break;
                case 't': v.str += '\t'; break;
                case 'r': v.str += '\r'; break;
                case 'b': v.str += '\b'; break;
                case 'f': v.str += '\f'; break;
                case 'u': {
                    if (i + 4 > t.size()) throw std::runtime_error("json: bad \\u escape");
                    uint32_t cp = (uint32_t)std::strtoul(std::string(t.substr(i, 4)).c_str(), nullptr, 16);
                    i += 4;
                    put_utf8(v.str, cp);
                    break;
                }
                default: v.str += e;
            }
        }
        if (i >= t.size()) throw std::runtime_error("json: unterminated string");
        ++i;
        return v;
    }
};

}  // namespace qlm
