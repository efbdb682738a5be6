// Host-side file helpers shared by the export loader and the tokenizer: SHA-256
// (FIPS 180-4), CRC-32 (IEEE 802.3, reflected polynomial 0xEDB88320), a JSON reader
// whose values are held as the reference's Json holds them (numbers as doubles, objects
// with sorted keys), the reference's dump conventions for strings and numbers
// (src/core/json.cpp:222-293) and whole-file reads.
#pragma once

#include <algorithm>
#include <cerrno>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <map>
#include <stdexcept>
#include <string>
#include <variant>
#include <vector>

namespace mla {
namespace io {

// ------------------------------------------------------------- hashes ----
class Sha256 {
  public:
    Sha256() { reset(); }
    void update(const uint8_t* p, size_t n) {
        total_ += n;
        while (n) {
            const size_t take = std::min(n, (size_t)64 - fill_);
            std::memcpy(block_ + fill_, p, take);
            fill_ += take;
            p += take;
            n -= take;
            if (fill_ == 64) {
                compress(block_);
                fill_ = 0;
            }
        }
    }
    std::string hex_digest() {
        const uint64_t bits = total_ * 8;
        const uint8_t one = 0x80, zero = 0;
        update(&one, 1);
        while (fill_ != 56)
            update(&zero, 1);
        uint8_t len[8];
        for (int i = 0; i < 8; ++i)
            len[i] = (uint8_t)(bits >> (56 - 8 * i));
        update(len, 8);
        static const char* digits = "0123456789abcdef";
        std::string s;
        for (uint32_t w : h_)
            for (int i = 3; i >= 0; --i) {
                const uint8_t b = (uint8_t)(w >> (8 * i));
                s += digits[b >> 4];
                s += digits[b & 15];
            }
        return s;
    }

  private:
    static uint32_t rotr(uint32_t x, int r) { return (x >> r) | (x << (32 - r)); }
    void reset() {
        static const uint32_t init[8] = {0x6a09e667, 0xbb67ae85, 0x3c6ef372, 0xa54ff53a,
                                         0x510e527f, 0x9b05688c, 0x1f83d9ab, 0x5be0cd19};
        std::memcpy(h_, init, sizeof h_);
        fill_ = 0;
        total_ = 0;
    }
    void compress(const uint8_t* b) {
        // The first 32 bits of the fractional parts of the cube roots of the first 64
        // primes (FIPS 180-4, section 4.2.2).
        static const uint32_t k[64] = {
            0x428a2f98, 0x71374491, 0xb5c0fbcf, 0xe9b5dba5, 0x3956c25b, 0x59f111f1, 0x923f82a4,
            0xab1c5ed5, 0xd807aa98, 0x12835b01, 0x243185be, 0x550c7dc3, 0x72be5d74, 0x80deb1fe,
            0x9bdc06a7, 0xc19bf174, 0xe49b69c1, 0xefbe4786, 0x0fc19dc6, 0x240ca1cc, 0x2de92c6f,
            0x4a7484aa, 0x5cb0a9dc, 0x76f988da, 0x983e5152, 0xa831c66d, 0xb00327c8, 0xbf597fc7,
            0xc6e00bf3, 0xd5a79147, 0x06ca6351, 0x14292967, 0x27b70a85, 0x2e1b2138, 0x4d2c6dfc,
            0x53380d13, 0x650a7354, 0x766a0abb, 0x81c2c92e, 0x92722c85, 0xa2bfe8a1, 0xa81a664b,
            0xc24b8b70, 0xc76c51a3, 0xd192e819, 0xd6990624, 0xf40e3585, 0x106aa070, 0x19a4c116,
            0x1e376c08, 0x2748774c, 0x34b0bcb5, 0x391c0cb3, 0x4ed8aa4a, 0x5b9cca4f, 0x682e6ff3,
            0x748f82ee, 0x78a5636f, 0x84c87814, 0x8cc70208, 0x90befffa, 0xa4506ceb, 0xbef9a3f7,
            0xc67178f2};
        uint32_t w[64];
        for (int t = 0; t < 16; ++t)
            w[t] = (uint32_t)b[4 * t] << 24 | (uint32_t)b[4 * t + 1] << 16 |
                   (uint32_t)b[4 * t + 2] << 8 | (uint32_t)b[4 * t + 3];
        for (int t = 16; t < 64; ++t) {
            const uint32_t s0 = rotr(w[t - 15], 7) ^ rotr(w[t - 15], 18) ^ (w[t - 15] >> 3);
            const uint32_t s1 = rotr(w[t - 2], 17) ^ rotr(w[t - 2], 19) ^ (w[t - 2] >> 10);
            w[t] = w[t - 16] + s0 + w[t - 7] + s1;
        }
        uint32_t a = h_[0], bb = h_[1], c = h_[2], d = h_[3], e = h_[4], f = h_[5], g = h_[6],
                 h = h_[7];
        for (int t = 0; t < 64; ++t) {
            const uint32_t t1 = h + (rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25)) +
                                ((e & f) ^ (~e & g)) + k[t] + w[t];
            const uint32_t t2 =
                (rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22)) + ((a & bb) ^ (a & c) ^ (bb & c));
            h = g;
            g = f;
            f = e;
            e = d + t1;
            d = c;
            c = bb;
            bb = a;
            a = t1 + t2;
        }
        h_[0] += a;
        h_[1] += bb;
        h_[2] += c;
        h_[3] += d;
        h_[4] += e;
        h_[5] += f;
        h_[6] += g;
        h_[7] += h;
    }
    uint32_t h_[8];
    uint8_t block_[64];
    size_t fill_;
    uint64_t total_;
};

inline std::string sha256_hex(const std::string& bytes) {
    Sha256 s;
    s.update(reinterpret_cast<const uint8_t*>(bytes.data()), bytes.size());
    return s.hex_digest();
}

inline uint32_t crc32(const uint8_t* p, size_t n) {
    static const std::vector<uint32_t> table = [] {
        std::vector<uint32_t> t(256);
        for (uint32_t i = 0; i < 256; ++i) {
            uint32_t x = i;
            for (int k = 0; k < 8; ++k)
                x = (x & 1) ? (x >> 1) ^ 0xEDB88320u : x >> 1;
            t[i] = x;
        }
        return t;
    }();
    uint32_t c = 0xFFFFFFFFu;
    for (size_t i = 0; i < n; ++i)
        c = table[(c ^ p[i]) & 0xFF] ^ (c >> 8);
    return ~c;
}

// --------------------------------------------------------------- JSON ----
// Values as the reference's Json holds them: every number is a double, objects keep
// their keys sorted (so a dump is canonical), strings are UTF-8 bytes.
struct Json {
    using Array = std::vector<Json>;
    using Object = std::map<std::string, Json, std::less<>>;
    std::variant<std::monostate, bool, double, std::string, Array, Object> v;

    const Object& object() const {
        if (auto p = std::get_if<Object>(&v))
            return *p;
        throw std::invalid_argument("Expected JSON object");
    }
    const Array& array() const {
        if (auto p = std::get_if<Array>(&v))
            return *p;
        throw std::invalid_argument("Expected JSON array");
    }
    const std::string& string() const {
        if (auto p = std::get_if<std::string>(&v))
            return *p;
        throw std::invalid_argument("Expected JSON string");
    }
    double number() const {
        if (auto p = std::get_if<double>(&v))
            return *p;
        throw std::invalid_argument("Expected JSON number");
    }
    bool boolean() const {
        if (auto p = std::get_if<bool>(&v))
            return *p;
        throw std::invalid_argument("Expected JSON boolean");
    }
    int integer() const {  // json.cpp: an integral value in int range
        const double x = number();
        if (!(x >= -2147483648.0 && x <= 2147483647.0) || std::floor(x) != x)
            throw std::invalid_argument("Expected bounded integer");
        return (int)x;
    }
    size_t size_integer() const {  // an exact non-negative integer (below 2^53)
        const double x = number();
        if (!(x >= 0 && x <= 9007199254740992.0) || std::floor(x) != x)
            throw std::invalid_argument("Expected exact nonnegative integer");
        return (size_t)x;
    }
    bool contains(const std::string& key) const {
        const Object& o = object();
        return o.find(key) != o.end();
    }
    const Json& at(const std::string& key) const {
        const Object& o = object();
        auto it = o.find(key);
        if (it == o.end())
            throw std::invalid_argument("Missing JSON field: " + key);
        return it->second;
    }
    std::string str_or(const std::string& key, const std::string& fallback) const {
        return contains(key) ? at(key).string() : fallback;
    }
    double num_or(const std::string& key, double fallback) const {
        return contains(key) ? at(key).number() : fallback;
    }
    bool bool_or(const std::string& key, bool fallback) const {
        return contains(key) ? at(key).boolean() : fallback;
    }
};

class JsonReader {
  public:
    explicit JsonReader(const std::string& t) : s_(t) {}
    Json parse() {
        Json j = value(0);
        skip();
        if (i_ != s_.size())
            fail("Trailing data");
        return j;
    }

  private:
    [[noreturn]] void fail(const char* why) const {
        throw std::invalid_argument(std::string(why) + " at JSON byte " + std::to_string(i_));
    }
    void skip() {
        while (i_ < s_.size() && (s_[i_] == ' ' || s_[i_] == '\t' || s_[i_] == '\n' || s_[i_] == '\r'))
            ++i_;
    }
    bool literal(const char* word) {
        const size_t n = std::strlen(word);
        if (s_.compare(i_, n, word) != 0)
            return false;
        i_ += n;
        return true;
    }
    Json value(int depth) {
        if (depth > 256)
            fail("JSON nesting too deep");
        skip();
        if (i_ >= s_.size())
            fail("Unexpected end of JSON");
        Json j;
        const char c = s_[i_];
        if (c == '{') {
            ++i_;
            Json::Object o;
            skip();
            if (i_ < s_.size() && s_[i_] == '}') {
                ++i_;
                j.v = std::move(o);
                return j;
            }
            for (;;) {
                skip();
                if (i_ >= s_.size() || s_[i_] != '"')
                    fail("Expected object key");
                std::string key = string_value();
                skip();
                if (i_ >= s_.size() || s_[i_] != ':')
                    fail("Unexpected character");
                ++i_;
                Json item = value(depth + 1);
                if (!o.emplace(std::move(key), std::move(item)).second)
                    fail("Duplicate JSON key");
                skip();
                if (i_ < s_.size() && s_[i_] == ',') {
                    ++i_;
                    continue;
                }
                if (i_ < s_.size() && s_[i_] == '}') {
                    ++i_;
                    break;
                }
                fail("Unexpected character");
            }
            j.v = std::move(o);
        } else if (c == '[') {
            ++i_;
            Json::Array a;
            skip();
            if (i_ < s_.size() && s_[i_] == ']') {
                ++i_;
                j.v = std::move(a);
                return j;
            }
            for (;;) {
                a.push_back(value(depth + 1));
                skip();
                if (i_ < s_.size() && s_[i_] == ',') {
                    ++i_;
                    continue;
                }
                if (i_ < s_.size() && s_[i_] == ']') {
                    ++i_;
                    break;
                }
                fail("Unexpected character");
            }
            j.v = std::move(a);
        } else if (c == '"') {
            j.v = string_value();
        } else if (literal("true")) {
            j.v = true;
        } else if (literal("false")) {
            j.v = false;
        } else if (literal("null")) {
            j.v = std::monostate{};
        } else {
            j.v = number_value();
        }
        return j;
    }
    double number_value() {
        // JSON grammar: -? (0 | [1-9][0-9]*) (. [0-9]+)? ([eE] [+-]? [0-9]+)?
        const size_t start = i_;
        auto digits = [&] {
            const size_t b = i_;
            while (i_ < s_.size() && s_[i_] >= '0' && s_[i_] <= '9')
                ++i_;
            return i_ > b;
        };
        if (i_ < s_.size() && s_[i_] == '-')
            ++i_;
        if (i_ < s_.size() && s_[i_] == '0')
            ++i_;
        else if (!digits())
            fail("Invalid JSON number");
        if (i_ < s_.size() && s_[i_] == '.') {
            ++i_;
            if (!digits())
                fail("Invalid JSON number");
        }
        if (i_ < s_.size() && (s_[i_] == 'e' || s_[i_] == 'E')) {
            ++i_;
            if (i_ < s_.size() && (s_[i_] == '+' || s_[i_] == '-'))
                ++i_;
            if (!digits())
                fail("Invalid JSON number");
        }
        const std::string text = s_.substr(start, i_ - start);
        const double x = std::strtod(text.c_str(), nullptr);
        if (!std::isfinite(x))
            fail("Invalid JSON number");
        return x;
    }
    unsigned hex4() {
        if (i_ + 4 > s_.size())
            fail("Truncated Unicode escape");
        unsigned n = 0;
        for (int k = 0; k < 4; ++k) {
            const char c = s_[i_++];
            n <<= 4;
            if (c >= '0' && c <= '9')
                n |= (unsigned)(c - '0');
            else if (c >= 'a' && c <= 'f')
                n |= (unsigned)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F')
                n |= (unsigned)(c - 'A' + 10);
            else
                fail("Invalid Unicode escape");
        }
        return n;
    }
    static void utf8(std::string& out, unsigned cp) {
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
    std::string string_value() {
        ++i_;  // opening quote
        std::string out;
        for (;;) {
            if (i_ >= s_.size())
                fail("Unterminated JSON string");
            const unsigned char c = (unsigned char)s_[i_++];
            if (c == '"')
                return out;
            if (c < 0x20)
                fail("Control character in JSON string");
            if (c != '\\') {
                out += (char)c;
                continue;
            }
            if (i_ >= s_.size())
                fail("Unterminated JSON string");
            const char e = s_[i_++];
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
                unsigned cp = hex4();
                if (cp >= 0xD800 && cp < 0xDC00) {  // high surrogate: a low one must follow
                    if (i_ + 2 > s_.size() || s_[i_] != '\\' || s_[i_ + 1] != 'u')
                        fail("Invalid Unicode surrogate");
                    i_ += 2;
                    const unsigned lo = hex4();
                    if (lo < 0xDC00 || lo >= 0xE000)
                        fail("Invalid Unicode surrogate");
                    cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                } else if (cp >= 0xDC00 && cp < 0xE000) {
                    fail("Invalid Unicode surrogate");
                }
                utf8(out, cp);
                break;
            }
            default:
                fail("Invalid JSON escape");
            }
        }
    }
    const std::string& s_;
    size_t i_ = 0;
};

// Json::dump's form (src/core/json.cpp:222-293): numbers with 17 significant digits,
// keys in sorted order, the reference's string escapes.
inline std::string dump_string(const std::string& s) {
    static const char* hex = "0123456789abcdef";
    std::string out = "\"";
    for (const char ch : s) {
        const unsigned char c = (unsigned char)ch;
        if (c == '"')
            out += "\\\"";
        else if (c == '\\')
            out += "\\\\";
        else if (c == '\n')
            out += "\\n";
        else if (c == '\r')
            out += "\\r";
        else if (c == '\t')
            out += "\\t";
        else if (c < 32) {
            out += "\\u00";
            out += hex[c >> 4];
            out += hex[c & 15];
        } else
            out += ch;
    }
    return out + '"';
}

inline std::string dump_number(double x) {
    char buf[40];
    std::snprintf(buf, sizeof buf, "%.17g", x);
    return buf;
}

// ----------------------------------------------------------- files ----
// Whole-file reads; `what` names the file in the reference's io_error form
// ("<path>: <strerror>").
inline bool read_file(const std::string& path, std::string& out, std::string& err) {
    std::ifstream f(path, std::ios::binary);
    if (!f) {
        err = path + ": " + std::strerror(errno);
        return false;
    }
    f.seekg(0, std::ios::end);
    const std::streamoff n = f.tellg();
    f.seekg(0, std::ios::beg);
    out.resize((size_t)n);
    if (n > 0 && !f.read(&out[0], n)) {
        err = path + ": read failed";
        return false;
    }
    return true;
}

inline std::string join(const std::string& dir, const char* name) {
    if (dir.empty() || dir.back() == '/')
        return dir + name;
    return dir + "/" + name;
}

}  // namespace io
}  // namespace mla
