// Model exports and checkpoints into the device model (host code only).
//
// The reference's inference side loads weights with load_checkpoint(path, training =
// false) (src/train/checkpoint.cpp:186-324); the directory format is
// docs/file_formats.md ("Checkpoint directory"): manifest.json (format, version, the
// architecture and tokenizer hashes, parameter count, per-file SHA-256, one entry per
// tensor with name, role, shape, dtype, file, offset, byte count and CRC-32), COMPLETE
// (SHA-256 of the manifest text), config.json, tokenizer.json and weights.bin (f32 or
// f16 weights; a training checkpoint adds optimizer.bin and trainer_state.json).  This
// file checks a directory the same way, in the same order and with the same error
// codes and messages, converts the weights to fp32 in the registry order and hands them
// to mla_model_create / mla_engine_create.
//
// SHA-256 (FIPS 180-4), CRC-32 (IEEE 802.3, reflected polynomial 0xEDB88320) and a
// JSON reader are implemented here; the reference uses CommonCrypto, its own CRC table
// and its own JSON class (src/core/io.cpp:111-150, src/core/json.cpp).
#include "mla_capi_util.hpp"
#include "mla_hip.h"

#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <map>
#include <memory>
#include <set>
#include <stdexcept>
#include <string>
#include <utility>
#include <variant>
#include <vector>

namespace mla {
namespace {

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

std::string sha256_hex(const std::string& bytes) {
    Sha256 s;
    s.update(reinterpret_cast<const uint8_t*>(bytes.data()), bytes.size());
    return s.hex_digest();
}

uint32_t crc32(const uint8_t* p, size_t n) {
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
std::string dump_string(const std::string& s) {
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

std::string dump_number(double x) {
    char buf[40];
    std::snprintf(buf, sizeof buf, "%.17g", x);
    return buf;
}

// ----------------------------------------------------------- files ----
// Whole-file reads; `what` names the file in the reference's io_error form
// ("<path>: <strerror>").
bool read_file(const std::string& path, std::string& out, std::string& err) {
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

std::string join(const std::string& dir, const char* name) {
    if (dir.empty() || dir.back() == '/')
        return dir + name;
    return dir + "/" + name;
}

// ---------------------------------------------------- configuration ----
// ModelConfig::json().dump() (src/model/config.cpp:49-70): the architecture's identity.
std::string config_dump(const mla_model_config& c) {
    std::map<std::string, std::string> kv = {
        {"model_type", dump_string("mla_dense_decoder")},
        {"version", dump_number(1)},
        {"vocab_size", dump_number(c.vocab_size)},
        {"max_sequence_length", dump_number(c.max_sequence_length)},
        {"n_layers", dump_number(c.n_layers)},
        {"d_model", dump_number(c.d_model)},
        {"n_heads", dump_number(c.n_heads)},
        {"head_dim_nope", dump_number(c.head_dim_nope)},
        {"head_dim_rope", dump_number(c.head_dim_rope)},
        {"head_dim_value", dump_number(c.head_dim_value)},
        {"q_lora_rank", dump_number(c.q_lora_rank)},
        {"kv_lora_rank", dump_number(c.kv_lora_rank)},
        {"d_ff", dump_number(c.d_ff)},
        {"norm_epsilon", dump_number((double)c.norm_epsilon)},
        {"rope_theta", dump_number((double)c.rope_theta)},
        {"norm", dump_string("rmsnorm")},
        {"activation", dump_string("swiglu")},
        {"mla_latent_norms", "true"},
        {"bias", "false"},
        {"tie_word_embeddings", "true"}};
    std::string s = "{";
    for (const auto& [k, v] : kv) {
        if (s.size() > 1)
            s += ',';
        s += dump_string(k) + ':' + v;
    }
    return s + '}';
}

// ModelConfig::from_json (src/model/config.cpp:74-107): MLA_OK or the reference's code
// and message.
int config_from_json(const Json& j, mla_model_config& c) {
    try {
        c.vocab_size = j.at("vocab_size").integer();
        c.max_sequence_length = j.at("max_sequence_length").integer();
        c.n_layers = j.at("n_layers").integer();
        c.d_model = j.at("d_model").integer();
        c.n_heads = j.at("n_heads").integer();
        c.head_dim_nope = j.at("head_dim_nope").integer();
        c.head_dim_rope = j.at("head_dim_rope").integer();
        c.head_dim_value = j.at("head_dim_value").integer();
        c.q_lora_rank = j.at("q_lora_rank").integer();
        c.kv_lora_rank = j.at("kv_lora_rank").integer();
        c.d_ff = j.at("d_ff").integer();
        c.norm_epsilon = (float)j.at("norm_epsilon").number();
        c.rope_theta = (float)j.at("rope_theta").number();
        if (j.str_or("model_type", "mla_dense_decoder") != "mla_dense_decoder" ||
            j.num_or("version", 1) != 1 || j.str_or("norm", "rmsnorm") != "rmsnorm" ||
            j.str_or("activation", "swiglu") != "swiglu" || j.bool_or("bias", false) ||
            !j.bool_or("tie_word_embeddings", true) || !j.bool_or("mla_latent_norms", true))
            return fail(MLA_ERR_UNSUPPORTED,
                        "Only v1 tied-embedding, bias-free MLA with latent RMSNorm and SwiGLU "
                        "is supported");
        const int st = mla_config_validate(&c);
        if (st != MLA_OK)
            return st;
        if (j.contains("expected_parameter_count") &&
            j.at("expected_parameter_count").size_integer() != mla_config_parameter_count(&c))
            return fail(MLA_ERR_INVALID_ARGUMENT,
                        "Expected parameter count disagrees with architecture");
        return MLA_OK;
    } catch (const std::exception& e) {
        return fail(MLA_ERR_INVALID_ARGUMENT, e.what());
    }
}

int parse_file(const std::string& path, Json& out) {  // read_json
    std::string text, err;
    if (!read_file(path, text, err))
        return fail(MLA_ERR_IO, err);
    try {
        out = JsonReader(text).parse();
    } catch (const std::exception& e) {
        return fail(MLA_ERR_INVALID_ARGUMENT, e.what());
    }
    return MLA_OK;
}

int load_config(const std::string& path, mla_model_config& c) {  // ModelConfig::load
    Json j;
    const int st = parse_file(path, j);
    return st != MLA_OK ? st : config_from_json(j, c);
}

// ------------------------------------------------------------ tokenizer ----
// Tokenizer::load's checks (src/infer/tokenizer.cpp:70-127); the tokenizer's identity is
// the SHA-256 of its file bytes.
int check_tokenizer(const std::string& path, int& vocab, std::string& hash) {
    std::string text, err;
    if (!read_file(path, text, err))
        return fail(MLA_ERR_IO, err);
    Json j;
    try {
        j = JsonReader(text).parse();
    } catch (const std::exception& e) {
        return fail(MLA_ERR_INVALID_ARGUMENT, e.what());
    }
    static const char* specials[8] = {"<|pad|>",       "<|bos|>",    "<|eos|>",  "<|user|>",
                                      "<|assistant|>", "<|system|>", "<|tool|>", "<|sep|>"};
    try {
        if (j.at("format").string() != "mini-mla-tokenizer" || j.at("version").integer() != 1 ||
            j.at("pretokenizer").string() != "bytes-v1")
            return fail(MLA_ERR_UNSUPPORTED, "Unsupported tokenizer format or pretokenizer");
        vocab = j.at("vocab_size").integer();
        if (vocab < 264 || vocab > 65535)
            return fail(MLA_ERR_INVALID_ARGUMENT, "Tokenizer vocabulary must be in [264,65535]");
        std::vector<size_t> length((size_t)vocab, 0);
        for (int i = 0; i < 256; ++i)
            length[(size_t)i] = 1;
        std::set<uint32_t> pairs;
        size_t id = 256;
        for (const Json& m : j.at("merges").array()) {
            const Json::Array& a = m.array();
            if (a.size() != 3 || id >= (size_t)(vocab - 8) || a[2].integer() != (int)id)
                throw std::invalid_argument("Malformed BPE merge");
            const int left = a[0].integer(), right = a[1].integer();
            if (left < 0 || right < 0 || (size_t)left >= id || (size_t)right >= id)
                throw std::invalid_argument("BPE merge references a future token");
            if (!pairs.insert((uint32_t)left << 16 | (uint32_t)right).second)
                throw std::invalid_argument("Duplicate BPE pair");
            length[id] = length[(size_t)left] + length[(size_t)right];
            if (length[id] > 1024 * 1024)
                throw std::invalid_argument("BPE token exceeds size limit");
            ++id;
        }
        if (j.at("specials").object().size() != 8)
            throw std::invalid_argument("Tokenizer must define exactly eight special tokens");
        for (int k = 0; k < 8; ++k)
            if (j.at("specials").at(specials[k]).integer() != vocab - 8 + k)
                throw std::invalid_argument(
                    "Special token IDs disagree with the native chat template");
    } catch (const std::exception& e) {
        return fail(MLA_ERR_INVALID_ARGUMENT, e.what());
    }
    hash = sha256_hex(text);
    return MLA_OK;
}

// ------------------------------------------------------------- registry ----
struct Slot {
    size_t offset, rows, cols;
    const char* role;
};

// Parameter names, roles and shapes in registry order (src/model/model.cpp:26-63).
std::map<std::string, Slot> registry(const mla_model_config& c) {
    static const char* names[13] = {"attn.norm",    "attn.w_dq", "attn.q_norm", "attn.w_uq",
                                    "attn.w_dkv",   "attn.kv_norm", "attn.w_uk", "attn.w_uv",
                                    "attn.w_o",     "ffn.norm",  "ffn.w_gate",  "ffn.w_up",
                                    "ffn.w_down"};
    static const char* roles[13] = {"norm_scale",    "hidden_matrix", "norm_scale",
                                    "hidden_matrix", "hidden_matrix", "norm_scale",
                                    "hidden_matrix", "hidden_matrix", "hidden_matrix",
                                    "norm_scale",    "hidden_matrix", "hidden_matrix",
                                    "hidden_matrix"};
    const size_t d = c.d_model, q = c.q_lora_rank, kv = c.kv_lora_rank, H = c.n_heads;
    const size_t nope = c.head_dim_nope, rope = c.head_dim_rope, dv = c.head_dim_value,
                 ff = c.d_ff;
    const size_t shapes[13][2] = {{1, d},         {d, q},       {1, q},         {q, H * (nope + rope)},
                                  {d, kv + rope}, {1, kv},      {kv, H * nope}, {kv, H * dv},
                                  {H * dv, d},    {1, d},       {d, ff},        {d, ff},
                                  {ff, d}};
    std::map<std::string, Slot> r;
    size_t at = 0;
    auto add = [&](const std::string& name, const char* role, size_t rows, size_t cols) {
        r.emplace(name, Slot{at, rows, cols, role});
        at += rows * cols;
    };
    add("token_embedding", "token_embedding", (size_t)c.vocab_size, d);
    add("final_norm", "norm_scale", 1, d);
    for (int l = 0; l < c.n_layers; ++l)
        for (int k = 0; k < 13; ++k)
            add("layers." + std::to_string(l) + "." + names[k], roles[k], shapes[k][0],
                shapes[k][1]);
    return r;
}

float half_to_float(uint16_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

// load_checkpoint(path, training = false) (src/train/checkpoint.cpp:186-324).
int read_export(const std::string& dir, mla_model_config& cfg, float* params, size_t count) {
    std::string raw, err;
    if (!read_file(join(dir, "manifest.json"), raw, err))
        return fail(MLA_ERR_IO, err);
    std::string complete;
    if (!read_file(join(dir, "COMPLETE"), complete, err) || complete != sha256_hex(raw) + "\n")
        return fail(MLA_ERR_IO, "Checkpoint is incomplete or manifest checksum failed");
    Json manifest;
    try {
        manifest = JsonReader(raw).parse();
    } catch (const std::exception& e) {
        return fail(MLA_ERR_INVALID_ARGUMENT, e.what());
    }
    try {
        const std::string format = manifest.at("format").string();
        if ((format != "mini-mla-checkpoint" && format != "mini-mla-model") ||
            manifest.at("version").integer() != 1)
            return fail(MLA_ERR_UNSUPPORTED,
                        "Unsupported model format or inference export used for resume");
        int st = load_config(join(dir, "config.json"), cfg);
        if (st != MLA_OK)
            return st;
        const size_t n_params = mla_config_parameter_count(&cfg);
        if (sha256_hex(config_dump(cfg)) != manifest.at("model_config_sha256").string() ||
            n_params != manifest.at("parameter_count").size_integer())
            return fail(MLA_ERR_INVALID_ARGUMENT, "Checkpoint model configuration mismatch");
        int vocab = 0;
        std::string tok_hash;
        st = check_tokenizer(join(dir, "tokenizer.json"), vocab, tok_hash);
        if (st != MLA_OK)
            return st;
        if (tok_hash != manifest.at("tokenizer_sha256").string() || vocab != cfg.vocab_size)
            return fail(MLA_ERR_INVALID_ARGUMENT, "Checkpoint tokenizer mismatch");
        if (params && count != n_params)
            return fail(MLA_ERR_INVALID_ARGUMENT,
                        "parameter buffer holds " + std::to_string(count) +
                            " floats; the export has " + std::to_string(n_params));
        std::map<std::string, std::string> files;
        for (const auto& [name, hash] : manifest.at("sha256").object()) {
            if (name != "weights.bin" && name != "optimizer.bin" && name != "trainer_state.json")
                throw std::invalid_argument("Invalid checkpoint filename");
            std::string bytes;
            if (!read_file(join(dir, name.c_str()), bytes, err))
                return fail(MLA_ERR_IO, err);
            if (sha256_hex(bytes) != hash.string())
                throw std::invalid_argument("Checkpoint file checksum failed: " + name);
            files.emplace(name, std::move(bytes));
        }
        std::map<std::string, Slot> expected = registry(cfg);
        std::set<std::string> seen;
        std::map<std::string, size_t> ends;
        for (const Json& entry : manifest.at("tensors").array()) {
            const std::string name = entry.at("name").string(), file = entry.at("file").string(),
                              dtype = entry.at("dtype").string();
            if (file != "weights.bin" && file != "optimizer.bin")
                throw std::invalid_argument("Invalid tensor filename");
            if (!seen.insert(name).second)
                throw std::invalid_argument("Duplicate named tensor");
            const size_t offset = entry.at("offset").size_integer(),
                         nbytes = entry.at("nbytes").size_integer();
            auto fit = files.find(file);
            if (fit == files.end() || offset != ends[file] || offset > fit->second.size() ||
                nbytes > fit->second.size() - offset)
                throw std::invalid_argument("Invalid tensor extent or missing tensor file");
            const uint8_t* bytes = reinterpret_cast<const uint8_t*>(fit->second.data()) + offset;
            ends[file] = offset + nbytes;
            if (crc32(bytes, nbytes) != entry.at("crc32").size_integer())
                throw std::invalid_argument("Tensor checksum failed: " + name);
            auto it = expected.find(name);
            if (it == expected.end()) {
                if (file == "optimizer.bin" && format == "mini-mla-checkpoint")
                    continue;  // training state: not needed for inference
                throw std::invalid_argument("Unexpected tensor: " + name);
            }
            const Slot slot = it->second;
            const Json::Array& shape = entry.at("shape").array();
            const size_t item = dtype == "f32" ? 4 : dtype == "f16" ? 2 : 0;
            if (!item || file != "weights.bin" || shape.size() != 2 ||
                shape[0].integer() != (int)slot.rows || shape[1].integer() != (int)slot.cols ||
                nbytes != slot.rows * slot.cols * item || entry.at("role").string() != slot.role)
                throw std::invalid_argument("Tensor shape, dtype, role, or file mismatch: " +
                                            name);
            const size_t n = slot.rows * slot.cols;
            bool finite = true;
            for (size_t k = 0; k < n; ++k) {
                float x;
                if (item == 4) {
                    std::memcpy(&x, bytes + 4 * k, 4);
                } else {
                    uint16_t h;
                    std::memcpy(&h, bytes + 2 * k, 2);
                    x = half_to_float(h);
                }
                finite = finite && std::isfinite(x);
                if (params)
                    params[slot.offset + k] = x;
            }
            if (!finite)
                throw std::invalid_argument("Nonfinite checkpoint tensor: " + name);
            expected.erase(it);
        }
        if (!expected.empty())
            throw std::invalid_argument("Checkpoint is missing tensor: " + expected.begin()->first);
        for (const auto& [file, end] : ends)
            if (end != files.at(file).size())
                throw std::invalid_argument("Unindexed trailing tensor data");
        return MLA_OK;
    } catch (const std::exception& e) {
        return fail(MLA_ERR_IO, e.what());
    }
}

}  // namespace
}  // namespace mla

using namespace mla;

extern "C" {

int mla_export_read_config(const char* dir, mla_model_config* config) {
    if (!dir || !config)
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_export_read_config: null argument");
    return load_config(join(dir, "config.json"), *config);
}

int mla_export_read(const char* dir, mla_model_config* config, float* params,
                    size_t params_count) {
    if (!dir || !config)
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_export_read: null argument");
    return read_export(dir, *config, params, params_count);
}

int mla_config_hash(const mla_model_config* config, char* hex_out) {
    if (!config || !hex_out)
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_config_hash: null argument");
    const std::string h = sha256_hex(config_dump(*config));
    std::memcpy(hex_out, h.c_str(), 65);
    return MLA_OK;
}

int mla_model_load(const char* dir, int max_batch, int page_size, mla_model_config* config,
                   void** model) {
    if (!dir || !config || !model)
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_model_load: null argument");
    mla_model_config c{};
    int st = load_config(join(dir, "config.json"), c);
    if (st != MLA_OK)
        return st;
    std::vector<float> params(mla_config_parameter_count(&c));
    st = read_export(dir, c, params.data(), params.size());
    if (st != MLA_OK)
        return st;
    *config = c;
    return mla_model_create(&c, params.data(), max_batch, page_size, model);
}

int mla_engine_load(const char* dir, int max_sessions, int max_rows, int num_pages,
                    int page_size, mla_model_config* config, void** engine) {
    if (!dir || !config || !engine)
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_engine_load: null argument");
    mla_model_config c{};
    int st = load_config(join(dir, "config.json"), c);
    if (st != MLA_OK)
        return st;
    std::vector<float> params(mla_config_parameter_count(&c));
    st = read_export(dir, c, params.data(), params.size());
    if (st != MLA_OK)
        return st;
    *config = c;
    return mla_engine_create(&c, params.data(), max_sessions, max_rows, num_pages, page_size,
                             engine);
}

}  // extern "C"
