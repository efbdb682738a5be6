// Byte-level BPE tokenizer of the reference (src/infer/tokenizer.cpp), host code: the
// mini-mla-tokenizer JSON format (docs/file_formats.md, "Tokenizer"), its validation,
// encode (ranked merges applied lowest id first, leftmost first on ties; optional
// special-token parsing), decode, and the file's SHA-256 identity.  Prompts for
// generation are BOS + encode(text) (inference.cpp:461-468).
#include "mla_capi_util.hpp"
#include "mla_hip.h"
#include "mla_io.hpp"
#include "mla_tokenizer.hpp"

#include <memory>
#include <set>

namespace mla {

namespace {

// The eight role tokens; they own the last eight ids of the vocabulary in this order
// (docs/file_formats.md, "Tokenizer").
const char* const kSpecialNames[8] = {"<|pad|>",       "<|bos|>",    "<|eos|>",  "<|user|>",
                                      "<|assistant|>", "<|system|>", "<|tool|>", "<|sep|>"};
constexpr int kSpecials = 8;
constexpr size_t kMaxTokenBytes = size_t(1) << 20;

// A load failure: an ErrorCode status and the message the reference gives for it.
struct Rejection {
    int code = MLA_OK;
    std::string message;
    explicit operator bool() const { return code != MLA_OK; }
};
Rejection reject(int code, std::string message) { return {code, std::move(message)}; }
Rejection invalid(std::string message) { return reject(MLA_ERR_INVALID_ARGUMENT, std::move(message)); }

// The header fields a version-1 bytes tokenizer must carry, then its vocabulary size.
Rejection read_header(const io::Json& j, int& vocab) {
    struct Field {
        const char* key;
        const char* text;  // expected string, or null for the integer below
        int number;
    };
    static const Field kAccepted[] = {{"format", "mini-mla-tokenizer", 0},
                                      {"version", nullptr, 1},
                                      {"pretokenizer", "bytes-v1", 0}};
    for (const Field& f : kAccepted) {
        const io::Json& v = j.at(f.key);
        if (f.text ? v.string() != f.text : v.integer() != f.number)
            return reject(MLA_ERR_UNSUPPORTED, "Unsupported tokenizer format or pretokenizer");
    }
    vocab = j.at("vocab_size").integer();
    if (vocab < 256 + kSpecials || vocab > 65535)
        return invalid("Tokenizer vocabulary must be in [264,65535]");
    return {};
}

// Builds the id -> bytes table and the pair -> id map from the sequential merge list:
// merge k creates id 256 + k, from two ids created before it, below the special range.
class MergeBuilder {
  public:
    MergeBuilder(Tokenizer& t, int vocab) : t_(t), first_special_((size_t)vocab - kSpecials) {
        t_.bytes.assign((size_t)vocab, std::string());
        for (int b = 0; b < 256; ++b)
            t_.bytes[(size_t)b].assign(1, (char)b);
    }
    Rejection add(const io::Json& merge) {
        const io::Json::Array& triple = merge.array();
        const size_t made = next_;
        if (triple.size() != 3 || made >= first_special_ || triple[2].integer() != (int)made)
            return invalid("Malformed BPE merge");
        const int lhs = triple[0].integer(), rhs = triple[1].integer();
        if (!earlier(lhs) || !earlier(rhs))
            return invalid("BPE merge references a future token");
        const uint32_t key = (uint32_t)lhs << 16 | (uint32_t)rhs;
        if (t_.merges.count(key))
            return invalid("Duplicate BPE pair");
        t_.merges.emplace(key, (uint16_t)made);
        std::string& text = t_.bytes[made];
        text = t_.bytes[(size_t)lhs];
        text += t_.bytes[(size_t)rhs];
        if (text.size() > kMaxTokenBytes)
            return invalid("BPE token exceeds size limit");
        ++next_;
        return {};
    }

  private:
    bool earlier(int id) const { return id >= 0 && (size_t)id < next_; }
    Tokenizer& t_;
    size_t first_special_, next_ = 256;
};

// The specials object names exactly the eight role tokens, each at its fixed id.
Rejection read_specials(const io::Json& j, int vocab, Tokenizer& t) {
    const io::Json& specials = j.at("specials");
    if (specials.object().size() != kSpecials)
        return invalid("Tokenizer must define exactly eight special tokens");
    for (int k = 0; k < kSpecials; ++k) {
        const int want = vocab - kSpecials + k;
        if (specials.at(kSpecialNames[k]).integer() != want)
            return invalid("Special token IDs disagree with the native chat template");
        t.specials.emplace_back(kSpecialNames[k], (uint16_t)want);
        t.bytes[(size_t)want] = kSpecialNames[k];
    }
    return {};
}

Rejection build(const io::Json& j, Tokenizer& t) {
    int vocab = 0;
    if (Rejection r = read_header(j, vocab))
        return r;
    t.vocab = vocab;
    MergeBuilder merges(t, vocab);
    for (const io::Json& m : j.at("merges").array())
        if (Rejection r = merges.add(m))
            return r;
    return read_specials(j, vocab, t);
}

}  // namespace

// Tokenizer::load (tokenizer.cpp:70-127): the file's bytes are its identity; JSON that
// does not parse, or lacks a field or has one of the wrong type, is invalid_argument.
int tokenizer_load(const std::string& path, Tokenizer& t) {
    std::string text, err;
    if (!io::read_file(path, text, err))
        return fail(MLA_ERR_IO, err);
    Tokenizer built;
    Rejection r;
    try {
        r = build(io::JsonReader(text).parse(), built);
    } catch (const std::exception& e) {
        r = invalid(e.what());
    }
    if (r)
        return fail(r.code, r.message);
    built.hash = io::sha256_hex(text);
    t = std::move(built);
    return MLA_OK;
}

bool tokenizer_decode(const Tokenizer& t, const uint16_t* ids, size_t n, bool skip_special,
                      std::string& out) {
    out.clear();
    for (size_t k = 0; k < n; ++k) {
        const uint16_t id = ids[k];
        if (id >= t.bytes.size() || t.bytes[id].empty())
            return false;
        if (!skip_special || id < t.vocab - 8)  // the specials are the last eight ids
            out += t.bytes[id];
    }
    return true;
}

int tokenizer_special(const Tokenizer& t, const std::string& name) {
    for (const auto& [n, sid] : t.specials)
        if (n == name)
            return sid;
    return -1;
}

namespace {

// Ranked BPE over one run of bytes.  Every adjacent pair that has a merge is a candidate
// keyed by (merged id, left position); the smallest key is merged first.  A merged id is
// always larger than both of its parts' ids (merges reference earlier ids only), so a
// merge never creates a candidate that ranks before the one just taken, and taking the
// smallest key each time applies the merges in id order, leftmost first within an id.
void encode_run(const Tokenizer& t, const char* s, size_t n, std::vector<uint16_t>& out) {
    if (t.merges.empty()) {
        for (size_t i = 0; i < n; ++i)
            out.push_back((uint8_t)s[i]);
        return;
    }
    const size_t none = (size_t)-1;
    std::vector<uint16_t> id(n);
    std::vector<size_t> next(n), prev(n);
    std::vector<int> cand(n, -1);  // merged id of the pair starting here, -1 for none
    for (size_t i = 0; i < n; ++i) {
        id[i] = (uint8_t)s[i];
        next[i] = i + 1 < n ? i + 1 : none;
        prev[i] = i ? i - 1 : none;
    }
    std::set<std::pair<int, size_t>> agenda;
    auto refresh = [&](size_t i) {
        if (i == none)
            return;
        if (cand[i] >= 0)
            agenda.erase({cand[i], i});
        cand[i] = -1;
        if (next[i] == none)
            return;
        auto it = t.merges.find((uint32_t)id[i] << 16 | id[next[i]]);
        if (it != t.merges.end()) {
            cand[i] = it->second;
            agenda.insert({cand[i], i});
        }
    };
    for (size_t i = 0; i < n; ++i)
        refresh(i);
    while (!agenda.empty()) {
        const auto [merged, i] = *agenda.begin();
        agenda.erase(agenda.begin());
        cand[i] = -1;
        const size_t r = next[i];
        if (cand[r] >= 0) {  // the right part's own pair disappears with it
            agenda.erase({cand[r], r});
            cand[r] = -1;
        }
        id[i] = (uint16_t)merged;
        next[i] = next[r];
        if (next[r] != none)
            prev[next[r]] = i;
        refresh(prev[i]);
        refresh(i);
    }
    for (size_t i = 0; n && i != none; i = next[i])
        out.push_back(id[i]);
}

// Tokenizer::encode (tokenizer.cpp:183-205): with allow_special, a special token's exact
// spelling becomes its id; everything else is bytes merged by encode_run.
std::vector<uint16_t> encode(const Tokenizer& t, const char* s, size_t n, bool allow_special) {
    std::vector<uint16_t> out;
    if (!allow_special) {
        encode_run(t, s, n, out);
        return out;
    }
    size_t begin = 0, i = 0;
    while (i < n) {
        bool hit = false;
        if (s[i] == '<')
            for (const auto& [name, sid] : t.specials)
                if (n - i >= name.size() && std::memcmp(s + i, name.data(), name.size()) == 0) {
                    encode_run(t, s + begin, i - begin, out);
                    out.push_back(sid);
                    i += name.size();
                    begin = i;
                    hit = true;
                    break;
                }
        if (!hit)
            ++i;
    }
    encode_run(t, s + begin, n - begin, out);
    return out;
}

}  // namespace
}  // namespace mla

using namespace mla;

extern "C" {

int mla_tokenizer_load(const char* path, void** tokenizer) {
    if (!path || !tokenizer)
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_tokenizer_load: null argument");
    auto t = std::make_unique<Tokenizer>();
    const int st = tokenizer_load(path, *t);
    if (st != MLA_OK)
        return st;
    *tokenizer = t.release();
    return MLA_OK;
}

int mla_tokenizer_destroy(void* tokenizer) {
    delete static_cast<Tokenizer*>(tokenizer);
    return MLA_OK;
}

int mla_tokenizer_info(void* tokenizer, int* vocab_size, char* sha256_hex) {
    const Tokenizer* t = static_cast<Tokenizer*>(tokenizer);
    if (!t || !vocab_size || !sha256_hex)
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_tokenizer_info: null argument");
    *vocab_size = t->vocab;
    std::memcpy(sha256_hex, t->hash.c_str(), 65);
    return MLA_OK;
}

int mla_tokenizer_special(void* tokenizer, const char* name, uint16_t* id) {
    const Tokenizer* t = static_cast<Tokenizer*>(tokenizer);
    if (!t || !name || !id)
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_tokenizer_special: null argument");
    const int sid = tokenizer_special(*t, name);
    if (sid < 0)
        return fail(MLA_ERR_INVALID_ARGUMENT, "Unknown special token");
    *id = (uint16_t)sid;
    return MLA_OK;
}

int mla_tokenizer_encode(void* tokenizer, const char* text, size_t len, int allow_special,
                         uint16_t* ids, size_t capacity, size_t* n_ids) {
    const Tokenizer* t = static_cast<Tokenizer*>(tokenizer);
    if (!t || (!text && len) || !n_ids)
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_tokenizer_encode: null argument");
    const std::vector<uint16_t> out = encode(*t, text ? text : "", len, allow_special != 0);
    *n_ids = out.size();
    if (!ids)
        return MLA_OK;  // size query
    if (capacity < out.size())
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_tokenizer_encode: needs " +
                                                  std::to_string(out.size()) + " ids");
    if (!out.empty())
        std::memcpy(ids, out.data(), out.size() * sizeof(uint16_t));
    return MLA_OK;
}

int mla_tokenizer_decode(void* tokenizer, const uint16_t* ids, size_t n, int skip_special,
                         char* text, size_t capacity, size_t* len) {
    const Tokenizer* t = static_cast<Tokenizer*>(tokenizer);
    if (!t || (!ids && n) || !len)
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_tokenizer_decode: null argument");
    std::string out;
    if (!tokenizer_decode(*t, ids, n, skip_special != 0, out))
        return fail(MLA_ERR_INVALID_ARGUMENT, "Unknown token ID");
    *len = out.size();
    if (!text)
        return MLA_OK;  // size query
    if (capacity < out.size())
        return fail(MLA_ERR_INVALID_ARGUMENT,
                    "mla_tokenizer_decode: needs " + std::to_string(out.size()) + " bytes");
    if (!out.empty())
        std::memcpy(text, out.data(), out.size());
    return MLA_OK;
}

}  // extern "C"
