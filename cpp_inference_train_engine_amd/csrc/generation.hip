// Token selection and the generation loop (src/infer/inference.cpp:330-579), host code.
// The greedy rule here is the one the device applies in the logits kernel (lowest id
// among the maxima of the ids not banned); this copy serves the cases the device rule
// does not cover (repetition penalty, temperature sampling) and drivers that hold host
// logits.
#include "mla_capi_util.hpp"
#include "mla_generation.hpp"
#include "mla_hip.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <limits>
#include <memory>

namespace mla {

int validate(const GenConfig& c) {
    if (c.max_new_tokens < 0 || c.max_new_tokens > 65535 || c.top_k < 0 ||
        !std::isfinite(c.temperature) || c.temperature < 0 || !std::isfinite(c.top_p) ||
        c.top_p <= 0 || c.top_p > 1 || !std::isfinite(c.repetition_penalty) ||
        c.repetition_penalty <= 0)
        return fail(MLA_ERR_INVALID_ARGUMENT, "Invalid generation settings");
    for (const std::string& s : c.stop)
        if (s.empty() || s.size() > 4096)
            return fail(MLA_ERR_INVALID_ARGUMENT, "Stop strings must be nonempty and <=4096 bytes");
    for (const auto& s : c.stop_tokens)
        if (s.empty())
            return fail(MLA_ERR_INVALID_ARGUMENT, "Stop token sequences must be nonempty");
    return MLA_OK;
}

namespace {
float penalised(float score, float penalty) {
    return score > 0 ? score / penalty : score * penalty;
}

// One 64-bit key per id whose ascending order is sample_token's order: higher score
// first, then lower id (-0 and +0 tie, as they compare equal).
uint64_t order_key(float score, uint16_t id) {
    if (score == 0.0f)
        score = 0.0f;
    uint32_t u;
    std::memcpy(&u, &score, sizeof(u));
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);  // ascending in the score
    return ((uint64_t)~u << 16) | id;
}

// LSD radix sort of 48-bit keys, 12 bits per pass.
void radix_sort48(std::vector<uint64_t>& keys, std::vector<uint64_t>& tmp) {
    constexpr int kBits = 12, kBuckets = 1 << kBits;
    tmp.resize(keys.size());
    std::vector<uint32_t> count(kBuckets);
    for (int shift = 0; shift < 48; shift += kBits) {
        std::fill(count.begin(), count.end(), 0u);
        for (const uint64_t k : keys)
            ++count[(k >> shift) & (kBuckets - 1)];
        uint32_t sum = 0;
        for (uint32_t& c : count) {
            const uint32_t n = c;
            c = sum;
            sum += n;
        }
        for (const uint64_t k : keys)
            tmp[count[(k >> shift) & (kBuckets - 1)]++] = k;
        keys.swap(tmp);
    }
}
}  // namespace

int sample_token(const float* logits, size_t vocab, const uint16_t* history, size_t n_history,
                 const GenConfig& c, SplitMix64& rng, const uint16_t* banned, size_t n_banned,
                 uint16_t& token) {
    if (const int st = validate(c))
        return st;
    if (vocab == 0 || vocab > 65535 || !logits)
        return fail(MLA_ERR_NUMERICAL, "Invalid sampler logits");
    for (size_t i = 0; i < vocab; ++i)
        if (!std::isfinite(logits[i]))
            return fail(MLA_ERR_NUMERICAL, "Invalid sampler logits");
    const bool penalty = c.repetition_penalty != 1.0f;
    if (c.temperature == 0) {
        // Greedy: the first id with the largest (penalised) score among those not banned.
        std::vector<char> skip(n_banned ? vocab : 0, 0), repeated(penalty ? vocab : 0, 0);
        for (size_t k = 0; k < n_banned; ++k)
            if (banned[k] < vocab)
                skip[banned[k]] = 1;
        for (size_t k = 0; penalty && k < n_history; ++k)
            if (history[k] < vocab)
                repeated[history[k]] = 1;
        size_t best = vocab;
        float top = -std::numeric_limits<float>::infinity();
        for (size_t i = 0; i < vocab; ++i) {
            if (n_banned && skip[i])
                continue;
            const float score = penalty && repeated[i] ? penalised(logits[i], c.repetition_penalty)
                                                       : logits[i];
            if (best == vocab || score > top) {
                best = i;
                top = score;
            }
        }
        if (best == vocab)
            return fail(MLA_ERR_INVALID_ARGUMENT, "All tokens are banned");
        token = (uint16_t)best;
        return MLA_OK;
    }
    // Sampling: penalise each id of the history once, drop banned ids, order the rest by
    // score (ties: lower id first), keep the top_k, then the smallest prefix whose
    // probability mass reaches top_p of the kept ones' total, and draw from it.
    std::vector<float> score(logits, logits + vocab);
    if (penalty) {
        std::vector<char> seen(vocab, 0);
        for (size_t k = 0; k < n_history; ++k)
            if (history[k] < vocab && !seen[history[k]]) {
                seen[history[k]] = 1;
                score[history[k]] = penalised(score[history[k]], c.repetition_penalty);
            }
    }
    for (size_t k = 0; k < n_banned; ++k)
        if (banned[k] < vocab)
            score[banned[k]] = -std::numeric_limits<float>::infinity();
    // The order is a strict total order, so the first top_k ids are the same whichever
    // selection or sorting algorithm finds them.
    thread_local std::vector<uint64_t> keys, tmp;
    keys.clear();
    for (size_t i = 0; i < vocab; ++i)
        if (std::isfinite(score[i]))
            keys.push_back(order_key(score[i], (uint16_t)i));
    if (keys.empty())
        return fail(MLA_ERR_INVALID_ARGUMENT, "All tokens are banned");
    if (c.top_k > 0 && (size_t)c.top_k < keys.size()) {
        std::partial_sort(keys.begin(), keys.begin() + c.top_k, keys.end());
        keys.resize((size_t)c.top_k);
    } else {
        radix_sort48(keys, tmp);
    }
    thread_local std::vector<uint16_t> order;
    thread_local std::vector<double> prob;
    order.resize(keys.size());
    prob.resize(keys.size());
    for (size_t i = 0; i < keys.size(); ++i)
        order[i] = (uint16_t)(keys[i] & 0xffff);
    // exp of an argument below -746 is 0 in double precision; skipping the call for
    // those terms leaves every probability and the sum unchanged.
    const float top = score[order[0]];
    double sum = 0;
    for (size_t i = 0; i < order.size(); ++i) {
        const double z = (double)(score[order[i]] - top) / c.temperature;
        prob[i] = z < -746.0 ? 0.0 : std::exp(z);
        sum += prob[i];
    }
    double kept = 0;
    size_t count = 0;
    do {
        kept += prob[count++];
    } while (count < order.size() && kept < (double)c.top_p * sum);
    double draw = (double)rng.uniform() * kept;
    for (size_t i = 0; i < count; ++i) {
        draw -= prob[i];
        if (draw <= 0) {
            token = order[i];
            return MLA_OK;
        }
    }
    token = order[count - 1];
    return MLA_OK;
}

std::vector<uint16_t> banned_tokens(const Tokenizer& t) {
    std::vector<uint16_t> out;
    const int eos = tokenizer_special(t, "<|eos|>");
    for (int i = 0; i < t.vocab; ++i)
        if ((i >= t.vocab - 8 && i != eos) || t.bytes[(size_t)i].empty())
            out.push_back((uint16_t)i);
    return out;
}

namespace {
// Length of the valid UTF-8 sequence at s[i], 0 when none (no overlong forms, no
// surrogates, nothing above U+10FFFF).
size_t utf8_length(std::string_view s, size_t i) {
    const unsigned c = (unsigned char)s[i];
    if (c < 0x80)
        return 1;
    const size_t n = c >= 0xc2 && c <= 0xdf ? 2 : c >= 0xe0 && c <= 0xef ? 3 : c >= 0xf0 && c <= 0xf4 ? 4 : 0;
    if (!n || i + n > s.size())
        return 0;
    for (size_t k = 1; k < n; ++k) {
        const unsigned b = (unsigned char)s[i + k];
        if (b < 0x80 || b > 0xbf)
            return 0;
    }
    const unsigned b = (unsigned char)s[i + 1];
    if ((c == 0xe0 && b < 0xa0) || (c == 0xed && b >= 0xa0) || (c == 0xf0 && b < 0x90) ||
        (c == 0xf4 && b >= 0x90))
        return 0;
    return n;
}
}  // namespace

std::string clean_utf8(std::string_view s) {
    std::string out;
    out.reserve(s.size());
    for (size_t i = 0; i < s.size();) {
        const size_t n = utf8_length(s, i);
        if (n) {
            out.append(s.substr(i, n));
            i += n;
        } else {
            out += "\xef\xbf\xbd";
            ++i;
        }
    }
    return out;
}

size_t stream_prefix(std::string_view s, size_t limit) {
    size_t i = 0;
    while (i < limit) {
        const unsigned c = (unsigned char)s[i];
        const size_t n = c < 0xc0 ? 1 : c < 0xe0 ? 2 : c < 0xf0 ? 3 : c <= 0xf4 ? 4 : 1;
        if (i + n > limit)
            break;
        i += n;
    }
    return i;
}

int Generation::start(const Tokenizer& t, const GenConfig& c, const uint16_t* prompt, size_t n,
                      int max_sequence_length, const std::vector<uint16_t>* banned, Callback cb) {
    if (const int st = validate(c))
        return st;
    if (n == 0 || n + (size_t)c.max_new_tokens > (size_t)std::max(max_sequence_length, 0))
        return fail(MLA_ERR_INVALID_ARGUMENT, "Prompt plus requested tokens exceeds context");
    size_t hold = 0;
    for (const std::string& s : c.stop)
        hold = std::max(hold, s.size());
    for (const auto& seq : c.stop_tokens) {
        size_t bytes = 0;
        for (const uint16_t tok : seq) {
            if (tok >= t.vocab)
                return fail(MLA_ERR_INVALID_ARGUMENT, "Stop token exceeds vocabulary");
            bytes += t.bytes[tok].size();
        }
        hold = std::max(hold, bytes);
    }
    t_ = &t;
    c_ = c;
    banned_ = banned;
    cb_ = std::move(cb);
    rng_.state = c.seed;
    history_.assign(prompt, prompt + n);
    tokens_.clear();
    text_.clear();
    reason_ = "length";
    hold_ = hold;
    emitted_ = 0;
    prompt_tokens_ = n;
    eos_ = tokenizer_special(t, "<|eos|>");
    done_ = false;
    if (c.max_new_tokens == 0)
        finish();
    return MLA_OK;
}

bool Generation::go_on(std::string_view text) { return !cb_ || cb_(text); }

int Generation::step(const float* logits, size_t vocab, int32_t* next) {
    if (!t_ || done_)
        return fail(MLA_ERR_INVALID_ARGUMENT, "generation step: not running");
    if (!go_on({})) {
        reason_ = "cancelled";
        finish();
        *next = -1;
        return MLA_OK;
    }
    uint16_t token = 0;
    const int st = sample_token(logits, vocab, history_.data(), history_.size(), c_, rng_,
                                banned_ ? banned_->data() : nullptr, banned_ ? banned_->size() : 0,
                                token);
    if (st) {
        done_ = true;
        return st;
    }
    return advance(token, next);
}

int Generation::step_token(uint16_t token, int32_t* next) {
    if (!t_ || done_ || !greedy_on_device() || token >= t_->vocab)
        return fail(MLA_ERR_INVALID_ARGUMENT, "generation step: not running");
    if (!go_on({})) {
        reason_ = "cancelled";
        finish();
        *next = -1;
        return MLA_OK;
    }
    return advance(token, next);
}

int Generation::advance(uint16_t token, int32_t* next) {
    *next = -1;
    tokens_.push_back(token);
    history_.push_back(token);
    if (token == eos_) {
        reason_ = "stop";
        finish();
        return MLA_OK;
    }
    const auto ends_with = [&](const std::vector<uint16_t>& seq) {
        return tokens_.size() >= seq.size() &&
               std::equal(seq.rbegin(), seq.rend(), tokens_.rbegin());
    };
    for (const auto& seq : c_.stop_tokens)
        if (ends_with(seq)) {
            // The whole text again without special tokens, less the sequence's own text.
            if (!tokenizer_decode(*t_, tokens_.data(), tokens_.size(), true, text_)) {
                done_ = true;
                return fail(MLA_ERR_INVALID_ARGUMENT, "Unknown token ID");
            }
            std::string tail;
            if (tokenizer_decode(*t_, seq.data(), seq.size(), true, tail) &&
                tail.size() <= text_.size())
                text_.resize(text_.size() - tail.size());
            reason_ = "stop";
            finish();
            return MLA_OK;
        }
    text_ += t_->bytes[token];
    bool stopped = false;
    for (const std::string& s : c_.stop) {  // the first listed stop string that occurs
        const size_t p = text_.find(s);
        if (p != std::string::npos) {
            text_.resize(p);
            reason_ = "stop";
            stopped = true;
            break;
        }
    }
    // Text that a later stop string or stop sequence could still remove is held back.
    const size_t limit = stopped ? text_.size() : text_.size() > hold_ ? text_.size() - hold_ : 0;
    const size_t safe = stream_prefix(text_, limit);
    if (cb_ && safe > emitted_) {
        if (!cb_(clean_utf8(std::string_view(text_).substr(emitted_, safe - emitted_)))) {
            reason_ = "cancelled";
            finish();
            return MLA_OK;
        }
        emitted_ = safe;
    }
    if (stopped || tokens_.size() >= (size_t)c_.max_new_tokens) {
        finish();
        return MLA_OK;
    }
    *next = token;
    return MLA_OK;
}

void Generation::finish() {
    if (cb_ && reason_ != "cancelled" && text_.size() > emitted_ &&
        !cb_(clean_utf8(std::string_view(text_).substr(emitted_))))
        reason_ = "cancelled";
    text_ = clean_utf8(text_);
    done_ = true;
}

int gen_config_from_c(const mla_generation_config* in, GenConfig& c) {
    if (!in)
        return fail(MLA_ERR_INVALID_ARGUMENT, "generation config: null");
    c = GenConfig();
    c.max_new_tokens = in->max_new_tokens;
    c.top_k = in->top_k;
    c.temperature = in->temperature;
    c.top_p = in->top_p;
    c.repetition_penalty = in->repetition_penalty;
    c.seed = in->seed;
    if (in->n_stop < 0 || in->n_stop_tokens < 0 || (in->n_stop && (!in->stop || !in->stop_len)) ||
        (in->n_stop_tokens && (!in->stop_tokens_len || !in->stop_tokens)))
        return fail(MLA_ERR_INVALID_ARGUMENT, "generation config: null stop list");
    for (int i = 0; i < in->n_stop; ++i) {
        if (!in->stop[i] && in->stop_len[i])
            return fail(MLA_ERR_INVALID_ARGUMENT, "generation config: null stop string");
        c.stop.emplace_back(in->stop[i] ? in->stop[i] : "", in->stop_len[i]);
    }
    size_t at = 0;
    for (int i = 0; i < in->n_stop_tokens; ++i) {
        if (in->stop_tokens_len[i] < 0)
            return fail(MLA_ERR_INVALID_ARGUMENT, "generation config: negative stop length");
        c.stop_tokens.emplace_back(in->stop_tokens + at, in->stop_tokens + at + in->stop_tokens_len[i]);
        at += (size_t)in->stop_tokens_len[i];
    }
    return MLA_OK;
}

namespace {
struct CGeneration {
    const Tokenizer* tok = nullptr;
    std::vector<uint16_t> banned;
    Generation gen;
};
}  // namespace

}  // namespace mla

using namespace mla;

extern "C" {

void mla_generation_config_init(mla_generation_config* c) {
    if (!c)
        return;
    std::memset(c, 0, sizeof(*c));
    const GenConfig d;
    c->max_new_tokens = d.max_new_tokens;
    c->top_k = d.top_k;
    c->temperature = d.temperature;
    c->top_p = d.top_p;
    c->repetition_penalty = d.repetition_penalty;
    c->seed = d.seed;
}

int mla_generation_config_validate(const mla_generation_config* config) {
    GenConfig c;
    if (const int st = gen_config_from_c(config, c))
        return st;
    return validate(c);
}

int mla_sample_token(const float* logits, size_t vocab, const uint16_t* history,
                     size_t n_history, const mla_generation_config* config, uint64_t* rng_state,
                     const uint16_t* banned, size_t n_banned, uint16_t* token) {
    if (!rng_state || !token || (!history && n_history) || (!banned && n_banned))
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_sample_token: null argument");
    GenConfig c;
    if (const int st = gen_config_from_c(config, c))
        return st;
    SplitMix64 rng{*rng_state};
    const int st = sample_token(logits, vocab, history, n_history, c, rng, banned, n_banned, *token);
    *rng_state = rng.state;
    return st;
}

int mla_tokenizer_banned(void* tokenizer, uint16_t* ids, size_t capacity, size_t* n) {
    const Tokenizer* t = static_cast<Tokenizer*>(tokenizer);
    if (!t || !n)
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_tokenizer_banned: null argument");
    const std::vector<uint16_t> b = banned_tokens(*t);
    *n = b.size();
    if (!ids)
        return MLA_OK;
    if (capacity < b.size())
        return fail(MLA_ERR_INVALID_ARGUMENT,
                    "mla_tokenizer_banned: needs " + std::to_string(b.size()) + " ids");
    std::memcpy(ids, b.data(), b.size() * sizeof(uint16_t));
    return MLA_OK;
}

int mla_generation_create(void* tokenizer, const mla_generation_config* config,
                          const uint16_t* prompt, size_t n, int max_sequence_length,
                          mla_text_callback callback, void* user, void** generation) {
    const Tokenizer* t = static_cast<Tokenizer*>(tokenizer);
    if (!t || !generation || (!prompt && n))
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_generation_create: null argument");
    GenConfig c;
    if (const int st = gen_config_from_c(config, c))
        return st;
    auto g = std::make_unique<CGeneration>();
    g->tok = t;
    g->banned = banned_tokens(*t);
    Generation::Callback cb;
    if (callback)
        cb = [callback, user](std::string_view s) { return callback(user, s.data(), s.size()) != 0; };
    if (const int st = g->gen.start(*t, c, prompt, n, max_sequence_length, &g->banned, std::move(cb)))
        return st;
    *generation = g.release();
    return MLA_OK;
}

int mla_generation_step(void* generation, const float* logits, size_t vocab, int32_t* next_token) {
    CGeneration* g = static_cast<CGeneration*>(generation);
    if (!g || !next_token)
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_generation_step: null argument");
    return g->gen.step(logits, vocab, next_token);
}

int mla_generation_result(void* generation, char* text, size_t text_capacity, size_t* text_len,
                          uint16_t* tokens, size_t tokens_capacity, size_t* n_tokens,
                          char* finish_reason) {
    const CGeneration* g = static_cast<CGeneration*>(generation);
    if (!g || !text_len || !n_tokens)
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_generation_result: null argument");
    const Generation& r = g->gen;
    *text_len = r.text().size();
    *n_tokens = r.tokens().size();
    if (finish_reason) {
        std::memset(finish_reason, 0, 16);
        std::memcpy(finish_reason, r.finish_reason().data(), std::min<size_t>(15, r.finish_reason().size()));
    }
    if (text) {
        if (text_capacity < r.text().size())
            return fail(MLA_ERR_INVALID_ARGUMENT, "mla_generation_result: text buffer too small");
        std::memcpy(text, r.text().data(), r.text().size());
    }
    if (tokens) {
        if (tokens_capacity < r.tokens().size())
            return fail(MLA_ERR_INVALID_ARGUMENT, "mla_generation_result: token buffer too small");
        std::memcpy(tokens, r.tokens().data(), r.tokens().size() * sizeof(uint16_t));
    }
    return MLA_OK;
}

int mla_generation_finished(void* generation) {
    const CGeneration* g = static_cast<CGeneration*>(generation);
    return g && g->gen.finished() ? 1 : 0;
}

int mla_generation_destroy(void* generation) {
    delete static_cast<CGeneration*>(generation);
    return MLA_OK;
}

}  // extern "C"
