// Token selection and the per-request generation loop of the reference
// (src/infer/inference.cpp:330-579), host side: GenerationConfig and its checks,
// sample_token (greedy with bans and repetition penalty; temperature, top-k and top-p
// sampling from the seeded SplitMix64 stream), the banned-token list of
// InferenceEngine::load, and generate_tokens' loop as a state machine driven one set of
// logits at a time, so that one session or a continuous batch can run it.
#pragma once

#include "mla_hip.h"
#include "mla_tokenizer.hpp"

#include <cstddef>
#include <cstdint>
#include <functional>
#include <string>
#include <string_view>
#include <vector>

namespace mla {

// GenerationConfig (include/mini_mla/inference.hpp:27-34), with the reference's defaults.
struct GenConfig {
    int max_new_tokens = 128, top_k = 0;
    float temperature = 0.8f, top_p = 0.95f, repetition_penalty = 1.0f;
    uint64_t seed = 42;
    std::vector<std::string> stop;
    std::vector<std::vector<uint16_t>> stop_tokens;
};

// GenerationConfig::validate (inference.cpp:330-344): MLA_OK or the reference's message.
int validate(const GenConfig& c);
// The C form of a configuration (mla_generation_config) into a GenConfig; not validated.
int gen_config_from_c(const mla_generation_config* in, GenConfig& c);

// Rng::next / Rng::uniform (include/mini_mla/rng.hpp): SplitMix64, and a float in (0, 1)
// from the top 24 bits.
struct SplitMix64 {
    uint64_t state;
    uint64_t next() {
        uint64_t z = (state += 0x9e3779b97f4a7c15ULL);
        z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
        z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
        return z ^ (z >> 31);
    }
    float uniform() { return ((float)(next() >> 40) + 0.5f) / 16777216.0f; }
};

// sample_token (inference.cpp:345-412).  history: the prompt and the tokens generated so
// far; banned ids never win.  MLA_OK with `token`, or MLA_ERR_NUMERICAL ("Invalid
// sampler logits") / MLA_ERR_INVALID_ARGUMENT (settings, "All tokens are banned").
int sample_token(const float* logits, size_t vocab, const uint16_t* history, size_t n_history,
                 const GenConfig& c, SplitMix64& rng, const uint16_t* banned, size_t n_banned,
                 uint16_t& token);

// The ids InferenceEngine::load bans (inference.cpp:441-447): the special tokens other
// than <|eos|>, and the ids with no bytes.
std::vector<uint16_t> banned_tokens(const Tokenizer& t);

// clean_utf8 (tokenizer.cpp:13-57): each byte that starts no valid UTF-8 sequence
// becomes U+FFFD.
std::string clean_utf8(std::string_view s);
// stream_prefix (inference.cpp:253-263): the longest prefix of s[0, limit) that ends on a
// sequence boundary, judged from lead bytes.
size_t stream_prefix(std::string_view s, size_t limit);

// generate_tokens (inference.cpp:469-579) one token at a time.  start() makes the checks
// the reference makes before its prefill; the driver then runs the prompt and passes the
// last position's logits to step(), which samples, applies the stop rules, streams text
// through the callback (text "" asks whether to go on; false cancels) and returns the
// token to decode next, or -1 once the generation has finished.
class Generation {
  public:
    using Callback = std::function<bool(std::string_view)>;
    int start(const Tokenizer& t, const GenConfig& c, const uint16_t* prompt, size_t n,
              int max_sequence_length, const std::vector<uint16_t>* banned, Callback cb);
    int step(const float* logits, size_t vocab, int32_t* next);
    // step() for a token already chosen by the device's greedy rule: only valid when
    // greedy_on_device() (temperature 0 and no repetition penalty, where the choice does
    // not depend on the history).
    int step_token(uint16_t token, int32_t* next);
    bool greedy_on_device() const { return c_.temperature == 0.0f && c_.repetition_penalty == 1.0f; }
    bool finished() const { return done_; }
    const std::vector<uint16_t>& tokens() const { return tokens_; }
    const std::string& text() const { return text_; }
    const std::string& finish_reason() const { return reason_; }
    size_t prompt_tokens() const { return prompt_tokens_; }

  private:
    bool go_on(std::string_view text);
    int advance(uint16_t token, int32_t* next);
    void finish();

    const Tokenizer* t_ = nullptr;
    GenConfig c_;
    const std::vector<uint16_t>* banned_ = nullptr;
    Callback cb_;
    SplitMix64 rng_{42};
    std::vector<uint16_t> history_, tokens_;
    std::string text_, reason_ = "length";
    size_t hold_ = 0, emitted_ = 0, prompt_tokens_ = 0;
    int eos_ = -1;
    bool done_ = false;
};

}  // namespace mla
