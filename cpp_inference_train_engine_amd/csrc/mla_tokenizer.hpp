// The reference's byte-level BPE tokenizer (src/infer/tokenizer.cpp), host side.
#pragma once

#include <cstdint>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

namespace mla {

struct Tokenizer {
    int vocab = 0;
    std::vector<std::string> bytes;                        // token id -> its bytes
    std::unordered_map<uint32_t, uint16_t> merges;         // (left << 16 | right) -> id
    std::vector<std::pair<std::string, uint16_t>> specials;  // the eight role tokens
    std::string hash;                                      // SHA-256 of the file bytes
};

// Tokenizer::load (tokenizer.cpp:70-127): MLA_OK, or the reference's code and message
// (recorded as this thread's last error).
int tokenizer_load(const std::string& path, Tokenizer& t);

}  // namespace mla
