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
// Tokenizer::decode (tokenizer.cpp:206-218): false on an id with no bytes ("Unknown token
// ID"); with skip_special the eight special tokens are left out.
bool tokenizer_decode(const Tokenizer& t, const uint16_t* ids, size_t n, bool skip_special,
                      std::string& out);
// Tokenizer::special (tokenizer.cpp:219-224): the id of a special token's name, -1 if none.
int tokenizer_special(const Tokenizer& t, const std::string& name);

}  // namespace mla
