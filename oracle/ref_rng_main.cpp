// Driver for the reference's header-only Rng (include/mini_mla/rng.hpp:7-38).
// Built into oracle/_ref/rng_ref straight from the reference checkout; prints
// known-answer vectors that pin oracle/mla_oracle.c's Rng restatement.
// TEST INFRASTRUCTURE ONLY.
#include "mini_mla/rng.hpp"

#include <cstdio>
#include <cstdlib>
#include <cstring>

int main(int argc, char** argv) {
    if (argc != 5) {
        std::fprintf(stderr, "usage: rng_ref next|uniform|normal|bounded SEED COUNT BOUND\n");
        return 2;
    }
    mini_mla::Rng rng(std::strtoull(argv[2], nullptr, 10));
    const long count = std::strtol(argv[3], nullptr, 10);
    const unsigned long long bound = std::strtoull(argv[4], nullptr, 10);
    for (long i = 0; i < count; ++i) {
        if (!std::strcmp(argv[1], "next"))
            std::printf("%llu\n", static_cast<unsigned long long>(rng.next()));
        else if (!std::strcmp(argv[1], "uniform"))
            std::printf("%.9g\n", static_cast<double>(rng.uniform()));
        else if (!std::strcmp(argv[1], "normal"))
            std::printf("%.9g\n", static_cast<double>(rng.normal()));
        else
            std::printf("%llu\n", static_cast<unsigned long long>(rng.bounded(bound)));
    }
    return 0;
}
