// Compares hf::glibc_expf and hf::router_sigmoid with the C library's expf and
// 1.0f / (1.0f + expf(-x)) (moe_router.h:19-21) over a range of float bit
// patterns, in parallel.
//   check table           -> prints the 32 table entries (hex), one a line
//   check exhaustive      -> every float (NaN aside): "<checked> <expf_bad> <sigmoid_bad> <first_bad_bits>"
//   check range LO HI     -> bit patterns LO..HI-1 only (same output)
//   check cr LO HI        -> as range, with a correctly rounded exp,
//                            (float)exp((double)x), in place of hf::glibc_expf:
//                            a planted mistake the comparison must catch
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "hf_expf.h"

static float bits_to_float(uint32_t u) {
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}
static uint32_t float_bits(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    return u;
}

int main(int argc, char** argv) {
    if (argc >= 2 && !std::strcmp(argv[1], "table")) {
        for (int i = 0; i < 32; ++i) std::printf("%016llx\n", (unsigned long long)hf::expf_detail::kTab[i]);
        return 0;
    }
    uint64_t lo = 0, hi = 1ull << 32;
    const bool cr = argc >= 2 && !std::strcmp(argv[1], "cr");
    if (argc >= 4 && (!std::strcmp(argv[1], "range") || cr)) {
        lo = std::strtoull(argv[2], nullptr, 0);
        hi = std::strtoull(argv[3], nullptr, 0);
    } else if (argc < 2 || std::strcmp(argv[1], "exhaustive")) {
        std::fprintf(stderr, "usage: check table | exhaustive | range LO HI\n");
        return 2;
    }
    long long checked = 0, bad_exp = 0, bad_sig = 0;
    uint64_t first_bad = ~0ull;
#pragma omp parallel for schedule(static) reduction(+ : checked, bad_exp, bad_sig) reduction(min : first_bad)
    for (long long i = (long long)lo; i < (long long)hi; ++i) {
        const float x = bits_to_float((uint32_t)i);
        if (x != x) continue;
        ++checked;
        const float e_lib = expf(x);
        const float e_hf = cr ? (float)std::exp((double)x) : hf::glibc_expf(x);
        const float s_lib = 1.0f / (1.0f + expf(-x));
        const float s_hf = cr ? (float)(1.0 / (double)(1.0f + (float)std::exp(-(double)x))) : hf::router_sigmoid(x);
        const bool be = float_bits(e_lib) != float_bits(e_hf);
        const bool bs = float_bits(s_lib) != float_bits(s_hf);
        bad_exp += be;
        bad_sig += bs;
        if ((be || bs) && (uint64_t)i < first_bad) first_bad = (uint64_t)i;
    }
    std::printf("%lld %lld %lld %llx\n", checked, bad_exp, bad_sig, (unsigned long long)first_bad);
    return 0;
}
