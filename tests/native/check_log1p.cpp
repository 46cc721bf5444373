// Exhaustive host check: npa_log1pf (burn_automata_amd/csrc/npa_math.hpp) against the host libm's
// log1pf for every float bit pattern in [lo_bits, hi_bits] (default: all of [+0, +inf]). Prints the mismatch count and the
// first mismatching inputs. Build: g++ -O2 -std=c++17 -fopenmp -ffp-contract=off.
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../../burn_automata_amd/csrc/npa_math.hpp"

static float from_bits(uint32_t b) { float f; memcpy(&f, &b, 4); return f; }
static uint32_t to_bits(float f) { uint32_t b; memcpy(&b, &f, 4); return b; }

int main(int argc, char** argv) {
    uint32_t lo = argc > 1 ? (uint32_t)strtoul(argv[1], 0, 0) : 0u;
    uint32_t hi = argc > 2 ? (uint32_t)strtoul(argv[2], 0, 0) : 0x7f800000u;
    unsigned long long bad = 0;
    uint32_t first[16];
    int nf = 0;
#pragma omp parallel for schedule(dynamic, 1 << 16) reduction(+ : bad)
    for (long long b = lo; b <= (long long)hi; ++b) {
        float x = from_bits((uint32_t)b);
        float a = npa::npa_log1pf(x), c = log1pf(x);
        if (to_bits(a) != to_bits(c) && !(a != a && c != c)) {
            bad++;
#pragma omp critical
            if (nf < 16) first[nf++] = (uint32_t)b;
        }
    }
    printf("range 0x%08x..0x%08x mismatches %llu\n", lo, hi, bad);
    for (int k = 0; k < nf; ++k) {
        float x = from_bits(first[k]);
        printf("  x=%a (%.9g): npa=%a libm=%a\n", x, x, npa::npa_log1pf(x), log1pf(x));
    }
    return bad ? 1 : 0;
}
