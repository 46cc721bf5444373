// npa_math.hpp - float log1p with the host libm's exact results, identical on host and device.
//
// The perception's log-normalisation (crates/burn_automata_kernels/src/reference/normalize.rs:60-69)
// calls f32::ln_1p, which on Linux is glibc's log1pf. That function is not correctly rounded (it is
// 1 ulp off for ~0.75% of inputs in [1e-6, inf)), and the NPA rollout is chaotic: a single 1-ulp
// difference grows to ~15% relative position error within 64 steps. The device therefore uses the
// same algorithm glibc's float log1pf is built on - FDLIBM's s_log1pf (Sun Microsystems; "permission
// to use, copy, modify, and distribute this software is freely granted, provided that this notice is
// preserved") - evaluated in float with the same operation order and no FMA contraction. The test
// tests/test_abi.py (via tests/native/check_log1p.cpp) compiles this header on the host and compares it with the host libm's log1pf
// for every float bit pattern in [-1, +inf]; the recorded result is zero mismatches.
//
// Outline: for x outside (-0.2929, 0.41422) reduce 1+x = 2^k * u with u in [sqrt(2)/2, sqrt(2)),
// carrying the rounding error of 1+x in a correction term c; then log(u) = f - hfsq + s*(hfsq + R)
// with f = u - 1, hfsq = f^2/2, s = f/(2+f) and R a degree-7 polynomial in s^2 (minimax
// coefficients, about 2/3, 2/5, 2/7, ...), and log1p(x) = k*ln2 + log(u) + c with ln2 split hi/lo.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define NPA_HD __host__ __device__
#else
#define NPA_HD
#endif

namespace npa {

NPA_HD inline int32_t f2i_bits(float f) { return __builtin_bit_cast(int32_t, f); }
NPA_HD inline float i2f_bits(int32_t i) { return __builtin_bit_cast(float, i); }

NPA_HD inline float npa_log1pf(float x) {
    const float ln2_hi = i2f_bits(0x3f317180), ln2_lo = i2f_bits(0x3717f7d1);
    const float Lp1 = i2f_bits(0x3F2AAAAB), Lp2 = i2f_bits(0x3ECCCCCD), Lp3 = i2f_bits(0x3E924925),
                Lp4 = i2f_bits(0x3E638E29), Lp5 = i2f_bits(0x3E3A3325), Lp6 = i2f_bits(0x3E1CD04F),
                Lp7 = i2f_bits(0x3E178897);
    float hfsq, f = 0.0f, c = 0.0f, s, z, R, u;
    int32_t k, hu = 0;
    const int32_t hx = f2i_bits(x);
    const int32_t ax = hx & 0x7fffffff;
    k = 1;
    if (hx < 0x3ed413d7) {  // x < 0.41422 (also every negative x)
        if (ax >= 0x3f800000) {  // x <= -1
            if (x == -1.0f) return -__builtin_inff();
            return __builtin_nanf("");
        }
        if (ax < 0x31000000) {  // |x| < 2^-29
            if (ax < 0x24800000) return x;  // |x| < 2^-54
            return x - x * x * 0.5f;
        }
        if (hx > 0 || hx <= (int32_t)0xbe95f61f) {  // -0.2929 < x < 0.41422
            k = 0;
            f = x;
            hu = 1;
        }
    } else if (hx >= 0x7f800000) {
        return x + x;  // +inf or NaN
    }
    if (k != 0) {
        if (hx < 0x5a000000) {  // x < 2^53
            u = 1.0f + x;
            hu = f2i_bits(u);
            k = (hu >> 23) - 127;
            c = (k > 0) ? 1.0f - (u - x) : x - (u - 1.0f);  // rounding error of 1 + x
            c /= u;
        } else {
            u = x;
            hu = f2i_bits(u);
            k = (hu >> 23) - 127;
            c = 0.0f;
        }
        hu &= 0x007fffff;
        if (hu < 0x3504f7) {
            u = i2f_bits(hu | 0x3f800000);  // u in [1, sqrt 2)
        } else {
            k += 1;
            u = i2f_bits(hu | 0x3f000000);  // u/2 in [sqrt(2)/2, 1)
            hu = (0x00800000 - hu) >> 2;
        }
        f = u - 1.0f;
    }
    hfsq = 0.5f * f * f;
    if (hu == 0) {  // f == 0 or |f| tiny
        if (f == 0.0f) {
            if (k == 0) return 0.0f;
            c += (float)k * ln2_lo;
            return (float)k * ln2_hi + c;
        }
        R = hfsq * (1.0f - 0.66666666666666666f * f);
        if (k == 0) return f - R;
        return (float)k * ln2_hi - ((R - ((float)k * ln2_lo + c)) - f);
    }
    s = f / (2.0f + f);
    z = s * s;
    R = z * (Lp1 + z * (Lp2 + z * (Lp3 + z * (Lp4 + z * (Lp5 + z * (Lp6 + z * Lp7))))));
    if (k == 0) return f - (hfsq - s * (hfsq + R));
    return (float)k * ln2_hi - ((hfsq - (s * (hfsq + R) + ((float)k * ln2_lo + c))) - f);
}

}  // namespace npa
