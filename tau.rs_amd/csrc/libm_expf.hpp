// f32 exp with the results of glibc's expf, bit for bit, on host and device.
//
// The reference's f32 CPU routing (tau.rs crates/models/src/components/
// sparse_moe/routing.rs:139-141, candle_nn::ops::softmax_last_dim) takes
// exp(x - max) with Rust's f32::exp, which on linux-gnu is glibc's expf.
// Which experts a token selects is decided by comparing the resulting f32
// probabilities (routing.rs:239-257: larger probability first, lower id on
// equal probabilities), so a distinct pair of logits whose exp rounds to the
// same float is a tie the reference breaks by id.  Reproducing those ties
// needs the same exp bits, which HIP's expf (a different approximation) does
// not give.
//
// Method (the published glibc/ARM optimized-routines expf design, glibc
// 2.27+ sysdeps/ieee754/flt-32/e_expf.c, here written from its description):
// in double precision, z = x * 32/ln2, k = round(z) (round-to-nearest-even
// through the 1.5*2^52 shift), r = z - k (z fused into both, as the FMA
// build of glibc contracts them), 2^(k/32) = 2^(k>>5) * T[k&31] with
// T[i] = 2^(i/32) rounded to double, and 2^(r/32) ~ 1 + c2 r + c1 r^2 + c0 r^3
// evaluated as fma(fma(c0, r, c1), r*r, fma(c2, r, 1)), the fused form glibc's
// x86-64 FMA build runs.  The result is rounded to float once.  Inputs below
// -0x1.9fe368p6 give +0 and above 0x1.62e42ep6 give +inf, as glibc.
//
// Checked on the host against the system expf for every finite float and
// both infinities (tests/test_libm_expf.py); the device code is the same
// source.
#pragma once
#include <stdint.h>

#include "host_device.hpp"

namespace tau_amd {

// 2^(i/32), i = 0..31, as IEEE double bit patterns.
static constexpr uint64_t kExp2Over32[32] = {
    0x3ff0000000000000ull, 0x3ff059b0d3158574ull, 0x3ff0b5586cf9890full, 0x3ff11301d0125b51ull,
    0x3ff172b83c7d517bull, 0x3ff1d4873168b9aaull, 0x3ff2387a6e756238ull, 0x3ff29e9df51fdee1ull,
    0x3ff306fe0a31b715ull, 0x3ff371a7373aa9cbull, 0x3ff3dea64c123422ull, 0x3ff44e086061892dull,
    0x3ff4bfdad5362a27ull, 0x3ff5342b569d4f82ull, 0x3ff5ab07dd485429ull, 0x3ff6247eb03a5585ull,
    0x3ff6a09e667f3bcdull, 0x3ff71f75e8ec5f74ull, 0x3ff7a11473eb0187ull, 0x3ff82589994cce13ull,
    0x3ff8ace5422aa0dbull, 0x3ff93737b0cdc5e5ull, 0x3ff9c49182a3f090ull, 0x3ffa5503b23e255dull,
    0x3ffae89f995ad3adull, 0x3ffb7f76f2fb5e47ull, 0x3ffc199bdd85529cull, 0x3ffcb720dcef9069ull,
    0x3ffd5818dcfba487ull, 0x3ffdfc97337b9b5full, 0x3ffea4afa2a490daull, 0x3fff50765b6e4540ull,
};

TAU_HOST_DEVICE inline float expf_glibc(float x) {
    constexpr double kN = 32.0;
    constexpr double kInvLn2N = 0x1.71547652b82fep+0 * kN;
    constexpr double kC0 = 0x1.c6af84b912394p-5 / kN / kN / kN;
    constexpr double kC1 = 0x1.ebfce50fac4f3p-3 / kN / kN;
    constexpr double kC2 = 0x1.62e42ff0c52d6p-1 / kN;
    constexpr double kShift = 0x1.8p+52;
    if (x < -0x1.9fe368p6f) return 0.0f;  // underflows to +0 (and -inf)
    if (x > 0x1.62e42ep6f) return __builtin_inff();
    const double xd = (double)x;
    // k = nearest integer to z = x * 32/ln2, which lands in the low mantissa
    // bits of z + 1.5*2^52; z is never rounded on its own (both uses are fused).
    double kd = __builtin_fma(kInvLn2N, xd, kShift);
    const int64_t k = (int64_t)(__builtin_bit_cast(uint64_t, kd) & 0xfffffffffffffull) - (1ll << 51);
    kd -= kShift;
    const double r = __builtin_fma(kInvLn2N, xd, -kd);
    const double s = __builtin_bit_cast(double, kExp2Over32[k & 31] + ((uint64_t)(k >> 5) << 52));
    const double p = __builtin_fma(kC0, r, kC1);
    double y = __builtin_fma(kC2, r, 1.0);
    y = __builtin_fma(p, r * r, y);
    return (float)(y * s);
}

}  // namespace tau_amd
