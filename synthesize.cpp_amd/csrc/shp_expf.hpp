// e^x for f32 x, rounded to f32 from a double evaluation (the exp of the
// softmax, of SnakeBeta's curves and of ggml_exp).
//
// Method: Tang's table-driven exponential (P. T. P. Tang, ACM TOMS 15(2),
// 1989), with 64 table entries and the work in double:
//   z = x * 64/ln2 (double), k = rint(z), r = z - k (|r| <= 1/2),
//   e^x = 2^(k/64) * 2^(r/64) = 2^floor(k/64) * T[k mod 64] * p(r),
//   T[j] = 2^(j/64) rounded to double, p(r) = 1 + c1 r + c2 r^2 + c3 r^3 + c4 r^4
//   with c_n = (ln2/64)^n / n!, the Taylor series of e^(r ln2/64).
// Error of the double result before the f32 rounding: truncation
// (|r ln2/64| <= 0.0055)^5/5! < 4e-14, z's rounding (|z| < 9600) < 2e-14 in
// the result, table and product roundings ~2^-52: about 2^-44 relative, so
// the f32 rounding is the correct one unless e^x lies within ~2^-44 of an f32
// rounding boundary. tests/host/expf_check.cpp compares every f32 input with
// the double exp rounded once.
// Range: x is clamped to [-104, 89] (e^-104 rounds to +0 and e^89 overflows
// to inf in f32, as every x beyond them does); NaN returns NaN.
//
// The table and coefficients are the correctly rounded doubles of the exact
// values (computed to 60 digits). The table lookup is a parameter: device
// code holds entry `lane` in a register and shuffles it to the lane that needs
// it; host code indexes the array.
#pragma once

#include <cmath>

#if defined(__HIPCC__)
#    include <hip/hip_runtime.h>
#endif

#ifndef SHP_HD
#    if defined(__HIPCC__)
#        define SHP_HD __host__ __device__
#    else
#        define SHP_HD
#    endif
#endif

namespace shp {

constexpr double kExpTable[64] = {
    0x1.0000000000000p+0, 0x1.02c9a3e778061p+0, 0x1.059b0d3158574p+0, 0x1.0874518759bc8p+0,
    0x1.0b5586cf9890fp+0, 0x1.0e3ec32d3d1a2p+0, 0x1.11301d0125b51p+0, 0x1.1429aaea92de0p+0,
    0x1.172b83c7d517bp+0, 0x1.1a35beb6fcb75p+0, 0x1.1d4873168b9aap+0, 0x1.2063b88628cd6p+0,
    0x1.2387a6e756238p+0, 0x1.26b4565e27cddp+0, 0x1.29e9df51fdee1p+0, 0x1.2d285a6e4030bp+0,
    0x1.306fe0a31b715p+0, 0x1.33c08b26416ffp+0, 0x1.371a7373aa9cbp+0, 0x1.3a7db34e59ff7p+0,
    0x1.3dea64c123422p+0, 0x1.4160a21f72e2ap+0, 0x1.44e086061892dp+0, 0x1.486a2b5c13cd0p+0,
    0x1.4bfdad5362a27p+0, 0x1.4f9b2769d2ca7p+0, 0x1.5342b569d4f82p+0, 0x1.56f4736b527dap+0,
    0x1.5ab07dd485429p+0, 0x1.5e76f15ad2148p+0, 0x1.6247eb03a5585p+0, 0x1.6623882552225p+0,
    0x1.6a09e667f3bcdp+0, 0x1.6dfb23c651a2fp+0, 0x1.71f75e8ec5f74p+0, 0x1.75feb564267c9p+0,
    0x1.7a11473eb0187p+0, 0x1.7e2f336cf4e62p+0, 0x1.82589994cce13p+0, 0x1.868d99b4492edp+0,
    0x1.8ace5422aa0dbp+0, 0x1.8f1ae99157736p+0, 0x1.93737b0cdc5e5p+0, 0x1.97d829fde4e50p+0,
    0x1.9c49182a3f090p+0, 0x1.a0c667b5de565p+0, 0x1.a5503b23e255dp+0, 0x1.a9e6b5579fdbfp+0,
    0x1.ae89f995ad3adp+0, 0x1.b33a2b84f15fbp+0, 0x1.b7f76f2fb5e47p+0, 0x1.bcc1e904bc1d2p+0,
    0x1.c199bdd85529cp+0, 0x1.c67f12e57d14bp+0, 0x1.cb720dcef9069p+0, 0x1.d072d4a07897cp+0,
    0x1.d5818dcfba487p+0, 0x1.da9e603db3285p+0, 0x1.dfc97337b9b5fp+0, 0x1.e502ee78b3ff6p+0,
    0x1.ea4afa2a490dap+0, 0x1.efa1bee615a27p+0, 0x1.f50765b6e4540p+0, 0x1.fa7c1819e90d8p+0,
};

constexpr double kExp64OverLn2 = 0x1.71547652b82fep+6;
constexpr double kExpC1        = 0x1.62e42fefa39efp-7;
constexpr double kExpC2        = 0x1.ebfbdff82c58fp-15;
constexpr double kExpC3        = 0x1.c6b08d704a0c0p-23;
constexpr double kExpC4        = 0x1.3b2ab6fba4e77p-31;

// tab(j) must return kExpTable[j] for j in [0, 63].
// Branch-free (a NaN is carried through a select, not an early return), so a
// caller's loop over independent elements stays straight-line code whose
// table reads overlap.
template <class Tab> SHP_HD inline float exp_f32_rn(float x, const Tab & tab) {
    const bool   nan = x != x;
    const float  xc  = std::fmin(std::fmax(x, -104.0f), 89.0f);  // max/min instructions; a NaN gives -104
    const double z  = static_cast<double>(xc) * kExp64OverLn2;
    const double kd = std::rint(z);
    const double r  = z - kd;
    double       p  = std::fma(r, kExpC4, kExpC3);
    p               = std::fma(p, r, kExpC2);
    p               = std::fma(p, r, kExpC1);
    p               = std::fma(p, r, 1.0);
    const int k     = static_cast<int>(kd);
    const int j     = k & 63;
    const float  e  = static_cast<float>(std::ldexp(tab(j) * p, (k - j) / 64));
    return nan ? x : e;
}

// Host form: the table indexed directly.
inline float exp_f32_rn_host(float x) {
    return exp_f32_rn(x, [](int j) { return kExpTable[j]; });
}

#if defined(__HIPCC__)
// Device forms with the table in the calling wave's own LDS copy: one
// ds_read_b64 per lookup, valid whichever lanes are active (measured ~3 %
// faster on the softmax than reading the table from memory or shuffling a
// per-lane entry, and the read is not a memory round trip in front of the
// first exp).
__device__ __forceinline__ float exp_f32_lds(float x, const double * tab) {
    return exp_f32_rn(x, [tab](int j) { return tab[j]; });
}

// Lane l's entry of the table, loaded early (with the kernel's first data
// loads) so that the table costs no round trip of its own.
__device__ __forceinline__ double exp_table_entry(int lane) {
    return kExpTable[lane];
}

// Fills the calling wave's 64-entry table (s_tab[wave]) with the entries its
// lanes loaded (lane l holds entry l; every lane of the wave active) and
// makes it visible to the whole wave.
__device__ __forceinline__ const double * wave_exp_table(double (*s_tab)[64], int lane, double entry) {
    double * t = s_tab[threadIdx.x / 64];
    t[lane]    = entry;
    __syncwarp();
    return t;
}
#endif

}  // namespace shp
