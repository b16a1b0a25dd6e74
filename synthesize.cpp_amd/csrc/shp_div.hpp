// IEEE f32 division q / a from a double reciprocal of a, for many q per a.
//
// r = (float)((double)q * y), with y within 1 ulp (double) of 1/a, equals the
// correctly rounded f32 quotient RN(q / a) for every f32 q and every finite,
// nonzero f32 a:
//   - the double product is within ~2^-51.4 (relative) of q / a: y's error
//     plus the product's rounding;
//   - an exact quotient of two 24-bit significands is either an f32 rounding
//     midpoint itself or at least 2^-49 (relative) away from every midpoint
//     (q - m*a is a nonzero multiple of the coarser of the two grids), so the
//     double product rounds to f32 on the same side as q / a does;
//   - a quotient that is exactly a midpoint needs a's significand to be a
//     power of two, and then y = 1/a and the product are exact, so the final
//     conversion rounds the tie to even like the division.
// Snake divides by one alpha per channel, so the reciprocal is formed once per
// lane and channel and each element costs a convert, a multiply and a convert
// instead of the ~12-instruction f32 division sequence. The host test
// tests/host/div_check.cpp checks the identity, including a reciprocal that
// is one ulp off, against the hardware f32 division.
#pragma once

#include <cmath>

#ifndef SHP_HD
#    if defined(__HIPCC__)
#        define SHP_HD __host__ __device__
#    else
#        define SHP_HD
#    endif
#endif

namespace shp {

// a finite and nonzero: the reciprocal route applies (else use q / a itself).
SHP_HD inline bool rcp_route_ok(float a) {
    return a != 0.0f && std::isfinite(a);
}

// 1/a to within 1 ulp: the hardware estimate refined by two Newton steps
// (each roughly doubles the correct bits), or the IEEE division on the host.
SHP_HD inline double rcp_d(double a) {
#if defined(__HIP_DEVICE_COMPILE__)
    double y = __builtin_amdgcn_rcp(a);
    double e = __builtin_fma(-a, y, 1.0);
    y        = __builtin_fma(y, e, y);
    e        = __builtin_fma(-a, y, 1.0);
    y        = __builtin_fma(y, e, y);
    return y;
#else
    return 1.0 / a;
#endif
}

SHP_HD inline float div_by_rcp(float q, double rcp) {
    return static_cast<float>(static_cast<double>(q) * rcp);
}

}  // namespace shp
