// cos/sin of an f32 angle, evaluated in double and rounded once to f32.
//
// Rope needs cos/sin of angles up to the largest position (thousands of
// radians) to the last f32 bit. The reduction r = x - k*pi/2 uses pi/2 split
// into two 33-bit pieces and a 53-bit tail (Cody-Waite): for |k| <= 2^19 the
// products k*P1 and k*P2 are exact, so r carries ~100 bits of pi/2 and its
// absolute error is below 2^-78. sin and cos of r in [-pi/4, pi/4] are Taylor
// polynomials through r^19 / r^20 (truncation < 1e-18), evaluated in double
// with FMA. The f32 result equals the correctly rounded value except when the
// exact value lies within ~2^-50 relative of an f32 rounding midpoint.
//
// Compiles for host and device, so the host test suite checks it against
// libm's double sin/cos.
#pragma once

#include <cmath>

#if defined(__HIPCC__)
#    define SHP_HD __host__ __device__
#else
#    define SHP_HD
#endif

namespace shp {

// pi/2 = P1 + P2 + P3: P1, P2 hold 33 significant bits each, P3 is the rest.
constexpr double kPio2P1  = 1.5707963267341256;     // 0x3ff921fb54400000
constexpr double kPio2P2  = 6.077100506303966e-11;  // 0x3dd0b4611a600000
constexpr double kPio2P3  = 2.0222662487959506e-21; // 0x3ba3198a2e037073
constexpr double kInvPio2 = 0.6366197723675814;     // 2/pi
constexpr double kMaxK    = 524288.0;               // 2^19

// Returns false (outputs untouched) when |th| is beyond the exact-reduction range.
SHP_HD inline bool sincos_f32_rn(float th, float & s_out, float & c_out) {
    if (th == 0.0f) {
        s_out = th;  // keeps the sign of zero, as sin(-0) = -0
        c_out = 1.0f;
        return true;
    }
    const double x = static_cast<double>(th);
    const double k = std::rint(x * kInvPio2);
    if (!(std::fabs(k) <= kMaxK)) {
        return false;
    }
    double r = std::fma(-k, kPio2P1, x);
    r        = std::fma(-k, kPio2P2, r);
    r        = std::fma(-k, kPio2P3, r);
    const double z = r * r;
    // sin r = r + r z (s3 + z (s5 + ... + z s19))
    double ps = -8.22063524662433e-18;
    ps        = std::fma(ps, z, 2.8114572543455206e-15);
    ps        = std::fma(ps, z, -7.647163731819816e-13);
    ps        = std::fma(ps, z, 1.6059043836821613e-10);
    ps        = std::fma(ps, z, -2.505210838544172e-08);
    ps        = std::fma(ps, z, 2.7557319223985893e-06);
    ps        = std::fma(ps, z, -0.0001984126984126984);
    ps        = std::fma(ps, z, 0.008333333333333333);
    ps        = std::fma(ps, z, -0.16666666666666666);
    const double sr = std::fma(r * z, ps, r);
    // cos r = 1 + z (-1/2 + z (c4 + ... + z c20))
    double pc = 4.110317623312165e-19;
    pc        = std::fma(pc, z, -1.5619206968586225e-16);
    pc        = std::fma(pc, z, 4.779477332387385e-14);
    pc        = std::fma(pc, z, -1.1470745597729725e-11);
    pc        = std::fma(pc, z, 2.08767569878681e-09);
    pc        = std::fma(pc, z, -2.755731922398589e-07);
    pc        = std::fma(pc, z, 2.48015873015873e-05);
    pc        = std::fma(pc, z, -0.001388888888888889);
    pc        = std::fma(pc, z, 0.041666666666666664);
    pc        = std::fma(pc, z, -0.5);
    const double cr = std::fma(z, pc, 1.0);
    const int    q  = static_cast<int>(static_cast<long long>(k) & 3);
    double       s, c;
    switch (q) {
        case 0:
            s = sr;
            c = cr;
            break;
        case 1:
            s = cr;
            c = -sr;
            break;
        case 2:
            s = -sr;
            c = -cr;
            break;
        default:
            s = -cr;
            c = sr;
            break;
    }
    s_out = static_cast<float>(s);
    c_out = static_cast<float>(c);
    return true;
}

}  // namespace shp
