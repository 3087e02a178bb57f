// Deterministic float64 arithmetic shared by the coders' decisions (detmath.py:20-58): log2 / exp2
// from IEEE basic operations only (odd atanh series, Taylor series of e^t around the nearest
// integer), round half to even by the 2^52 addition. Built without contraction, these are the same
// bits as the reference's GPU and --cpu builds.
#pragma once
#include <hip/hip_runtime.h>

namespace spa {
namespace dm {

__device__ __forceinline__ double dm_rint(double x) {
    if (!(fabs(x) < 4503599627370496.0)) return x;
    double y = fabs(x) + 4503599627370496.0;
    y = y - 4503599627370496.0;
    return copysign(y, x);
}

__device__ inline double dm_log2(double x) {
    if (isnan(x)) return x;
    if (x < 0.0) return __longlong_as_double(0x7ff8000000000000LL);
    if (x == 0.0) return __longlong_as_double((long long)0xfff0000000000000ULL);
    if (isinf(x)) return x;
    long long u = __double_as_longlong(x);
    int e = (int)((u >> 52) & 0x7ff);
    if (e == 0) {                               // subnormal: scaled by 2^54
        x = x * 18014398509481984.0;
        u = __double_as_longlong(x);
        e = (int)((u >> 52) & 0x7ff) - 54;
    }
    e -= 1023;
    double m = __longlong_as_double((u & 0x000fffffffffffffLL) | 0x3ff0000000000000LL);
    if (m > 1.4142135623730951) { m = m * 0.5; e += 1; }
    const double s = (m - 1.0) / (m + 1.0), z = s * s;     // ln m = 2 atanh s
    constexpr double C[12] = {0.043478260869565216, 0.047619047619047616, 0.05263157894736842, 0.058823529411764705,
                              0.06666666666666667,  0.07692307692307693,  0.09090909090909091, 0.1111111111111111,
                              0.14285714285714285,  0.2,                  0.3333333333333333,  1.0};
    double p = 0.04;
#pragma unroll
    for (int i = 0; i < 12; ++i) p = p * z + C[i];
    return (double)e + (2.0 * s * p) * 1.4426950408889634;
}

__device__ inline double dm_exp2(double y) {
    if (isnan(y)) return y;
    if (y >= 1024.0) return __longlong_as_double(0x7ff0000000000000LL);
    if (y < -1075.0) return 0.0;
    const double n = dm_rint(y), t = (y - n) * 0.6931471805599453;
    constexpr double C[17] = {4.779477332387385e-14,  7.647163731819816e-13, 1.1470745597729725e-11, 1.6059043836821613e-10,
                              2.08767569878681e-09,   2.505210838544172e-08, 2.7557319223985893e-07, 2.755731922398589e-06,
                              2.48015873015873e-05,   0.0001984126984126984, 0.001388888888888889,   0.008333333333333333,
                              0.041666666666666664,   0.16666666666666666,   0.5,                    1.0,
                              1.0};
    double p = 2.8114572543455206e-15;
#pragma unroll
    for (int i = 0; i < 17; ++i) p = p * t + C[i];
    const int k = (int)n, k1 = k / 2, k2 = k - k1;
    return p * __longlong_as_double((long long)(k1 + 1023) << 52) * __longlong_as_double((long long)(k2 + 1023) << 52);
}

}  // namespace dm
}  // namespace spa
