/*
 * mdnav_math.h — elementary functions with one definition for CPU and GPU.
 *
 * The reference evaluates exp/log/sin/cos/tanh with the platform libm (Apple
 * libm on the CPU path, Metal "precise" on the GPU path), so its two paths
 * already differ in the last bits.  Here both paths compile the functions
 * below, built only from IEEE operations that are correctly rounded on x86-64
 * SSE and on gfx950 (+, -, *, /, sqrt, floor, ldexp) with contraction off.
 * The same input therefore gives the same bits on the host and the device,
 * which is what lets integer outcomes (contact/done flags, reset decisions,
 * RNG streams) agree exactly between the HIP path and the CPU oracle.
 *
 * Methods (published, restated from the mathematics):
 *   exp, expm1  Cody–Waite reduction x = k ln2 + r, |r| <= ln2/2 (ln2 split in
 *               a 16-bit head and a tail), Taylor polynomial of degree 7/8 in r
 *               (truncation < 1e-8 relative), scaling by 2^k with ldexp.
 *   log         x = 2^e m, m in [sqrt(1/2), sqrt(2)), log m = 2 atanh(s),
 *               s = (m-1)/(m+1), odd series to s^11 (|s| <= 0.1716).
 *   sin, cos    Cody–Waite reduction by pi/2 with the three-part split of
 *               Cephes (Moshier), Taylor polynomials on [-pi/4, pi/4].
 *   tanh        t = expm1(2|x|), tanh = sign(x) t / (t + 2).
 * Accuracy is a few ulp against glibc (checked in tests/test_oracle_math.py);
 * the reference's own CPU/GPU tolerance is 2e-5 absolute.
 *
 * Build rule: every translation unit that includes this header must be
 * compiled with -ffp-contract=off and without fast-math.
 */
#ifndef MDNAV_MATH_H
#define MDNAV_MATH_H

#include <stdint.h>

#include <cmath>
#include <cstring>
#if defined(__HIPCC__) || defined(__HIP__)
#include <hip/hip_runtime.h>
#define MDN_HD __host__ __device__ __forceinline__
#else
#define MDN_HD inline
#endif

#ifdef __clang__
#pragma clang fp contract(off)
#endif

namespace mdn {

MDN_HD float floor_f(float x) {
#if defined(__HIP_DEVICE_COMPILE__)
    return floorf(x);
#else
    return std::floor(x);
#endif
}

MDN_HD float ldexp_f(float x, int k) {
#if defined(__HIP_DEVICE_COMPILE__)
    return ldexpf(x, k);
#else
    return std::ldexp(x, k);
#endif
}

MDN_HD float sqrt_f(float x) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __builtin_sqrtf(x);
#else
    return std::sqrt(x);
#endif
}

// Fused multiply-add with one rounding (IEEE fma).  Dot products and
// weight-gradient sums on both sides are sequential chains of it, which is
// also exactly what the fp32 matrix-core instructions compute.
MDN_HD float fma_f(float a, float b, float c) { return __builtin_fmaf(a, b, c); }

MDN_HD float fabs_f(float x) { return __builtin_fabsf(x); }  // the sign bit cleared

MDN_HD uint32_t float_bits(float x) {
    uint32_t u;
#if defined(__HIP_DEVICE_COMPILE__)
    u = __float_as_uint(x);
#else
    std::memcpy(&u, &x, 4);
#endif
    return u;
}

MDN_HD float bits_float(uint32_t u) {
    float x;
#if defined(__HIP_DEVICE_COMPILE__)
    x = __uint_as_float(u);
#else
    std::memcpy(&x, &u, 4);
#endif
    return x;
}

MDN_HD float inf_f() { return bits_float(0x7f800000u); }
MDN_HD float nan_f() { return bits_float(0x7fc00000u); }
MDN_HD bool isfinite_f(float x) { return (float_bits(x) & 0x7f800000u) != 0x7f800000u; }

// ln2 = LN2_HI + LN2_LO; LN2_HI has 16 significant bits so k*LN2_HI is exact.
constexpr float LN2_HI = 0.693145751953125f;
constexpr float LN2_LO = 1.42860677e-06f;
constexpr float LOG2E = 1.44269502f;

MDN_HD float exp_f(float x) {
    // straight-line: the argument is clamped with min/max, the function
    // evaluated, and the special cases selected at the end (no branches)
    const bool nan = !(x == x);
    const float xc = nan ? 0.0f : __builtin_fminf(__builtin_fmaxf(x, -104.0f), 88.8f);
    const float k = floor_f(xc * LOG2E + 0.5f);
    const float r = (xc - k * LN2_HI) - k * LN2_LO;
    float p = 1.98412698e-04f;      // 1/7!
    p = p * r + 1.38888889e-03f;    // 1/6!
    p = p * r + 8.33333333e-03f;    // 1/5!
    p = p * r + 4.16666667e-02f;    // 1/4!
    p = p * r + 1.66666667e-01f;    // 1/3!
    p = p * r + 0.5f;
    p = p * r + 1.0f;
    p = p * r + 1.0f;
    const float v = ldexp_f(p, (int)k);
    const float lo = x < -104.0f ? 0.0f : v;
    const float hi = x > 88.8f ? inf_f() : lo;
    return nan ? x : hi;
}

// expm1 of an argument already in [-18, 88] (not NaN)
MDN_HD float expm1_core(float xc) {
    const float k = floor_f(xc * LOG2E + 0.5f);
    const float r = (xc - k * LN2_HI) - k * LN2_LO;
    float p = 2.48015873e-05f;      // 1/8!
    p = p * r + 1.98412698e-04f;    // 1/7!
    p = p * r + 1.38888889e-03f;    // 1/6!
    p = p * r + 8.33333333e-03f;    // 1/5!
    p = p * r + 4.16666667e-02f;    // 1/4!
    p = p * r + 1.66666667e-01f;    // 1/3!
    p = p * r + 0.5f;               // 1/2!
    const float em1 = r + (r * r) * p;
    const float scale = ldexp_f(1.0f, (int)k);
    const float big = scale * em1 + (scale - 1.0f);
    return k == 0.0f ? em1 : big;
}

MDN_HD float expm1_f(float x) {
    const bool nan = !(x == x);
    const float v = expm1_core(nan ? 0.0f : __builtin_fminf(__builtin_fmaxf(x, -18.0f), 88.0f));
    const float lo = x < -18.0f ? -1.0f : v;
    const float hi = x > 88.0f ? inf_f() : lo;
    return nan ? x : hi;
}

MDN_HD float log_f(float x) {
    const bool sub = x < 1.17549435e-38f;
    const float xs = sub ? x * 8388608.0f : x;
    const uint32_t bits = float_bits(xs);
    int e = (sub ? -23 : 0) + (int)((bits >> 23) & 0xffu) - 127;
    float m = bits_float((bits & 0x007fffffu) | 0x3f800000u);
    const bool high = m > 1.41421356f;
    m = high ? m * 0.5f : m;
    e += high ? 1 : 0;
    const float s = (m - 1.0f) / (m + 1.0f);
    const float z = s * s;
    float p = 9.09090909e-02f;      // 1/11
    p = p * z + 1.11111111e-01f;    // 1/9
    p = p * z + 1.42857143e-01f;    // 1/7
    p = p * z + 2.0e-01f;           // 1/5
    p = p * z + 3.33333333e-01f;    // 1/3
    p = p * z + 1.0f;
    const float lm = (2.0f * s) * p;
    const float ef = (float)e;
    const float v = ef * LN2_HI + (ef * LN2_LO + lm);
    // special cases as single selects (no branches): +-0 -> -inf, negative
    // or NaN -> NaN, +inf -> +inf
    const float fin = isfinite_f(x) ? v : x;
    const float pos = x > 0.0f ? fin : nan_f();
    return x == 0.0f ? -inf_f() : pos;
}

// Cephes pi/2 split: PIO2_1 + PIO2_2 + PIO2_3 = pi/2; k*PIO2_1 is exact.
MDN_HD void sincos_f(float x, float* s_out, float* c_out) {
    const float k = floor_f(x * 0.636619772f + 0.5f);
    const float r = ((x - k * 1.5703125f) - k * 4.83751297e-04f) - k * 7.54978995e-08f;
    const float z = r * r;
    float sp = 2.75573192e-06f;     // 1/9!
    sp = sp * z - 1.98412698e-04f;  // 1/7!
    sp = sp * z + 8.33333333e-03f;  // 1/5!
    sp = sp * z - 1.66666667e-01f;  // 1/3!
    const float sr = r + (r * z) * sp;
    float cp = -2.75573192e-07f;    // 1/10!
    cp = cp * z + 2.48015873e-05f;  // 1/8!
    cp = cp * z - 1.38888889e-03f;  // 1/6!
    cp = cp * z + 4.16666667e-02f;  // 1/4!
    cp = cp * z - 0.5f;
    const float cr = 1.0f + z * cp;
    const int q = (k == k && k > -2147483648.0f && k < 2147483648.0f) ? (((int)k) & 3) : 0;
    const bool odd = (q & 1) != 0, neg_s = q >= 2, neg_c = q == 1 || q == 2;
    const float s = odd ? cr : sr, c = odd ? sr : cr;
    *s_out = neg_s ? -s : s;
    *c_out = neg_c ? -c : c;
}

MDN_HD float sin_f(float x) { float s, c; sincos_f(x, &s, &c); return s; }
MDN_HD float cos_f(float x) { float s, c; sincos_f(x, &s, &c); return c; }

// 1/d correctly rounded when 1/d is a normal number: the division on the
// host; on the device v_rcp_f32 and one Newton step, which equals it for every
// such d (checked on the GPU over all 2^32 inputs)
MDN_HD float recip_normal_f(float d) {
#if defined(__HIP_DEVICE_COMPILE__)
    const float y = __builtin_amdgcn_rcpf(d);
    return __builtin_fmaf(__builtin_fmaf(-d, y, 1.0f), y, y);
#else
    return 1.0f / d;
#endif
}

MDN_HD float tanh_f(float x) {
    // 2 min(|x|, 10) is inside expm1_core's range; NaN takes 0 and is
    // selected out at the end
    const float a = fabs_f(x);
    const float e = expm1_core(2.0f * (a == a ? __builtin_fminf(a, 10.0f) : 0.0f));
    // e / (e + 2) for e in [0, expm1(20)] by one correction step from the
    // correctly rounded reciprocal (Markstein): q0 = e y, r = e - q0 d exactly,
    // q = q0 + r y rounded once.  Equal to the correctly rounded quotient for
    // every float e in that range (all 1,307,025,409 checked on the host).
    const float d = e + 2.0f;
    const float y = recip_normal_f(d);
    const float q0 = e * y;
    const float q = fma_f(fma_f(-q0, d, e), y, q0);
    const float t = a > 10.0f ? 1.0f : q;
    const float v = x < 0.0f ? -t : t;
    return !(a == a) ? x : v;
}

MDN_HD float sigmoid_f(float x) { return 1.0f / (1.0f + exp_f(-x)); }

// atan: Cephes atanf (S. L. Moshier, Cephes Math Library): reduction at
// tan(3 pi/8) and tan(pi/8), then a degree-4 polynomial in x^2; selects
// instead of branches.
MDN_HD float atan_f(float x) {
    const float ax = fabs_f(x);
    const bool big = ax > 2.414213562373095f, mid = ax > 0.4142135623730950f;
    const float xr = big ? -1.0f / ax : (mid ? (ax - 1.0f) / (ax + 1.0f) : ax);
    const float y0 = big ? 1.5707963267948966f : (mid ? 0.7853981633974483f : 0.0f);
    const float z = xr * xr;
    const float p = (((8.05374449538e-2f * z - 1.38776856032e-1f) * z + 1.99777106478e-1f) * z - 3.33329491539e-1f) *
                    z * xr + xr;
    const float r = y0 + p;
    return x < 0.0f ? -r : r;
}
// atan2 with the special values of C99 Annex F.9.1.4: a = atan_f(|y| / |x|)
// in [0, pi/2] (pi/4 when both are infinite, 0 when both are zero), then
// pi - a when x is negative or -0, with the sign of y.  For finite nonzero
// operands this is the quadrant rule t, t + pi, t - pi on t = atan_f(y / x)
// operation for operation (atan_f is odd and -(pi - a) = a - pi exactly).
MDN_HD float atan2_f(float y, float x) {
    const float pi = 3.14159265358979f, quarter_pi = 0.7853981633974483f;
    const float ay = fabs_f(y), ax = fabs_f(x);
    const float t = atan_f(ay / ax);
    const bool both_inf = ay == inf_f() && ax == inf_f(), both_zero = ay == 0.0f && ax == 0.0f;
    const float a0 = both_inf ? quarter_pi : (both_zero ? 0.0f : t);
    const float a = (float_bits(x) >> 31) != 0u ? pi - a0 : a0;
    const float r = bits_float(float_bits(a) | (float_bits(y) & 0x80000000u));
    return (x == x && y == y) ? r : x + y;
}

MDN_HD float min_f(float a, float b) { return b < a ? b : a; }
MDN_HD float max_f(float a, float b) { return a < b ? b : a; }
MDN_HD float clamp_f(float x, float lo, float hi) { return max_f(lo, min_f(hi, x)); }
// C fmin/fmax semantics (a NaN operand yields the other operand).
MDN_HD float fmin_f(float a, float b) { return (b < a || !(a == a)) ? b : a; }
MDN_HD float fmax_f(float a, float b) { return (a < b || !(a == a)) ? b : a; }

} // namespace mdn

#endif /* MDNAV_MATH_H */
