// activations.hip -- the ten tensor-level activations plus sigmoid.
//
// Formulas are those of activations_c.c:124-158 (and node_sigmoid,
// activations.asm:352-413): each element is widened to double, the formula is
// evaluated in double, and f32 tensors store one final rounding to float
// (activations_c.c:71-77).
//
// The piecewise-linear ones (leaky_relu, hardswish, hardtanh) and the exp-based
// ones (elu, selu, swish, sigmoid) evaluate the reference expression as
// written (f32 tensors: in float where the reference's double rounding is
// invisible at 1e-5, see the *F32 functors).  tanh, gelu, mish and softplus are evaluated by closed forms built
// on one double exp, which costs a fifth to a third of the device library's
// double tanh / log on gfx950 (measured ~141 and ~70 FP64 instructions per
// element for tanh and log, ~18 for exp), while keeping the two roundings of
// the reference that decide its low-order result:
//
//   u = 1.0 + exp(x)   (softplus, mish): for x << 0, u - 1 is exp(x) quantized to
//                       multiples of 2^-52; the closed forms take t = u - 1 (exact)
//                       so the result carries the reference's quantization;
//   1.0 + tanh(z)       (gelu, z << 0): tanh(z) rounds to a multiple of 2^-53 in
//                       [-1, -0.5], so 1 + tanh(z) is that multiple; it is
//                       rebuilt as rint(eps * 2^53) * 2^-53 from eps = 1 - |tanh z|
//                       computed to a few ulp (a few 2^-53 steps at most).
//
// Everything else matches the reference's value to ~1e-14 relative or better
// (libm differences aside), far inside the 1e-5 (f32) / 1e-12 + 1e-15 (f64) bars.
// f32 tensors use the float-output paths below.
#include <cmath>

#include "ew_impl.hpp"

namespace nh {

constexpr double kGelu = 0.7978845608028654;
constexpr double kSeluL = 1.0507009873554804934193349852946;
constexpr double kSeluA = 1.6732632423543772848170429916717;
// 1 / d for normal d of moderate size (2^-1000 < |d| < 2^1000) from the
// hardware reciprocal seed.  AMD does not publish a bound for the f64 seed;
// a GPU probe measured 2^-24.4 relative over 16 M values in [1, 4].
//   rcp_nr2: two Newton steps (5 instructions instead of a division's ~12):
//            a seed even as coarse as 2^-12 ends within ~2^-48, and a seed
//            within 2^-22 ends at the rounding error of the last FMA (~1 ulp).
//            Used by tanh, gelu and mish, whose quotients feed the result
//            directly.
//   rcp_nr1: one Newton step (3 instructions): the seed's error squared, so
//            ~2^-44 for a 2^-22 seed.  Used only by softplus, where the
//            reciprocal enters the atanh series of log m through s = (m - 1) /
//            (m + 1), |s| <= 0.172: checked on the CPU over 4e7 values of u
//            with a seed perturbed by 2^-22, the log stays within 5.8e-14.
NH_DEV double rcp_nr1(double d)
{
    const double r = __builtin_amdgcn_rcp(d);
    return __builtin_fma(r, __builtin_fma(-d, r, 1.0), r);
}
NH_DEV double rcp_nr2(double d)
{
    double r = __builtin_amdgcn_rcp(d);
    r = __builtin_fma(r, __builtin_fma(-d, r, 1.0), r);
    return __builtin_fma(r, __builtin_fma(-d, r, 1.0), r);
}

// e^a for a in [0, 44] (tanh's argument): a = k ln2 + r, |r| <= ln2/2, e^r by
// its Taylor polynomial through r^11 (truncation below 7e-15 relative), scaled
// by 2^k; ~17 instructions without the device library's range selects.  Its
// error (up to ~30 ulp) is fine where e^a enters a quotient, not where the
// reference rounds 1 + e^a (softplus, mish) or 1 + tanh (gelu): there an
// exponential a few ulp off moves the rounded sum across a rounding boundary
// about once per 10^4 elements, an error of up to 1e-11 relative after it
// (measured on mish), so those keep the device library's exp.
NH_DEV double exp_in_range(double a)
{
    const double k = __builtin_rint(a * 0x1.71547652b82fep+0);  // 1 / ln 2
    double r = __builtin_fma(-k, kLn2Hi, a);                     // exact for |k| < 2^21
    r = __builtin_fma(-k, kLn2Lo, r);
    double p = 1.0 / 39916800.0;
    p = __builtin_fma(p, r, 1.0 / 3628800.0);
    p = __builtin_fma(p, r, 1.0 / 362880.0);
    p = __builtin_fma(p, r, 1.0 / 40320.0);
    p = __builtin_fma(p, r, 1.0 / 5040.0);
    p = __builtin_fma(p, r, 1.0 / 720.0);
    p = __builtin_fma(p, r, 1.0 / 120.0);
    p = __builtin_fma(p, r, 1.0 / 24.0);
    p = __builtin_fma(p, r, 1.0 / 6.0);
    p = __builtin_fma(p, r, 0.5);
    p = __builtin_fma(p, r, 1.0);
    p = __builtin_fma(p, r, 1.0);
    return __builtin_ldexp(p, int(k));
}

// tanh(x) = (E - 1) / (E + 1), E = exp(2|x|), with |x| clamped to 22 (where
// the double result is already +-1); |x| < 2^-7 uses the Taylor series through
// x^7 (truncation below 3e-19 relative; zeros keep their sign, denormals are
// returned unchanged).
// E - 1 is exact, so the relative error is ~1 ulp(E) / (E - 1) < 1.5e-14 (plus
// ~1 ulp from the reciprocal).
NH_DEV double tanh_d(double x)
{
    const double a = __builtin_fabs(x);
    const double x2 = x * x;
    const double small = __builtin_copysign(
        __builtin_fma(x * x2, __builtin_fma(x2, __builtin_fma(x2, -17.0 / 315.0, 2.0 / 15.0), -1.0 / 3.0), x), x);
    const double c = a < 22.0 ? a : 22.0;
    const double e = exp_in_range(c + c);
    const double big = __builtin_copysign((e - 1.0) * rcp_nr2(e + 1.0), x);
    return (a < 0x1p-7 || x != x) ? small : big;
}

// 1 + tanh(z) as the reference's double tanh leaves it, from w = exp(-2|z|):
//   z >= 0:  1 + (1 - w)/(1 + w) = 2/(1 + w)                     (no cancellation)
//   z < 0:   eps = 1 - |tanh z| = 2w/(1 + w); while tanh z is in [-1, -0.5]
//            it is a multiple of 2^-53, so 1 + tanh z is eps rounded to a
//            multiple of 2^-53 (round-half-even on the multiple =
//            round-half-even on tanh z).
// Both sides share one reciprocal and no branch: a wave holds both signs.
// An ulp of error in eps matters to rint only where eps * 2^53 is large, i.e.
// where one multiple of 2^-53 is far below 1e-12 of the result.
// The exponent is clamped at -40 (w >= 4.2e-18): beyond it the result is
// already exactly 2 (z > 0) or 0 (z < 0, eps * 2^53 < 0.08 rounds to 0), and
// cfg3's +-30 inputs (z = +-987) would otherwise drive exp into underflow.
NH_DEV double one_plus_tanh(double z)
{
    const double a = -2.0 * __builtin_fabs(z);
    const double w = exp(a > -40.0 ? a : -40.0);
    const double r = rcp_nr2(1.0 + w);
    const double eps = (w + w) * r;
    // eps rounded to a multiple of 2^-53, ties to even: 0.5 + eps (in [0.5, 1),
    // ulp 2^-53) rounds exactly so, and subtracting 0.5 is exact
    const double q = eps < 0.5 ? (eps + 0.5) - 0.5 : eps;
    return z >= 0.0 ? r + r : q;
}

NH_DEV double gelu_d(double x)
{
    const double z = kGelu * (x + 0.044715 * x * x * x);  // activations_c.c:130-131, same order
    return 0.5 * x * one_plus_tanh(z);
}

// softplus = log(u), u = 1.0 + exp(x) rounded as in the reference, from one
// exponential t = e^{-|x|} <= 1:
//   x <= 0:  u = 1 + t is the reference's u exactly;
//   x > 0:   log(1 + e^x) = x + log(1 + t); the rounding of 1 + t moves that
//            by at most 2^-53, below 1.6e-16 of a result > log 2;
// log of u in [1, 2]: m = u, or u / 2 above sqrt 2 (then + ln 2), and
// log m = 2 atanh(s) = 2s + 2s^3 g(s^2), s = (m - 1) / (m + 1) in
// [-0.172, 0.172] (m - 1 exact), g by a degree-5 polynomial in w = s^2 fitted
// near-minimax on [0, 0.0295] (7e-16 relative on log m with an exact
// quotient, against 3.4e-14 for the Taylor series through s^15 it replaces).
// The quotient's reciprocal has one Newton step: even a seed within only
// 2^-22 would leave 5.8e-14 relative on log m (checked over 4e7 values of u
// on the CPU).  The reference's double exp
// overflows above 709.78 (+inf).
NH_DEV double softplus_d(double x)
{
    const double t = exp(-__builtin_fabs(x));
    const double u = 1.0 + t;
    const bool hi = u > 0x1.6a09e667f3bcdp+0;  // sqrt 2
    const double m = u * (hi ? 0.5 : 1.0);     // exact
    const double s = (m - 1.0) * rcp_nr1(m + 1.0);
    const double w = s * s;
    double q = 0x1.58e1eaa5792a2p-4;
    q = __builtin_fma(q, w, 0x1.732185997e49ap-4);
    q = __builtin_fma(q, w, 0x1.c722e0b18874dp-4);
    q = __builtin_fma(q, w, 0x1.2492408227507p-3);
    q = __builtin_fma(q, w, 0x1.999999a4af1eap-3);
    q = __builtin_fma(q, w, 0x1.5555555552c78p-2);
    const double s_2 = s + s;
    const double l = __builtin_fma(s_2 * w, q, s_2) + (hi ? 0x1.62e42fefa39efp-1 : 0.0);  // + ln 2
    const double r = __builtin_fmax(x, 0.0) + l;  // x <= 0: l exactly
    return x > 0x1.62e42fefa39efp+9 ? __builtin_inf() : r;  // 709.782712893384
}

// mish = x * tanh(log u), u = 1 + e^x, tanh(log u) = (u^2 - 1)/(u^2 + 1), from
// one exponential s = e^{-|x|} and one division, no branch (a wave holds both
// signs):
//   x <= 0:  t = (1 + s) - 1, the reference's rounding of u kept exactly;
//            g = t(2 + t) / (t(2 + t) + 2)
//   x > 0:   with t = 1/s:  g = (1 + 2s) / (1 + 2s + 2s^2)  (no overflow for
//            large x; u's rounding moves g by ~1e-16 here, where g ~ 1)
NH_DEV double mish_d(double x)
{
    const double s = exp(-__builtin_fabs(x));
    const bool pos = x > 0.0;
    const double t = (1.0 + s) - 1.0;
    const double num = pos ? __builtin_fma(2.0, s, 1.0) : t * (2.0 + t);
    const double den = num + (pos ? 2.0 * (s * s) : 2.0);
    return x * (num * rcp_nr2(den));
}

// ---- f32 outputs ----------------------------------------------------------------
// An f32 result only needs the reference's value to 1e-5 relative, so where the
// reference's double roundings are invisible at that level the formula runs in
// float (device expf / log1pf / tanhf, a few ulp), and the double closed forms
// above take over only where the quantization shows:
//   softplus, mish: x < -20, where 1 + exp(x) keeps fewer than 31 bits of exp(x)
//                   (above it the quantization is < 5.4e-8 relative);
//   gelu:           z < -8, where 1 + tanh(z) < 2.3e-7 is a multiple of 2^-53
//                   (quantization < 4.9e-10 relative) and the float head's
//                   error would approach the bar;
//   swish:          x < -80, where exp(-x) leaves float's range.
// Inputs of magnitude below 2^-30 (where outputs can be denormal, so a second
// rounding would show) take the double formula's linear term exactly.

NH_DEV float rcp_f32(float a) { return __builtin_amdgcn_rcpf(a); }  // 1 ulp, a in [1, 2^126)

// log(1 + e) for e in [0, 1] in float: 2 atanh(s), s = e / (2 + e) <= 1/3, odd
// series through s^13 (truncation below 1.5e-8 relative).
NH_DEV float log1p_01(float e)
{
    const float s = e * rcp_f32(2.0f + e);
    const float s2 = s * s;
    float q = 1.0f / 13.0f;
    q = __builtin_fmaf(q, s2, 1.0f / 11.0f);
    q = __builtin_fmaf(q, s2, 1.0f / 9.0f);
    q = __builtin_fmaf(q, s2, 1.0f / 7.0f);
    q = __builtin_fmaf(q, s2, 1.0f / 5.0f);
    q = __builtin_fmaf(q, s2, 1.0f / 3.0f);
    const float s_2 = s + s;
    return __builtin_fmaf(s_2 * s2, q, s_2);
}

// Each f32 activation below is a head (float formula, every element, with the
// `need` flag for the region where the reference's double rounding shows) and
// a tail (the exact double evaluation for those elements).
struct GeluF32 {
    static constexpr bool kHeadTail = true;
    NH_DEV float head(float xf, bool &need) const
    {
        // z in float: x + 0.044715 x^3 adds terms of one sign (no
        // cancellation), so z is within ~3 ulp (3.6e-7 relative) of the
        // reference's double z; w = exp(-2|z|) = 2^a with a rounded to float:
        // |a| <= 23.1 where the head is used, so w (and 1 + tanh z = 2w / (1 + w)
        // for z < 0) is off by at most 2 |dz| + 9.5e-7 <= 6.7e-6 relative at
        // the tail threshold z = -8, a third inside the 1e-5 f32 bar.  Below
        // it (1 + tanh z < 2.3e-7, where the bound would grow towards the bar)
        // the double tail takes over.
        const float z = float(kGelu) * (xf + 0.044715f * xf * xf * xf);
        need = z < -8.0f;
        const float w = __builtin_amdgcn_exp2f(-2.0f * 1.44269504f * __builtin_fabsf(z));
        const float r = rcp_f32(1.0f + w);
        const float onept = z >= 0.0f ? 2.0f * r : (w + w) * r;
        return (0.5f * xf) * onept;
    }
    NH_DEV float tail(float xf) const
    {
        const double x = double(xf);
        const double z = kGelu * (x + 0.044715 * x * x * x);
        // 1 + tanh z, a multiple of 2^-53 in the reference (tanh z in [-1, -0.5])
        const double w = exp(z + z);               // < 1.2e-7 (z < -8 within float's error)
        const double eps = (w + w) * (1.0 - w);   // 2w / (1 + w) to 2 w^3 < 3.4e-21 absolute
        return float(0.5 * x * (__builtin_rint(eps * 0x1p53) * 0x1p-53));
    }
};

// softplus = max(x, 0) + log1p(s), s = e^{-|x|} as one hardware exp2 (as in
// mish: within ~8e-7 relative for |x| <= 20; for x > 0 the error of s is
// damped by the + x); no branch.
struct SoftplusF32 {
    static constexpr bool kHeadTail = true;
    NH_DEV float head(float x, bool &need) const
    {
        need = x < -20.0f;  // 1 + exp(x) keeps < 31 bits of exp(x) in the reference
        const float s = __builtin_amdgcn_exp2f(-1.44269504f * __builtin_fabsf(x));
        const float y = __builtin_fmaxf(x, 0.0f) + log1p_01(s);
        return x >= 709.78271484375f ? __builtin_inff() : y;  // the reference's double exp overflows there
    }
    NH_DEV float tail(float x) const
    {
        const double t = (1.0 + exp(double(x))) - 1.0;  // the reference's quantized exp(x); t < 2.1e-9
        return float(t - 0.5 * t * t);                  // log1p(t), truncation t^3/3
    }
};

// mish: tanh(log u) from t = u - 1: t(2+t) / (t(2+t) + 2) for t <= 1, else
// 1 - 2/(u^2 + 1).
NH_DEV float mish_from_t(float x, float t)
{
    float g;
    if (t <= 1.0f) {
        const float a = t * (2.0f + t);
        g = a * rcp_f32(a + 2.0f);
    } else {
        const float u = 1.0f + t;
        g = 1.0f - 2.0f * rcp_f32(__builtin_fmaf(u, u, 1.0f));
    }
    return x * g;
}

// The head is the branch-free form of mish_d in float: s = e^{-|x|} as one
// hardware exp2 (the product |x| log2 e rounds to within 9.5e-7 of the
// exponent for |x| <= 20, so s and, for x <= 0, g ~ s are within ~8e-7
// relative; for x > 0, g ~ 1 - 2s^2 hides s's error).  Near 0, g is 0.6
// to a few float ulps, so x * g rounds like the reference's x * 0.6 except
// where x * 0.6 lies within g's error of a rounding midpoint: for denormal
// outputs k ulps long that needs k > 2.8e5 (0.6 k is at least 0.1 ulp from a
// midpoint), an error below 4e-6 relative.
struct MishF32 {
    static constexpr bool kHeadTail = true;
    NH_DEV float head(float x, bool &need) const
    {
        need = x < -20.0f;
        const float s = __builtin_amdgcn_exp2f(-1.44269504f * __builtin_fabsf(x));
        const bool pos = x > 0.0f;
        const float num = pos ? __builtin_fmaf(2.0f, s, 1.0f) : s * (s + 2.0f);
        const float den = num + (pos ? 2.0f * (s * s) : 2.0f);
        return x * (num * rcp_f32(den));
    }
    NH_DEV float tail(float x) const { return mish_from_t(x, float((1.0 + exp(double(x))) - 1.0)); }
};

struct SwishF32 {
    static constexpr bool kHeadTail = true;
    NH_DEV float head(float x, bool &need) const
    {
        need = x < -80.0f;  // exp(-x) leaves float's range
        return x * rcp_f32(1.0f + expf(-x));
    }
    NH_DEV float tail(float x) const { return float(double(x) / (1.0 + exp(-double(x)))); }
};

// elu / selu, f32: x > 0 is the reference's double product; below, the
// reference's alpha * (exp(x) - 1.0) with the float expm1.  The reference's
// double exp(x) - 1.0 carries an absolute error of ~1.1e-16, below 1e-8
// relative for |x| >= 2^-26, so there the float result matches it to ~2 float
// ulps; smaller |x| (and zeros) keep the double formula.
struct EluF32 {
    double alpha;
    static constexpr bool kHeadTail = true;
    NH_DEV float head(float x, bool &need) const
    {
        need = x <= 0.0f && x > -0x1p-26f;
        return x > 0.0f ? x : float(alpha * double(expm1f(x)));
    }
    NH_DEV float tail(float x) const { return float(alpha * (exp(double(x)) - 1.0)); }
};

struct SeluF32 {
    static constexpr bool kHeadTail = true;
    NH_DEV float head(float x, bool &need) const
    {
        need = x <= 0.0f && x > -0x1p-26f;
        return x > 0.0f ? float(kSeluL * double(x)) : float(kSeluL * kSeluA * double(expm1f(x)));
    }
    NH_DEV float tail(float x) const { return float(kSeluL * kSeluA * (exp(double(x)) - 1.0)); }
};

// ---- functors ----------------------------------------------------------------------

// Reference formula (or its closed form) in double; f32 tensors round once.
struct ATanh { NH_DEV double f(double x) const { return tanh_d(x); } };
struct AGelu { NH_DEV double f(double x) const { return gelu_d(x); } };
struct ALeaky { double alpha; NH_DEV double f(double x) const { return x >= 0 ? x : alpha * x; } };
struct AElu { double alpha; NH_DEV double f(double x) const { return x > 0 ? x : alpha * (exp(x) - 1.0); } };
struct ASelu { NH_DEV double f(double x) const { return x > 0 ? kSeluL * x : kSeluL * kSeluA * (exp(x) - 1.0); } };
struct ASwish { NH_DEV double f(double x) const { return x / (1.0 + exp(-x)); } };
struct AMish { NH_DEV double f(double x) const { return mish_d(x); } };
struct AHardswish { NH_DEV double f(double x) const { return x <= -3.0 ? 0.0 : (x >= 3.0 ? x : x * (x + 3.0) / 6.0); } };
struct ASoftplus { NH_DEV double f(double x) const { return softplus_d(x); } };
struct AHardtanh { NH_DEV double f(double x) const { return x < -1.0 ? -1.0 : (x > 1.0 ? 1.0 : x); } };
struct ASigmoid { NH_DEV double f(double x) const { return 1.0 / (1.0 + exp(x * -1.0)); } };

// Elementwise functor over both dtypes from a double formula.
template <class A>
struct ActFn {
    A a;
    NH_DEV float operator()(float x) const { return float(a.f(double(x))); }
    NH_DEV double operator()(double x) const { return a.f(x); }
};

// f32 functor from a head/tail pair (k_map1_f32_tail on aligned contiguous
// tensors; per element otherwise).
template <class H>
struct HeadTailFn {
    H h;
    static constexpr bool kHeadTail = true;
    NH_DEV float head(float x, bool &need) const { return h.head(x, need); }
    NH_DEV float tail(float x) const { return h.tail(x); }
    NH_DEV float operator()(float x) const
    {
        bool need = false;
        const float y = h.head(x, need);
        return need ? h.tail(x) : y;
    }
};

// hardswish on f32 tensors: the reference's double x * (x + 3.0) / 6.0 with
// the division by 6 replaced by the product with RN(1/6).  The double results
// can differ in the last bit, but after the rounding to float they agree for
// every float input (checked exhaustively against the reference expression
// over (-3, 3) on the CPU, zero signs included): one FP64 multiply in place of
// the division's ten instructions.
struct HardswishF32Fn {
    NH_DEV float operator()(float xf) const
    {
        const double x = double(xf);
        const double d = (x * (x + 3.0)) * (1.0 / 6.0);
        return xf <= -3.0f ? 0.0f : (xf >= 3.0f ? xf : float(d));
    }
};

// tanh on f32 tensors, in float: |x| < 0.1 by the odd Taylor series through
// x^7 (truncation below 3e-10 relative; the sign of zeros kept); above it
// (1 - e) / (1 + e) with e = e^{-2|x|} as one hardware exp2 (~2e-7 relative,
// amplified at most 5.5x by the exact subtraction 1 - e for |x| >= 0.1) and
// the hardware reciprocal, then the sign of x.  Within ~1.2e-6 of the
// reference's (float) tanh((double) x); NaN stays NaN, large |x| gives +-1.
struct TanhF32Fn {
    NH_DEV float operator()(float x) const
    {
        const float a = __builtin_fabsf(x);
        const float x2 = x * x;
        const float small = __builtin_copysignf(
            __builtin_fmaf(x * x2, __builtin_fmaf(x2, __builtin_fmaf(x2, -17.0f / 315.0f, 2.0f / 15.0f), -1.0f / 3.0f),
                           x),
            x);
        const float e = __builtin_amdgcn_exp2f(-2.88539008f * a);  // 2 / ln 2
        const float big = __builtin_copysignf((1.0f - e) * rcp_f32(1.0f + e), x);
        return a < 0.1f ? small : big;
    }
};

template <class A, class F32>
static int act2(void *out, const void *in, F32 f32, A a = A{})
{
    if (!out || !in) return set_error(NEURAL_ERR_NULL_POINTER);
    ActFn<A> f64{a};
    return run_unary(static_cast<NeuralTensor *>(out), static_cast<const NeuralTensor *>(in), f32, f64);
}

template <class A>
static int act(void *out, const void *in, A a = A{})
{
    return act2<A>(out, in, ActFn<A>{a}, a);
}

static int act_gelu_impl(void *out, const void *in) { return act2<AGelu>(out, in, HeadTailFn<GeluF32>{}); }
static int act_swish_impl(void *out, const void *in) { return act2<ASwish>(out, in, HeadTailFn<SwishF32>{}); }
static int act_mish_impl(void *out, const void *in) { return act2<AMish>(out, in, HeadTailFn<MishF32>{}); }
static int act_softplus_impl(void *out, const void *in) { return act2<ASoftplus>(out, in, HeadTailFn<SoftplusF32>{}); }
static int act_tanh_impl(void *out, const void *in) { return act2<ATanh>(out, in, TanhF32Fn{}); }
static int act_elu_impl(void *out, const void *in, double alpha)
{
    return act2<AElu>(out, in, HeadTailFn<EluF32>{EluF32{alpha}}, AElu{alpha});
}
static int act_selu_impl(void *out, const void *in) { return act2<ASelu>(out, in, HeadTailFn<SeluF32>{}); }

// Bias add then activation, one pass: y = act(x + b) with x + b rounded in
// the tensor's dtype first (nn_layers.asm:472-539 then activations_c.c), so
// the result equals neural_bias_add followed by the activation bit for bit.
template <class F32, class F64>
struct OpAddAct {
    using F32T = F32;
    F32 f32;
    F64 f64;
    NH_DEV float operator()(float x, float b) const { return f32(x + b); }
    NH_DEV double operator()(double x, double b) const { return f64(x + b); }
};
template <class F32, class F64>
OpAddAct<F32, F64> add_act(F32 f32, F64 f64) { return {f32, f64}; }

struct FnReluAct {
    NH_DEV float operator()(float x) const { return x > 0.0f ? x : 0.0f; }
    NH_DEV double operator()(double x) const { return x > 0.0 ? x : 0.0; }
};
struct FnIdentity {
    template <class T> NH_DEV T operator()(T x) const { return x; }
};

static int bias_add_act(NeuralTensor *out, const NeuralTensor *x, const NeuralTensor *bias, int act, double alpha)
{
    if (!out || !x || !bias) return set_error(NEURAL_ERR_NULL_POINTER);
    if (bias->ndim < 1 || x->ndim < 1 || numel(bias) != x->shape[x->ndim - 1])
        return set_error(NEURAL_ERR_SHAPE_MISMATCH);
    if (out->ndim != x->ndim) return set_error(NEURAL_ERR_SHAPE_MISMATCH);
    for (int64_t i = 0; i < x->ndim; i++)
        if (out->shape[i] != x->shape[i]) return set_error(NEURAL_ERR_SHAPE_MISMATCH);
    switch (act) {
    case NEURAL_ACT_NONE: return binary_api(out, x, bias, add_act(FnIdentity{}, FnIdentity{}));
    case NEURAL_ACT_RELU: return binary_api(out, x, bias, add_act(FnReluAct{}, FnReluAct{}));
    case NEURAL_ACT_SIGMOID: return binary_api(out, x, bias, add_act(ActFn<ASigmoid>{}, ActFn<ASigmoid>{}));
    case NEURAL_ACT_TANH: return binary_api(out, x, bias, add_act(TanhF32Fn{}, ActFn<ATanh>{}));
    case NEURAL_ACT_GELU: return binary_api(out, x, bias, add_act(HeadTailFn<GeluF32>{}, ActFn<AGelu>{}));
    case NEURAL_ACT_LEAKY_RELU:
        return binary_api(out, x, bias, add_act(ActFn<ALeaky>{ALeaky{alpha}}, ActFn<ALeaky>{ALeaky{alpha}}));
    case NEURAL_ACT_ELU:
        return binary_api(out, x, bias, add_act(HeadTailFn<EluF32>{EluF32{alpha}}, ActFn<AElu>{AElu{alpha}}));
    case NEURAL_ACT_SELU: return binary_api(out, x, bias, add_act(HeadTailFn<SeluF32>{}, ActFn<ASelu>{}));
    case NEURAL_ACT_SWISH: return binary_api(out, x, bias, add_act(HeadTailFn<SwishF32>{}, ActFn<ASwish>{}));
    case NEURAL_ACT_MISH: return binary_api(out, x, bias, add_act(HeadTailFn<MishF32>{}, ActFn<AMish>{}));
    case NEURAL_ACT_HARDSWISH: return binary_api(out, x, bias, add_act(HardswishF32Fn{}, ActFn<AHardswish>{}));
    case NEURAL_ACT_SOFTPLUS:
        return binary_api(out, x, bias, add_act(HeadTailFn<SoftplusF32>{}, ActFn<ASoftplus>{}));
    case NEURAL_ACT_HARDTANH: return binary_api(out, x, bias, add_act(ActFn<AHardtanh>{}, ActFn<AHardtanh>{}));
    default: return set_error(NEURAL_ERR_INVALID_ARGUMENT);
    }
}

}  // namespace nh

using namespace nh;

extern "C" {

int act_tanh(void *out, const void *in) { return act_tanh_impl(out, in); }
int act_gelu(void *out, const void *in) { return act_gelu_impl(out, in); }
int act_leaky_relu(void *out, const void *in, double alpha) { return act<ALeaky>(out, in, ALeaky{alpha}); }
int act_elu(void *out, const void *in, double alpha) { return act_elu_impl(out, in, alpha); }
int act_selu(void *out, const void *in) { return act_selu_impl(out, in); }
int act_swish(void *out, const void *in) { return act_swish_impl(out, in); }
int act_mish(void *out, const void *in) { return act_mish_impl(out, in); }
int act_hardswish(void *out, const void *in) { return act2<AHardswish>(out, in, HardswishF32Fn{}); }
int act_softplus(void *out, const void *in) { return act_softplus_impl(out, in); }
int act_hardtanh(void *out, const void *in) { return act<AHardtanh>(out, in); }

// Tensor-typed aliases of the header's neural_* activations
// (neural_api.h:387-486).
int neural_sigmoid(NeuralTensor *out, const NeuralTensor *in) { return act<ASigmoid>(out, in); }
int neural_tanh(NeuralTensor *out, const NeuralTensor *in) { return act_tanh_impl(out, in); }
int neural_gelu(NeuralTensor *out, const NeuralTensor *in) { return act_gelu_impl(out, in); }
int neural_leaky_relu(NeuralTensor *out, const NeuralTensor *in, double alpha) { return act<ALeaky>(out, in, ALeaky{alpha}); }
int neural_elu(NeuralTensor *out, const NeuralTensor *in, double alpha) { return act_elu_impl(out, in, alpha); }
int neural_selu(NeuralTensor *out, const NeuralTensor *in) { return act_selu_impl(out, in); }
int neural_swish(NeuralTensor *out, const NeuralTensor *in) { return act_swish_impl(out, in); }
int neural_mish(NeuralTensor *out, const NeuralTensor *in) { return act_mish_impl(out, in); }
int neural_hardswish(NeuralTensor *out, const NeuralTensor *in) { return act2<AHardswish>(out, in, HardswishF32Fn{}); }
int neural_softplus(NeuralTensor *out, const NeuralTensor *in) { return act_softplus_impl(out, in); }
int neural_hardtanh(NeuralTensor *out, const NeuralTensor *in) { return act<AHardtanh>(out, in); }

int neural_bias_add_act(NeuralTensor *out, const NeuralTensor *x, const NeuralTensor *bias, int act, double alpha)
{
    return bias_add_act(out, x, bias, act, alpha);
}

}  // extern "C"
