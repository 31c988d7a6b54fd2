/* Exhaustive CPU checks of arithmetic identities the device kernels rely on.
 *
 * Built by tests/test_identities.py with the reference's flags plus
 * -ffp-contract=off (no contraction: every a * b + c below is two roundings
 * unless written as fma()).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static float f32_of_bits(uint32_t u)
{
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static uint32_t bits_of_f32(float f)
{
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

/* bitwise equal, NaN compared by class */
static int same_f32(float a, float b)
{
    return (a != a && b != b) || bits_of_f32(a) == bits_of_f32(b);
}

/* activations_c.c:154 (hardswish) on a float widened to double, stored as
 * float (activations_c.c:71-77). */
static float hardswish_reference(float xf)
{
    const double x = (double)xf;
    return (float)(x <= -3.0 ? 0.0 : (x >= 3.0 ? x : x * (x + 3.0) / 6.0));
}

/* The f32 kernel's form (activations.hip, HardswishF32Fn): the division by
 * 6 replaced by the product with RN(1/6). */
static float hardswish_kernel(float xf, double sixth)
{
    const double x = (double)xf;
    const double d = (x * (x + 3.0)) * sixth;
    return xf <= -3.0f ? 0.0f : (xf >= 3.0f ? xf : (float)d);
}

/* Number of float bit patterns u in [lo, hi) whose two hardswish results
 * differ (bitwise, NaN by class), the kernel form taking `sixth` as its
 * constant (the kernel's is 1.0 / 6.0); the first one found is stored in
 * *first. */
int64_t hardswish_f32_mismatches(uint64_t lo, uint64_t hi, double sixth, uint32_t *first)
{
    int64_t bad = 0;
    for (uint64_t u = lo; u < hi; u++) {
        const float x = f32_of_bits((uint32_t)u);
        if (!same_f32(hardswish_reference(x), hardswish_kernel(x, sixth))) {
            if (bad == 0) *first = (uint32_t)u;
            bad++;
        }
    }
    return bad;
}

/* The same comparison for the formula evaluated in float arithmetic (a
 * plausible slip for an f32 kernel), so the test shows the check catches it. */
int64_t hardswish_f32_mismatches_planted(uint64_t lo, uint64_t hi)
{
    int64_t bad = 0;
    for (uint64_t u = lo; u < hi; u++) {
        const float xf = f32_of_bits((uint32_t)u);
        const float k = xf <= -3.0f ? 0.0f : (xf >= 3.0f ? xf : xf * (xf + 3.0f) / 6.0f);
        if (!same_f32(hardswish_reference(xf), k)) bad++;
    }
    return bad;
}
