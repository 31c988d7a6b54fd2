/*
 * cpu_baseline.c -- the reference's host SIMD loops, restated in C with
 * intrinsics, for the CPU baseline that bench.py reports beside the GPU.
 *
 * TEST INFRASTRUCTURE ONLY, like neural_oracle.c: loaded by bench.py's
 * cpu_baseline legs and by tests/ (which check these loops against the oracle
 * bit for bit); the product never loads it.
 *
 * Each function keeps the reference loop's instruction-set width, lane order
 * and pass structure, so its time is what the reference's own code costs on
 * the host it runs on:
 *   - ew_add / ew_mul f32: 8-wide vmovups/vaddps (vmulps) + a scalar tail
 *     (math_kernels.asm:98-131, 292-...);
 *   - reduce_sum f32 (axis -1): one 8-lane ymm accumulator, vextractf128 +
 *     vaddps, two vhaddps, then the scalar tail (math_kernels.asm:1124-1161);
 *   - simd.asm's AVX-512 path (get_simd_level == 4): 16-wide add / mul
 *     (simd.asm:190-306) and the zmm sum folded 16 -> 8 -> 4 -> hadd x2
 *     (simd.asm:684-784); exported but never called in the reference tree;
 *   - tensor_grad_l2_norm: a 4-lane SSE mulps/addps accumulator, movhlps +
 *     addps + shufps 0x55 + addss, the scalar tail, sqrtss
 *     (training_ops.asm:636-696);
 *   - neural_relu -> node_relu: a zero-filled 32-byte-aligned temporary
 *     (tensor_create), the scalar maxss loop, then neural_tensor_copy into the
 *     caller's tensor (neural_api.asm:1218-1274, activations.asm:114-200).
 * Each intrinsics function carries its own target attribute; callers check
 * cpu_has_avx() / cpu_has_avx512f() first (bench.py does).
 */
#include <immintrin.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

int cpu_has_avx(void) { return __builtin_cpu_supports("avx"); }
int cpu_has_avx512f(void) { return __builtin_cpu_supports("avx512f"); }

/* ---- math_kernels.asm: AVX-256 ------------------------------------------------ */

__attribute__((target("avx"))) void cpu_ew_add_avx(const float *a, const float *b, float *out, int64_t n)
{
    int64_t nv = n >> 3, i = 0;
    for (int64_t k = 0; k < nv; k++, i += 8)
        _mm256_storeu_ps(out + i, _mm256_add_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i)));
    for (; i < n; i++) out[i] = a[i] + b[i];
    _mm256_zeroupper();
}

__attribute__((target("avx"))) void cpu_ew_mul_avx(const float *a, const float *b, float *out, int64_t n)
{
    int64_t nv = n >> 3, i = 0;
    for (int64_t k = 0; k < nv; k++, i += 8)
        _mm256_storeu_ps(out + i, _mm256_mul_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i)));
    for (; i < n; i++) out[i] = a[i] * b[i];
    _mm256_zeroupper();
}

__attribute__((target("avx"))) float cpu_reduce_sum_avx(const float *x, int64_t n)
{
    __m128 acc = _mm_setzero_ps();
    int64_t nv = n >> 3, i = 0;
    if (nv > 0) {
        __m256 l = _mm256_setzero_ps();
        for (int64_t k = 0; k < nv; k++, i += 8) l = _mm256_add_ps(l, _mm256_loadu_ps(x + i));
        __m128 lo = _mm256_castps256_ps128(l), hi = _mm256_extractf128_ps(l, 1);
        acc = _mm_add_ps(lo, hi);
        acc = _mm_hadd_ps(acc, acc);
        acc = _mm_hadd_ps(acc, acc);
    }
    float s = _mm_cvtss_f32(acc);
    for (; i < n; i++) s = s + x[i];
    _mm256_zeroupper();
    return s;
}

/* ---- simd.asm: the AVX-512 path ------------------------------------------------ */

__attribute__((target("avx512f"))) void cpu_simd_add_avx512(const float *a, const float *b, float *out, int64_t n)
{
    int64_t nv = n >> 4, i = 0;
    for (int64_t k = 0; k < nv; k++, i += 16)
        _mm512_storeu_ps(out + i, _mm512_add_ps(_mm512_loadu_ps(a + i), _mm512_loadu_ps(b + i)));
    for (; i < n; i++) out[i] = a[i] + b[i];
    _mm256_zeroupper();
}

__attribute__((target("avx512f"))) void cpu_simd_mul_avx512(const float *a, const float *b, float *out, int64_t n)
{
    int64_t nv = n >> 4, i = 0;
    for (int64_t k = 0; k < nv; k++, i += 16)
        _mm512_storeu_ps(out + i, _mm512_mul_ps(_mm512_loadu_ps(a + i), _mm512_loadu_ps(b + i)));
    for (; i < n; i++) out[i] = a[i] * b[i];
    _mm256_zeroupper();
}

__attribute__((target("avx512f"))) float cpu_simd_sum_avx512(const float *x, int64_t n)
{
    __m128 acc = _mm_setzero_ps();
    int64_t nv = n >> 4, i = 0;
    if (nv > 0) {
        __m512 l = _mm512_setzero_ps();
        for (int64_t k = 0; k < nv; k++, i += 16) l = _mm512_add_ps(l, _mm512_loadu_ps(x + i));
        /* vextractf32x8 + vaddps (16 -> 8), vextractf128 + vaddps (8 -> 4) */
        __m256 lo8 = _mm512_castps512_ps256(l);
        __m256 hi8 = _mm256_castpd_ps(_mm512_extractf64x4_pd(_mm512_castps_pd(l), 1));
        __m256 s8 = _mm256_add_ps(lo8, hi8);
        acc = _mm_add_ps(_mm256_castps256_ps128(s8), _mm256_extractf128_ps(s8, 1));
        acc = _mm_hadd_ps(acc, acc);
        acc = _mm_hadd_ps(acc, acc);
    }
    float s = _mm_cvtss_f32(acc);
    for (; i < n; i++) s = s + x[i];
    _mm256_zeroupper();
    return s;
}

/* ---- training_ops.asm: SSE 4-lane L2 norm -------------------------------------- */

float cpu_l2_sse(const float *x, uint64_t n)
{
    if (!x || n == 0) return 0.0f;
    __m128 acc = _mm_setzero_ps();
    uint64_t nv = n >> 2, i = 0;
    for (uint64_t k = 0; k < nv; k++, i += 4) {
        __m128 v = _mm_loadu_ps(x + i);
        acc = _mm_add_ps(acc, _mm_mul_ps(v, v));
    }
    if (nv > 0) {
        __m128 h = _mm_movehl_ps(acc, acc);                   /* movhlps: lanes 2,3 -> 0,1 */
        acc = _mm_add_ps(acc, h);                             /* (l0+l2), (l1+l3) */
        __m128 e1 = _mm_shuffle_ps(acc, acc, 0x55);           /* element 1 */
        acc = _mm_add_ss(acc, e1);
    }
    for (; i < n; i++) {
        __m128 v = _mm_load_ss(x + i);
        acc = _mm_add_ss(acc, _mm_mul_ss(v, v));
    }
    return _mm_cvtss_f32(_mm_sqrt_ss(acc));
}

/* ---- neural_relu -> node_relu --------------------------------------------------- */

int cpu_relu_node(const float *x, float *out, int64_t n)
{
    size_t bytes = (size_t)(n > 0 ? n : 1) * sizeof(float);
    bytes = (bytes + 31) & ~(size_t)31;
    float *tmp = (float *)aligned_alloc(32, bytes);
    if (!tmp) return -1;
    memset(tmp, 0, bytes); /* tensor_create zero-fills */
    const __m128 z = _mm_setzero_ps();
    for (int64_t i = 0; i < n; i++) /* maxss x, 0: NaN and -0 give +0 */
        _mm_store_ss(tmp + i, _mm_max_ss(_mm_load_ss(x + i), z));
    memcpy(out, tmp, (size_t)n * sizeof(float)); /* neural_tensor_copy */
    free(tmp);
    return 0;
}
