/*
 * neural_oracle.c -- CPU restatement of the Neural-Assembly tensor hot path.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the product).  See
 * neural_oracle.h for what pins each function.  Build: oracle/Makefile,
 * -O2 -std=c11 -ffp-contract=off, no -ffast-math, no -march (SSE2 only, as
 * the reference's own C flags in Makefile:12).
 *
 * Reference paths below are relative to the Neural-Assembly source tree.
 */
#include "neural_oracle.h"

#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* Elementwise: src/asm/math_kernels.asm:66-945                              */
/* ------------------------------------------------------------------------ */

/* ew_add/sub/mul/div/max (math_kernels.asm:66-507,730-835): out[i] = a[i] op b[i]
 * over the flat element range.  vmaxps/maxss return the second operand
 * unless the first is strictly greater, so max(a,b) = (a > b) ? a : b. */
void ora_ew_f32(int op, const float *a, const float *b, float *out, int64_t n)
{
    for (int64_t i = 0; i < n; i++) {
        float x = a[i], y = b[i];
        switch (op) {
        case ORA_ADD: out[i] = x + y; break;
        case ORA_SUB: out[i] = x - y; break;
        case ORA_MUL: out[i] = x * y; break;
        case ORA_DIV: out[i] = x / y; break;
        default:      out[i] = (x > y) ? x : y; break;
        }
    }
}

void ora_ew_f64(int op, const double *a, const double *b, double *out, int64_t n)
{
    for (int64_t i = 0; i < n; i++) {
        double x = a[i], y = b[i];
        switch (op) {
        case ORA_ADD: out[i] = x + y; break;
        case ORA_SUB: out[i] = x - y; break;
        case ORA_MUL: out[i] = x * y; break;
        case ORA_DIV: out[i] = x / y; break;
        default:      out[i] = (x > y) ? x : y; break;
        }
    }
}

/* ew_scalar_add / ew_scalar_mul (math_kernels.asm:516-725): the scalar arrives
 * as a double and is rounded to float once (cvtsd2ss, :544/:653) for f32. */
void ora_scalar_f32(int op, const float *a, double s, float *out, int64_t n)
{
    float sf = (float)s;
    for (int64_t i = 0; i < n; i++)
        out[i] = (op == ORA_ADD) ? a[i] + sf : a[i] * sf;
}

void ora_scalar_f64(int op, const double *a, double s, double *out, int64_t n)
{
    for (int64_t i = 0; i < n; i++)
        out[i] = (op == ORA_ADD) ? a[i] + s : a[i] * s;
}

/* ew_neg (math_kernels.asm:843-945): xor with the sign-bit mask, which also
 * flips the sign of NaNs and zeros. */
void ora_neg_f32(const float *a, float *out, int64_t n)
{
    for (int64_t i = 0; i < n; i++) {
        uint32_t u;
        memcpy(&u, &a[i], 4);
        u ^= 0x80000000u;
        memcpy(&out[i], &u, 4);
    }
}

void ora_neg_f64(const double *a, double *out, int64_t n)
{
    for (int64_t i = 0; i < n; i++) {
        uint64_t u;
        memcpy(&u, &a[i], 8);
        u ^= 0x8000000000000000ull;
        memcpy(&out[i], &u, 8);
    }
}

/* node_relu (activations.asm:153-171): maxss x, 0 -> (x > 0) ? x : +0.0, so
 * NaN -> +0 and -0 -> +0. */
void ora_relu_f32(const float *a, float *out, int64_t n)
{
    for (int64_t i = 0; i < n; i++) out[i] = (a[i] > 0.0f) ? a[i] : 0.0f;
}

void ora_relu_f64(const double *a, double *out, int64_t n)
{
    for (int64_t i = 0; i < n; i++) out[i] = (a[i] > 0.0) ? a[i] : 0.0;
}

/* Row-broadcast bias add inside linear_forward_fn (nn_layers.asm:472-539):
 * out[i*cols + j] = mm[i*cols + j] + bias[j]. */
void ora_bias_add_f32(const float *x, const float *b, float *out, int64_t rows, int64_t cols)
{
    for (int64_t i = 0; i < rows; i++)
        for (int64_t j = 0; j < cols; j++)
            out[i * cols + j] = x[i * cols + j] + b[j];
}

void ora_bias_add_f64(const double *x, const double *b, double *out, int64_t rows, int64_t cols)
{
    for (int64_t i = 0; i < rows; i++)
        for (int64_t j = 0; j < cols; j++)
            out[i * cols + j] = x[i * cols + j] + b[j];
}

/* ------------------------------------------------------------------------ */
/* Reductions: src/asm/math_kernels.asm:956-1264, main.asm:3245-3292,3598-3640 */
/* ------------------------------------------------------------------------ */

/* reduce_sum axis=-1, f32 (math_kernels.asm:1124-1161): eight running lanes
 * (vaddps), then (l0+l4),(l1+l5),(l2+l6),(l3+l7) (vextractf128 + vaddps),
 * two vhaddps -> ((s0+s1)+(s2+s3)), then the n%8 tail added one by one.
 * With n < 8 the vector block is skipped and the tail starts from 0. */
float ora_sum_ref_f32(const float *x, int64_t n)
{
    float l[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int64_t nv = n / 8;
    for (int64_t i = 0; i < nv; i++)
        for (int k = 0; k < 8; k++) l[k] = l[k] + x[i * 8 + k];
    float acc = 0.0f;
    if (nv > 0) {
        float s0 = l[0] + l[4], s1 = l[1] + l[5], s2 = l[2] + l[6], s3 = l[3] + l[7];
        acc = (s0 + s1) + (s2 + s3);
    }
    for (int64_t i = nv * 8; i < n; i++) acc = acc + x[i];
    return acc;
}

/* reduce_sum axis=-1, f64 (math_kernels.asm:1163-1196): four lanes,
 * (l0+l2),(l1+l3), one vhaddpd, then the n%4 tail. */
double ora_sum_ref_f64(const double *x, int64_t n)
{
    double l[4] = {0, 0, 0, 0};
    int64_t nv = n / 4;
    for (int64_t i = 0; i < nv; i++)
        for (int k = 0; k < 4; k++) l[k] = l[k] + x[i * 4 + k];
    double acc = 0.0;
    if (nv > 0) acc = (l[0] + l[2]) + (l[1] + l[3]);
    for (int64_t i = nv * 4; i < n; i++) acc = acc + x[i];
    return acc;
}

/* Neumaier-compensated double sum: the "fp64-exact" value the reduction
 * contract compares against (error below 2^-104 * sum|x| plus one final
 * rounding; f32 inputs are exact in double). */
#define NEUMAIER(T, x, n, out)                                           \
    do {                                                                 \
        double s_ = 0.0, c_ = 0.0;                                       \
        for (int64_t i_ = 0; i_ < (n); i_++) {                           \
            double v_ = (double)(x)[i_];                                 \
            double t_ = s_ + v_;                                         \
            if (fabs(s_) >= fabs(v_)) c_ += (s_ - t_) + v_;              \
            else c_ += (v_ - t_) + s_;                                   \
            s_ = t_;                                                     \
        }                                                                \
        (out) = s_ + c_;                                                 \
    } while (0)

double ora_sum_exact_f32(const float *x, int64_t n) { double r; NEUMAIER(float, x, n, r); return r; }
double ora_sum_exact_f64(const double *x, int64_t n) { double r; NEUMAIER(double, x, n, r); return r; }

void ora_rowsum_exact_f32(const float *x, int64_t rows, int64_t cols, double *out)
{
    for (int64_t i = 0; i < rows; i++) NEUMAIER(float, x + i * cols, cols, out[i]);
}

void ora_rowsum_exact_f64(const double *x, int64_t rows, int64_t cols, double *out)
{
    for (int64_t i = 0; i < rows; i++) NEUMAIER(double, x + i * cols, cols, out[i]);
}

/* reduce_sum axis=1 (math_kernels.asm:1061-1107): one strictly sequential
 * scalar accumulator per row, starting at +0. */
void ora_rowsum_ref_f32(const float *x, int64_t rows, int64_t cols, float *out)
{
    for (int64_t i = 0; i < rows; i++) {
        float acc = 0.0f;
        for (int64_t j = 0; j < cols; j++) acc = acc + x[i * cols + j];
        out[i] = acc;
    }
}

void ora_rowsum_ref_f64(const double *x, int64_t rows, int64_t cols, double *out)
{
    for (int64_t i = 0; i < rows; i++) {
        double acc = 0.0;
        for (int64_t j = 0; j < cols; j++) acc = acc + x[i * cols + j];
        out[i] = acc;
    }
}

/* reduce_sum axis=0 (math_kernels.asm:995-1058): zero out[cols], then add the
 * rows in order. */
void ora_colsum_ref_f32(const float *x, int64_t rows, int64_t cols, float *out)
{
    for (int64_t j = 0; j < cols; j++) out[j] = 0.0f;
    for (int64_t i = 0; i < rows; i++)
        for (int64_t j = 0; j < cols; j++) out[j] = x[i * cols + j] + out[j];
}

void ora_colsum_ref_f64(const double *x, int64_t rows, int64_t cols, double *out)
{
    for (int64_t j = 0; j < cols; j++) out[j] = 0.0;
    for (int64_t i = 0; i < rows; i++)
        for (int64_t j = 0; j < cols; j++) out[j] = x[i * cols + j] + out[j];
}

/* Running max as the softmax max pass does it (activations.asm:815-823 f64,
 * 888-895 f32): m = x0; m = maxss(m, x_j) = (m > x_j) ? m : x_j. */
float ora_max_chain_f32(const float *x, int64_t n)
{
    float m = x[0];
    for (int64_t j = 1; j < n; j++) m = (m > x[j]) ? m : x[j];
    return m;
}

double ora_max_chain_f64(const double *x, int64_t n)
{
    double m = x[0];
    for (int64_t j = 1; j < n; j++) m = (m > x[j]) ? m : x[j];
    return m;
}

void ora_rowmax_chain_f32(const float *x, int64_t rows, int64_t cols, float *out)
{
    for (int64_t i = 0; i < rows; i++) out[i] = ora_max_chain_f32(x + i * cols, cols);
}

void ora_rowmax_chain_f64(const double *x, int64_t rows, int64_t cols, double *out)
{
    for (int64_t i = 0; i < rows; i++) out[i] = ora_max_chain_f64(x + i * cols, cols);
}

/* tensor_argmax (main.asm:3598-3640) and the per-row argmax of
 * calculate_batch_accuracy (main.asm:3245-3270): idx = 0, m = x0; comiss/jbe
 * updates only when x_j > m (ordered), so ties keep the first index and NaNs
 * never win. */
int64_t ora_argmax_f32(const float *x, int64_t n)
{
    int64_t idx = 0;
    float m = x[0];
    for (int64_t j = 1; j < n; j++)
        if (x[j] > m) { m = x[j]; idx = j; }
    return idx;
}

int64_t ora_argmax_f64(const double *x, int64_t n)
{
    int64_t idx = 0;
    double m = x[0];
    for (int64_t j = 1; j < n; j++)
        if (x[j] > m) { m = x[j]; idx = j; }
    return idx;
}

void ora_rowargmax_f32(const float *x, int64_t rows, int64_t cols, int64_t *out)
{
    for (int64_t i = 0; i < rows; i++) out[i] = ora_argmax_f32(x + i * cols, cols);
}

void ora_rowargmax_f64(const double *x, int64_t rows, int64_t cols, int64_t *out)
{
    for (int64_t i = 0; i < rows; i++) out[i] = ora_argmax_f64(x + i * cols, cols);
}

/* ------------------------------------------------------------------------ */
/* Softmax / log-softmax rows                                                */
/* ------------------------------------------------------------------------ */

/* node_softmax, f32 (activations.asm:874-952), intended semantics (the asm
 * keeps max and sum in one stack slot, :900/:927-929): m = running maxss;
 * e_j = (float)exp((double)x_j - (double)m); s = sequential float sum of e_j;
 * y_j = e_j / s in float. */
void ora_softmax_rows_f32(const float *x, int64_t rows, int64_t cols, float *out)
{
    for (int64_t i = 0; i < rows; i++) {
        const float *r = x + i * cols;
        float *o = out + i * cols;
        float m = ora_max_chain_f32(r, cols);
        float s = 0.0f;
        for (int64_t j = 0; j < cols; j++) {
            float e = (float)exp((double)r[j] - (double)m);
            o[j] = e;
            s = s + e;
        }
        for (int64_t j = 0; j < cols; j++) o[j] = o[j] / s;
    }
}

/* node_softmax, f64 (activations.asm:800-871): m = running maxsd;
 * e_j = exp(x_j - m); s = sequential sum; y_j = e_j / s. */
void ora_softmax_rows_f64(const double *x, int64_t rows, int64_t cols, double *out)
{
    for (int64_t i = 0; i < rows; i++) {
        const double *r = x + i * cols;
        double *o = out + i * cols;
        double m = ora_max_chain_f64(r, cols);
        double s = 0.0;
        for (int64_t j = 0; j < cols; j++) {
            double e = exp(r[j] - m);
            o[j] = e;
            s = s + e;
        }
        for (int64_t j = 0; j < cols; j++) o[j] = o[j] / s;
    }
}

/* Log-softmax rows, formula of label_smoothing_ce_forward
 * (src/c/metrics_losses.c:47-64), in double: m = max (strict >, first wins),
 * L = log(sum_c exp(x_c - m)) sequential, y_c = (x_c - m) - L.  f32 tensors
 * widen on load and round the double result once. */
void ora_log_softmax_rows_f64(const double *x, int64_t rows, int64_t cols, double *out)
{
    for (int64_t i = 0; i < rows; i++) {
        const double *r = x + i * cols;
        double m = r[0];
        for (int64_t c = 1; c < cols; c++) if (r[c] > m) m = r[c];
        double lse = 0.0;
        for (int64_t c = 0; c < cols; c++) lse += exp(r[c] - m);
        lse = log(lse);
        for (int64_t c = 0; c < cols; c++) out[i * cols + c] = (r[c] - m) - lse;
    }
}

void ora_log_softmax_rows_f32(const float *x, int64_t rows, int64_t cols, float *out)
{
    for (int64_t i = 0; i < rows; i++) {
        const float *r = x + i * cols;
        double m = (double)r[0];
        for (int64_t c = 1; c < cols; c++) if ((double)r[c] > m) m = (double)r[c];
        double lse = 0.0;
        for (int64_t c = 0; c < cols; c++) lse += exp((double)r[c] - m);
        lse = log(lse);
        for (int64_t c = 0; c < cols; c++) out[i * cols + c] = (float)(((double)r[c] - m) - lse);
    }
}

/* ------------------------------------------------------------------------ */
/* Activations: src/c/activations_c.c:63-158 (double math, one rounding to   */
/* float for f32 tensors); sigmoid: activations.asm:352-413                  */
/* ------------------------------------------------------------------------ */

static const double K_GELU = 0.7978845608028654;
static const double K_SELU_L = 1.0507009873554804934193349852946;
static const double K_SELU_A = 1.6732632423543772848170429916717;

static double act_eval(int which, double x, double alpha)
{
    switch (which) {
    case ORA_TANH:       return tanh(x);
    case ORA_GELU:       return 0.5 * x * (1.0 + tanh(K_GELU * (x + 0.044715 * x * x * x)));
    case ORA_LEAKY_RELU: return x >= 0 ? x : alpha * x;
    case ORA_ELU:        return x > 0 ? x : alpha * (exp(x) - 1.0);
    case ORA_SELU:       return x > 0 ? K_SELU_L * x : K_SELU_L * K_SELU_A * (exp(x) - 1.0);
    case ORA_SWISH:      return x / (1.0 + exp(-x));
    case ORA_MISH:       return x * tanh(log(1.0 + exp(x)));
    case ORA_HARDSWISH:  return x <= -3.0 ? 0.0 : (x >= 3.0 ? x : x * (x + 3.0) / 6.0);
    case ORA_SOFTPLUS:   return log(1.0 + exp(x));
    case ORA_HARDTANH:   return x < -1.0 ? -1.0 : (x > 1.0 ? 1.0 : x);
    default:             return 1.0 / (1.0 + exp(x * -1.0));
    }
}

void ora_act_f32(int which, const float *in, float *out, int64_t n, double alpha)
{
    for (int64_t i = 0; i < n; i++) out[i] = (float)act_eval(which, (double)in[i], alpha);
}

void ora_act_f64(int which, const double *in, double *out, int64_t n, double alpha)
{
    for (int64_t i = 0; i < n; i++) out[i] = act_eval(which, in[i], alpha);
}

/* ------------------------------------------------------------------------ */
/* INT8 quantization: src/c/quantize.c:39-84,144-174,222-269                 */
/* ------------------------------------------------------------------------ */

/* (int32_t)round(v) as gcc emits it on x86-64: libm round, then cvttsd2si,
 * which yields INT32_MIN for NaN and for values outside int32 range. */
static int32_t x86_round_to_i32(double v)
{
    double r = round(v);
    if (!(r > -2147483649.0 && r < 2147483648.0)) return INT32_MIN;
    return (int32_t)r;
}

/* q = (int32)round(x * inv_scale) + zp with the x86 wrap-around add, then the
 * clamp to [-128, 127] (quantize.c:151-156). */
static int8_t quant_one(double x, double inv_scale, int32_t zp)
{
    int32_t q = (int32_t)((uint32_t)x86_round_to_i32(x * inv_scale) + (uint32_t)zp);
    if (q < -128) q = -128;
    if (q > 127) q = 127;
    return (int8_t)q;
}

/* Scalar epilogue of calibrate_minmax (quantize.c:62-82). */
static void minmax_params(double mn, double mx, int symmetric, OraQuantParams *out)
{
    if (symmetric) {
        double am = fmax(fabs(mn), fabs(mx));
        if (am < 1e-30) am = 1e-30;
        out->scale = am / 127.0;
        out->zero_point = 0;
        out->min_val = -am;
        out->max_val = am;
        out->symmetric = 1;
    } else {
        if (mn == mx) { mn -= 0.5; mx += 0.5; }
        out->scale = (mx - mn) / 255.0;
        if (out->scale < 1e-30) out->scale = 1e-30;
        out->zero_point = x86_round_to_i32(-128.0 - mn / out->scale);
        if (out->zero_point < -128) out->zero_point = -128;
        if (out->zero_point > 127) out->zero_point = 127;
        out->min_val = mn;
        out->max_val = mx;
        out->symmetric = 0;
    }
}

/* calibrate_minmax (quantize.c:52-60): strict-compare running min/max from
 * d[0] (NaNs are skipped unless d[0] is NaN). */
int ora_calibrate_minmax(const double *d, int64_t n, int symmetric, OraQuantParams *out)
{
    if (!d || n <= 0 || !out) return -1;
    double mn = d[0], mx = d[0];
    for (int64_t i = 1; i < n; i++) {
        if (d[i] < mn) mn = d[i];
        if (d[i] > mx) mx = d[i];
    }
    minmax_params(mn, mx, symmetric, out);
    return 0;
}

int ora_calibrate_minmax_f32(const float *d, int64_t n, int symmetric, OraQuantParams *out)
{
    if (!d || n <= 0 || !out) return -1;
    double mn = d[0], mx = d[0];
    for (int64_t i = 1; i < n; i++) {
        double v = (double)d[i];
        if (v < mn) mn = v;
        if (v > mx) mx = v;
    }
    minmax_params(mn, mx, symmetric, out);
    return 0;
}

/* quantize_tensor (quantize.c:144-158). */
int ora_quantize(const double *d, int8_t *out, int64_t n, const OraQuantParams *p)
{
    if (!d || !out || n <= 0 || !p) return -1;
    double inv = 1.0 / p->scale;
    for (int64_t i = 0; i < n; i++) out[i] = quant_one(d[i], inv, p->zero_point);
    return 0;
}

int ora_quantize_f32(const float *d, int8_t *out, int64_t n, const OraQuantParams *p)
{
    if (!d || !out || n <= 0 || !p) return -1;
    double inv = 1.0 / p->scale;
    for (int64_t i = 0; i < n; i++) out[i] = quant_one((double)d[i], inv, p->zero_point);
    return 0;
}

/* dequantize_tensor (quantize.c:163-174): ((double)q - (double)zp) * scale. */
int ora_dequantize(const int8_t *q, double *out, int64_t n, const OraQuantParams *p)
{
    if (!q || !out || n <= 0 || !p) return -1;
    for (int64_t i = 0; i < n; i++) out[i] = ((double)q[i] - (double)p->zero_point) * p->scale;
    return 0;
}

int ora_dequantize_f32(const int8_t *q, float *out, int64_t n, const OraQuantParams *p)
{
    if (!q || !out || n <= 0 || !p) return -1;
    for (int64_t i = 0; i < n; i++)
        out[i] = (float)(((double)q[i] - (double)p->zero_point) * p->scale);
    return 0;
}

/* quantization_error / quantization_snr (quantize.c:222-269): fused
 * quantize -> dequantize -> squared error, sequential double sums. */
#define QERR_BODY(T)                                                       \
    double inv = 1.0 / p->scale, sig = 0.0, noise = 0.0;                   \
    for (int64_t i = 0; i < n; i++) {                                      \
        double x = (double)d[i];                                           \
        sig += x * x;                                                      \
        int8_t q = quant_one(x, inv, p->zero_point);                       \
        double rec = ((double)q - (double)p->zero_point) * p->scale;       \
        double diff = x - rec;                                             \
        noise += diff * diff;                                              \
    }

double ora_quant_error(const double *d, int64_t n, const OraQuantParams *p)
{
    if (!d || n <= 0 || !p) return -1.0;
    QERR_BODY(double)
    (void)sig;
    return noise / (double)n;
}

double ora_quant_snr(const double *d, int64_t n, const OraQuantParams *p)
{
    if (!d || n <= 0 || !p) return -1.0;
    QERR_BODY(double)
    if (noise < 1e-30) return 999.0;
    return 10.0 * log10(sig / noise);
}

double ora_quant_error_f32(const float *d, int64_t n, const OraQuantParams *p)
{
    if (!d || n <= 0 || !p) return -1.0;
    QERR_BODY(float)
    (void)sig;
    return noise / (double)n;
}

double ora_quant_snr_f32(const float *d, int64_t n, const OraQuantParams *p)
{
    if (!d || n <= 0 || !p) return -1.0;
    QERR_BODY(float)
    if (noise < 1e-30) return 999.0;
    return 10.0 * log10(sig / noise);
}

/* ------------------------------------------------------------------------ */
/* Optimizers: src/c/optimizers_c.c:218-348                                  */
/* ------------------------------------------------------------------------ */

/* bc = 1 - pow(beta, t) (optimizers_c.c:258-260, 302-304). */
double ora_bias_correction(double beta, int64_t t) { return 1.0 - pow(beta, (double)t); }

/* sgd_step_impl (optimizers_c.c:218-249). */
void ora_sgd_f32(float *p, const float *g, double *vel, int64_t n, double lr, double mom)
{
    for (int64_t j = 0; j < n; j++) {
        double grad = (double)g[j];
        vel[j] = mom * vel[j] + grad;
        p[j] -= (float)(lr * vel[j]);
    }
}

void ora_sgd_f64(double *p, const double *g, double *vel, int64_t n, double lr, double mom)
{
    for (int64_t j = 0; j < n; j++) {
        vel[j] = mom * vel[j] + g[j];
        p[j] -= lr * vel[j];
    }
}

/* adam_step_impl (optimizers_c.c:251-293): the f32 update is subtracted in
 * float after one rounding of the double step. */
void ora_adam_f32(float *p, const float *g, double *m, double *v, int64_t n, double lr,
                  double b1, double b2, double eps, double bc1, double bc2)
{
    for (int64_t j = 0; j < n; j++) {
        double grad = (double)g[j];
        m[j] = b1 * m[j] + (1.0 - b1) * grad;
        v[j] = b2 * v[j] + (1.0 - b2) * grad * grad;
        double mh = m[j] / bc1;
        double vh = v[j] / bc2;
        p[j] -= (float)(lr * mh / (sqrt(vh) + eps));
    }
}

void ora_adam_f64(double *p, const double *g, double *m, double *v, int64_t n, double lr,
                  double b1, double b2, double eps, double bc1, double bc2)
{
    for (int64_t j = 0; j < n; j++) {
        double grad = g[j];
        m[j] = b1 * m[j] + (1.0 - b1) * grad;
        v[j] = b2 * v[j] + (1.0 - b2) * grad * grad;
        double mh = m[j] / bc1;
        double vh = v[j] / bc2;
        p[j] -= lr * mh / (sqrt(vh) + eps);
    }
}

/* adamw_step_impl (optimizers_c.c:295-348): decoupled decay on the double
 * copy of the parameter, then the Adam step, one rounding at the end. */
void ora_adamw_f32(float *p, const float *g, double *m, double *v, int64_t n, double lr,
                   double b1, double b2, double eps, double wd, double bc1, double bc2)
{
    for (int64_t j = 0; j < n; j++) {
        double param = (double)p[j];
        double grad = (double)g[j];
        param -= lr * wd * param;
        m[j] = b1 * m[j] + (1.0 - b1) * grad;
        v[j] = b2 * v[j] + (1.0 - b2) * grad * grad;
        double mh = m[j] / bc1;
        double vh = v[j] / bc2;
        param -= lr * mh / (sqrt(vh) + eps);
        p[j] = (float)param;
    }
}

void ora_adamw_f64(double *p, const double *g, double *m, double *v, int64_t n, double lr,
                   double b1, double b2, double eps, double wd, double bc1, double bc2)
{
    for (int64_t j = 0; j < n; j++) {
        double param = p[j];
        double grad = g[j];
        param -= lr * wd * param;
        m[j] = b1 * m[j] + (1.0 - b1) * grad;
        v[j] = b2 * v[j] + (1.0 - b2) * grad * grad;
        double mh = m[j] / bc1;
        double vh = v[j] / bc2;
        param -= lr * mh / (sqrt(vh) + eps);
        p[j] = param;
    }
}

/* ------------------------------------------------------------------------ */
/* NaN / Inf scans and the L2 norm: src/asm/training_ops.asm:544-696         */
/* ------------------------------------------------------------------------ */

/* tensor_has_nan (training_ops.asm:544-574): ucomiss x,x unordered. */
int ora_has_nan_f32(const float *x, uint64_t n)
{
    if (!x || n == 0) return 0;
    for (uint64_t i = 0; i < n; i++) if (x[i] != x[i]) return 1;
    return 0;
}

/* tensor_has_inf (training_ops.asm:585-621): (bits & 0x7fffffff) == 0x7f800000. */
int ora_has_inf_f32(const float *x, uint64_t n)
{
    if (!x || n == 0) return 0;
    for (uint64_t i = 0; i < n; i++) {
        uint32_t u;
        memcpy(&u, &x[i], 4);
        if ((u & 0x7fffffffu) == 0x7f800000u) return 1;
    }
    return 0;
}

/* tensor_grad_l2_norm (training_ops.asm:636-696): four float lanes of x*x
 * (mulps/addps), then (l0+l2)+(l1+l3) (movhlps/addps/shufps/addss), then the
 * n%4 tail squared and added one by one, then sqrtss. */
float ora_l2_ref_f32(const float *x, uint64_t n)
{
    if (!x || n == 0) return 0.0f;
    float l[4] = {0, 0, 0, 0};
    uint64_t nv = n / 4;
    for (uint64_t i = 0; i < nv; i++)
        for (int k = 0; k < 4; k++) {
            float sq = x[i * 4 + k] * x[i * 4 + k];
            l[k] = l[k] + sq;
        }
    float s = 0.0f;
    if (nv > 0) s = (l[0] + l[2]) + (l[1] + l[3]);
    for (uint64_t i = nv * 4; i < n; i++) {
        float sq = x[i] * x[i];
        s = s + sq;
    }
    return sqrtf(s);
}

/* Exact sum of squares in double (squares of floats are exact in double). */
double ora_sumsq_exact_f32(const float *x, uint64_t n)
{
    double s = 0.0, c = 0.0;
    for (uint64_t i = 0; i < n; i++) {
        double v = (double)x[i] * (double)x[i];
        double t = s + v;
        if (fabs(s) >= fabs(v)) c += (s - t) + v;
        else c += (v - t) + s;
        s = t;
    }
    return s + c;
}

/* ------------------------------------------------------------------------ */
/* 2-D f64 copies: src/c/tensor_ops.c:15-148                                 */
/* ------------------------------------------------------------------------ */

int ora_concat_2d(const double *a, const double *b, int64_t ra, int64_t ca, int64_t rb,
                  int64_t cb, int64_t axis, double *out, int64_t *orows, int64_t *ocols)
{
    if (!a || !b || !out || !orows || !ocols) return -1;
    if (ra <= 0 || ca <= 0 || rb <= 0 || cb <= 0) return -1;
    if (axis == 0) {
        if (ca != cb) return -1;
        *orows = ra + rb;
        *ocols = ca;
        for (int64_t i = 0; i < ra * ca; i++) out[i] = a[i];
        for (int64_t i = 0; i < rb * cb; i++) out[ra * ca + i] = b[i];
        return 0;
    }
    if (axis != 1 || ra != rb) return -1;
    *orows = ra;
    *ocols = ca + cb;
    for (int64_t r = 0; r < ra; r++) {
        for (int64_t c = 0; c < ca; c++) out[r * (ca + cb) + c] = a[r * ca + c];
        for (int64_t c = 0; c < cb; c++) out[r * (ca + cb) + ca + c] = b[r * cb + c];
    }
    return 0;
}

int ora_split_2d(const double *in, int64_t rows, int64_t cols, int64_t axis, int64_t split,
                 double *oa, double *ob, int64_t *ra, int64_t *ca, int64_t *rb, int64_t *cb)
{
    if (!in || !oa || !ob || !ra || !ca || !rb || !cb) return -1;
    if (rows <= 0 || cols <= 0) return -1;
    if (axis == 0) {
        if (split <= 0 || split >= rows) return -1;
        *ra = split; *ca = cols; *rb = rows - split; *cb = cols;
        for (int64_t i = 0; i < split * cols; i++) oa[i] = in[i];
        for (int64_t i = 0; i < (rows - split) * cols; i++) ob[i] = in[split * cols + i];
        return 0;
    }
    if (axis != 1) return -1;
    if (split <= 0 || split >= cols) return -1;
    *ra = rows; *ca = split; *rb = rows; *cb = cols - split;
    for (int64_t r = 0; r < rows; r++) {
        for (int64_t c = 0; c < split; c++) oa[r * split + c] = in[r * cols + c];
        for (int64_t c = split; c < cols; c++) ob[r * (cols - split) + c - split] = in[r * cols + c];
    }
    return 0;
}

int ora_pad_2d(const double *in, int64_t rows, int64_t cols, int64_t pt, int64_t pb,
               int64_t pl, int64_t pr, double value, double *out, int64_t *orows, int64_t *ocols)
{
    if (!in || !out || !orows || !ocols) return -1;
    if (rows <= 0 || cols <= 0) return -1;
    if (pt < 0 || pb < 0 || pl < 0 || pr < 0) return -1;
    int64_t R = rows + pt + pb, C = cols + pl + pr;
    *orows = R;
    *ocols = C;
    for (int64_t i = 0; i < R * C; i++) out[i] = value;
    for (int64_t r = 0; r < rows; r++)
        for (int64_t c = 0; c < cols; c++) out[(r + pt) * C + pl + c] = in[r * cols + c];
    return 0;
}

int ora_transpose_2d(const double *in, int64_t rows, int64_t cols, double *out)
{
    if (!in || !out) return -1;
    if (rows <= 0 || cols <= 0) return -1;
    for (int64_t r = 0; r < rows; r++)
        for (int64_t c = 0; c < cols; c++) out[c * rows + r] = in[r * cols + c];
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Cross-entropy losses                                                     */
/* ------------------------------------------------------------------------ */

/* Label-smoothed cross-entropy, forward (metrics_losses.c:28-77): per row
 * max by strict compare from row[0]; lse = log(sum exp(x - max)) in index
 * order; sample_loss -= smooth_t * log_soft over c in index order, with
 * smooth_t = smoothing / K (+ 1 - smoothing at the target); loss = total / B. */
int ora_ls_ce_forward(const double *logits, const int64_t *targets, int64_t batch, int64_t classes,
                      double smoothing, double *loss_out)
{
    if (!logits || !targets || !loss_out) return -1;
    if (batch <= 0 || classes <= 0) return -1;
    if (smoothing < 0.0 || smoothing > 1.0) return -1;
    double total = 0.0;
    for (int64_t i = 0; i < batch; i++) {
        const double *row = logits + i * classes;
        double mx = row[0];
        for (int64_t c = 1; c < classes; c++)
            if (row[c] > mx) mx = row[c];
        double lse = 0.0;
        for (int64_t c = 0; c < classes; c++) lse += exp(row[c] - mx);
        lse = log(lse);
        const int64_t t = targets[i];
        if (t < 0 || t >= classes) return -1;
        double sample = 0.0;
        for (int64_t c = 0; c < classes; c++) {
            const double ls = (row[c] - mx) - lse;
            double st = smoothing / (double)classes;
            if (c == t) st += (1.0 - smoothing);
            sample -= st * ls;
        }
        total += sample;
    }
    *loss_out = total / (double)batch;
    return 0;
}

/* Label-smoothed cross-entropy, backward (metrics_losses.c:80-125):
 * grad = (1/B) * (exp(x - max) / sum - smooth_t), the division per element. */
int ora_ls_ce_backward(const double *logits, const int64_t *targets, int64_t batch, int64_t classes,
                       double smoothing, double *grad)
{
    if (!logits || !targets || !grad) return -1;
    if (batch <= 0 || classes <= 0) return -1;
    if (smoothing < 0.0 || smoothing > 1.0) return -1;
    const double inv_n = 1.0 / (double)batch;
    for (int64_t i = 0; i < batch; i++) {
        const double *row = logits + i * classes;
        double *g = grad + i * classes;
        double mx = row[0];
        for (int64_t c = 1; c < classes; c++)
            if (row[c] > mx) mx = row[c];
        double s = 0.0;
        for (int64_t c = 0; c < classes; c++) {
            g[c] = exp(row[c] - mx);
            s += g[c];
        }
        for (int64_t c = 0; c < classes; c++) g[c] /= s;
        const int64_t t = targets[i];
        if (t < 0 || t >= classes) return -1;
        for (int64_t c = 0; c < classes; c++) {
            double st = smoothing / (double)classes;
            if (c == t) st += (1.0 - smoothing);
            g[c] = inv_n * (g[c] - st);
        }
    }
    return 0;
}

/* cross_entropy_loss (losses.asm:315-613), intended semantics: per row the
 * maxss chain from x[0] (the running max of ora_max_chain), e_j =
 * (float)exp((double)x_j - (double)max) summed sequentially in float
 * (addss), p = e / sum (divss); the target index is the truncation of the
 * target tensor's float value (cvttss2si); per-row loss
 * (float)(-log((double)p_t + 1e-7)) summed sequentially in float, divided by
 * (float)B.  Returns -1 for a target outside [0, K). */
int ora_ce_loss_f32(const float *x, const float *tgt, int64_t batch, int64_t classes, double *loss)
{
    float total = 0.0f;
    for (int64_t i = 0; i < batch; i++) {
        const float *row = x + i * classes;
        const float mx = ora_max_chain_f32(row, classes);
        float s = 0.0f;
        for (int64_t c = 0; c < classes; c++) s += (float)exp((double)row[c] - (double)mx);
        if (!(tgt[i] > -1.0f && tgt[i] < (float)classes)) return -1;
        const int32_t t = (int32_t)tgt[i];  /* in range: truncation, as cvttss2si */
        const float et = (float)exp((double)row[t] - (double)mx);
        const float p = et / s;
        total += (float)(-log((double)p + 1e-7));
    }
    *loss = (double)(total / (float)batch);
    return 0;
}

/* f64 path of the same routine: exp / log in double, sums in double. */
int ora_ce_loss_f64(const double *x, const double *tgt, int64_t batch, int64_t classes, double *loss)
{
    double total = 0.0;
    for (int64_t i = 0; i < batch; i++) {
        const double *row = x + i * classes;
        const double mx = ora_max_chain_f64(row, classes);
        double s = 0.0;
        for (int64_t c = 0; c < classes; c++) s += exp(row[c] - mx);
        if (!(tgt[i] > -1.0 && tgt[i] < (double)classes)) return -1;
        const int64_t t = (int64_t)tgt[i];
        const double p = exp(row[t] - mx) / s;
        total += -log(p + 1e-7);
    }
    *loss = total / (double)batch;
    return 0;
}

/* ---- gradient clipping ---------------------------------------------------------- */

/* clip_grad_norm_ (optimizers.asm:1370-1516) over a list of gradient buffers
 * (dtypes[i]: 0 f32, 1 f64; NULL entries skipped as the asm skips parameter
 * nodes without a gradient, 1396-1403).  One sequential double sum of
 * (double)g * (double)g over the list in order (mulsd + addsd, 1410-1436),
 * sqrtsd (1444), then clip only when norm > max_norm: ucomisd + jbe
 * (1448-1449) skips on <= and on unordered.  scale = max_norm / norm (divsd,
 * 1452); f64 gradients g * scale (1480-1487), f32 gradients g * (float)scale
 * in float (cvtsd2ss + mulss, 1489-1499).  Returns the pre-clip norm. */
double ora_clip_grad_norm(void **grads, const int *dtypes, const int64_t *ns, int64_t count, double max_norm)
{
    double total = 0.0;
    for (int64_t i = 0; i < count; i++) {
        if (!grads[i]) continue;
        if (dtypes[i] == 0) {
            const float *g = (const float *)grads[i];
            for (int64_t j = 0; j < ns[i]; j++) {
                const double d = (double)g[j];
                total += d * d;
            }
        } else {
            const double *g = (const double *)grads[i];
            for (int64_t j = 0; j < ns[i]; j++) total += g[j] * g[j];
        }
    }
    const double norm = sqrt(total);
    if (norm > max_norm) {
        const double scale = max_norm / norm;
        for (int64_t i = 0; i < count; i++) {
            if (!grads[i]) continue;
            if (dtypes[i] == 0) {
                float *g = (float *)grads[i];
                const float sf = (float)scale;
                for (int64_t j = 0; j < ns[i]; j++) g[j] = g[j] * sf;
            } else {
                double *g = (double *)grads[i];
                for (int64_t j = 0; j < ns[i]; j++) g[j] = g[j] * scale;
            }
        }
    }
    return norm;
}

/* clip_grad_value_ (optimizers.asm:1527-1620): maxsd then minsd, i.e.
 * t = g > lo ? g : lo; g = t < hi ? t : hi (the SSE rule returns the second
 * operand when the compare is false, NaN included).  f32 bounds are rounded to
 * float first (cvtsd2ss, 1587-1591); maxsd / minsd at 1579-1581. */
void ora_clip_grad_value(void **grads, const int *dtypes, const int64_t *ns, int64_t count, double lo, double hi)
{
    for (int64_t i = 0; i < count; i++) {
        if (!grads[i]) continue;
        if (dtypes[i] == 0) {
            float *g = (float *)grads[i];
            const float l = (float)lo, h = (float)hi;
            for (int64_t j = 0; j < ns[i]; j++) {
                const float t = g[j] > l ? g[j] : l;
                g[j] = t < h ? t : h;
            }
        } else {
            double *g = (double *)grads[i];
            for (int64_t j = 0; j < ns[i]; j++) {
                const double t = g[j] > lo ? g[j] : lo;
                g[j] = t < hi ? t : hi;
            }
        }
    }
}

/* calibrate_percentile (quantize.c:89-132): a sorted copy by the C
 * library's qsort with the reference's comparator (equal elements, e.g. -0
 * and +0, keep the order qsort gives them), sorted[lo] / sorted[hi] with
 * lo = (int64)(n p), hi = (int64)(n (1 - p)), then the minmax expressions. */
static int ora_cmp_double_asc(const void *a, const void *b)
{
    const double da = *(const double *)a, db = *(const double *)b;
    return (da > db) - (da < db);
}

int ora_calibrate_percentile(const double *data, int64_t n, double percentile, int symmetric, OraQuantParams *out)
{
    if (!data || n <= 0 || !out) return -1;
    if (percentile != percentile) return -1; /* the reference reads out of bounds here */
    if (percentile < 0.0 || percentile > 0.5) percentile = 0.01;
    double *sorted = (double *)malloc((size_t)n * sizeof(double));
    if (!sorted) return -1;
    memcpy(sorted, data, (size_t)n * sizeof(double));
    qsort(sorted, (size_t)n, sizeof(double), ora_cmp_double_asc);
    int64_t lo_idx = (int64_t)(n * percentile);
    int64_t hi_idx = (int64_t)(n * (1.0 - percentile));
    if (lo_idx < 0) lo_idx = 0;
    if (hi_idx >= n) hi_idx = n - 1;
    double cmin = sorted[lo_idx], cmax = sorted[hi_idx];
    free(sorted);
    if (symmetric) {
        double am = fmax(fabs(cmin), fabs(cmax));
        if (am < 1e-30) am = 1e-30;
        out->scale = am / 127.0;
        out->zero_point = 0;
        out->min_val = -am;
        out->max_val = am;
        out->symmetric = 1;
    } else {
        if (cmin == cmax) {
            cmin -= 0.5;
            cmax += 0.5;
        }
        out->scale = (cmax - cmin) / 255.0;
        if (out->scale < 1e-30) out->scale = 1e-30;
        out->zero_point = x86_round_to_i32(-128.0 - cmin / out->scale);
        if (out->zero_point < -128) out->zero_point = -128;
        if (out->zero_point > 127) out->zero_point = 127;
        out->min_val = cmin;
        out->max_val = cmax;
        out->symmetric = 0;
    }
    return 0;
}

/* quantized_matmul (quantize.c:191-214): combined_scale = sa * sb;
 * acc = sum_k ((int32)A[i][k] - za) * ((int32)B[k][j] - zb) in int32, the
 * reference's loop order; the adds and multiplies wrap mod 2^32 (the compiled
 * reference's behaviour; written in uint32 here so that C defines it);
 * C[i][j] = (double)acc * combined_scale. */
int ora_quantized_matmul(const int8_t *A, const int8_t *B, double *C, int64_t M, int64_t K, int64_t N,
                         const OraQuantParams *pa, const OraQuantParams *pb)
{
    if (!A || !B || !C || !pa || !pb) return -1;
    if (M <= 0 || K <= 0 || N <= 0) return -1;
    const double cs = pa->scale * pb->scale;
    const uint32_t za = (uint32_t)pa->zero_point, zb = (uint32_t)pb->zero_point;
    for (int64_t i = 0; i < M; i++)
        for (int64_t j = 0; j < N; j++) {
            uint32_t acc = 0;
            for (int64_t k = 0; k < K; k++) {
                const uint32_t a = (uint32_t)(int32_t)A[i * K + k] - za;
                const uint32_t b = (uint32_t)(int32_t)B[k * N + j] - zb;
                acc += a * b;
            }
            C[i * N + j] = (double)(int32_t)acc * cs;
        }
    return 0;
}

/* ---- dropout and the fused add + relu -------------------------------------------- */

/* cvtsd2si under the default MXCSR rounding (nearest even); NaN and values
 * outside int64 give the integer indefinite INT64_MIN. */
static int64_t ora_cvtsd2si(double v)
{
    if (!(v >= -0x1p63 && v < 0x1p63)) return INT64_MIN;
    return (int64_t)nearbyint(v);
}

void ora_srand(unsigned seed) { srand(seed); }

/* dropout_forward (training_ops.asm:718-790) with the C library's rand(), as
 * the reference calls it: p widened to double (cvtss2sd, 734);
 * scale = (float)(1.0 / (1.0 - p)) (divsd + cvtsd2ss, 736-739); threshold =
 * cvtsd2si(p * 2147483647.0) (743-744); per element one rand() (753),
 * sign-extended and compared signed (757-759): r < threshold drops (mask 0,
 * out +0.0f, 768-772), else mask 1 and out = in * scale (mulss, 762-765). */
int ora_dropout_forward(const float *in, float *out, uint8_t *mask, uint64_t n, float p)
{
    const double pd = (double)p;
    const float scale = (float)(1.0 / (1.0 - pd));
    const int64_t th = ora_cvtsd2si(pd * 2147483647.0);
    for (uint64_t i = 0; i < n; i++) {
        const int64_t r = (int64_t)rand();
        if (r < th) {
            mask[i] = 0;
            out[i] = 0.0f;
        } else {
            mask[i] = 1;
            out[i] = in[i] * scale;
        }
    }
    return 0;
}

/* dropout_backward (training_ops.asm:804-858): any nonzero mask byte keeps
 * (movzx + test, 832-834),
 * grad_in = grad_out * scale (mulss); else +0.0f. */
int ora_dropout_backward(const float *go, float *gi, const uint8_t *mask, uint64_t n, float p)
{
    const float scale = (float)(1.0 / (1.0 - (double)p));
    for (uint64_t i = 0; i < n; i++) gi[i] = mask[i] ? go[i] * scale : 0.0f;
    return 0;
}

/* The C library's rand() n times (the process-wide stream, as the reference
 * draws it). */
void ora_rand_n(uint64_t n, uint32_t *out)
{
    for (uint64_t i = 0; i < n; i++) out[i] = (uint32_t)rand();
}

/* glibc's TYPE_3 stream at any position without stepping to it.
 * srand(s): r[0] = s (0 taken as 1), r[i] = 16807 r[i-1] mod (2^31 - 1) for
 * i < 31 (Schrage's method on int32, as glibc's srandom_r), r[31..33] =
 * r[0..2], r[i] = r[i-31] + r[i-3] mod 2^32 for i >= 34; rand() number k
 * (k = 0, 1, ...) is r[k + 344] >> 1.  The recurrence is linear with
 * characteristic polynomial P(x) = x^31 - x^28 - 1, so with the anchor
 * window W = r[313 .. 343], r[313 + j] = sum_m (x^j mod P)_m W[m]
 * (coefficients mod 2^32): the window at any offset follows from
 * x^skip mod P by square-and-multiply. */
static void ora_pmul(uint32_t *a, const uint32_t *b) /* a = a * b mod P; b may alias a */
{
    uint32_t prod[61] = {0};
    for (int i = 0; i < 31; i++)
        for (int j = 0; j < 31; j++) prod[i + j] += a[i] * b[j];
    for (int d = 60; d >= 31; d--) { /* x^d = x^(d-3) + x^(d-31) */
        prod[d - 31] += prod[d];
        prod[d - 3] += prod[d];
    }
    memcpy(a, prod, 31 * sizeof(uint32_t));
}

void ora_glibc_window(uint32_t seed, uint64_t skip, uint64_t n, uint32_t *out)
{
    uint32_t r[344];
    r[0] = seed == 0 ? 1u : seed;
    int32_t word = (int32_t)r[0];
    for (int i = 1; i < 31; i++) {
        const int32_t hi = word / 127773, lo = word % 127773;
        word = 16807 * lo - 2836 * hi;
        if (word < 0) word += 2147483647;
        r[i] = (uint32_t)word;
    }
    for (int i = 31; i < 34; i++) r[i] = r[i - 31];
    for (int i = 34; i < 344; i++) r[i] = r[i - 31] + r[i - 3];
    const uint32_t *W = r + 313;
    /* window at r[344 + skip - 31 ..]: offset j = skip + 0 .. 30 from the anchor */
    uint32_t c[31] = {0}, base[31] = {0}, w[31];
    c[0] = 1u;
    base[1] = 1u;
    for (uint64_t k = skip; k; k >>= 1) {
        if (k & 1) ora_pmul(c, base);
        ora_pmul(base, base);
    }
    for (int t = 0; t < 31; t++) {
        uint32_t v = 0;
        for (int m = 0; m < 31; m++) v += c[m] * W[m];
        w[t] = v;
        const uint32_t top = c[30]; /* c <- c * x mod P */
        for (int m = 30; m > 0; m--) c[m] = c[m - 1];
        c[0] = top;
        c[28] += top;
    }
    for (uint64_t j = 0; j < n; j++) {
        const int a = (int)(j % 31), b = (int)((j + 28) % 31);
        const uint32_t v = w[a] + w[b];
        w[a] = v;
        out[j] = v >> 1;
    }
}

/* ora_dropout_forward on draws skip .. skip + n - 1 after srand(seed), the
 * draws taken from ora_glibc_window instead of the C library. */
int ora_dropout_window(uint32_t seed, uint64_t skip, const float *in, float *out, uint8_t *mask, uint64_t n,
                       float p)
{
    uint32_t *r = (uint32_t *)malloc(n * sizeof(uint32_t) + 4);
    if (!r) return -1;
    ora_glibc_window(seed, skip, n, r);
    const double pd = (double)p;
    const float scale = (float)(1.0 / (1.0 - pd));
    const int64_t th = ora_cvtsd2si(pd * 2147483647.0);
    for (uint64_t i = 0; i < n; i++) {
        if ((int64_t)r[i] < th) {
            mask[i] = 0;
            out[i] = 0.0f;
        } else {
            mask[i] = 1;
            out[i] = in[i] * scale;
        }
    }
    free(r);
    return 0;
}

/* vec_add_relu_fusion (fusion.asm:200-226): addss then maxss with +0, i.e.
 * s = a + b; c = s > 0 ? s : +0 (NaN and -0 give +0). */
void ora_add_relu_f32(const float *a, const float *b, float *c, int64_t n)
{
    for (int64_t i = 0; i < n; i++) {
        const float s = a[i] + b[i];
        c[i] = s > 0.0f ? s : 0.0f;
    }
}

/* ---- per-feature transforms (transforms.c) ----------------------------------------- */

/* transform_compute_stats (transforms.c:27-62): per feature, one pass over the
 * rows in order: sum += v, sum2 += v * v, mn starts at 1e308 and takes v only
 * when v < mn (mx: -1e308, v > mx), so NaN never enters, the first of equal
 * values (+0 / -0) stays, and values beyond +-1e308 leave the start value.
 * mean = sum / b; var = sum2 / b - mean * mean, clamped at 0 (a NaN var
 * stays NaN); std = sqrt(var).  NULL outputs are skipped. */
int ora_transform_stats(const double *data, int64_t b, int64_t nf, double *mean, double *std, double *mn_out,
                        double *mx_out)
{
    if (!data || b <= 0 || nf <= 0) return -1;
    for (int64_t f = 0; f < nf; f++) {
        double sum = 0.0, sum2 = 0.0, mn = 1e308, mx = -1e308;
        for (int64_t i = 0; i < b; i++) {
            const double v = data[i * nf + f];
            sum += v;
            sum2 += v * v;
            if (v < mn) mn = v;
            if (v > mx) mx = v;
        }
        const double m = sum / (double)b;
        double var = sum2 / (double)b - m * m;
        if (var < 0.0) var = 0.0;
        if (mean) mean[f] = m;
        if (std) std[f] = sqrt(var);
        if (mn_out) mn_out[f] = mn;
        if (mx_out) mx_out[f] = mx;
    }
    return 0;
}

/* transform_normalize / _unnormalize / _minmax (transforms.c:68-143):
 * (x - mean) / (std + eps); x * (std + eps) + mean; (x - min) / (max - min + eps).
 * mode 0, 1, 2 respectively; -1 on NULL pointers or non-positive sizes. */
int ora_transform_apply(int mode, const double *data, double *out, int64_t b, int64_t nf, const double *p0,
                        const double *p1, double eps)
{
    if (!data || !out || !p0 || !p1) return -1;
    if (b <= 0 || nf <= 0) return -1;
    for (int64_t i = 0; i < b; i++) {
        for (int64_t f = 0; f < nf; f++) {
            const int64_t idx = i * nf + f;
            if (mode == 0) out[idx] = (data[idx] - p0[f]) / (p1[f] + eps);
            else if (mode == 1) out[idx] = data[idx] * (p1[f] + eps) + p0[f];
            else {
                const double range = p1[f] - p0[f] + eps;
                out[idx] = (data[idx] - p0[f]) / range;
            }
        }
    }
    return 0;
}
