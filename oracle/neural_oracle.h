/*
 * neural_oracle.h -- CPU restatement of the Neural-Assembly tensor hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker the HIP kernels in
 * libneural_hip.so are compared against.  Only tests/, the smoke() entry and
 * bench.py's cpu_baseline leg may load it; the product path never does.
 *
 * Every function restates one reference loop (file:line under the reference
 * tree) with the same operation order, the same widths and the same
 * double-precision intermediates, compiled with -O2 -std=c11
 * -ffp-contract=off (the reference C is built with -O2 -std=c11 and no -march,
 * so SSE2 arithmetic and no FMA contraction).
 *
 * Pinning (what each function is checked against, in tests/test_oracle_*.py):
 *   - ora_ew_*, ora_scalar_*, ora_neg_*, ora_relu_*, ora_bias_add_f32/f64,
 *     ora_has_nan/inf: IEEE-754 closed forms (numpy) plus the reference
 *     unit-test values (src/asm/tests.asm:337-405,470-519).
 *   - ora_max_chain_f32/f64, ora_rowmax_chain_*, ora_argmax_f32/f64,
 *     ora_rowargmax_*: brute force over every array of length 1-4 drawn
 *     from {NaN, -0, +0, 1, -1, 2} in float32 AND float64 against the
 *     maxss/maxsd and comiss/comisd rules, plus closed forms (rightmost
 *     maximum after the last NaN; first index of the non-NaN maximum).
 *   - ora_sum_ref_*, ora_l2_ref_f32, ora_rowsum_ref_*: a Python lane-by-lane
 *     emulation of the asm order on tiny inputs and the fp64-exact value
 *     (math.fsum) within the rounding bound of the order.
 *   - ora_calibrate_minmax_f32, ora_quantize_f32, ora_dequantize_f32,
 *     ora_quant_error_f32, ora_quant_snr_f32: bit-for-bit against the
 *     reference's quantize.c run on the float32 values widened to double
 *     (exact), incl. NaN / +-Inf / +-50 / 2^31 overflow (the dequantized
 *     floats against (float) of the reference's double).
 *   - ora_act_*, ora_quant*, ora_calibrate*, ora_dequant*, ora_adam*,
 *     ora_sgd*, ora_log_softmax_rows_*, ora_concat/split/pad/transpose,
 *     ora_transform_*: bit-for-bit against the reference's own C
 *     (activations_c.c, quantize.c, optimizers_c.c, metrics_losses.c,
 *     tensor_ops.c, transforms.c) compiled unchanged into
 *     oracle/_ref/libneural_ref.so.
 *   - ora_softmax_rows_*: fp64 closed form (numpy) within the f32 rounding
 *     bound; the f64 path also equals an unrolled numpy restatement bit for
 *     bit when the same libm exp is used.
 */
#ifndef NEURAL_ORACLE_H
#define NEURAL_ORACLE_H

#include <stdint.h>

/* binary op codes shared by ora_ew_* */
enum { ORA_ADD = 0, ORA_SUB = 1, ORA_MUL = 2, ORA_DIV = 3, ORA_MAX = 4 };

/* activation codes shared by ora_act_* */
enum {
    ORA_TANH = 0, ORA_GELU = 1, ORA_LEAKY_RELU = 2, ORA_ELU = 3, ORA_SELU = 4,
    ORA_SWISH = 5, ORA_MISH = 6, ORA_HARDSWISH = 7, ORA_SOFTPLUS = 8,
    ORA_HARDTANH = 9, ORA_SIGMOID = 10
};

typedef struct {
    double  scale;
    int32_t zero_point;
    double  min_val;
    double  max_val;
    int     symmetric;
} OraQuantParams;

void ora_ew_f32(int op, const float *a, const float *b, float *out, int64_t n);
void ora_ew_f64(int op, const double *a, const double *b, double *out, int64_t n);
void ora_scalar_f32(int op, const float *a, double s, float *out, int64_t n);
void ora_scalar_f64(int op, const double *a, double s, double *out, int64_t n);
void ora_neg_f32(const float *a, float *out, int64_t n);
void ora_neg_f64(const double *a, double *out, int64_t n);
void ora_relu_f32(const float *a, float *out, int64_t n);
void ora_relu_f64(const double *a, double *out, int64_t n);
void ora_bias_add_f32(const float *x, const float *b, float *out, int64_t rows, int64_t cols);
void ora_bias_add_f64(const double *x, const double *b, double *out, int64_t rows, int64_t cols);

float  ora_sum_ref_f32(const float *x, int64_t n);
double ora_sum_ref_f64(const double *x, int64_t n);
double ora_sum_exact_f32(const float *x, int64_t n);
double ora_sum_exact_f64(const double *x, int64_t n);
void   ora_rowsum_ref_f32(const float *x, int64_t rows, int64_t cols, float *out);
void   ora_rowsum_ref_f64(const double *x, int64_t rows, int64_t cols, double *out);
void   ora_colsum_ref_f32(const float *x, int64_t rows, int64_t cols, float *out);
void   ora_colsum_ref_f64(const double *x, int64_t rows, int64_t cols, double *out);
void   ora_rowsum_exact_f32(const float *x, int64_t rows, int64_t cols, double *out);
void   ora_rowsum_exact_f64(const double *x, int64_t rows, int64_t cols, double *out);
float  ora_max_chain_f32(const float *x, int64_t n);
double ora_max_chain_f64(const double *x, int64_t n);
void   ora_rowmax_chain_f32(const float *x, int64_t rows, int64_t cols, float *out);
void   ora_rowmax_chain_f64(const double *x, int64_t rows, int64_t cols, double *out);
int64_t ora_argmax_f32(const float *x, int64_t n);
int64_t ora_argmax_f64(const double *x, int64_t n);
void   ora_rowargmax_f32(const float *x, int64_t rows, int64_t cols, int64_t *out);
void   ora_rowargmax_f64(const double *x, int64_t rows, int64_t cols, int64_t *out);

void ora_softmax_rows_f32(const float *x, int64_t rows, int64_t cols, float *out);
void ora_softmax_rows_f64(const double *x, int64_t rows, int64_t cols, double *out);
void ora_log_softmax_rows_f32(const float *x, int64_t rows, int64_t cols, float *out);
void ora_log_softmax_rows_f64(const double *x, int64_t rows, int64_t cols, double *out);

void ora_act_f32(int which, const float *in, float *out, int64_t n, double alpha);
void ora_act_f64(int which, const double *in, double *out, int64_t n, double alpha);

int    ora_calibrate_minmax(const double *d, int64_t n, int symmetric, OraQuantParams *out);
int    ora_calibrate_minmax_f32(const float *d, int64_t n, int symmetric, OraQuantParams *out);
int    ora_quantize(const double *d, int8_t *out, int64_t n, const OraQuantParams *p);
int    ora_quantize_f32(const float *d, int8_t *out, int64_t n, const OraQuantParams *p);
int    ora_dequantize(const int8_t *q, double *out, int64_t n, const OraQuantParams *p);
int    ora_dequantize_f32(const int8_t *q, float *out, int64_t n, const OraQuantParams *p);
double ora_quant_error(const double *d, int64_t n, const OraQuantParams *p);
/* calibrate_percentile (quantize.c:89-132) and quantized_matmul
 * (quantize.c:191-214).  Pinned bit-exact against the reference's quantize.c
 * (oracle/_ref) in tests/test_oracle_vs_ref.py -- runs of mixed-sign zeros at
 * the selected ranks (glibc's qsort is a stable merge sort), an infinite range,
 * percentiles outside [0, 0.5], a K = 40,000 product whose int32 sums wrap --
 * and by the golden fixtures pct_params / qmm_c. */
int    ora_calibrate_percentile(const double *data, int64_t n, double percentile, int symmetric,
                                OraQuantParams *out);
int    ora_quantized_matmul(const int8_t *A, const int8_t *B, double *C, int64_t M, int64_t K, int64_t N,
                            const OraQuantParams *pa, const OraQuantParams *pb);
double ora_quant_snr(const double *d, int64_t n, const OraQuantParams *p);
double ora_quant_error_f32(const float *d, int64_t n, const OraQuantParams *p);
double ora_quant_snr_f32(const float *d, int64_t n, const OraQuantParams *p);

double ora_bias_correction(double beta, int64_t t);
void ora_sgd_f32(float *p, const float *g, double *vel, int64_t n, double lr, double mom);
void ora_sgd_f64(double *p, const double *g, double *vel, int64_t n, double lr, double mom);
void ora_adam_f32(float *p, const float *g, double *m, double *v, int64_t n, double lr,
                  double b1, double b2, double eps, double bc1, double bc2);
void ora_adam_f64(double *p, const double *g, double *m, double *v, int64_t n, double lr,
                  double b1, double b2, double eps, double bc1, double bc2);
void ora_adamw_f32(float *p, const float *g, double *m, double *v, int64_t n, double lr,
                   double b1, double b2, double eps, double wd, double bc1, double bc2);
void ora_adamw_f64(double *p, const double *g, double *m, double *v, int64_t n, double lr,
                   double b1, double b2, double eps, double wd, double bc1, double bc2);

int   ora_has_nan_f32(const float *x, uint64_t n);
int   ora_has_inf_f32(const float *x, uint64_t n);
float ora_l2_ref_f32(const float *x, uint64_t n);
double ora_sumsq_exact_f32(const float *x, uint64_t n);

int ora_concat_2d(const double *a, const double *b, int64_t ra, int64_t ca, int64_t rb,
                  int64_t cb, int64_t axis, double *out, int64_t *orows, int64_t *ocols);
int ora_split_2d(const double *in, int64_t rows, int64_t cols, int64_t axis, int64_t split,
                 double *oa, double *ob, int64_t *ra, int64_t *ca, int64_t *rb, int64_t *cb);
int ora_pad_2d(const double *in, int64_t rows, int64_t cols, int64_t pt, int64_t pb,
               int64_t pl, int64_t pr, double value, double *out, int64_t *orows, int64_t *ocols);
int ora_transpose_2d(const double *in, int64_t rows, int64_t cols, double *out);

/* Cross-entropy losses (metrics_losses.c:28-125, losses.asm:315-613).
 * ora_ls_ce_*: pinned bit-exact against the reference's metrics_losses.c
 * (oracle/_ref).  ora_ce_loss_*: pinned by a closed form (fp64 log-softmax
 * at the target) and a small hand-checked case (tests/test_oracle_losses.py). */
int ora_ls_ce_forward(const double *logits, const int64_t *targets, int64_t batch, int64_t classes,
                      double smoothing, double *loss_out);
int ora_ls_ce_backward(const double *logits, const int64_t *targets, int64_t batch, int64_t classes,
                       double smoothing, double *grad);
int ora_ce_loss_f32(const float *x, const float *tgt, int64_t batch, int64_t classes, double *loss);
int ora_ce_loss_f64(const double *x, const double *tgt, int64_t batch, int64_t classes, double *loss);

/* Gradient clipping (optimizers.asm:1370-1620).  Pinned by invariants in
 * tests/test_oracle_clip.py: the pre-clip norm against math.fsum, the
 * post-clip norm equal to max_norm, bitwise no-op below the threshold and for
 * a NaN norm, hand-computed NaN / reversed-bound cases for the value clip. */
double ora_clip_grad_norm(void **grads, const int *dtypes, const int64_t *ns, int64_t count, double max_norm);
void   ora_clip_grad_value(void **grads, const int *dtypes, const int64_t *ns, int64_t count, double lo, double hi);

/* Dropout (training_ops.asm:717-858) with the C library's rand() -- the
 * reference's own generator -- and vec_add_relu_fusion (fusion.asm:200-226).
 * Pinned in tests/test_oracle_dropout.py: rand() against a restatement of
 * glibc's TYPE_3 generator, hand-derived thresholds (p = 0.5 rounds half to
 * even), keep rates, the closed forms of out and the backward. */
void ora_srand(unsigned seed);
int  ora_dropout_forward(const float *in, float *out, uint8_t *mask, uint64_t n, float p);
int  ora_dropout_backward(const float *go, float *gi, const uint8_t *mask, uint64_t n, float p);
void ora_rand_n(uint64_t n, uint32_t *out);
void ora_glibc_window(uint32_t seed, uint64_t skip, uint64_t n, uint32_t *out);
int  ora_dropout_window(uint32_t seed, uint64_t skip, const float *in, float *out, uint8_t *mask, uint64_t n,
                        float p);
void ora_add_relu_f32(const float *a, const float *b, float *c, int64_t n);

/* Per-feature transforms (transforms.c:27-143): statistics and the three
 * per-feature affine maps (mode 0 normalize, 1 unnormalize, 2 min-max).
 * Pinned bit-exact against the reference's transforms.c (oracle/_ref). */
int ora_transform_stats(const double *data, int64_t b, int64_t nf, double *mean, double *std, double *mn_out,
                        double *mx_out);
int ora_transform_apply(int mode, const double *data, double *out, int64_t b, int64_t nf, const double *p0,
                        const double *p1, double eps);

#endif
