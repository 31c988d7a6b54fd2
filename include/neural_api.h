/*
 * neural_api.h -- C ABI of libneural_hip.so, the MI355X (gfx950) implementation
 * of Neural-Assembly's tensor hot path.
 *
 * Drop-in for the reference's neural_api.h on this path: same names, argument
 * meaning, error codes and ownership rules, so the reference's ctypes layer
 * (pyneural/core.py) can bind this library instead of libneural.so.  Each
 * declaration names the reference interface it replaces (paths relative to
 * the Neural-Assembly tree).  Declarations marked NEW have no reference
 * counterpart; they are additive.
 *
 * Memory model (differs from the all-host reference):
 *   - Tensors created by the library keep their data in device memory (HBM).
 *     neural_tensor_data() / neural_buffer_info() return a host pointer and
 *     synchronise device -> host first.  The pointer is valid for host reads
 *     and writes until the next library call that takes the tensor; the next
 *     such call uploads the host copy.  (The reference Python layer calls
 *     neural_tensor_data() right before every memmove, which fits this.)
 *   - neural_tensor_from_buffer() accepts a host pointer (kept host-
 *     authoritative: uploaded before and written back after every call) or a
 *     device pointer (used in place, no copies).
 *   - Raw-pointer entry points (quantize_*, calibrate_*, *_has_nan, ...) accept
 *     host or device pointers; host buffers are staged through HBM.
 *   - Calls are stream-ordered on one HIP stream; results that come back by
 *     value or through host pointers are synchronised before return.
 */
#ifndef NEURAL_HIP_API_H
#define NEURAL_HIP_API_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif
#if defined(__GNUC__)
#pragma GCC visibility push(default)
#endif

/* Error codes: neural_api.h:15-35 (error.asm:11-29). */
typedef enum {
    NEURAL_OK                   = 0,
    NEURAL_ERR_NULL_POINTER     = 1,
    NEURAL_ERR_OUT_OF_MEMORY    = 2,
    NEURAL_ERR_INVALID_ARGUMENT = 3,
    NEURAL_ERR_SHAPE_MISMATCH   = 4,
    NEURAL_ERR_DTYPE_MISMATCH   = 5,
    NEURAL_ERR_FILE_NOT_FOUND   = 6,
    NEURAL_ERR_FILE_READ        = 7,
    NEURAL_ERR_FILE_WRITE       = 8,
    NEURAL_ERR_PARSE_ERROR      = 9,
    NEURAL_ERR_INVALID_CONFIG   = 10,
    NEURAL_ERR_TENSOR_TOO_LARGE = 11,
    NEURAL_ERR_INVALID_DTYPE    = 12,
    NEURAL_ERR_DIM_MISMATCH     = 13,
    NEURAL_ERR_NOT_IMPLEMENTED  = 14,
    NEURAL_ERR_INTERNAL         = 15,
    NEURAL_ERR_GRAD_CHECK       = 16,
    NEURAL_ERR_NAN_DETECTED     = 17,
    NEURAL_ERR_INF_DETECTED     = 18
} NeuralError;

/* dtype codes: neural_api.h:41-44. */
typedef enum { NEURAL_DTYPE_FLOAT32 = 0, NEURAL_DTYPE_FLOAT64 = 1 } NeuralDtype;

/* Opaque 64-byte tensor descriptor.  Offsets 0..39 keep the reference layout
 * (tensor.asm:7-24): data@0, ndim@8, shape@16, stride@24 (bytes, the unit
 * neural_tensor_stride() reports), dtype@32, flags@36. */
typedef struct NeuralTensor NeuralTensor;

/* ---- Framework / errors --------------------------------------------------- */
int         neural_init(void);                       /* neural_api.h:68  (neural_api.asm:297-331) */
void        neural_shutdown(void);                   /* neural_api.h:73 */
const char *neural_version(void);                    /* neural_api.h:79 */
void        neural_clear_error(void);                /* neural_api.h:88 */
int         neural_get_last_error(void);             /* neural_api.h:94 (thread-local here; global at neural_api.asm:56) */
const char *neural_get_error_message(int error_code);/* neural_api.h:101 (error.asm:32-50) */

/* ---- Tensor API: neural_api.h:130-302, neural_api.asm:392-967,2293-2426 ---- */
NeuralTensor   *neural_tensor_create(const uint64_t *shape, uint64_t ndim, int dtype);   /* neural_api.h:130 */
NeuralTensor   *neural_tensor_zeros(const uint64_t *shape, uint64_t ndim, int dtype);    /* neural_api.h:139 */
NeuralTensor   *neural_tensor_ones(const uint64_t *shape, uint64_t ndim, int dtype);     /* neural_api.h:148 */
NeuralTensor   *neural_tensor_from_data(const void *data, const uint64_t *shape,
                                        uint64_t ndim, int dtype);                       /* neural_api.h:167 */
NeuralTensor   *neural_tensor_from_buffer(void *buffer, const uint64_t *shape, uint64_t ndim,
                                          int dtype, const int64_t *strides);            /* neural_api.h:183 */
const int64_t  *neural_tensor_stride(NeuralTensor *tensor);                              /* neural_api.h:190 */
int             neural_tensor_is_contiguous(NeuralTensor *tensor);                       /* neural_api.h:197 */
NeuralTensor   *neural_tensor_make_contiguous(NeuralTensor *tensor);                     /* neural_api.h:204 */

/* neural_api.h:209-217; layout: data@0 itemsize@8 ndim@16 shape@24 strides@32
 * readonly@40 format@44 (neural_api.asm:840-890). */
typedef struct {
    void           *data;
    uint64_t        itemsize;
    uint64_t        ndim;
    const uint64_t *shape;
    const int64_t  *strides;
    int             readonly;
    char            format[8];
} NeuralBufferInfo;
int             neural_buffer_info(NeuralTensor *tensor, NeuralBufferInfo *info);        /* neural_api.h:229 */

void            neural_tensor_free(NeuralTensor *tensor);                                /* neural_api.h:235 */
void           *neural_tensor_data(NeuralTensor *tensor);                                /* neural_api.h:242 */
uint64_t        neural_tensor_ndim(NeuralTensor *tensor);                                /* neural_api.h:249 */
const uint64_t *neural_tensor_shape(NeuralTensor *tensor);                               /* neural_api.h:256 */
uint64_t        neural_tensor_numel(NeuralTensor *tensor);                               /* neural_api.h:263 */
int             neural_tensor_dtype(NeuralTensor *tensor);                               /* neural_api.h:270 */
uint64_t        neural_tensor_bytes(NeuralTensor *tensor);                               /* neural_api.h:277 */
int             neural_tensor_fill(NeuralTensor *tensor, double value);                  /* neural_api.h:285 (tensor.asm:531-589) */
int             neural_tensor_copy(NeuralTensor *dst, const NeuralTensor *src);          /* neural_api.h:293 (neural_api.asm:905-967) */
NeuralTensor   *neural_tensor_reshape(NeuralTensor *tensor, const uint64_t *new_shape,
                                      uint64_t new_ndim);                                /* neural_api.h:302 (tensor.asm:600-680) */

/* NEW: explicit transfers and the device address, for callers that manage
 * their own host buffers or hand the data to other HIP code. */
int   neural_tensor_upload(NeuralTensor *tensor, const void *host_src, uint64_t bytes);
int   neural_tensor_download(NeuralTensor *tensor, void *host_dst, uint64_t bytes);
void *neural_tensor_device_data(NeuralTensor *tensor);

/* ---- Elementwise / broadcast: neural_api.h:315-349, math_kernels.asm:66-945 */
/* Shapes: equal element counts run flat (the reference loop, math_kernels.asm:
 * 105-131); otherwise numpy broadcasting over up to 4 dims, honouring strides. */
int neural_add(NeuralTensor *out, const NeuralTensor *a, const NeuralTensor *b);  /* neural_api.h:315, ew_add  math_kernels.asm:66 */
int neural_sub(NeuralTensor *out, const NeuralTensor *a, const NeuralTensor *b);  /* neural_api.h:324, ew_sub  math_kernels.asm:182 */
int neural_mul(NeuralTensor *out, const NeuralTensor *a, const NeuralTensor *b);  /* neural_api.h:333, ew_mul  math_kernels.asm:292 */
int neural_div(NeuralTensor *out, const NeuralTensor *a, const NeuralTensor *b);  /* neural_api.h:342, ew_div  math_kernels.asm:402 */
int neural_maximum(NeuralTensor *out, const NeuralTensor *a, const NeuralTensor *b); /* ew_max math_kernels.asm:730 */
int neural_scalar_add(NeuralTensor *out, const NeuralTensor *a, double s);        /* ew_scalar_add math_kernels.asm:516 */
int neural_scalar_mul(NeuralTensor *out, const NeuralTensor *a, double s);        /* ew_scalar_mul math_kernels.asm:625 */
int neural_neg(NeuralTensor *out, const NeuralTensor *a);                         /* ew_neg math_kernels.asm:843 */
/* Row-broadcast bias add out[i,j] = x[i,j] + bias[j]: nn_layers.asm:472-539. */
int neural_bias_add(NeuralTensor *out, const NeuralTensor *x, const NeuralTensor *bias);
/* NEW out = max(0, a + b) in one pass (addss then maxss with +0, as
 * vec_add_relu_fusion, fusion.asm:200-226); b broadcasts as in neural_add, so
 * a [.., C] bias gives the bias + ReLU epilogue of matmul_bias_relu_fusion
 * (fusion.asm:110-190). */
int neural_add_relu(NeuralTensor *out, const NeuralTensor *a, const NeuralTensor *b);
/* NEW fused bias add + activation: out = act(x + bias) with x + bias rounded
 * in the tensor's dtype first (nn_layers.asm:472-539, then the activation
 * formulas of activations_c.c), bit-identical to neural_bias_add followed by
 * the activation.  alpha is used by LEAKY_RELU and ELU. */
typedef enum {
    NEURAL_ACT_NONE = 0, NEURAL_ACT_RELU = 1, NEURAL_ACT_SIGMOID = 2, NEURAL_ACT_TANH = 3,
    NEURAL_ACT_GELU = 4, NEURAL_ACT_LEAKY_RELU = 5, NEURAL_ACT_ELU = 6, NEURAL_ACT_SELU = 7,
    NEURAL_ACT_SWISH = 8, NEURAL_ACT_MISH = 9, NEURAL_ACT_HARDSWISH = 10, NEURAL_ACT_SOFTPLUS = 11,
    NEURAL_ACT_HARDTANH = 12
} NeuralActivation;
int neural_bias_add_act(NeuralTensor *out, const NeuralTensor *x, const NeuralTensor *bias, int act,
                        double alpha);

/* Raw-pointer f32 kernels of simd.asm:190-784, destination first as there
 * (host or device pointers; the reference returns void, these return 0 or an
 * error code). */
int   simd_add_f32(float *dst, const float *a, const float *b, uint64_t n);       /* simd.asm:190 */
int   simd_mul_f32(float *dst, const float *a, const float *b, uint64_t n);       /* simd.asm:316 */
int   simd_fma_f32(float *dst, const float *a, const float *b, const float *c,
                   uint64_t n);                                                   /* simd.asm:436 (fused a*b+c) */
float simd_dot_f32(const float *a, const float *b, uint64_t n);                   /* simd.asm:551 */
float simd_sum_f32(const float *a, uint64_t n);                                   /* simd.asm:684 */
/* c[i] = max(0, a[i] + b[i]); nothing for length <= 0 (host or device pointers). */
void  vec_add_relu_fusion(const float *a, const float *b, float *c, int64_t length);  /* fusion.asm:200 */

/* ---- Reductions ------------------------------------------------------------- */
/* neural_sum / neural_mean: neural_api.h:359,367 (stubs returning 14 at
 * neural_api.asm:2446-2454; implemented here).  Result in double. */
int neural_sum(const NeuralTensor *tensor, double *result);
int neural_mean(const NeuralTensor *tensor, double *result);
/* NEW full-tensor max (running-max semantics of activations.asm:888-895) and
 * argmax (tensor_argmax, main.asm:3598-3640). */
int neural_max(const NeuralTensor *tensor, double *result);
int neural_argmax(const NeuralTensor *tensor, int64_t *result);
/* reduce_sum / reduce_mean (math_kernels.asm:956-1264): axis -1 = all,
 * 0 = column sums of a 2-D tensor, 1 = row sums; other ranks reduce the
 * last dim when axis == ndim-1, else all.  Mean divides each output by its
 * own count (the asm divides only out[0] by the total, math_kernels.asm:
 * 1232-1256). */
int neural_reduce_sum(const NeuralTensor *in, int64_t axis, NeuralTensor *out);
int neural_reduce_mean(const NeuralTensor *in, int64_t axis, NeuralTensor *out);
/* NEW row max (running maxss over the row, activations.asm:888-895) and row
 * argmax (main.asm:3245-3270) over the last dim; indices are int64 written to
 * a host or device pointer with rows entries.  axis is -1 or ndim - 1, both
 * the last dim (unlike neural_reduce_sum, -1 is not the whole tensor: that is
 * neural_max / neural_argmax); other axes return NEURAL_ERR_DIM_MISMATCH. */
int neural_reduce_max(const NeuralTensor *in, int64_t axis, NeuralTensor *out);
int neural_reduce_argmax(const NeuralTensor *in, int64_t axis, int64_t *out_indices);
/* NEW, no counterpart in the reference: the row sum, mean, max and argmax over
 * the last dim from ONE read of `in`, each bit-identical to the matching
 * neural_reduce_sum / _mean / _max (axis = last dim) and neural_reduce_argmax
 * call.  Any output may be NULL (skipped), not all of them (NULL_POINTER);
 * sum / mean / max: contiguous, `rows` elements, the input's dtype; argmax:
 * `rows` int64 at a host or device pointer.  Outputs must not overlap. */
int neural_row_stats(const NeuralTensor *in, NeuralTensor *sum, NeuralTensor *mean, NeuralTensor *max,
                     int64_t *argmax);
/* NEW, no counterpart in the reference: out = in + bias exactly as
 * neural_bias_add, and the row statistics of out exactly as neural_row_stats,
 * reading `in` once and writing `out` once (contiguous tensors whose rows the
 * stand-alone reductions give one wave or block each; otherwise the two calls
 * in sequence, same results).  `out` may be `in` (the in-place bias add of a
 * linear layer) or overlap `in` or `bias`: such calls take the two-call route.
 * The statistics outputs must not overlap `out`, `in`, `bias` or each other. */
int neural_bias_add_row_stats(NeuralTensor *out, const NeuralTensor *in, const NeuralTensor *bias,
                              NeuralTensor *sum, NeuralTensor *mean, NeuralTensor *max, int64_t *argmax);

/* ---- Activations -------------------------------------------------------------- */
int neural_relu(NeuralTensor *out, const NeuralTensor *input);      /* neural_api.h:379, node_relu activations.asm:114-200 */
int neural_sigmoid(NeuralTensor *out, const NeuralTensor *input);   /* neural_api.h:387, node_sigmoid activations.asm:318-413 */
int neural_tanh(NeuralTensor *out, const NeuralTensor *input);      /* neural_api.h:395 */
int neural_softmax(NeuralTensor *out, const NeuralTensor *input);   /* neural_api.h:403, node_softmax activations.asm:761-987 */
/* NEW log-softmax rows, formula of metrics_losses.c:47-64. */
int neural_log_softmax(NeuralTensor *out, const NeuralTensor *input);
int neural_gelu(NeuralTensor *out, const NeuralTensor *input);                    /* neural_api.h:412 */
int neural_leaky_relu(NeuralTensor *out, const NeuralTensor *input, double alpha);/* neural_api.h:421 */
int neural_elu(NeuralTensor *out, const NeuralTensor *input, double alpha);       /* neural_api.h:431 */
int neural_selu(NeuralTensor *out, const NeuralTensor *input);                    /* neural_api.h:441 */
int neural_swish(NeuralTensor *out, const NeuralTensor *input);                   /* neural_api.h:450 */
int neural_mish(NeuralTensor *out, const NeuralTensor *input);                    /* neural_api.h:459 */
int neural_hardswish(NeuralTensor *out, const NeuralTensor *input);               /* neural_api.h:468 */
int neural_softplus(NeuralTensor *out, const NeuralTensor *input);                /* neural_api.h:477 */
int neural_hardtanh(NeuralTensor *out, const NeuralTensor *input);                /* neural_api.h:486 */
/* Tensor-level activations (neural_api.h:494-503, activations_c.c:124-158). */
int act_tanh(void *out, const void *in);
int act_gelu(void *out, const void *in);
int act_leaky_relu(void *out, const void *in, double alpha);
int act_elu(void *out, const void *in, double alpha);
int act_selu(void *out, const void *in);
int act_swish(void *out, const void *in);
int act_mish(void *out, const void *in);
int act_hardswish(void *out, const void *in);
int act_softplus(void *out, const void *in);
int act_hardtanh(void *out, const void *in);

/* ---- Optimizers: neural_api.h:510-517, optimizers_c.c:135-562 ----------------- */
void   *opt_sgd_create(double lr, double momentum);                                   /* optimizers_c.c:135 */
void   *opt_adam_create(double lr, double beta1, double beta2, double epsilon);       /* optimizers_c.c:145 */
void   *opt_adamw_create(double lr, double beta1, double beta2, double epsilon,
                         double weight_decay);                                        /* optimizers_c.c:158 */
int     opt_step(void *opt, void **params, void **grads, int64_t n);                  /* optimizers_c.c:353 */
void    opt_free(void *opt);                                                          /* optimizers_c.c:370 */
double  opt_get_lr(void *opt);                                                        /* optimizers_c.c:378 */
void    opt_set_lr(void *opt, double lr);                                             /* optimizers_c.c:384 */
int64_t opt_state_bytes(void *opt);                                                   /* optimizers_c.c:398 */
int     opt_state_export(void *opt, void *buffer, int64_t size);                      /* optimizers_c.c:417 */
int     opt_state_import(void *opt, const void *buffer, int64_t size);                /* optimizers_c.c:480 */

/* Gradient clipping: neural_api.h:731,741 (neural_api.asm:1677-1720 ->
 * clip_grad_norm_ / clip_grad_value_, optimizers.asm:1370-1620).  On an
 * optimizer handle, they act on the gradient tensors passed to its latest
 * opt_step (none before the first step: NEURAL_OK, nothing done).  Global-norm
 * clip: norm = sqrt(sum double(g)^2); when norm > max_norm every gradient is
 * multiplied by max_norm / norm (f32: that scale rounded to float).  Value
 * clip: g = min(max(g, lo), hi) with SSE maxsd/minsd operand rules (a NaN
 * gradient becomes lo); f32 bounds rounded to float. */
int     neural_clip_grad_norm(void *optimizer, double max_norm);                     /* neural_api.h:731 */
int     neural_clip_grad_value(void *optimizer, double min_val, double max_val);     /* neural_api.h:741 */
/* NEW: the same on an explicit gradient list (NULL entries skipped); total_norm
 * (may be NULL) receives the pre-clip norm -- when NULL the call does not wait
 * for the device.  At most 16384 non-empty tensors per call. */
int     neural_clip_grad_norm_list(NeuralTensor **grads, int64_t n, double max_norm, double *total_norm);
int     neural_clip_grad_value_list(NeuralTensor **grads, int64_t n, double min_val, double max_val);

/* ---- INT8 quantization: neural_api.h:1008-1065, quantize.c:39-269 ------------- */
/* Same 40-byte layout as the reference (scale@0 zero_point@8 min_val@16
 * max_val@24 symmetric@32). */
typedef struct {
    double  scale;
    int32_t zero_point;
    double  min_val;
    double  max_val;
    int     symmetric;
} QuantParams;
int    calibrate_minmax(const double *data, int64_t n, int symmetric, QuantParams *out); /* quantize.c:52 */
/* quantized_matmul (quantize.c:191-214): C[M x N] = (double)acc * (sa * sb),
 * acc = sum_k (A[i][k] - za)(B[k][j] - zb) in int32 (wrapping), A [M x K] and
 * B [K x N] row-major int8; host or device pointers; 0, or -1 for NULL
 * pointers / non-positive sizes / more than 8,388,480 rows or 1,048,560
 * columns of A. */
int    quantized_matmul(const int8_t *A, const int8_t *B, double *C, int64_t M, int64_t K, int64_t N,
                        const QuantParams *params_a, const QuantParams *params_b);
/* calibrate_percentile (quantize.c:89-132): calibrate on [sorted[lo], sorted[hi]]
 * of the data in the order of quantize.c's comparator, lo = (int64)(n p),
 * hi = (int64)(n (1 - p)), p outside [0, 0.5] taken as 0.01; host or device
 * data; 0, or -1 for NULL / n <= 0 / a NaN p (which the reference does not
 * survive). */
int    calibrate_percentile(const double *data, int64_t n, double percentile, int symmetric, QuantParams *out);
int    quantize_tensor(const double *data, int8_t *out, int64_t n, const QuantParams *p);/* quantize.c:144 */
int    dequantize_tensor(const int8_t *data, double *out, int64_t n, const QuantParams *p);/* quantize.c:163 */
double quantization_error(const double *original, int64_t n, const QuantParams *p);   /* quantize.c:222 */
double quantization_snr(const double *original, int64_t n, const QuantParams *p);     /* quantize.c:247 */
/* NEW fp32 variants (input widened to double exactly; same arithmetic). */
int    calibrate_minmax_f32(const float *data, int64_t n, int symmetric, QuantParams *out);
int    quantize_tensor_f32(const float *data, int8_t *out, int64_t n, const QuantParams *p);
int    dequantize_tensor_f32(const int8_t *data, float *out, int64_t n, const QuantParams *p);
double quantization_error_f32(const float *original, int64_t n, const QuantParams *p);
double quantization_snr_f32(const float *original, int64_t n, const QuantParams *p);
/* NEW device-resident pipeline: params are produced and consumed in device
 * memory (no host round trip between calibration and quantization). */
int    calibrate_minmax_f32_dev(const float *data, int64_t n, int symmetric, QuantParams *dev_params);
int    quantize_tensor_f32_dev(const float *data, int8_t *out, int64_t n, const QuantParams *dev_params);
int    dequantize_tensor_f32_dev(const int8_t *data, float *out, int64_t n, const QuantParams *dev_params);
/* NEW, no counterpart in the reference: calibrate_minmax_f32_dev for callers
 * that cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same result, bit for bit; data and
 * dev_params must be device pointers (host pointers: -1,
 * NEURAL_ERR_INVALID_ARGUMENT).  Allocates nothing and never initialises the
 * library: before neural_init() it returns -1 with NEURAL_ERR_INVALID_CONFIG.
 * The segment summaries use a static 64 KiB device buffer per GPU (held until
 * the process ends); a launch whose summaries would not fit it returns -1
 * with NEURAL_ERR_TENSOR_TOO_LARGE (never on MI355X: at most 4 per CU).
 * Calls enqueued on one stream are ordered; calls that overlap on one GPU
 * (e.g. captured graphs replayed concurrently on two streams) race on the
 * buffer. */
int    calibrate_minmax_f32_dev_noalloc(const float *data, int64_t n, int symmetric, QuantParams *dev_params);

/* ---- Training ops: training_ops.asm:544-696 (neural_api.asm:2786-2791) -------- */
int   neural_tensor_has_nan(const float *data, uint64_t n);      /* training_ops.asm:544 */
int   neural_tensor_has_inf(const float *data, uint64_t n);      /* training_ops.asm:585 */
float neural_tensor_grad_l2_norm(const float *data, uint64_t n); /* training_ops.asm:636 */
/* NEW fused single pass: NaN flag, Inf flag and sum of squares (double). */
int   neural_scan_nan_inf_l2(const float *data, uint64_t n, int *has_nan, int *has_inf,
                             double *sumsq);
/* NEW tensor-level forms (no host round trip for device-resident tensors). */
int   neural_tensor_scan(NeuralTensor *t, int *has_nan, int *has_inf, double *sumsq);

/* Inverted dropout (training_ops.asm:718-858; neural_api.asm:2797-2803; bound
 * at pyneural/core.py:499-515).  Forward draws one value of the library's
 * copy of glibc's rand() stream per element: dropped when the draw is below
 * cvtsd2si(p * 2147483647.0) (mask 0, out +0.0f), else mask 1 and
 * out = x * (float)(1 / (1 - p)).  Backward: grad_in = mask ? grad_out * scale
 * : +0.0f.  Host or device pointers. */
int   neural_dropout_forward(const float *input, float *output, uint8_t *mask, uint64_t num_elements,
                             float p);
int   neural_dropout_backward(const float *grad_output, float *grad_input, const uint8_t *mask,
                              uint64_t num_elements, float p);
/* NEW: position the dropout stream as srand(seed) positions glibc's rand()
 * (the reference seeds through srand, training_ops.asm:943); the stream
 * starts as srand(1).  neural_dropout_draws: draws taken since the last seed. */
int      neural_dropout_seed(uint32_t seed);
uint64_t neural_dropout_draws(void);

/* ---- 2-D f64 tensor ops: neural_api.h:1273-1305, tensor_ops.c:15-148 ---------- */
int tensor_concat_2d(const double *a, const double *b, int64_t rows_a, int64_t cols_a,
                     int64_t rows_b, int64_t cols_b, int64_t axis, double *out,
                     int64_t *out_rows, int64_t *out_cols);
int tensor_split_2d(const double *in, int64_t rows, int64_t cols, int64_t axis,
                    int64_t split_index, double *out_a, double *out_b, int64_t *rows_a,
                    int64_t *cols_a, int64_t *rows_b, int64_t *cols_b);
int tensor_pad_2d(const double *in, int64_t in_rows, int64_t in_cols, int64_t pad_top,
                  int64_t pad_bottom, int64_t pad_left, int64_t pad_right, double pad_value,
                  double *out, int64_t *out_rows, int64_t *out_cols);
int tensor_transpose2d_array(const double *in, int64_t rows, int64_t cols, double *out);

/* ---- Per-feature transforms: neural_api.h:1115-1126, transforms.c:27-143 ---- */
/* [batch, features] row-major float64, host or device pointers; 0 or -1 as
 * the reference (NULL data / non-positive sizes).  compute_stats: any output
 * may be NULL; min / max start at +-1e308 and keep the first of equal values;
 * std is the population std sqrt(max(sum2/b - mean^2, 0)). */
int transform_compute_stats(const double *data, int64_t batch_size, int64_t num_features, double *mean_out,
                            double *std_out, double *min_out, double *max_out);          /* transforms.c:26 */
int transform_normalize(const double *data, double *output, int64_t batch_size, int64_t num_features,
                        const double *mean, const double *std, double eps);              /* transforms.c:69 */
int transform_unnormalize(const double *data, double *output, int64_t batch_size, int64_t num_features,
                          const double *mean, const double *std, double eps);            /* transforms.c:95 */
int transform_minmax(const double *data, double *output, int64_t batch_size, int64_t num_features,
                     const double *min_val, const double *max_val, double eps);          /* transforms.c:122 */

/* ---- Cross-entropy losses --------------------------------------------------------- */
/* Label-smoothed cross-entropy (replaces metrics_losses.c:28-125, declared at
 * neural_api.h:1101-1106): f64 logits [batch, num_classes], int64 targets;
 * smoothed target (1 - a) * one_hot + a / K; loss_out = mean over rows of
 * -sum_c target_c * log_softmax_c; grad_out = (softmax - target) / batch.
 * Pointers may be host or device memory.  Returns 0, or -1 on NULL, batch or
 * num_classes <= 0, smoothing outside [0, 1], or a target outside [0, K). */
int label_smoothing_ce_forward(const double *logits, const int64_t *targets, int64_t batch_size,
                               int64_t num_classes, double smoothing, double *loss_out);
int label_smoothing_ce_backward(const double *logits, const int64_t *targets, int64_t batch_size,
                                int64_t num_classes, double smoothing, double *grad_out);
/* NEW: forward and backward in one pass over the logits.  The gradient bits
 * equal label_smoothing_ce_backward's; the loss agrees with
 * label_smoothing_ce_forward's to a few ulps of the row terms (the f64
 * forward takes exp from a table, this form the library's exp). */
int label_smoothing_ce_fused(const double *logits, const int64_t *targets, int64_t batch_size,
                             int64_t num_classes, double smoothing, double *loss_out, double *grad_out);
/* NEW: the same on f32 logits (widened exactly to double, as the reference's
 * f32 paths do), gradient rounded to float. */
int label_smoothing_ce_fused_f32(const float *logits, const int64_t *targets, int64_t batch_size,
                                 int64_t num_classes, double smoothing, double *loss_out, float *grad_out);
/* NEW, no counterpart in the reference (for GPU training loops that read the
 * loss only now and then): the forward, fused and f32 fused forms with the
 * mean loss left in device memory (*loss_dev, one double) instead of
 * returned to the host.  The call returns once its launches are enqueued on
 * the library's stream; the loss and gradient bits equal those of the
 * host-returning form of the same name without _dev.  Every pointer must be device memory, aligned to its element
 * (targets and loss_dev to 8 bytes).  Returns 0, or -1 on NULL, a host or
 * misaligned pointer, batch or num_classes <= 0, or smoothing outside
 * [0, 1]; a target outside [0, K) cannot be reported without waiting: it
 * makes the loss NaN and leaves that row's gradient unwritten. */
int label_smoothing_ce_forward_dev(const double *logits, const int64_t *targets, int64_t batch_size,
                                   int64_t num_classes, double smoothing, double *loss_dev);
int label_smoothing_ce_fused_dev(const double *logits, const int64_t *targets, int64_t batch_size,
                                 int64_t num_classes, double smoothing, double *loss_dev, double *grad_dev);
int label_smoothing_ce_fused_f32_dev(const float *logits, const int64_t *targets, int64_t batch_size,
                                     int64_t num_classes, double smoothing, double *loss_dev, float *grad_dev);
/* Cross-entropy of softmax(prediction) (replaces neural_api.h:674,
 * neural_api.asm:2546 -> losses.asm:315-613, intended semantics): prediction
 * [batch, K], target [batch] holding class indices as values of the same
 * dtype (truncated); *loss = mean over rows of -log(softmax[target] + 1e-7).
 * NULL_POINTER / DTYPE_MISMATCH / DIM_MISMATCH (prediction not 2-D) /
 * SHAPE_MISMATCH (target numel != batch) / INVALID_ARGUMENT (target out of
 * range, or non-contiguous tensors). */
int neural_cross_entropy_loss(const NeuralTensor *prediction, const NeuralTensor *target, double *loss);

/* ---- Reference entry points outside the hot path ---------------------------------
 * The reference's Python layer binds every one of these names at import
 * (pyneural/core.py; the line of each binding is given), so the library
 * exports them for that loader to succeed.  The subsystems behind them
 * (layers, recurrent cells, pooling, attention, fuzzy logic, pruning,
 * datasets, config, metrics, TensorBoard writer, weight init, LR schedules,
 * the asm optimizer handles) are outside
 * this library's scope.  Each records NEURAL_ERR_NOT_IMPLEMENTED as the last
 * error and returns: NEURAL_ERR_NOT_IMPLEMENTED (int neural_* functions), -1
 * (other int and int64_t functions, the C modules' failure value), NULL
 * (pointers), 0 (uint64_t), NaN (double).  The *_free functions and
 * neural_optimizer_set_lr do nothing (no stub hands out an object);
 * neural_get_simd_level / _name report that no host SIMD path exists. */
int attention_scaled_dot_product(void *, void *, void *, void *, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, void *, void *);  /* core.py:1336 */
int batchnorm1d_backward(void *, void *, void *, void *, void *, int64_t);  /* core.py:812 */
int batchnorm1d_forward(void *, void *, void *, int64_t, int);  /* core.py:803 */
int64_t batchnorm1d_num_features(void *);  /* core.py:834 */
void *batchnorm1d_beta(void *);  /* core.py:825 */
void *batchnorm1d_create(int64_t, double, double);  /* core.py:797 */
void *batchnorm1d_gamma(void *);  /* core.py:822 */
void *batchnorm1d_running_mean(void *);  /* core.py:828 */
void *batchnorm1d_running_var(void *);  /* core.py:831 */
void batchnorm1d_free(void *);  /* core.py:800 */
int conv2d_layer_backward(void *, void *, void *, int64_t, int64_t, int64_t, void *, void *, void *);  /* core.py:1150 */
int conv2d_layer_forward(void *, void *, int64_t, int64_t, int64_t, void *);  /* core.py:1140 */
int64_t conv2d_layer_in_channels(void *);  /* core.py:1178 */
int64_t conv2d_layer_kernel_h(void *);  /* core.py:1184 */
int64_t conv2d_layer_kernel_w(void *);  /* core.py:1187 */
int64_t conv2d_layer_out_channels(void *);  /* core.py:1181 */
int64_t conv2d_layer_out_h(void *, int64_t);  /* core.py:1169 */
int64_t conv2d_layer_out_w(void *, int64_t);  /* core.py:1172 */
int64_t conv2d_layer_padding(void *);  /* core.py:1193 */
int64_t conv2d_layer_stride(void *);  /* core.py:1190 */
int64_t conv2d_layer_weight_size(void *);  /* core.py:1175 */
int64_t conv2d_output_size(int64_t, int64_t, int64_t, int64_t);  /* core.py:1118 */
void *conv2d_layer_bias(void *);  /* core.py:1166 */
void *conv2d_layer_create(int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int);  /* core.py:1126 */
void *conv2d_layer_weight(void *);  /* core.py:1163 */
void conv2d_layer_free(void *);  /* core.py:1137 */
int embedding_backward(void *, void *, int64_t, void *, void *);  /* core.py:961 */
int embedding_forward(void *, void *, int64_t, void *);  /* core.py:953 */
int64_t embedding_dim(void *);  /* core.py:976 */
int64_t embedding_num_embeddings(void *);  /* core.py:973 */
void *embedding_create(int64_t, int64_t);  /* core.py:947 */
void *embedding_weight(void *);  /* core.py:970 */
void embedding_free(void *);  /* core.py:950 */
double fuzzy_and(double, double);  /* core.py:1007 */
double fuzzy_defuzz_bisector(void *, void *, int64_t);  /* core.py:1024 */
double fuzzy_defuzz_centroid(void *, void *, int64_t);  /* core.py:1017 */
double fuzzy_defuzz_mom(void *, void *, int64_t);  /* core.py:1031 */
double fuzzy_gaussian(double, double, double);  /* core.py:999 */
double fuzzy_not(double);  /* core.py:1013 */
double fuzzy_or(double, double);  /* core.py:1010 */
double fuzzy_trapezoidal(double, double, double, double, double);  /* core.py:990 */
double fuzzy_triangular(double, double, double, double);  /* core.py:982 */
int fuzzy_system_add_input_mf(void *, int, int, double, double, double, double);  /* core.py:1065 */
int fuzzy_system_add_output_mf(void *, int, double, double, double, double);  /* core.py:1076 */
int fuzzy_system_add_rule(void *, void *, void *, int, int, double);  /* core.py:1086 */
int fuzzy_system_defuzz_method(void *);  /* core.py:1113 */
int fuzzy_system_evaluate(void *, void *, void *);  /* core.py:1096 */
int fuzzy_system_n_inputs(void *);  /* core.py:1104 */
int fuzzy_system_n_rules(void *);  /* core.py:1107 */
int fuzzy_system_resolution(void *);  /* core.py:1110 */
int fuzzy_system_set_input_range(void *, int, double, double);  /* core.py:1050 */
int fuzzy_system_set_output_range(void *, double, double);  /* core.py:1058 */
void *fuzzy_system_create(int, int, int);  /* core.py:1039 */
void fuzzy_system_free(void *);  /* core.py:1046 */
double *gru_bias_hh(void *);  /* core.py:364 */
double *gru_bias_ih(void *);  /* core.py:362 */
double *gru_weight_hh(void *);  /* core.py:360 */
double *gru_weight_ih(void *);  /* core.py:358 */
int gru_forward(void *, double *, double *, double *, double *, int64_t, int64_t);  /* core.py:347 */
int64_t gru_hidden_size(void *);  /* core.py:368 */
int64_t gru_input_size(void *);  /* core.py:366 */
void *gru_create(int64_t, int64_t);  /* core.py:341 */
void gru_free(void *);  /* core.py:344 */
int layernorm_backward(void *, void *, void *, void *, void *, int64_t);  /* core.py:852 */
int layernorm_forward(void *, void *, void *, int64_t);  /* core.py:844 */
int64_t layernorm_num_features(void *);  /* core.py:868 */
void *layernorm_beta(void *);  /* core.py:865 */
void *layernorm_create(int64_t, double);  /* core.py:838 */
void *layernorm_gamma(void *);  /* core.py:862 */
void layernorm_free(void *);  /* core.py:841 */
double *lstm_bias_hh(void *);  /* core.py:334 */
double *lstm_bias_ih(void *);  /* core.py:332 */
double *lstm_weight_hh(void *);  /* core.py:330 */
double *lstm_weight_ih(void *);  /* core.py:328 */
int lstm_forward(void *, double *, double *, double *, double *, double *, double *, int64_t, int64_t);  /* core.py:315 */
int64_t lstm_hidden_size(void *);  /* core.py:338 */
int64_t lstm_input_size(void *);  /* core.py:336 */
void *lstm_create(int64_t, int64_t);  /* core.py:309 */
void lstm_free(void *);  /* core.py:312 */
const char *neural_get_simd_name(void);  /* core.py:113 */
double compute_sparsity(void *, int64_t);  /* core.py:705 */
double compute_threshold_for_sparsity(void *, int64_t, double);  /* core.py:711 */
int neural_get_simd_level(void);  /* core.py:110 */
int neural_matmul(void *, void *, void *);  /* core.py:178 */
int neural_mse_loss(void *, void *, double *);  /* core.py:372 */
int neural_weighted_sample_indices(void *, uint64_t, uint64_t, void *, int);  /* core.py:618 */
int roc_auc_score(void *, void *, int64_t, double *);  /* core.py:893 */
int64_t count_nonzero(void *, int64_t);  /* core.py:708 */
void apply_mask(void *, void *, int64_t);  /* core.py:718 */
void *neural_adam_create(double, double, double, double);  /* core.py:243 */
void *neural_adamw_create(double, double, double, double, double);  /* core.py:251 */
double neural_compute_accuracy_from_matrix(void *, int);  /* core.py:450 */
double neural_compute_class_f1(void *, int, int);  /* core.py:443 */
double neural_compute_class_precision(void *, int, int);  /* core.py:429 */
double neural_compute_class_recall(void *, int, int);  /* core.py:436 */
int neural_compute_class_weights(void *, uint64_t, uint64_t, void *);  /* core.py:601 */
int neural_compute_sample_weights(void *, uint64_t, void *, uint64_t, void *);  /* core.py:609 */
void *neural_config_load(const char *);  /* core.py:411 */
void neural_config_free(void *);  /* core.py:414 */
int neural_confusion_matrix_update(void *, void *, void *, uint64_t, uint64_t);  /* core.py:420 */
int neural_dataset_get_batch(void *, uint64_t, uint64_t, void **, void **);  /* core.py:401 */
uint64_t neural_dataset_size(void *);  /* core.py:398 */
void *neural_dataset_load_csv(const char *, const char *, uint64_t, uint32_t);  /* core.py:387 */
void neural_dataset_free(void *);  /* core.py:395 */
int neural_init_he_normal(void *, uint64_t, uint64_t, int);  /* core.py:554 */
int neural_init_he_uniform(void *, uint64_t, uint64_t, int);  /* core.py:537 */
int neural_init_kaiming_uniform(void *, uint64_t, uint64_t, uint64_t, int, int);  /* core.py:571 */
int neural_init_normal_range(void *, uint64_t, float, float, int);  /* core.py:528 */
int neural_init_uniform_range(void *, uint64_t, float, float, int);  /* core.py:519 */
int neural_init_xavier_normal(void *, uint64_t, uint64_t, uint64_t, int);  /* core.py:562 */
int neural_init_xavier_uniform(void *, uint64_t, uint64_t, uint64_t, int);  /* core.py:545 */
int neural_linear_forward(void *, void *, void *);  /* core.py:229 */
void *neural_linear_bias(void *);  /* core.py:236 */
void *neural_linear_create(uint64_t, uint64_t, int);  /* core.py:223 */
void *neural_linear_weight(void *);  /* core.py:233 */
void neural_linear_free(void *);  /* core.py:226 */
double neural_lr_cosine_annealing(double, int, int, double);  /* core.py:472 */
double neural_lr_exponential_decay(double, int, double);  /* core.py:465 */
double neural_lr_step_decay(double, int, int, double);  /* core.py:457 */
double neural_optimizer_get_lr(void *);  /* core.py:588 */
void neural_optimizer_free(void *);  /* core.py:260 */
void neural_optimizer_set_lr(void *, double);  /* core.py:582 */
void *neural_sgd_create(double, double);  /* core.py:240 */
int avgpool2d_backward(void *, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, void *);  /* core.py:1242 */
int avgpool2d_forward(void *, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, void *);  /* core.py:1228 */
int maxpool2d_backward(void *, void *, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, void *);  /* core.py:1213 */
int maxpool2d_forward(void *, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, void *, void *);  /* core.py:1198 */
int64_t prune_cols(void *, int64_t, int64_t, double, void *);  /* core.py:696 */
int64_t prune_magnitude(void *, void *, int64_t, double);  /* core.py:671 */
int64_t prune_rows(void *, int64_t, int64_t, double, void *);  /* core.py:687 */
int64_t prune_topk(void *, void *, int64_t, double);  /* core.py:679 */
const char *tb_get_filepath(int);  /* core.py:667 */
const char *tb_get_logdir(int);  /* core.py:664 */
int tb_add_histogram_stats(int, const char *, void *, int, int64_t);  /* core.py:649 */
int tb_add_scalar(int, const char *, float, int64_t);  /* core.py:631 */
int tb_add_scalars(int, const char *, void *, void *, int, int64_t);  /* core.py:639 */
int tb_close(int);  /* core.py:661 */
int tb_create_writer(const char *);  /* core.py:628 */
int tb_flush(int);  /* core.py:658 */
int transformer_block_forward(void *, int64_t, int64_t, int64_t, int64_t, void *, void *, void *, void *, void *, void *, void *, void *, void *, void *, void *, void *, double, void *);  /* core.py:1352 */
int upsample2d_nearest_backward(void *, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, void *);  /* core.py:1268 */
int upsample2d_nearest_forward(void *, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, void *);  /* core.py:1256 */

/* ---- HIP runtime controls (NEW) ------------------------------------------------- */
/* Threads: every entry point may be called from several host threads at
 * once (the reference is single-threaded; ctypes releases the GIL around
 * each call).  The last error is per thread.  Calls that use the shared
 * reduction workspace (whole-tensor and per-row reductions over few rows, the
 * NaN/Inf/L2 scan, calibration, quantization error, the CE losses, gradient
 * clipping, simd_sum/dot) hold one process-wide lock from their first launch
 * until their result has been read back, so they serialise; everything else
 * only shares the stream.  One tensor must not be written by one thread while
 * another reads or writes it. */
/* Use an existing HIP stream (e.g. torch.cuda.current_stream().cuda_stream) for
 * all later launches; NULL selects the HIP null stream.  The previous stream
 * is synchronised first.  neural_hip_reset_stream() returns to the library's
 * own stream, a blocking one: it orders implicitly with the legacy null stream
 * (torch's default stream), so kernels on it follow earlier null-stream work
 * and later null-stream work waits for them. */
/* NEW (no reference counterpart; for measurement): attach two hipEvent_t to
 * one later kernel launch made by the CALLING thread: the launch after the
 * next `skip` launches (skip = 0: the next launch; the second kernel of a
 * two-kernel call is skip = 1).  That launch is made with
 * hipExtLaunchKernelGGL, so hipEventElapsedTime(start, stop) is that
 * kernel's own execution time on its stream, without the latency of separate
 * event records around the call.  The events are used once, then cleared;
 * neural_hip_time_cancel() clears them unused.  Returns
 * NEURAL_ERR_NULL_POINTER for a null event, NEURAL_ERR_INVALID_ARGUMENT for
 * skip < 0. */
int   neural_hip_time_next_launch(void *start_event, void *stop_event, int skip);
/* NEW (no reference counterpart; for measurement): the same over a span of
 * launches: after `skip` launches, the next one records start_event when it
 * starts executing and the launch `count` - 1 later records stop_event when it
 * ends, so hipEventElapsedTime spans every kernel of a multi-launch call and
 * the gaps between them (count = 1 is neural_hip_time_next_launch).  Returns
 * NEURAL_ERR_INVALID_ARGUMENT for skip < 0 or count < 1. */
int   neural_hip_time_launches(void *start_event, void *stop_event, int skip, int count);
int   neural_hip_time_cancel(void);
/* NEW (no reference counterpart; for measurement): kernel launches the
 * calling thread has made so far (the difference around a call is the number
 * of launches the call makes). */
unsigned long long neural_hip_launch_count(void);
/* NEW (no reference counterpart; diagnostics): device allocations the
 * library has requested so far from its caching allocator (every request)
 * and, among them, those that called hipMalloc (cache misses); either
 * pointer may be NULL.  Process-wide counts. */
int   neural_hip_alloc_stats(unsigned long long *dev_allocs, unsigned long long *hip_mallocs);
/* NEW (no reference counterpart; a bandwidth reference for measurement):
 * dst = src over `bytes` bytes with the library's flat streaming kernel
 * (16-byte non-temporal loads and stores).  Device pointers only, 16-byte
 * aligned, bytes a multiple of 16; otherwise NEURAL_ERR_INVALID_ARGUMENT. */
int   neural_hip_stream_copy(void *dst, const void *src, uint64_t bytes);
int   neural_hip_set_stream(void *hip_stream);
int   neural_hip_reset_stream(void);
void *neural_hip_get_stream(void);
int   neural_hip_synchronize(void);
/* Release cached device blocks back to the driver. */
int   neural_hip_empty_cache(void);
/* Device ordinal, compute-unit count and device name of the active GPU. */
int   neural_hip_device_info(int *ordinal, int *num_cus, char *name, int name_len);

#if defined(__GNUC__)
#pragma GCC visibility pop
#endif
#ifdef __cplusplus
}
#endif
#endif /* NEURAL_HIP_API_H */
