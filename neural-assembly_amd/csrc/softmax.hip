// softmax.hip -- row softmax and log-softmax over the last dimension.
//
// Softmax follows node_softmax (activations.asm:761-987) with its intended
// f32 semantics (the asm keeps the max and the running sum in one stack slot,
// activations.asm:900,927-929):
//   f32: m = row max; e_j = (float)exp((double)x_j - (double)m);
//        s = sum of e_j; y_j = e_j / s
//   f64: e_j = exp(x_j - m); y_j = e_j / s
// Here the f32 e_j come from the exact double difference x - m and the
// hardware exp2 (about 1.5e-7 relative, see exp_diff_f32) and y_j = e_j * (1/s).
// Log-softmax follows the formula of label_smoothing_ce_forward
// (metrics_losses.c:47-64) in double: y = (x - m) - log(sum exp(x - m)),
// rounded once for f32.
//
// The sum is accumulated in double with a fixed wave/block tree instead of the
// reference's sequential order; results are compared against the fp64-exact
// softmax.  A NaN anywhere in a row makes the whole row NaN, as in the
// reference (the NaN reaches the sum).
//
// Rows of up to 64*16 vectors (4096 f32 / 2048 f64 values) are register
// resident: one wave per row, a single HBM read and a single write.
#include <cmath>

#include <hip/hip_ext.h>

#include "common.hpp"

namespace nh {

constexpr int kSmBlock = 256;

template <typename T>
NH_DEV T neg_inf();
template <> NH_DEV float neg_inf<float>() { return -__builtin_inff(); }
template <> NH_DEV double neg_inf<double>() { return -__builtin_inf(); }

// exp(x - m) for f32 rows (x <= m, m the row max held in double): the
// difference is exact in double, so exp_d2f gives about 1.5e-7 relative
// against (float)exp((double)x - (double)m) for any spread of the row.  A NaN
// passes through and makes the row's sum NaN, as in the reference.
NH_DEV float exp_diff_f32(float x, double md) { return exp_d2f(double(x) - md); }

// One wave per row (RPW rows per wave: all loads of the wave's rows issued
// before any arithmetic).
template <bool LOG, int VPL, bool FULL>
NH_DEV void softmax_row_f32(f32x4 (&v)[VPL], f32x4 *__restrict__ yr, int64_t ncv, int lane)
{
    const auto in_row = [&](int k) { return FULL || lane + int64_t(k) * 64 < ncv; };
    float m = -__builtin_inff();
#pragma unroll
    for (int k = 0; k < VPL; k++) {
        if (in_row(k)) {
#pragma unroll
            for (int j = 0; j < 4; j++) m = __builtin_fmaxf(m, v[k][j]);
        }
    }
    const double md = double(wave_fmax(m));
    double s = 0.0;
    if (!LOG) {
        // e_j kept in the input registers, rounded to float as the reference does.
#pragma unroll
        for (int k = 0; k < VPL; k++) {
            if (in_row(k)) {
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const float e = exp_diff_f32(v[k][j], md);
                    v[k][j] = e;
                    s += double(e);
                }
            }
        }
        s = wave_dsum(s);
        const float rs = 1.0f / float(s);
#pragma unroll
        for (int k = 0; k < VPL; k++)
            if (in_row(k)) st_nt(yr + lane + k * 64, v[k] * rs);
    } else {
#pragma unroll
        for (int k = 0; k < VPL; k++) {
            if (in_row(k)) {
#pragma unroll
                for (int j = 0; j < 4; j++) s += double(exp_diff_f32(v[k][j], md));
            }
        }
        s = wave_dsum(s);
        // y = (x - m) - lse in float: x - m <= 0 and lse >= 0, so the two
        // terms never cancel and two float roundings (plus lse's) leave y
        // within ~2e-7 relative of the double expression; NaN / Inf rows give
        // the same NaNs as the double form.
        const float lse = float(log_ge1(s));  // s >= 1: the row maximum contributes exp(0) = 1
        const float mf = float(md);
#pragma unroll
        for (int k = 0; k < VPL; k++) {
            if (in_row(k)) st_nt(yr + lane + k * 64, (v[k] - mf) - lse);
        }
    }
}

template <bool LOG, int VPL, bool FULL, int RPW>
__global__ __launch_bounds__(kSmBlock) void k_softmax_wave_f32(const float *__restrict__ x, float *__restrict__ y,
                                                               int64_t rows, int64_t cols, int64_t r_base)
{
    using V = f32x4;
    const int lane = threadIdx.x & 63;
    const int64_t r0 = r_base + (int64_t(blockIdx.x) * (kSmBlock / 64) + (threadIdx.x >> 6)) * RPW;
    if (r0 >= rows) return;  // uniform per wave
    const int64_t ncv = cols / 4;
    V v[RPW][VPL];
#pragma unroll
    for (int q = 0; q < RPW; q++) {
        if (r0 + q < rows) {
            const V *xr = reinterpret_cast<const V *>(x + (r0 + q) * cols);
#pragma unroll
            for (int k = 0; k < VPL; k++)
                if (FULL || lane + int64_t(k) * 64 < ncv) v[q][k] = ld_nt(xr + lane + k * 64);
        }
    }
#pragma unroll
    for (int q = 0; q < RPW; q++)
        if (r0 + q < rows)
            softmax_row_f32<LOG, VPL, FULL>(v[q], reinterpret_cast<V *>(y + (r0 + q) * cols), ncv, lane);
}

template <bool LOG, int VPL>
__global__ __launch_bounds__(kSmBlock) void k_softmax_wave_f64(const double *__restrict__ x, double *__restrict__ y,
                                                               int64_t rows, int64_t cols, int64_t r_base)
{
    using V = f64x2;
    const int lane = threadIdx.x & 63;
    const int64_t r = r_base + int64_t(blockIdx.x) * (kSmBlock / 64) + (threadIdx.x >> 6);
    if (r >= rows) return;  // uniform per wave
    const V *xr = reinterpret_cast<const V *>(x + r * cols);
    V *yr = reinterpret_cast<V *>(y + r * cols);
    const int64_t ncv = cols / 2;

    V v[VPL];
#pragma unroll
    for (int k = 0; k < VPL; k++) {
        const int64_t c = lane + int64_t(k) * 64;
        if (c < ncv) v[k] = ld_nt(xr + c);
    }
    double m = -__builtin_inf();
#pragma unroll
    for (int k = 0; k < VPL; k++) {
        const int64_t c = lane + int64_t(k) * 64;
        if (c < ncv) {
#pragma unroll
            for (int j = 0; j < 2; j++) m = v[k][j] > m ? v[k][j] : m;
        }
    }
    m = wave_max_ignore_nan(m);
    double s = 0.0;
#pragma unroll
    for (int k = 0; k < VPL; k++) {
        const int64_t c = lane + int64_t(k) * 64;
        if (c < ncv) {
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const double e = exp(v[k][j] - m);
                if (!LOG) v[k][j] = e;
                s += e;
            }
        }
    }
    s = wave_sum(s);
    const double lse = LOG ? log_ge1(s) : 0.0;  // s >= 1 (the maximum contributes 1)
#pragma unroll
    for (int k = 0; k < VPL; k++) {
        const int64_t c = lane + int64_t(k) * 64;
        if (c < ncv) {
            V o;
#pragma unroll
            for (int j = 0; j < 2; j++) o[j] = LOG ? (v[k][j] - m) - lse : v[k][j] / s;
            st_nt(yr + c, o);
        }
    }
}

// General rows: one block per row, three passes over the row.
template <typename T>
NH_DEV T block_max_ignore_nan(T v)
{
    __shared__ T lds[kSmBlock / 64];
    v = wave_max_ignore_nan(v);
    if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = v;
    __syncthreads();
    T r = lds[0];
    for (int i = 1; i < kSmBlock / 64; i++) r = (lds[i] > r) ? lds[i] : r;
    __syncthreads();
    return r;
}

NH_DEV double block_sum(double v)
{
    __shared__ double lds[kSmBlock / 64];
    v = wave_sum(v);
    if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = v;
    __syncthreads();
    double r = lds[0];
    for (int i = 1; i < kSmBlock / 64; i++) r += lds[i];
    __syncthreads();
    return r;
}

NH_DEV float row_exp(float x, float m) { return exp_diff_f32(x, double(m)); }
NH_DEV double row_exp(double x, double m) { return exp(x - m); }

template <typename T, bool LOG>
__global__ __launch_bounds__(kSmBlock) void k_softmax_block(const T *__restrict__ x, T *__restrict__ y, int64_t cols,
                                                            int64_t r_base)
{
    const int64_t r = r_base + blockIdx.x;
    const T *xr = x + r * cols;
    T *yr = y + r * cols;
    T m = neg_inf<T>();
    for (int64_t j = threadIdx.x; j < cols; j += kSmBlock) m = xr[j] > m ? xr[j] : m;
    m = block_max_ignore_nan(m);
    const double md = double(m);
    double s = 0.0;
    for (int64_t j = threadIdx.x; j < cols; j += kSmBlock) s += double(row_exp(xr[j], m));
    s = block_sum(s);
    if (LOG) {
        const double lse = log(s);
        for (int64_t j = threadIdx.x; j < cols; j += kSmBlock) yr[j] = T((double(xr[j]) - md) - lse);
    } else {
        for (int64_t j = threadIdx.x; j < cols; j += kSmBlock) yr[j] = T(double(row_exp(xr[j], m)) / s);
    }
}

template <typename K, typename... Args>
static void launch_timed(K kernel, unsigned g, Args... args)
{
    NH_LAUNCH(kernel, dim3(g), dim3(kSmBlock), 0, stream(), args...);
}

template <typename T, bool LOG, int VPL>
static void launch_wave(const T *x, T *y, int64_t rows, int64_t cols)
{
    for_row_launches(rows, kSmBlock / 64, [&](unsigned g, int64_t base) {
        if constexpr (sizeof(T) == 4) {
            // (two rows per wave measured slower on MI355X: 89.7 vs 86.2 us at [65536,1024])
            if (cols == int64_t(VPL) * 256)
                launch_timed(k_softmax_wave_f32<LOG, VPL, true, 1>, g, x, y, rows, cols, base);
            else
                launch_timed(k_softmax_wave_f32<LOG, VPL, false, 1>, g, x, y, rows, cols, base);
        } else {
            launch_timed(k_softmax_wave_f64<LOG, VPL>, g, x, y, rows, cols, base);
        }
    });
}

template <typename T, bool LOG>
static int launch_softmax(const T *x, T *y, int64_t rows, int64_t cols)
{
    constexpr int VN = Vec16<T>::n;
    const bool vec = ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y)) & 15u) == 0 && cols % VN == 0;
    const int64_t ncv = cols / VN;
    if (vec && ncv <= 64 * 16) {
        if (ncv <= 64) launch_wave<T, LOG, 1>(x, y, rows, cols);
        else if (ncv <= 128) launch_wave<T, LOG, 2>(x, y, rows, cols);
        else if (ncv <= 256) launch_wave<T, LOG, 4>(x, y, rows, cols);
        else if (ncv <= 512) launch_wave<T, LOG, 8>(x, y, rows, cols);
        else launch_wave<T, LOG, 16>(x, y, rows, cols);
    } else {
        for_row_launches(rows, 1, [&](unsigned g, int64_t base) {
            NH_LAUNCH((k_softmax_block<T, LOG>), dim3(g), dim3(kSmBlock), 0, stream(), x, y, cols, base);
        });
    }
    return check_launch();
}

static int softmax_api(NeuralTensor *out, const NeuralTensor *in, bool log)
{
    NH_TRY(ensure_init());
    if (!out || !in) return set_error(NEURAL_ERR_NULL_POINTER);
    NH_TRY(check_tensor(in));
    NH_TRY(check_tensor(out));
    if (in->dtype != out->dtype) return set_error(NEURAL_ERR_DTYPE_MISMATCH);
    if (in->ndim < 1) return set_error(NEURAL_ERR_DIM_MISMATCH);
    const int64_t n = numel(in);
    if (numel(out) != n) return set_error(NEURAL_ERR_SHAPE_MISMATCH);
    if (!is_contiguous(in) || !is_contiguous(out)) return set_error(NEURAL_ERR_INVALID_ARGUMENT);
    const int64_t cols = in->shape[in->ndim - 1];
    if (n == 0 || cols == 0) return set_error(NEURAL_OK);
    const int64_t rows = n / cols;
    const void *src = nullptr;
    void *dst = nullptr;
    NH_TRY(dev_read(in, &src));
    NH_TRY(dev_write(out, &dst, true));
    if (in->dtype == NEURAL_DTYPE_FLOAT32) {
        if (log) NH_TRY((launch_softmax<float, true>(static_cast<const float *>(src), static_cast<float *>(dst), rows, cols)));
        else NH_TRY((launch_softmax<float, false>(static_cast<const float *>(src), static_cast<float *>(dst), rows, cols)));
    } else {
        if (log) NH_TRY((launch_softmax<double, true>(static_cast<const double *>(src), static_cast<double *>(dst), rows, cols)));
        else NH_TRY((launch_softmax<double, false>(static_cast<const double *>(src), static_cast<double *>(dst), rows, cols)));
    }
    NH_TRY(dev_written(out));
    return set_error(NEURAL_OK);
}

}  // namespace nh

extern "C" {

// neural_softmax (neural_api.asm:1340-1396): rows over the last dimension
// (the reference handles 2-D [batch, classes] only).
int neural_softmax(NeuralTensor *out, const NeuralTensor *in) { return nh::softmax_api(out, in, false); }

int neural_log_softmax(NeuralTensor *out, const NeuralTensor *in) { return nh::softmax_api(out, in, true); }

}  // extern "C"
