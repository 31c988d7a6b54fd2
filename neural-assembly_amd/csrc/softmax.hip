// softmax.hip -- row softmax and log-softmax over the last dimension.
//
// Softmax follows node_softmax (activations.asm:761-987) with its intended
// f32 semantics (the asm keeps the max and the running sum in one stack slot,
// activations.asm:900,927-929):
//   f32: m = row max; e_j = (float)exp((double)x_j - (double)m);
//        s = sum of e_j; y_j = e_j / (float)s  (float division)
//   f64: e_j = exp(x_j - m); y_j = e_j / s
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

#include "common.hpp"

namespace nh {

constexpr int kSmBlock = 256;

template <typename T>
NH_DEV T neg_inf();
template <> NH_DEV float neg_inf<float>() { return -__builtin_inff(); }
template <> NH_DEV double neg_inf<double>() { return -__builtin_inf(); }

template <typename T, bool LOG, int VPL>
__global__ __launch_bounds__(kSmBlock) void k_softmax_wave(const T *__restrict__ x, T *__restrict__ y, int64_t rows,
                                                           int64_t cols)
{
    using V = typename Vec16<T>::type;
    constexpr int VN = Vec16<T>::n;
    const int lane = threadIdx.x & 63;
    const int64_t r = int64_t(blockIdx.x) * (kSmBlock / 64) + (threadIdx.x >> 6);
    if (r >= rows) return;  // uniform per wave
    const V *xr = reinterpret_cast<const V *>(x + r * cols);
    V *yr = reinterpret_cast<V *>(y + r * cols);
    const int64_t ncv = cols / VN;

    V v[VPL];
#pragma unroll
    for (int k = 0; k < VPL; k++) {
        const int64_t c = lane + int64_t(k) * 64;
        if (c < ncv) v[k] = xr[c];
    }
    T m = neg_inf<T>();
#pragma unroll
    for (int k = 0; k < VPL; k++) {
        const int64_t c = lane + int64_t(k) * 64;
        if (c < ncv) {
#pragma unroll
            for (int j = 0; j < VN; j++) {
                const T e = vget(v[k], j);
                m = e > m ? e : m;
            }
        }
    }
    m = wave_max_ignore_nan(m);
    const double md = double(m);

    double s = 0.0;
    if (!LOG) {
        // Keep e_j (rounded to T) in the input registers.
#pragma unroll
        for (int k = 0; k < VPL; k++) {
            const int64_t c = lane + int64_t(k) * 64;
            if (c < ncv) {
#pragma unroll
                for (int j = 0; j < VN; j++) {
                    const T e = T(exp(double(vget(v[k], j)) - md));
                    vset(v[k], j, e);
                    s += double(e);
                }
            }
        }
        s = wave_sum(s);
        const T st = T(s);
#pragma unroll
        for (int k = 0; k < VPL; k++) {
            const int64_t c = lane + int64_t(k) * 64;
            if (c < ncv) {
                V o;
#pragma unroll
                for (int j = 0; j < VN; j++) vset(o, j, vget(v[k], j) / st);
                yr[c] = o;
            }
        }
    } else {
#pragma unroll
        for (int k = 0; k < VPL; k++) {
            const int64_t c = lane + int64_t(k) * 64;
            if (c < ncv) {
#pragma unroll
                for (int j = 0; j < VN; j++) s += exp(double(vget(v[k], j)) - md);
            }
        }
        s = wave_sum(s);
        const double lse = log(s);
#pragma unroll
        for (int k = 0; k < VPL; k++) {
            const int64_t c = lane + int64_t(k) * 64;
            if (c < ncv) {
                V o;
#pragma unroll
                for (int j = 0; j < VN; j++) vset(o, j, T((double(vget(v[k], j)) - md) - lse));
                yr[c] = o;
            }
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

template <typename T, bool LOG>
__global__ __launch_bounds__(kSmBlock) void k_softmax_block(const T *__restrict__ x, T *__restrict__ y, int64_t cols)
{
    const int64_t r = blockIdx.x;
    const T *xr = x + r * cols;
    T *yr = y + r * cols;
    T m = neg_inf<T>();
    for (int64_t j = threadIdx.x; j < cols; j += kSmBlock) m = xr[j] > m ? xr[j] : m;
    m = block_max_ignore_nan(m);
    const double md = double(m);
    double s = 0.0;
    for (int64_t j = threadIdx.x; j < cols; j += kSmBlock) {
        if (LOG) s += exp(double(xr[j]) - md);
        else s += double(T(exp(double(xr[j]) - md)));
    }
    s = block_sum(s);
    if (LOG) {
        const double lse = log(s);
        for (int64_t j = threadIdx.x; j < cols; j += kSmBlock) yr[j] = T((double(xr[j]) - md) - lse);
    } else {
        const T st = T(s);
        for (int64_t j = threadIdx.x; j < cols; j += kSmBlock) yr[j] = T(exp(double(xr[j]) - md)) / st;
    }
}

template <typename T, bool LOG>
static int launch_softmax(const T *x, T *y, int64_t rows, int64_t cols)
{
    constexpr int VN = Vec16<T>::n;
    const bool vec = ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y)) & 15u) == 0 && cols % VN == 0;
    const int64_t ncv = cols / VN;
    const unsigned g = unsigned(ceil_div(rows, kSmBlock / 64));
    if (vec && ncv <= 64 * 16) {
        if (ncv <= 64) hipLaunchKernelGGL((k_softmax_wave<T, LOG, 1>), dim3(g), dim3(kSmBlock), 0, stream(), x, y, rows, cols);
        else if (ncv <= 128) hipLaunchKernelGGL((k_softmax_wave<T, LOG, 2>), dim3(g), dim3(kSmBlock), 0, stream(), x, y, rows, cols);
        else if (ncv <= 256) hipLaunchKernelGGL((k_softmax_wave<T, LOG, 4>), dim3(g), dim3(kSmBlock), 0, stream(), x, y, rows, cols);
        else if (ncv <= 512) hipLaunchKernelGGL((k_softmax_wave<T, LOG, 8>), dim3(g), dim3(kSmBlock), 0, stream(), x, y, rows, cols);
        else hipLaunchKernelGGL((k_softmax_wave<T, LOG, 16>), dim3(g), dim3(kSmBlock), 0, stream(), x, y, rows, cols);
    } else {
        hipLaunchKernelGGL((k_softmax_block<T, LOG>), dim3(unsigned(rows)), dim3(kSmBlock), 0, stream(), x, y, cols);
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
