// tensor_ops.hip -- 2-D float64 concat / split / pad / transpose.
//
// Reference: tensor_ops.c:15-148 (same argument checks, -1 on invalid input,
// output extents through the pointer arguments).  Buffers may be host or
// device pointers; host buffers are staged through HBM.  Concat/split along
// rows are contiguous block copies; the column variants, pad and transpose
// are copy kernels (transpose through a padded 32x32 LDS tile so both the
// read and the write are coalesced).
#include "common.hpp"

namespace nh {

constexpr int kTile = 32;

__global__ __launch_bounds__(256) void k_concat_cols(const double *a, const double *b, double *o, int64_t rows,
                                                     int64_t ca, int64_t cb)
{
    const int64_t C = ca + cb;
    const int64_t n = rows * C;
    const int64_t stride = int64_t(gridDim.x) * 256;
    for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < n; i += stride) {
        const int64_t r = i / C, c = i % C;
        o[i] = c < ca ? a[r * ca + c] : b[r * cb + (c - ca)];
    }
}

__global__ __launch_bounds__(256) void k_split_cols(const double *in, double *oa, double *ob, int64_t rows,
                                                    int64_t cols, int64_t split)
{
    const int64_t n = rows * cols;
    const int64_t cb = cols - split;
    const int64_t stride = int64_t(gridDim.x) * 256;
    for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < n; i += stride) {
        const int64_t r = i / cols, c = i % cols;
        if (c < split) oa[r * split + c] = in[i];
        else ob[r * cb + (c - split)] = in[i];
    }
}

__global__ __launch_bounds__(256) void k_pad(const double *in, double *o, int64_t rows, int64_t cols, int64_t pt,
                                             int64_t pl, int64_t R, int64_t C, double value)
{
    const int64_t n = R * C;
    const int64_t stride = int64_t(gridDim.x) * 256;
    for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < n; i += stride) {
        const int64_t r = i / C - pt, c = i % C - pl;
        o[i] = (r >= 0 && r < rows && c >= 0 && c < cols) ? in[r * cols + c] : value;
    }
}

// out[c, r] = in[r, c]; block (32 x 8) moves 32x32 tiles, stepping through
// the tile grid by the launch grid (capped in both dimensions).
__global__ __launch_bounds__(256) void k_transpose(const double *in, double *o, int64_t rows, int64_t cols)
{
    __shared__ double tile[kTile][kTile + 1];
    const int tx = threadIdx.x % kTile, ty = threadIdx.x / kTile;
    const int64_t tcols = (cols + kTile - 1) / kTile, trows = (rows + kTile - 1) / kTile;
    for (int64_t by = blockIdx.y; by < trows; by += gridDim.y) {
        for (int64_t bx = blockIdx.x; bx < tcols; bx += gridDim.x) {
            const int64_t c0 = bx * kTile, r0 = by * kTile;
            for (int k = ty; k < kTile; k += 8) {
                const int64_t r = r0 + k, c = c0 + tx;
                if (r < rows && c < cols) tile[k][tx] = in[r * cols + c];
            }
            __syncthreads();
            for (int k = ty; k < kTile; k += 8) {
                const int64_t c = c0 + k, r = r0 + tx;
                if (c < cols && r < rows) o[c * rows + r] = tile[tx][k];
            }
            __syncthreads();  // the tile is rewritten by the next step
        }
    }
}

inline unsigned t_grid(int64_t n)
{
    int64_t g = ceil_div(n, 256);
    const int64_t cap = kMaxGridBlocks;
    if (g > cap) g = cap;
    return unsigned(g < 1 ? 1 : g);
}

}  // namespace nh

using namespace nh;

// a * b as an element count the raw-pointer paths can stage (no wrap).
static bool count_of(int64_t a, int64_t b, int64_t *out)
{
    return !__builtin_mul_overflow(a, b, out) && uint64_t(*out) <= kMaxRawCount;
}

extern "C" {

int tensor_concat_2d(const double *a, const double *b, int64_t rows_a, int64_t cols_a, int64_t rows_b,
                     int64_t cols_b, int64_t axis, double *out, int64_t *out_rows, int64_t *out_cols)
{
    if (!a || !b || !out || !out_rows || !out_cols) return -1;
    if (rows_a <= 0 || cols_a <= 0 || rows_b <= 0 || cols_b <= 0) return -1;
    if (axis != 0 && axis != 1) return -1;
    if (axis == 0 && cols_a != cols_b) return -1;
    if (axis == 1 && rows_a != rows_b) return -1;
    if (ensure_init() != NEURAL_OK) return -1;
    int64_t na, nb;
    if (!count_of(rows_a, cols_a, &na) || !count_of(rows_b, cols_b, &nb)) return -1;
    Staged sa, sb, so;
    if (sa.open(a, size_t(na) * 8, true) || sb.open(b, size_t(nb) * 8, true) || so.open(out, size_t(na + nb) * 8, false))
        return -1;
    double *O = static_cast<double *>(so.dev);
    if (axis == 0) {
        if (hipMemcpyAsync(O, sa.dev, size_t(na) * 8, hipMemcpyDeviceToDevice, stream()) != hipSuccess ||
            hipMemcpyAsync(O + na, sb.dev, size_t(nb) * 8, hipMemcpyDeviceToDevice, stream()) != hipSuccess)
            return -1;
        *out_rows = rows_a + rows_b;
        *out_cols = cols_a;
    } else {
        NH_LAUNCH(k_concat_cols, dim3(t_grid(na + nb)), dim3(256), 0, stream(),
                           static_cast<const double *>(sa.dev), static_cast<const double *>(sb.dev), O, rows_a,
                           cols_a, cols_b);
        if (check_launch() != NEURAL_OK) return -1;
        *out_rows = rows_a;
        *out_cols = cols_a + cols_b;
    }
    if (so.finish(true) || sa.finish(false) || sb.finish(false)) return -1;
    return 0;
}

int tensor_split_2d(const double *in, int64_t rows, int64_t cols, int64_t axis, int64_t split_index, double *out_a,
                    double *out_b, int64_t *rows_a, int64_t *cols_a, int64_t *rows_b, int64_t *cols_b)
{
    if (!in || !out_a || !out_b || !rows_a || !cols_a || !rows_b || !cols_b) return -1;
    if (rows <= 0 || cols <= 0) return -1;
    if (axis != 0 && axis != 1) return -1;
    const int64_t lim = axis == 0 ? rows : cols;
    if (split_index <= 0 || split_index >= lim) return -1;
    if (ensure_init() != NEURAL_OK) return -1;
    int64_t n;
    if (!count_of(rows, cols, &n)) return -1;
    const int64_t na = axis == 0 ? split_index * cols : rows * split_index;
    const int64_t nb = n - na;
    Staged si, sa, sb;
    if (si.open(in, size_t(n) * 8, true) || sa.open(out_a, size_t(na) * 8, false) || sb.open(out_b, size_t(nb) * 8, false))
        return -1;
    const double *I = static_cast<const double *>(si.dev);
    if (axis == 0) {
        if (hipMemcpyAsync(sa.dev, I, size_t(na) * 8, hipMemcpyDeviceToDevice, stream()) != hipSuccess ||
            hipMemcpyAsync(sb.dev, I + na, size_t(nb) * 8, hipMemcpyDeviceToDevice, stream()) != hipSuccess)
            return -1;
        *rows_a = split_index; *cols_a = cols; *rows_b = rows - split_index; *cols_b = cols;
    } else {
        NH_LAUNCH(k_split_cols, dim3(t_grid(n)), dim3(256), 0, stream(), I, static_cast<double *>(sa.dev),
                           static_cast<double *>(sb.dev), rows, cols, split_index);
        if (check_launch() != NEURAL_OK) return -1;
        *rows_a = rows; *cols_a = split_index; *rows_b = rows; *cols_b = cols - split_index;
    }
    if (sa.finish(true) || sb.finish(true) || si.finish(false)) return -1;
    return 0;
}

int tensor_pad_2d(const double *in, int64_t in_rows, int64_t in_cols, int64_t pad_top, int64_t pad_bottom,
                  int64_t pad_left, int64_t pad_right, double pad_value, double *out, int64_t *out_rows,
                  int64_t *out_cols)
{
    if (!in || !out || !out_rows || !out_cols) return -1;
    if (in_rows <= 0 || in_cols <= 0) return -1;
    if (pad_top < 0 || pad_bottom < 0 || pad_left < 0 || pad_right < 0) return -1;
    if (ensure_init() != NEURAL_OK) return -1;
    int64_t R, C, nin, nout;
    if (__builtin_add_overflow(in_rows, pad_top, &R) || __builtin_add_overflow(R, pad_bottom, &R) ||
        __builtin_add_overflow(in_cols, pad_left, &C) || __builtin_add_overflow(C, pad_right, &C) ||
        !count_of(in_rows, in_cols, &nin) || !count_of(R, C, &nout))
        return -1;
    Staged si, so;
    if (si.open(in, size_t(nin) * 8, true) || so.open(out, size_t(nout) * 8, false)) return -1;
    NH_LAUNCH(k_pad, dim3(t_grid(R * C)), dim3(256), 0, stream(), static_cast<const double *>(si.dev),
                       static_cast<double *>(so.dev), in_rows, in_cols, pad_top, pad_left, R, C, pad_value);
    if (check_launch() != NEURAL_OK) return -1;
    *out_rows = R;
    *out_cols = C;
    if (so.finish(true) || si.finish(false)) return -1;
    return 0;
}

int tensor_transpose2d_array(const double *in, int64_t rows, int64_t cols, double *out)
{
    if (!in || !out) return -1;
    if (rows <= 0 || cols <= 0) return -1;
    if (ensure_init() != NEURAL_OK) return -1;
    int64_t n;
    if (!count_of(rows, cols, &n)) return -1;
    const size_t bytes = size_t(n) * 8;
    Staged si, so;
    if (si.open(in, bytes, true) || so.open(out, bytes, false)) return -1;
    int64_t gx = ceil_div(cols, kTile), gy = ceil_div(rows, kTile);
    if (gx > 65535) gx = 65535;
    if (gy > 65535) gy = 65535;
    NH_LAUNCH(k_transpose, dim3(unsigned(gx), unsigned(gy)), dim3(256), 0, stream(),
                       static_cast<const double *>(si.dev), static_cast<double *>(so.dev), rows, cols);
    if (check_launch() != NEURAL_OK) return -1;
    if (so.finish(true) || si.finish(false)) return -1;
    return 0;
}

}  // extern "C"
