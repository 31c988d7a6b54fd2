// reduce.hip -- sum / mean / max / argmax over whole tensors, rows and columns.
//
// Reference semantics (math_kernels.asm:956-1264, activations.asm:888-895,
// main.asm:3245-3292,3598-3640):
//   sum      accumulated here in double (the reference's fp32 lane orders are
//            order-dependent; results are compared against the fp64-exact sum)
//   max      the running-max chain m = (m > x) ? m : x: equal values resolve to
//            the later element, and a NaN restarts the chain at the next
//            element.  Closed form: max over the elements after the last NaN
//            (later element on ties); NaN if the last element is NaN.
//   argmax   idx = 0, m = x0, update iff x_j > m: first index of the largest
//            non-NaN value, or 0 if x0 is NaN.
#include "kernels.hpp"
#include "reduce_impl.hpp"

namespace nh {

// ---- reducers -------------------------------------------------------------------

struct RedSum {
    struct S { double s; };
    static constexpr bool kSuffixPass = false;
    NH_DEV S init() const { return {0.0}; }
    NH_DEV void acc(S &st, double v, int64_t) const { st.s += v; }
    NH_DEV S comb(S a, S b) const { return {a.s + b.s}; }
    NH_DEV S shfl(S a, int off) const { return {__shfl_xor(a.s, off, 64)}; }
    NH_DEV void store(void *out, S st) const { *static_cast<double *>(out) = st.s; }
};

// Sum / mean written in the tensor's dtype (one rounding of the double
// result); `div` is the element count for a mean, 1 for a sum.
template <typename T>
struct RedRowSum : RedSum {
    int64_t div;
    NH_DEV void store_row(void *out, int64_t r, S st) const
    {
        const double v = div > 1 ? st.s / double(div) : st.s;
        static_cast<T *>(out)[r] = T(v);
    }
    NH_DEV void store(void *out, S st) const { store_row(out, 0, st); }
    NH_DEV void store_row_x(void *out, int64_t r, S st, const T *, int64_t) const { store_row(out, r, st); }
};

// Running-max chain m = (m > x) ? m : x as a reduction.  The chain's result
// is the largest value after the last NaN (NaN if the last element is NaN);
// equal values only differ in the sign of zero, where the chain keeps the
// later element.  State: largest non-NaN value, last NaN index, last zero
// index.  Every lane walks its elements in increasing index order, so "last"
// is a plain overwrite per lane and a max across lanes.  The element behind a
// zero result is re-read to get its sign.
struct RedMax {
    struct S { double v; int64_t nan_i; int64_t zero_i; };
    static constexpr bool kSuffixPass = true;
    const void *x;   // the reduced array (element 0), to read back a zero's sign
    int f64;         // element type of x
    NH_DEV S init() const { return {-__builtin_inf(), -1, -1}; }
    NH_DEV void acc(S &st, double v, int64_t i) const
    {
        st.nan_i = (v != v) ? i : st.nan_i;
        st.zero_i = (v == 0.0) ? i : st.zero_i;
        st.v = __builtin_fmax(st.v, v);
    }
    NH_DEV S comb(S a, S b) const
    {
        return {__builtin_fmax(a.v, b.v), a.nan_i > b.nan_i ? a.nan_i : b.nan_i,
                a.zero_i > b.zero_i ? a.zero_i : b.zero_i};
    }
    NH_DEV S shfl(S a, int off) const
    {
        return {__shfl_xor(a.v, off, 64), __shfl_xor(a.nan_i, off, 64), __shfl_xor(a.zero_i, off, 64)};
    }
    NH_DEV int64_t suffix_start(S st) const { return st.nan_i; }
    // Second pass over (L, cols) of the same row (no NaN there by
    // definition).  A row that ends with NaN has an empty suffix: its chain
    // value is NaN, marked by nan_i = kEndsWithNaN.
    static constexpr int64_t kEndsWithNaN = -3;
    NH_DEV S suffix_result(S first, S second, int64_t cols) const
    {
        if (first.nan_i == cols - 1) return {0.0, kEndsWithNaN, -1};
        S r = second;
        r.nan_i = -1;
        return r;
    }
    // Value of the chain given a first-pass state over x[0..n) (row base xr).
    NH_DEV double finish(S st, const void *xr) const
    {
        double v = st.v;
        if (v == 0.0 && st.zero_i >= 0)
            v = f64 ? static_cast<const double *>(xr)[st.zero_i] : double(static_cast<const float *>(xr)[st.zero_i]);
        return v;
    }
    NH_DEV void store(void *out, S st) const { *static_cast<S *>(out) = st; }
};

template <typename T>
struct RedRowMax : RedMax {
    NH_DEV void store_row_x(void *out, int64_t r, S st, const T *xr, int64_t cols) const
    {
        const double v = st.nan_i == kEndsWithNaN ? __longlong_as_double(0x7ff8000000000000ll) : finish(st, xr);
        static_cast<T *>(out)[r] = T(v);
    }
};

// Argmax: idx = 0, m = x0, update iff x_j > m.  Reduction state: largest
// non-NaN value and its first index (-1 while none beats -inf); x0 NaN, or no
// element above -inf, gives 0 (read from x in the epilogue).
struct RedArgmax {
    struct S { double v; int64_t i; };
    static constexpr bool kSuffixPass = false;
    NH_DEV S init() const { return {-__builtin_inf(), -1}; }
    NH_DEV void acc(S &st, double v, int64_t i) const
    {
        const bool up = v > st.v;
        st.v = up ? v : st.v;
        st.i = up ? i : st.i;
    }
    NH_DEV S comb(S a, S b) const
    {
        if (b.v > a.v || (b.v == a.v && b.i >= 0 && (a.i < 0 || b.i < a.i))) return b;
        return a;
    }
    NH_DEV S shfl(S a, int off) const { return {__shfl_xor(a.v, off, 64), __shfl_xor(a.i, off, 64)}; }
    template <typename T>
    NH_DEV static int64_t result(S st, const T *x0)
    {
        const T first = x0[0];
        return (first != first || st.i < 0) ? 0 : st.i;
    }
};

template <typename T>
struct RedRowArgmax : RedArgmax {
    NH_DEV void store_row_x(void *out, int64_t r, S st, const T *xr, int64_t) const
    {
        static_cast<int64_t *>(out)[r] = result(st, xr);
    }
};

template <typename T>
struct RedFullArgmax : RedArgmax {
    const T *x;
    NH_DEV void store(void *out, S st) const { *static_cast<int64_t *>(out) = result(st, x); }
};

// ---- column sums (reduce_sum axis=0) -------------------------------------------------
// Stage 1: grid (column groups of 256, row chunks) writes double partials
// [chunks][cols]; stage 2 adds the chunks in order per column.

__global__ __launch_bounds__(256) void k_colsum_stage1_f32(const float *x, int64_t rows, int64_t cols,
                                                           int64_t chunk, double *part)
{
    const int64_t c = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (c >= cols) return;
    const int64_t r0 = int64_t(blockIdx.y) * chunk;
    int64_t r1 = r0 + chunk;
    if (r1 > rows) r1 = rows;
    double s = 0.0;
    for (int64_t r = r0; r < r1; r++) s += double(x[r * cols + c]);
    part[int64_t(blockIdx.y) * cols + c] = s;
}

__global__ __launch_bounds__(256) void k_colsum_stage1_f64(const double *x, int64_t rows, int64_t cols,
                                                           int64_t chunk, double *part)
{
    const int64_t c = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (c >= cols) return;
    const int64_t r0 = int64_t(blockIdx.y) * chunk;
    int64_t r1 = r0 + chunk;
    if (r1 > rows) r1 = rows;
    double s = 0.0;
    for (int64_t r = r0; r < r1; r++) s += x[r * cols + c];
    part[int64_t(blockIdx.y) * cols + c] = s;
}

template <typename T>
__global__ __launch_bounds__(256) void k_colsum_stage2(const double *part, int64_t nchunks, int64_t cols,
                                                       int64_t div, T *out)
{
    const int64_t c = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (c >= cols) return;
    double s = 0.0;
    for (int64_t k = 0; k < nchunks; k++) s += part[k * cols + c];
    out[c] = T(div > 1 ? s / double(div) : s);
}

static int colsum(const NeuralTensor *in, const void *src, int64_t rows, int64_t cols, bool mean, void *dst)
{
    if (cols <= 0) return NEURAL_OK;
    // ~4 row chunks per CU-worth of column groups, at least 64 rows per chunk.
    const int64_t cgroups = ceil_div(cols, 256);
    int64_t nchunks = ceil_div(int64_t(num_cus()) * 4, cgroups);
    if (nchunks > ceil_div(rows, 64)) nchunks = ceil_div(rows, 64);
    if (nchunks < 1) nchunks = 1;
    if (nchunks > 65535) nchunks = 65535;
    const int64_t chunk = ceil_div(rows > 0 ? rows : 1, nchunks);
    double *part = static_cast<double *>(dev_alloc(size_t(nchunks * cols) * sizeof(double)));
    if (!part) return set_error(NEURAL_ERR_OUT_OF_MEMORY);
    const dim3 g1{unsigned(cgroups), unsigned(nchunks), 1u};
    if (in->dtype == NEURAL_DTYPE_FLOAT32)
        hipLaunchKernelGGL(k_colsum_stage1_f32, g1, dim3(256), 0, stream(), static_cast<const float *>(src), rows,
                           cols, chunk, part);
    else
        hipLaunchKernelGGL(k_colsum_stage1_f64, g1, dim3(256), 0, stream(), static_cast<const double *>(src), rows,
                           cols, chunk, part);
    const int64_t div = mean ? rows : 1;
    if (in->dtype == NEURAL_DTYPE_FLOAT32)
        hipLaunchKernelGGL((k_colsum_stage2<float>), dim3(unsigned(cgroups)), dim3(256), 0, stream(), part, nchunks,
                           cols, div, static_cast<float *>(dst));
    else
        hipLaunchKernelGGL((k_colsum_stage2<double>), dim3(unsigned(cgroups)), dim3(256), 0, stream(), part,
                           nchunks, cols, div, static_cast<double *>(dst));
    const int rc = check_launch();
    dev_free(part);
    return rc;
}

// ---- helpers ----------------------------------------------------------------------------

// Device copy of a (possibly strided) tensor in logical order, or the tensor's
// own buffer when it is contiguous.
struct Contig {
    const void *p = nullptr;
    void *tmp = nullptr;
    int open(const NeuralTensor *t)
    {
        NH_TRY(dev_read(t, &p));
        if (is_contiguous(t)) return NEURAL_OK;
        const int64_t n = numel(t);
        const int es = int(elem_size(t->dtype));
        tmp = dev_alloc(size_t(n) * size_t(es));
        if (!tmp) return set_error(NEURAL_ERR_OUT_OF_MEMORY);
        const int64_t one = n;
        const int64_t st = es;
        NH_TRY(launch_copy_nd(tmp, &one, &st, 1, p, t->shape, t->stride, int(t->ndim), es));
        p = tmp;
        return NEURAL_OK;
    }
    ~Contig() { if (tmp) dev_free(tmp); }
};

template <class Red, typename Out>
static int full_reduce(const NeuralTensor *t, const Red &red, Out *host_out)
{
    const int64_t n = numel(t);
    Contig c;
    NH_TRY(c.open(t));
    void *res = workspace().result;
    if (t->dtype == NEURAL_DTYPE_FLOAT32) NH_TRY(launch_reduce_full(static_cast<const float *>(c.p), n, red, res));
    else NH_TRY(launch_reduce_full(static_cast<const double *>(c.p), n, red, res));
    NH_HIP(hipMemcpyAsync(host_out, res, sizeof(Out), hipMemcpyDeviceToHost, stream()));
    NH_TRY(sync());
    return NEURAL_OK;
}

// Running-max over a whole tensor: the first pass finds the largest value,
// the last NaN and the last zero; if a NaN was seen a second pass runs on the
// suffix after it (the chain restarts there).
static int full_max(const NeuralTensor *t, double *result)
{
    const int64_t n = numel(t);
    Contig c;
    NH_TRY(c.open(t));
    const bool f64 = t->dtype == NEURAL_DTYPE_FLOAT64;
    const size_t es = elem_size(t->dtype);
    void *res = workspace().result;
    int64_t base = 0;
    for (int pass = 0; pass < 2; pass++) {
        const void *sp = static_cast<const char *>(c.p) + size_t(base) * es;
        RedMax red;
        red.x = sp;
        red.f64 = f64 ? 1 : 0;
        const int64_t m = n - base;
        if (f64) NH_TRY(launch_reduce_full(static_cast<const double *>(sp), m, red, res));
        else NH_TRY(launch_reduce_full(static_cast<const float *>(sp), m, red, res));
        RedMax::S st;
        NH_HIP(hipMemcpyAsync(&st, res, sizeof(st), hipMemcpyDeviceToHost, stream()));
        NH_TRY(sync());
        if (st.nan_i < 0) {
            double v = st.v;
            if (v == 0.0 && st.zero_i >= 0) {
                // the sign of the zero the chain keeps (the last one)
                const char *p = static_cast<const char *>(sp) + size_t(st.zero_i) * es;
                if (f64) NH_HIP(hipMemcpyAsync(&v, p, 8, hipMemcpyDeviceToHost, stream()));
                else {
                    float f;
                    NH_HIP(hipMemcpyAsync(&f, p, 4, hipMemcpyDeviceToHost, stream()));
                    NH_TRY(sync());
                    v = f;
                }
                NH_TRY(sync());
            }
            *result = v;
            return NEURAL_OK;
        }
        base += st.nan_i + 1;
        if (base >= n) {
            *result = __builtin_nan("");
            return NEURAL_OK;
        }
    }
    return set_error(NEURAL_ERR_INTERNAL);  // unreachable: the suffix holds no NaN
}

// Resolve (rows, cols) for a reduction over `axis` of `in`:
//   kind 0 = all elements, 1 = last dim (rows x cols), 2 = columns of 2-D.
static int resolve_axis(const NeuralTensor *in, int64_t axis, int &kind, int64_t &rows, int64_t &cols)
{
    const int64_t nd = in->ndim;
    if (axis < -1) return set_error(NEURAL_ERR_DIM_MISMATCH);
    if (axis == -1 || nd == 0) { kind = 0; rows = 1; cols = numel(in); return NEURAL_OK; }
    if (nd == 2 && axis == 0) { kind = 2; rows = in->shape[0]; cols = in->shape[1]; return NEURAL_OK; }
    if (axis == nd - 1) {
        kind = 1;
        cols = in->shape[nd - 1];
        rows = cols > 0 ? numel(in) / cols : 0;
        return NEURAL_OK;
    }
    // Other axes: the reference falls back to the full sum (math_kernels.asm:979-991).
    kind = 0; rows = 1; cols = numel(in);
    return NEURAL_OK;
}

static int reduce_sum_mean(const NeuralTensor *in, int64_t axis, NeuralTensor *out, bool mean)
{
    NH_TRY(ensure_init());
    if (!in || !out) return set_error(NEURAL_ERR_NULL_POINTER);
    NH_TRY(check_tensor(in));
    NH_TRY(check_tensor(out));
    if (in->dtype != out->dtype) return set_error(NEURAL_ERR_DTYPE_MISMATCH);
    int kind;
    int64_t rows, cols;
    NH_TRY(resolve_axis(in, axis, kind, rows, cols));
    const int64_t nout = kind == 0 ? 1 : (kind == 1 ? rows : cols);
    if (numel(out) != nout || !is_contiguous(out)) return set_error(NEURAL_ERR_SHAPE_MISMATCH);
    if (numel(in) == 0) return neural_tensor_fill(out, 0.0);
    Contig c;
    NH_TRY(c.open(in));
    void *dst = nullptr;
    NH_TRY(dev_write(out, &dst, true));
    if (kind == 0) {
        // Whole tensor: full-grid reduction storing straight into out[0].
        if (in->dtype == NEURAL_DTYPE_FLOAT32) {
            RedRowSum<float> red;
            red.div = mean ? cols : 1;
            NH_TRY(launch_reduce_full(static_cast<const float *>(c.p), cols, red, dst));
        } else {
            RedRowSum<double> red;
            red.div = mean ? cols : 1;
            NH_TRY(launch_reduce_full(static_cast<const double *>(c.p), cols, red, dst));
        }
    } else if (kind == 1) {
        if (in->dtype == NEURAL_DTYPE_FLOAT32) {
            RedRowSum<float> red;
            red.div = mean ? cols : 1;
            NH_TRY(launch_reduce_rows(static_cast<const float *>(c.p), rows, cols, red, dst));
        } else {
            RedRowSum<double> red;
            red.div = mean ? cols : 1;
            NH_TRY(launch_reduce_rows(static_cast<const double *>(c.p), rows, cols, red, dst));
        }
    } else {
        NH_TRY(colsum(in, c.p, rows, cols, mean, dst));
    }
    NH_TRY(dev_written(out));
    return set_error(NEURAL_OK);
}

}  // namespace nh

using namespace nh;

extern "C" {

int neural_sum(const NeuralTensor *t, double *result)
{
    NH_TRY(ensure_init());
    if (!t || !result) return set_error(NEURAL_ERR_NULL_POINTER);
    NH_TRY(check_tensor(t));
    if (numel(t) == 0) { *result = 0.0; return set_error(NEURAL_OK); }
    NH_TRY(full_reduce(t, RedSum{}, result));
    return set_error(NEURAL_OK);
}

int neural_mean(const NeuralTensor *t, double *result)
{
    NH_TRY(ensure_init());
    if (!t || !result) return set_error(NEURAL_ERR_NULL_POINTER);
    NH_TRY(check_tensor(t));
    const int64_t n = numel(t);
    if (n == 0) return set_error(NEURAL_ERR_INVALID_ARGUMENT);
    double s = 0.0;
    NH_TRY(full_reduce(t, RedSum{}, &s));
    *result = s / double(n);
    return set_error(NEURAL_OK);
}

int neural_max(const NeuralTensor *t, double *result)
{
    NH_TRY(ensure_init());
    if (!t || !result) return set_error(NEURAL_ERR_NULL_POINTER);
    NH_TRY(check_tensor(t));
    if (numel(t) == 0) return set_error(NEURAL_ERR_INVALID_ARGUMENT);
    NH_TRY(full_max(t, result));
    return set_error(NEURAL_OK);
}

int neural_argmax(const NeuralTensor *t, int64_t *result)
{
    NH_TRY(ensure_init());
    if (!t || !result) return set_error(NEURAL_ERR_NULL_POINTER);
    NH_TRY(check_tensor(t));
    if (numel(t) == 0) return set_error(NEURAL_ERR_INVALID_ARGUMENT);
    const void *p = nullptr;
    NH_TRY(dev_read(t, &p));
    if (t->dtype == NEURAL_DTYPE_FLOAT32) {
        RedFullArgmax<float> red;
        red.x = static_cast<const float *>(p);
        NH_TRY(full_reduce(t, red, result));
    } else {
        RedFullArgmax<double> red;
        red.x = static_cast<const double *>(p);
        NH_TRY(full_reduce(t, red, result));
    }
    return set_error(NEURAL_OK);
}

int neural_reduce_sum(const NeuralTensor *in, int64_t axis, NeuralTensor *out)
{
    return reduce_sum_mean(in, axis, out, false);
}

int neural_reduce_mean(const NeuralTensor *in, int64_t axis, NeuralTensor *out)
{
    return reduce_sum_mean(in, axis, out, true);
}

int neural_reduce_max(const NeuralTensor *in, int64_t axis, NeuralTensor *out)
{
    NH_TRY(ensure_init());
    if (!in || !out) return set_error(NEURAL_ERR_NULL_POINTER);
    NH_TRY(check_tensor(in));
    NH_TRY(check_tensor(out));
    if (in->dtype != out->dtype) return set_error(NEURAL_ERR_DTYPE_MISMATCH);
    if (in->ndim < 1 || (axis != -1 && axis != in->ndim - 1)) return set_error(NEURAL_ERR_DIM_MISMATCH);
    const int64_t cols = in->shape[in->ndim - 1];
    if (cols <= 0) return set_error(NEURAL_ERR_INVALID_ARGUMENT);
    const int64_t rows = numel(in) / cols;
    if (numel(out) != rows || !is_contiguous(out)) return set_error(NEURAL_ERR_SHAPE_MISMATCH);
    if (rows == 0) return set_error(NEURAL_OK);
    Contig c;
    NH_TRY(c.open(in));
    void *dst = nullptr;
    NH_TRY(dev_write(out, &dst, true));
    if (in->dtype == NEURAL_DTYPE_FLOAT32)
        NH_TRY(launch_reduce_rows(static_cast<const float *>(c.p), rows, cols, RedRowMax<float>{{nullptr, 0}}, dst));
    else
        NH_TRY(launch_reduce_rows(static_cast<const double *>(c.p), rows, cols, RedRowMax<double>{{nullptr, 1}}, dst));
    NH_TRY(dev_written(out));
    return set_error(NEURAL_OK);
}

int neural_reduce_argmax(const NeuralTensor *in, int64_t axis, int64_t *out_indices)
{
    NH_TRY(ensure_init());
    if (!in || !out_indices) return set_error(NEURAL_ERR_NULL_POINTER);
    NH_TRY(check_tensor(in));
    if (in->ndim < 1 || (axis != -1 && axis != in->ndim - 1)) return set_error(NEURAL_ERR_DIM_MISMATCH);
    const int64_t cols = in->shape[in->ndim - 1];
    if (cols <= 0) return set_error(NEURAL_ERR_INVALID_ARGUMENT);
    const int64_t rows = numel(in) / cols;
    if (rows == 0) return set_error(NEURAL_OK);
    Contig c;
    NH_TRY(c.open(in));
    Staged so;
    NH_TRY(so.open(out_indices, size_t(rows) * sizeof(int64_t), false));
    if (in->dtype == NEURAL_DTYPE_FLOAT32)
        NH_TRY(launch_reduce_rows(static_cast<const float *>(c.p), rows, cols, RedRowArgmax<float>{}, so.dev));
    else
        NH_TRY(launch_reduce_rows(static_cast<const double *>(c.p), rows, cols, RedRowArgmax<double>{}, so.dev));
    NH_TRY(so.finish(true));
    return set_error(NEURAL_OK);
}

// simd_sum_f32 / simd_dot_f32 (simd.asm:551-784): float result of a double
// accumulation (compared against the fp64-exact value).
float simd_sum_f32(const float *a, uint64_t n)
{
    if (ensure_init() != NEURAL_OK || !a || n == 0) return 0.0f;
    Staged sa;
    if (sa.open(a, size_t(n) * 4, true) != NEURAL_OK) return 0.0f;
    void *res = workspace().result;
    double s = 0.0;
    if (launch_reduce_full(static_cast<const float *>(sa.dev), int64_t(n), RedSum{}, res) != NEURAL_OK) return 0.0f;
    if (hipMemcpyAsync(&s, res, sizeof(s), hipMemcpyDeviceToHost, stream()) != hipSuccess || sync() != NEURAL_OK)
        return 0.0f;
    set_error(NEURAL_OK);
    return float(s);
}

}  // extern "C"

namespace nh {

// Dot product: sum of a[i]*b[i] in double (products of floats are exact).
__global__ __launch_bounds__(kRBlock) void k_dot_f32(const float *__restrict__ a, const float *__restrict__ b,
                                                     int64_t n, RedSum::S *partials, unsigned *counter, double *out)
{
    RedSum red;
    RedSum::S st = red.init();
    const int64_t stride = int64_t(gridDim.x) * kRBlock;
    for (int64_t i = int64_t(blockIdx.x) * kRBlock + threadIdx.x; i < n; i += stride)
        st.s += double(a[i]) * double(b[i]);
    st = block_reduce(red, st);
    __shared__ bool s_last;
    if (threadIdx.x == 0) {
        partials[blockIdx.x] = st;
        __threadfence();
        s_last = atomicAdd(counter, 1u) == gridDim.x - 1;
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    RedSum::S acc = red.init();
    for (int i = threadIdx.x; i < int(gridDim.x); i += kRBlock) acc = red.comb(acc, partials[i]);
    acc = block_reduce(red, acc);
    if (threadIdx.x == 0) {
        *out = acc.s;
        *counter = 0u;
    }
}

}  // namespace nh

extern "C" float simd_dot_f32(const float *a, const float *b, uint64_t n)
{
    if (ensure_init() != NEURAL_OK || !a || !b || n == 0) return 0.0f;
    Staged sa, sb;
    if (sa.open(a, size_t(n) * 4, true) != NEURAL_OK || sb.open(b, size_t(n) * 4, true) != NEURAL_OK) return 0.0f;
    Workspace &ws = workspace();
    int64_t g = ceil_div(int64_t(n), kRBlock);
    if (g > int64_t(num_cus()) * 4) g = int64_t(num_cus()) * 4;
    hipLaunchKernelGGL(k_dot_f32, dim3(unsigned(g)), dim3(kRBlock), 0, stream(), static_cast<const float *>(sa.dev),
                       static_cast<const float *>(sb.dev), int64_t(n), static_cast<RedSum::S *>(ws.partials),
                       ws.counter, static_cast<double *>(ws.result));
    double s = 0.0;
    if (check_launch() != NEURAL_OK ||
        hipMemcpyAsync(&s, ws.result, sizeof(s), hipMemcpyDeviceToHost, stream()) != hipSuccess || sync() != NEURAL_OK)
        return 0.0f;
    set_error(NEURAL_OK);
    return float(s);
}
