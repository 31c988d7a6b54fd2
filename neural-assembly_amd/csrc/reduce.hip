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

// Running-max chain m = (m > x) ? m : x (activations.asm:815-823,888-895).
// Closed form: NaN if the last element is NaN, else the largest value after
// the last NaN, the later element winning ties (which only matters for the
// sign of zero).  Lanes keep a NaN-ignoring max and a NaN/Inf sentinel
// (x * 0 is NaN exactly for NaN and +-Inf); a segment whose sentinel fired
// rescans itself for its last NaN, and a zero result rescans for the last
// zero.  Segment summary {v, nan, nonempty} composes in index order:
// a later segment that holds a NaN replaces everything before it.
enum { OUT_T = 0, OUT_F64 = 1 };
template <typename T, int MODE>
struct RedMaxChain {
    struct L { T m, nanacc; };
    struct B { T v; int32_t nan, nonempty; };
    static_assert(sizeof(B) % 4 == 0, "");
    NH_DEV L linit() const { return {-inf_t<T>(), T(0)}; }
    NH_DEV void lacc(L &s, T x, int64_t) const
    {
        s.m = fmax_nn(s.m, x);
        s.nanacc = fma_t(x, T(0), s.nanacc);
    }
    NH_DEV L lcomb(L a, L b) const { return {fmax_nn(a.m, b.m), a.nanacc + b.nanacc}; }
    // `row` is the row itself or a view that yields its elements by index
    template <int TPR, class R>
    NH_DEV B finish(L s, const R &row, int64_t lo, int64_t hi) const
    {
        using G = Grp<TPR>;
        B b{s.m, 0, hi > lo ? 1 : 0};
        int64_t from = lo;
        if (s.nanacc != s.nanacc) {
            int64_t ln = -1;
            for (int64_t j = lo + G::lane(); j < hi; j += TPR) ln = (row[j] != row[j]) ? j : ln;
            ln = G::max_i64(ln);
            if (ln >= 0) {
                b.nan = 1;
                if (ln == hi - 1) {
                    b.v = qnan_t<T>();
                    return b;
                }
                T m = -inf_t<T>();
                for (int64_t j = ln + 1 + G::lane(); j < hi; j += TPR) m = fmax_nn(m, row[j]);
                b.v = G::reduce(m, [](T a, T c) { return fmax_nn(a, c); });
                from = ln + 1;
            }
        }
        if (b.v == T(0)) {
            int64_t lz = -1;
            for (int64_t j = from + G::lane(); j < hi; j += TPR) lz = (row[j] == T(0)) ? j : lz;
            lz = G::max_i64(lz);
            if (lz >= 0) b.v = row[lz];
        }
        return b;
    }
    NH_DEV B bident() const { return {T(0), 0, 0}; }
    NH_DEV B bcomb(B a, B b) const
    {
        if (!b.nonempty) return a;
        if (!a.nonempty || b.nan) return b;
        return {(a.v > b.v) ? a.v : b.v, a.nan, 1};
    }
    NH_DEV void store(void *out, int64_t r, B b, const T *, int64_t) const
    {
        if (MODE == OUT_F64) static_cast<double *>(out)[r] = double(b.v);
        else static_cast<T *>(out)[r] = b.v;
    }
};

// Argmax: idx = 0, m = x0, update iff x_j > m (main.asm:3245-3292,3598-3640):
// the first index of the largest non-NaN value, or 0 when x0 is NaN or no
// element exceeds -inf.  Lane state {best value, its first index relative to
// the segment start} (8 bytes for f32: two dwords through every butterfly
// step); segment summary {row index, value}.  Ties go to the smaller index,
// so the combine is order-free.
template <typename T> struct ArgLane;
template <> struct ArgLane<float> { float v; int32_t i; };
template <> struct ArgLane<double> { double v; int32_t i, pad; };

template <typename T>
struct RedArgmax {
    static constexpr bool kRelIndex = true;
    static constexpr bool kStoreReadsFirst = true;
    using L = ArgLane<T>;
    struct B { int64_t i; T v; int32_t pad[sizeof(T) == 4 ? 1 : 2]; };
    NH_DEV L linit() const
    {
        L l{};
        l.v = -inf_t<T>();
        l.i = -1;
        return l;
    }
    NH_DEV void lacc(L &s, T x, int64_t i) const
    {
        const bool up = x > s.v;
        s.v = up ? x : s.v;
        s.i = up ? int32_t(i) : s.i;
    }
    NH_DEV L lcomb(L a, L b) const
    {
        if (b.v > a.v || (b.v == a.v && b.i >= 0 && (a.i < 0 || b.i < a.i))) return b;
        return a;
    }
    template <int TPR, class R>
    NH_DEV B finish(L s, const R &, int64_t lo, int64_t) const
    {
        B b{};
        b.i = s.i >= 0 ? lo + s.i : -1;
        b.v = s.v;
        return b;
    }
    NH_DEV B bident() const
    {
        B b{};
        b.i = -1;
        b.v = -inf_t<T>();
        return b;
    }
    NH_DEV B bcomb(B a, B b) const
    {
        if (b.v > a.v || (b.v == a.v && b.i >= 0 && (a.i < 0 || b.i < a.i))) return b;
        return a;
    }
    template <class R>
    NH_DEV void store(void *out, int64_t r, B b, const R &row, int64_t) const
    {
        const T first = row[0];
        static_cast<int64_t *>(out)[r] = (first != first || b.i < 0) ? 0 : b.i;
    }
};

// ---- row statistics in one pass (NEW: no counterpart in the reference) -------------
// Sum, mean, running-max chain and argmax of every row from one walk: the
// four reducers side by side, each fed exactly the values, in exactly the
// order, that it is fed by itself, so every output is bit-identical to the
// stand-alone reduce_sum / reduce_mean / reduce_max / reduce_argmax of the
// same rows.  Null output pointers are skipped.
template <typename T>
struct RedStats {
    static constexpr bool kRelIndex = true;
    static constexpr bool kStoreReadsFirst = true;
    using S = RedSum<T, SUM_OUT_T>;
    using M = RedMaxChain<T, OUT_T>;
    using A = RedArgmax<T>;
    // Lane state: the double sum and the argmax lane, whose best value is also
    // the max chain's NaN-ignoring lane maximum (x > v and fmax(v, x) agree
    // except on the sign of a zero, which the chain's zero rescan decides).
    // A NaN makes the double sum NaN, so a NaN sum stands for the chain's NaN
    // sentinel (it also fires for +Inf with -Inf; the rescan then finds no NaN
    // and changes nothing).  4 dwords for f32 instead of 8.
    struct L { double s; typename A::L a; };
    struct B { typename S::B s; typename M::B m; typename A::B a; };
    T *sum = nullptr, *mean = nullptr, *max = nullptr;
    int64_t *argmax = nullptr;
    int64_t cols = 1;

    NH_DEV L linit() const { return {0.0, A{}.linit()}; }
    NH_DEV void lacc(L &l, T x, int64_t i) const
    {
        l.s += double(x);
        A{}.lacc(l.a, x, i);
    }
    NH_DEV L lcomb(L a, L b) const { return {a.s + b.s, A{}.lcomb(a.a, b.a)}; }
    template <int TPR, class R>
    NH_DEV B finish(L l, const R &row, int64_t lo, int64_t hi) const
    {
        const typename M::L ml{l.a.v, l.s != l.s ? qnan_t<T>() : T(0)};
        return {l.s, M{}.template finish<TPR>(ml, row, lo, hi), A{}.template finish<TPR>(l.a, row, lo, hi)};
    }
    NH_DEV B bident() const { return {S{}.bident(), M{}.bident(), A{}.bident()}; }
    NH_DEV B bcomb(B a, B b) const { return {S{}.bcomb(a.s, b.s), M{}.bcomb(a.m, b.m), A{}.bcomb(a.a, b.a)}; }
    template <class R>
    NH_DEV void store(void *, int64_t r, B b, const R &row, int64_t) const
    {
        const T *none = nullptr;
        if (sum) S{}.store(sum, r, b.s, none, cols);
        if (mean) {
            S m;
            m.div = cols;
            m.store(mean, r, b.s, none, cols);
        }
        if (max) M{}.store(max, r, b.m, none, cols);
        if (argmax) A{}.store(argmax, r, b.a, row, cols);
    }
};

// The bias add as the walk's prologue: y = x + b per element (the rounding
// neural_bias_add does), stored non-temporally and then reduced.
template <typename T>
struct BiasPre {
    static constexpr bool kActive = true;
    using V = typename Vec16<T>::type;
    const T *bias;  // [cols]
    T *y;           // this row of the output
    NH_DEV V load(int64_t i) const { return reinterpret_cast<const V *>(bias)[i]; }
    NH_DEV V vec(const V &v, const V &b, int64_t i) const
    {
        V r;
#pragma unroll
        for (int k = 0; k < Vec16<T>::n; k++) r[k] = v[k] + b[k];
        st_nt(reinterpret_cast<V *>(y) + i, r);
        return r;
    }
    NH_DEV T one(T x, int64_t j) const
    {
        const T r = x + bias[j];
        y[j] = r;
        return r;
    }
};

// The output row as the rescans see it, recomputed from x and b (the same
// values the prologue stored; no wait for those stores is needed).
template <typename T>
struct BiasRow {
    const T *x, *bias;
    NH_DEV T operator[](int64_t j) const { return x[j] + bias[j]; }
};

// One group of TPR lanes per row, as k_reduce_rows: the row of x is read
// once, y = x + b written once, and the statistics of y stored.
template <typename T, int TPR>
__global__ __launch_bounds__(kRBlock) void k_bias_row_stats(const T *__restrict__ x, const T *__restrict__ bias,
                                                            T *__restrict__ y, int64_t rows, int64_t cols,
                                                            RedStats<T> red, bool vec)
{
    constexpr int RPB = kRBlock / TPR;
    for (int64_t r = int64_t(blockIdx.x) * RPB + threadIdx.x / TPR; r < rows; r += int64_t(gridDim.x) * RPB) {
        const T *xr = x + r * cols;
        const BiasPre<T> pre{bias, y + r * cols};
        T y0 = T(0);  // y[r][0] as lane 0 computed it
        const typename RedStats<T>::L l = seg_walk<T, RedStats<T>, TPR, true>(red, xr, 0, cols, vec, pre, &y0);
        const BiasRow<T> row{xr, bias};
        const typename RedStats<T>::B b = red.template finish<TPR>(l, row, 0, cols);
        if (Grp<TPR>::lane() == 0) red.store(nullptr, r, b, FirstOnly<T>{y0}, cols);
    }
}

// bias == nullptr: the statistics of x.  Otherwise y = x + bias and its
// statistics in one pass where the stand-alone reductions would use one group
// per row; where they would split rows into segments (few long rows) the
// bias add runs first and the statistics are reduced from y, so the split,
// and with it every result, stays the stand-alone one.
template <typename T>
static int row_stats_launch(const T *x, const T *bias, T *y, int64_t rows, int64_t cols, const RedStats<T> &red)
{
    if (!bias) return launch_reduce(x, rows, cols, cols, red, nullptr);
    const ReducePlan plan = reduce_plan<T>(rows, cols);
    if (plan.gx > 1) return NEURAL_ERR_NOT_IMPLEMENTED;  // the caller takes the two-pass route
    const bool vec = ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(bias) |
                       reinterpret_cast<uintptr_t>(y)) & 15u) == 0 && cols % Vec16<T>::n == 0;
    if (plan.tpr == 64)
        NH_LAUNCH((k_bias_row_stats<T, 64>), dim3(rows_grid(rows, kRBlock / 64)), dim3(kRBlock), 0, stream(), x,
                  bias, y, rows, cols, red, vec);
    else
        NH_LAUNCH((k_bias_row_stats<T, kRBlock>), dim3(rows_grid(rows, 1)), dim3(kRBlock), 0, stream(), x, bias,
                  y, rows, cols, red, vec);
    return check_launch();
}

// ---- column sums (reduce_sum axis=0) -------------------------------------------------
// Stage 1: grid (column groups of 256, row chunks) writes double partials
// [chunks][cols]; stage 2 adds the chunks in order per column.  Both step
// through column groups by the grid's width (capped at kMaxGridBlocks).

__global__ __launch_bounds__(256) void k_colsum_stage1_f32(const float *x, int64_t rows, int64_t cols,
                                                           int64_t chunk, double *part)
{
    const int64_t r0 = int64_t(blockIdx.y) * chunk;
    int64_t r1 = r0 + chunk;
    if (r1 > rows) r1 = rows;
    for (int64_t c = int64_t(blockIdx.x) * 256 + threadIdx.x; c < cols; c += int64_t(gridDim.x) * 256) {
        double s = 0.0;
        for (int64_t r = r0; r < r1; r++) s += double(x[r * cols + c]);
        part[int64_t(blockIdx.y) * cols + c] = s;
    }
}

__global__ __launch_bounds__(256) void k_colsum_stage1_f64(const double *x, int64_t rows, int64_t cols,
                                                           int64_t chunk, double *part)
{
    const int64_t r0 = int64_t(blockIdx.y) * chunk;
    int64_t r1 = r0 + chunk;
    if (r1 > rows) r1 = rows;
    for (int64_t c = int64_t(blockIdx.x) * 256 + threadIdx.x; c < cols; c += int64_t(gridDim.x) * 256) {
        double s = 0.0;
        for (int64_t r = r0; r < r1; r++) s += x[r * cols + c];
        part[int64_t(blockIdx.y) * cols + c] = s;
    }
}

template <typename T>
__global__ __launch_bounds__(256) void k_colsum_stage2(const double *part, int64_t nchunks, int64_t cols,
                                                       int64_t div, T *out)
{
    for (int64_t c = int64_t(blockIdx.x) * 256 + threadIdx.x; c < cols; c += int64_t(gridDim.x) * 256) {
        double s = 0.0;
        for (int64_t k = 0; k < nchunks; k++) s += part[k * cols + c];
        out[c] = T(div > 1 ? s / double(div) : s);
    }
}

static int colsum(const NeuralTensor *in, const void *src, int64_t rows, int64_t cols, bool mean, void *dst)
{
    if (cols <= 0) return NEURAL_OK;
    // ~4 row chunks per CU-worth of column groups, at least 64 rows per chunk.
    const int64_t cgroups = ceil_div(cols, 256);
    const unsigned gx = unsigned(cgroups < kMaxGridBlocks ? cgroups : kMaxGridBlocks);
    int64_t nchunks = ceil_div(int64_t(num_cus()) * 4, cgroups);
    if (nchunks > ceil_div(rows, 64)) nchunks = ceil_div(rows, 64);
    if (nchunks < 1) nchunks = 1;
    if (nchunks > 65535) nchunks = 65535;
    const int64_t chunk = ceil_div(rows > 0 ? rows : 1, nchunks);
    double *part = static_cast<double *>(dev_alloc(size_t(nchunks * cols) * sizeof(double)));
    if (!part) return set_error(NEURAL_ERR_OUT_OF_MEMORY);
    const dim3 g1{gx, unsigned(nchunks), 1u};
    if (in->dtype == NEURAL_DTYPE_FLOAT32)
        NH_LAUNCH(k_colsum_stage1_f32, g1, dim3(256), 0, stream(), static_cast<const float *>(src), rows,
                           cols, chunk, part);
    else
        NH_LAUNCH(k_colsum_stage1_f64, g1, dim3(256), 0, stream(), static_cast<const double *>(src), rows,
                           cols, chunk, part);
    const int64_t div = mean ? rows : 1;
    if (in->dtype == NEURAL_DTYPE_FLOAT32)
        NH_LAUNCH((k_colsum_stage2<float>), dim3(gx), dim3(256), 0, stream(), part, nchunks,
                           cols, div, static_cast<float *>(dst));
    else
        NH_LAUNCH((k_colsum_stage2<double>), dim3(gx), dim3(256), 0, stream(), part,
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

// Whole-tensor reduction returned to the host: the combine launch stores the
// result into the mapped host area, then one stream sync.
template <template <typename> class RedOf, typename Out>
static int full_to_host(const NeuralTensor *t, Out *host_out)
{
    const int64_t n = numel(t);
    Contig c;
    NH_TRY(c.open(t));
    WsGuard wg;
    if (t->dtype == NEURAL_DTYPE_FLOAT32)
        return reduce_full_to_host(static_cast<const float *>(c.p), n, RedOf<float>{}, host_out, sizeof(Out));
    return reduce_full_to_host(static_cast<const double *>(c.p), n, RedOf<double>{}, host_out, sizeof(Out));
}

template <typename T> using SumF64 = RedSum<T, SUM_OUT_F64>;
template <typename T> using MaxF64 = RedMaxChain<T, OUT_F64>;

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
        rows = 1;  // the leading dims' product (rows of zero length still count)
        for (int64_t i = 0; i + 1 < nd; i++) rows *= in->shape[i];
        return NEURAL_OK;
    }
    // Other axes: the reference falls back to the full sum (math_kernels.asm:979-991).
    kind = 0; rows = 1; cols = numel(in);
    return NEURAL_OK;
}

template <typename T>
static int rows_sum(const void *src, int64_t rows, int64_t cols, bool mean, void *dst)
{
    RedSum<T, SUM_OUT_T> red;
    red.div = mean ? cols : 1;
    return launch_reduce(static_cast<const T *>(src), rows, cols, cols, red, dst);
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
    // empty input: sums of no elements are 0, their means 0 / 0
    if (numel(in) == 0) return neural_tensor_fill(out, mean ? __builtin_nan("") : 0.0);
    Contig c;
    NH_TRY(c.open(in));
    void *dst = nullptr;
    NH_TRY(dev_write(out, &dst, true));
    if (kind == 2) {
        NH_TRY(colsum(in, c.p, rows, cols, mean, dst));
    } else {
        // kind 0 is the whole tensor as one row
        if (in->dtype == NEURAL_DTYPE_FLOAT32) NH_TRY(rows_sum<float>(c.p, rows, cols, mean, dst));
        else NH_TRY(rows_sum<double>(c.p, rows, cols, mean, dst));
    }
    NH_TRY(dev_written(out));
    return set_error(NEURAL_OK);
}

// The optional outputs of a row-statistics call on `in` (rows of its last
// dimension): sum / mean / max tensors of `rows` elements, contiguous, in the
// input's dtype; argmax `rows` int64 (host or device).  At least one is given.
struct StatsOut {
    NeuralTensor *t[3] = {nullptr, nullptr, nullptr};  // sum, mean, max
    void *dev[3] = {nullptr, nullptr, nullptr};
    int64_t *argmax = nullptr;
    Staged arg;

    int open(const NeuralTensor *in, int64_t rows, NeuralTensor *sum, NeuralTensor *mean, NeuralTensor *max,
             int64_t *argmax_out)
    {
        t[0] = sum;
        t[1] = mean;
        t[2] = max;
        argmax = argmax_out;
        if (!sum && !mean && !max && !argmax) return set_error(NEURAL_ERR_NULL_POINTER);
        for (NeuralTensor *o : t) {
            if (!o) continue;
            NH_TRY(check_tensor(o));
            if (o->dtype != in->dtype) return set_error(NEURAL_ERR_DTYPE_MISMATCH);
            if (numel(o) != rows || !is_contiguous(o)) return set_error(NEURAL_ERR_SHAPE_MISMATCH);
        }
        return NEURAL_OK;
    }
    // device destinations (after the argument checks of the call)
    int map(int64_t rows)
    {
        for (int k = 0; k < 3; k++)
            if (t[k]) NH_TRY(dev_write(t[k], &dev[k], true));
        if (argmax) NH_TRY(arg.open(argmax, size_t(rows) * sizeof(int64_t), false));
        return NEURAL_OK;
    }
    template <typename T>
    RedStats<T> reducer(int64_t cols) const
    {
        RedStats<T> r;
        r.sum = static_cast<T *>(dev[0]);
        r.mean = static_cast<T *>(dev[1]);
        r.max = static_cast<T *>(dev[2]);
        r.argmax = argmax ? static_cast<int64_t *>(arg.dev) : nullptr;
        r.cols = cols;
        return r;
    }
    int finish()
    {
        for (NeuralTensor *o : t)
            if (o) NH_TRY(dev_written(o));
        if (argmax) NH_TRY(arg.finish(true));
        return NEURAL_OK;
    }
};

// rows x cols of `in` over its last dimension (cols > 0).
static int stats_shape(const NeuralTensor *in, int64_t &rows, int64_t &cols)
{
    NH_TRY(check_tensor(in));
    if (in->ndim < 1) return set_error(NEURAL_ERR_DIM_MISMATCH);
    cols = in->shape[in->ndim - 1];
    if (cols <= 0) return set_error(NEURAL_ERR_INVALID_ARGUMENT);
    rows = numel(in) / cols;
    return NEURAL_OK;
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
    NH_TRY(full_to_host<SumF64>(t, result));
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
    NH_TRY(full_to_host<SumF64>(t, &s));
    *result = s / double(n);
    return set_error(NEURAL_OK);
}

int neural_max(const NeuralTensor *t, double *result)
{
    NH_TRY(ensure_init());
    if (!t || !result) return set_error(NEURAL_ERR_NULL_POINTER);
    NH_TRY(check_tensor(t));
    if (numel(t) == 0) return set_error(NEURAL_ERR_INVALID_ARGUMENT);
    NH_TRY(full_to_host<MaxF64>(t, result));
    return set_error(NEURAL_OK);
}

int neural_argmax(const NeuralTensor *t, int64_t *result)
{
    NH_TRY(ensure_init());
    if (!t || !result) return set_error(NEURAL_ERR_NULL_POINTER);
    NH_TRY(check_tensor(t));
    if (numel(t) == 0) return set_error(NEURAL_ERR_INVALID_ARGUMENT);
    NH_TRY(full_to_host<RedArgmax>(t, result));
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
        NH_TRY(launch_reduce(static_cast<const float *>(c.p), rows, cols, cols, RedMaxChain<float, OUT_T>{}, dst));
    else
        NH_TRY(launch_reduce(static_cast<const double *>(c.p), rows, cols, cols, RedMaxChain<double, OUT_T>{}, dst));
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
        NH_TRY(launch_reduce(static_cast<const float *>(c.p), rows, cols, cols, RedArgmax<float>{}, so.dev));
    else
        NH_TRY(launch_reduce(static_cast<const double *>(c.p), rows, cols, cols, RedArgmax<double>{}, so.dev));
    NH_TRY(so.finish(true));
    return set_error(NEURAL_OK);
}

// neural_row_stats (NEW: no counterpart in the reference): the sum, mean,
// max and argmax of every row over the last dimension from one read of the
// input, each bit-identical to neural_reduce_sum / neural_reduce_mean /
// neural_reduce_max (axis = last) and neural_reduce_argmax.
int neural_row_stats(const NeuralTensor *in, NeuralTensor *sum, NeuralTensor *mean, NeuralTensor *max,
                     int64_t *argmax)
{
    NH_TRY(ensure_init());
    if (!in) return set_error(NEURAL_ERR_NULL_POINTER);
    int64_t rows = 0, cols = 0;
    NH_TRY(stats_shape(in, rows, cols));
    StatsOut so;
    NH_TRY(so.open(in, rows, sum, mean, max, argmax));
    if (rows == 0) return set_error(NEURAL_OK);
    Contig c;
    NH_TRY(c.open(in));
    NH_TRY(so.map(rows));
    if (in->dtype == NEURAL_DTYPE_FLOAT32)
        NH_TRY(row_stats_launch(static_cast<const float *>(c.p), static_cast<const float *>(nullptr),
                                static_cast<float *>(nullptr), rows, cols, so.reducer<float>(cols)));
    else
        NH_TRY(row_stats_launch(static_cast<const double *>(c.p), static_cast<const double *>(nullptr),
                                static_cast<double *>(nullptr), rows, cols, so.reducer<double>(cols)));
    NH_TRY(so.finish());
    return set_error(NEURAL_OK);
}

// neural_bias_add_row_stats (NEW: no counterpart in the reference): out =
// in + bias as neural_bias_add computes it, and the row statistics of out as
// neural_row_stats computes them, with one read of `in` and one write of
// `out` (no re-read of out) wherever the stand-alone reductions would give
// each row one group of lanes; otherwise the two calls in sequence.
int neural_bias_add_row_stats(NeuralTensor *out, const NeuralTensor *in, const NeuralTensor *bias,
                              NeuralTensor *sum, NeuralTensor *mean, NeuralTensor *max, int64_t *argmax)
{
    NH_TRY(ensure_init());
    if (!out || !in || !bias) return set_error(NEURAL_ERR_NULL_POINTER);
    NH_TRY(check_tensor(out));
    NH_TRY(check_tensor(bias));
    int64_t rows = 0, cols = 0;
    NH_TRY(stats_shape(in, rows, cols));
    if (bias->ndim < 1 || numel(bias) != cols) return set_error(NEURAL_ERR_SHAPE_MISMATCH);
    if (out->ndim != in->ndim) return set_error(NEURAL_ERR_SHAPE_MISMATCH);
    for (int64_t i = 0; i < in->ndim; i++)
        if (out->shape[i] != in->shape[i]) return set_error(NEURAL_ERR_SHAPE_MISMATCH);
    if (in->dtype != out->dtype || bias->dtype != out->dtype) return set_error(NEURAL_ERR_DTYPE_MISMATCH);
    StatsOut so;
    NH_TRY(so.open(in, rows, sum, mean, max, argmax));
    if (rows == 0) return set_error(NEURAL_OK);
    // In place (out sharing bytes with in or bias) the one-pass kernel would
    // overwrite values its rare-case rescans read again: two calls instead.
    const bool fused = is_contiguous(in) && is_contiguous(out) && is_contiguous(bias) &&
                       !tensors_may_overlap(out, in) && !tensors_may_overlap(out, bias) &&
                       ((in->dtype == NEURAL_DTYPE_FLOAT32 ? reduce_plan<float>(rows, cols)
                                                           : reduce_plan<double>(rows, cols)).gx == 1);
    if (!fused) {
        NH_TRY(neural_bias_add(out, in, bias));
        return neural_row_stats(out, sum, mean, max, argmax);
    }
    const void *px = nullptr, *pb = nullptr;
    void *py = nullptr;
    NH_TRY(dev_read(in, &px));
    NH_TRY(dev_read(bias, &pb));
    NH_TRY(dev_write(out, &py, true));
    NH_TRY(so.map(rows));
    if (in->dtype == NEURAL_DTYPE_FLOAT32)
        NH_TRY(row_stats_launch(static_cast<const float *>(px), static_cast<const float *>(pb),
                                static_cast<float *>(py), rows, cols, so.reducer<float>(cols)));
    else
        NH_TRY(row_stats_launch(static_cast<const double *>(px), static_cast<const double *>(pb),
                                static_cast<double *>(py), rows, cols, so.reducer<double>(cols)));
    NH_TRY(dev_written(out));
    NH_TRY(so.finish());
    return set_error(NEURAL_OK);
}

// simd_sum_f32 / simd_dot_f32 (simd.asm:551-784): float result of a double
// accumulation (compared against the fp64-exact value).
float simd_sum_f32(const float *a, uint64_t n)
{
    if (ensure_init() != NEURAL_OK || !a || n == 0) return 0.0f;
    Staged sa;
    if (sa.open_n(a, n, 4, true) != NEURAL_OK) return 0.0f;
    WsGuard wg;
    double s = 0.0;
    if (reduce_full_to_host(static_cast<const float *>(sa.dev), int64_t(n), SumF64<float>{}, &s, sizeof(s)) !=
        NEURAL_OK)
        return 0.0f;
    set_error(NEURAL_OK);
    return float(s);
}

}  // extern "C"

namespace nh {

// Dot product: sum of a[i]*b[i] in double (products of floats are exact).
__global__ __launch_bounds__(kRBlock) void k_dot_f32(const float *__restrict__ a, const float *__restrict__ b,
                                                     int64_t n, double *partials, unsigned *counter, double *out)
{
    double s = 0.0;
    const int64_t stride = int64_t(gridDim.x) * kRBlock;
    for (int64_t i = int64_t(blockIdx.x) * kRBlock + threadIdx.x; i < n; i += stride)
        s = __builtin_fma(double(a[i]), double(b[i]), s);
    const auto add = [](double x, double y) { return x + y; };
    s = Grp<kRBlock>::reduce(s, add);
    __shared__ bool s_last;
    if (threadIdx.x == 0) {
        partials[blockIdx.x] = s;
        __threadfence();
        s_last = atomicAdd(counter, 1u) == gridDim.x - 1;
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    double acc = 0.0;
    for (int i = threadIdx.x; i < int(gridDim.x); i += kRBlock) acc += partials[i];
    acc = Grp<kRBlock>::reduce(acc, add);
    if (threadIdx.x == 0) {
        *out = acc;
        *counter = 0u;
    }
}

}  // namespace nh

extern "C" float simd_dot_f32(const float *a, const float *b, uint64_t n)
{
    if (ensure_init() != NEURAL_OK || !a || !b || n == 0) return 0.0f;
    Staged sa, sb;
    if (sa.open_n(a, n, 4, true) != NEURAL_OK || sb.open_n(b, n, 4, true) != NEURAL_OK) return 0.0f;
    WsGuard wg;
    Workspace &ws = workspace();
    int64_t g = ceil_div(int64_t(n), kRBlock);
    if (g > int64_t(num_cus()) * 4) g = int64_t(num_cus()) * 4;
    NH_LAUNCH(k_dot_f32, dim3(unsigned(g)), dim3(kRBlock), 0, stream(), static_cast<const float *>(sa.dev),
                       static_cast<const float *>(sb.dev), int64_t(n), static_cast<double *>(ws.partials), ws.counter,
                       static_cast<double *>(ws.host_result_dev));
    double s = 0.0;
    if (check_launch() != NEURAL_OK || host_result_fetch(&s, sizeof(s)) != NEURAL_OK) return 0.0f;
    set_error(NEURAL_OK);
    return float(s);
}
