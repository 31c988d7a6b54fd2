// scan.hip -- NaN / Inf detection and the gradient L2 norm in one pass.
//
// Reference: tensor_has_nan (training_ops.asm:544-574, NaN iff unordered),
// tensor_has_inf (585-621, |bits| == 0x7f800000), tensor_grad_l2_norm
// (636-696, sqrt of a 4-lane float sum of squares).  One grid reduction reads
// the data once and produces both flags and the sum of squares, accumulated
// in double (squares of floats are exact in double); the norm is the float
// rounding of sqrt of that sum.
#include <cmath>

#include "reduce_impl.hpp"

namespace nh {

// Lane state: sum of squares in double (fused x*x + s: the square of a
// float is exact in double, so this is the unfused sum) and the largest |x|
// (NaN-ignoring).  A NaN makes the sum NaN and nothing else does (all terms
// are >= 0, so no Inf - Inf); an infinity makes the largest |x| infinite.
struct ScanOut { double ss; int32_t flags; int32_t pad; };  // flags bit 0: NaN, bit 1: Inf

template <typename T>
struct RedScan {
    struct L { double ss; T amax; int32_t pad[sizeof(T) == 4 ? 1 : 2]; };
    using B = L;
    NH_DEV L linit() const { return {0.0, T(0), {}}; }
    NH_DEV void lacc(L &s, T x, int64_t) const
    {
        const double d = double(x);
        s.ss = __builtin_fma(d, d, s.ss);
        s.amax = fmax_nn(s.amax, fabs_t(x));
    }
    NH_DEV L lcomb(L a, L b) const { return {a.ss + b.ss, fmax_nn(a.amax, b.amax), {}}; }
    template <int TPR>
    NH_DEV B finish(L s, const T *, int64_t, int64_t) const { return s; }
    NH_DEV B bident() const { return linit(); }
    NH_DEV B bcomb(B a, B b) const { return lcomb(a, b); }
    NH_DEV void store(void *out, int64_t, B b, const T *, int64_t) const
    {
        ScanOut o;
        o.ss = b.ss;
        o.flags = (b.ss != b.ss ? 1 : 0) | (b.amax == inf_t<T>() ? 2 : 0);
        o.pad = 0;
        *static_cast<ScanOut *>(out) = o;
    }
};

template <typename T>
static int scan_dev(const T *x, int64_t n, ScanOut *st)
{
    WsGuard wg;
    return reduce_full_to_host(x, n, RedScan<T>{}, st, sizeof(*st));
}

static int scan_raw(const float *data, uint64_t n, ScanOut *st)
{
    NH_TRY(ensure_init());
    Staged s;
    NH_TRY(s.open_n(data, n, 4, true));
    NH_TRY(scan_dev(static_cast<const float *>(s.dev), int64_t(n), st));
    NH_TRY(s.finish(false));
    return NEURAL_OK;
}

}  // namespace nh

using namespace nh;

extern "C" {

int neural_tensor_has_nan(const float *data, uint64_t n)
{
    if (!data || n == 0) return 0;
    ScanOut st;
    if (scan_raw(data, n, &st) != NEURAL_OK) return 0;
    return (st.flags & 1) ? 1 : 0;
}

int neural_tensor_has_inf(const float *data, uint64_t n)
{
    if (!data || n == 0) return 0;
    ScanOut st;
    if (scan_raw(data, n, &st) != NEURAL_OK) return 0;
    return (st.flags & 2) ? 1 : 0;
}

float neural_tensor_grad_l2_norm(const float *data, uint64_t n)
{
    if (!data || n == 0) return 0.0f;
    ScanOut st;
    if (scan_raw(data, n, &st) != NEURAL_OK) return 0.0f;
    return float(std::sqrt(st.ss));
}

int neural_scan_nan_inf_l2(const float *data, uint64_t n, int *has_nan, int *has_inf, double *sumsq)
{
    if (!data && n > 0) return set_error(NEURAL_ERR_NULL_POINTER);
    ScanOut st{0.0, 0, 0};
    if (n > 0) NH_TRY(scan_raw(data, n, &st));
    if (has_nan) *has_nan = st.flags & 1;
    if (has_inf) *has_inf = (st.flags >> 1) & 1;
    if (sumsq) *sumsq = st.ss;
    return set_error(NEURAL_OK);
}

int neural_tensor_scan(NeuralTensor *t, int *has_nan, int *has_inf, double *sumsq)
{
    NH_TRY(ensure_init());
    NH_TRY(check_tensor(t));
    ScanOut st{0.0, 0, 0};
    const int64_t n = numel(t);
    if (n > 0) {
        if (!is_contiguous(t)) return set_error(NEURAL_ERR_INVALID_ARGUMENT);
        const void *p = nullptr;
        NH_TRY(dev_read(t, &p));
        if (t->dtype == NEURAL_DTYPE_FLOAT32) NH_TRY(scan_dev(static_cast<const float *>(p), n, &st));
        else NH_TRY(scan_dev(static_cast<const double *>(p), n, &st));
    }
    if (has_nan) *has_nan = st.flags & 1;
    if (has_inf) *has_inf = (st.flags >> 1) & 1;
    if (sumsq) *sumsq = st.ss;
    return set_error(NEURAL_OK);
}

}  // extern "C"
