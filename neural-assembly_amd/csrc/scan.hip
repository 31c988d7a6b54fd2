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

struct RedScan {
    struct S { double ss; int flags; };  // bit 0: NaN seen, bit 1: Inf seen
    static constexpr bool kSuffixPass = false;
    NH_DEV S init() const { return {0.0, 0}; }
    NH_DEV void acc(S &s, double v, int64_t) const
    {
        if (v != v) s.flags |= 1;
        else if (__builtin_isinf(v)) s.flags |= 2;
        s.ss += v * v;
    }
    NH_DEV S comb(S a, S b) const { return {a.ss + b.ss, a.flags | b.flags}; }
    NH_DEV S shfl(S a, int off) const { return {__shfl_xor(a.ss, off, 64), __shfl_xor(a.flags, off, 64)}; }
    NH_DEV void store(void *out, S s) const { *static_cast<S *>(out) = s; }
};

template <typename T>
static int scan_dev(const T *x, int64_t n, RedScan::S *st)
{
    void *res = workspace().result;
    NH_TRY(launch_reduce_full(x, n, RedScan{}, res));
    NH_HIP(hipMemcpyAsync(st, res, sizeof(*st), hipMemcpyDeviceToHost, stream()));
    NH_TRY(sync());
    return NEURAL_OK;
}

static int scan_raw(const float *data, uint64_t n, RedScan::S *st)
{
    NH_TRY(ensure_init());
    Staged s;
    NH_TRY(s.open(data, size_t(n) * 4, true));
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
    RedScan::S st;
    if (scan_raw(data, n, &st) != NEURAL_OK) return 0;
    return (st.flags & 1) ? 1 : 0;
}

int neural_tensor_has_inf(const float *data, uint64_t n)
{
    if (!data || n == 0) return 0;
    RedScan::S st;
    if (scan_raw(data, n, &st) != NEURAL_OK) return 0;
    return (st.flags & 2) ? 1 : 0;
}

float neural_tensor_grad_l2_norm(const float *data, uint64_t n)
{
    if (!data || n == 0) return 0.0f;
    RedScan::S st;
    if (scan_raw(data, n, &st) != NEURAL_OK) return 0.0f;
    return float(std::sqrt(st.ss));
}

int neural_scan_nan_inf_l2(const float *data, uint64_t n, int *has_nan, int *has_inf, double *sumsq)
{
    if (!data && n > 0) return set_error(NEURAL_ERR_NULL_POINTER);
    RedScan::S st{0.0, 0};
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
    RedScan::S st{0.0, 0};
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
