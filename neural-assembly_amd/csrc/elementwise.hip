// elementwise.hip -- elementwise, broadcast, fill and copy kernels.
//
// Semantics follow math_kernels.asm:66-945 (ew_*), activations.asm:153-171
// (ReLU via maxss), nn_layers.asm:472-539 (row-broadcast bias add),
// tensor.asm:531-589 (fill) and simd.asm:190-540 (raw-pointer add/mul/fma).
// Each output element is one IEEE operation on the same operands as the
// reference (no FMA contraction: built with -ffp-contract=off), so results
// are bit-identical.
#include <vector>

#include "ew_impl.hpp"
#include "kernels.hpp"

namespace nh {

// ---- operators ---------------------------------------------------------------

struct OpAdd { template <class T> NH_DEV T operator()(T x, T y) const { return x + y; } };
struct OpSub { template <class T> NH_DEV T operator()(T x, T y) const { return x - y; } };
struct OpMul { template <class T> NH_DEV T operator()(T x, T y) const { return x * y; } };
struct OpDiv { template <class T> NH_DEV T operator()(T x, T y) const { return x / y; } };
// vmaxps / maxss: second operand unless the first is strictly greater.
struct OpMax { template <class T> NH_DEV T operator()(T x, T y) const { return x > y ? x : y; } };

// ew_neg: sign-bit xor (math_kernels.asm:857-868), NaN sign flips too.
struct FnNeg {
    NH_DEV float operator()(float x) const { return __uint_as_float(__float_as_uint(x) ^ 0x80000000u); }
    NH_DEV double operator()(double x) const
    {
        return __longlong_as_double(__double_as_longlong(x) ^ (long long)0x8000000000000000ull);
    }
};

// node_relu: maxss x, 0 -> (x > 0) ? x : +0 (NaN -> +0, -0 -> +0).
struct FnRelu {
    NH_DEV float operator()(float x) const { return x > 0.0f ? x : 0.0f; }
    NH_DEV double operator()(double x) const { return x > 0.0 ? x : 0.0; }
};

// Identity: the streaming copy the flat kernels' tiling gives for a 1:1
// read / write stream (the bandwidth reference neural_hip_stream_copy times).
struct FnCopy {
    NH_DEV float operator()(float x) const { return x; }
};

// vec_add_relu_fusion (fusion.asm:200-226) and the bias + ReLU epilogue of
// matmul_bias_relu_fusion (fusion.asm:110-190): addss, then maxss with +0.
struct OpAddRelu {
    template <class T> NH_DEV T operator()(T x, T y) const
    {
        const T s = x + y;
        return s > T(0) ? s : T(0);
    }
};

// ew_scalar_add/mul: the f32 path rounds the double scalar to float once
// (cvtsd2ss, math_kernels.asm:544,653).
struct FnScalarAdd {
    float sf;
    double sd;
    NH_DEV float operator()(float x) const { return x + sf; }
    NH_DEV double operator()(double x) const { return x + sd; }
};
struct FnScalarMul {
    float sf;
    double sd;
    NH_DEV float operator()(float x) const { return x * sf; }
    NH_DEV double operator()(double x) const { return x * sd; }
};

// ---- fill / copy -----------------------------------------------------------------

template <typename T>
__global__ __launch_bounds__(kBlock) void k_fill(T *__restrict__ o, int64_t n, T v)
{
    using V = typename Vec16<T>::type;
    constexpr int VN = Vec16<T>::n;
    const int64_t nv = n / VN;
    V vv;
#pragma unroll
    for (int k = 0; k < VN; k++) vv[k] = v;
    V *ov = reinterpret_cast<V *>(o);
    const int64_t step = int64_t(gridDim.x) * (kBlock * kUnroll);
    for (int64_t base = int64_t(blockIdx.x) * (kBlock * kUnroll) + threadIdx.x; base < nv; base += step) {
#pragma unroll
        for (int u = 0; u < kUnroll; u++) {
            const int64_t i = base + int64_t(u) * kBlock;
            if (i < nv) st_nt(ov + i, vv);
        }
    }
    if (blockIdx.x == 0) {
        const int64_t j = nv * VN + threadIdx.x;
        if (j < n) o[j] = v;
    }
}

// Logical-order N-D addressing with element strides (up to 8 dims).
struct NDX {
    int nd;
    int64_t shape[8];
    int64_t stride[8];
};

NH_DEV int64_t ndx_offset(const NDX &d, int64_t idx)
{
    int64_t off = 0;
    for (int i = d.nd - 1; i >= 0; i--) {
        const int64_t s = d.shape[i];
        off += (idx % s) * d.stride[i];
        idx /= s;
    }
    return off;
}

template <typename U>
__global__ __launch_bounds__(kBlock) void k_fill_nd(U *o, int64_t n, NDX d, U v)
{
    const int64_t stride = int64_t(gridDim.x) * kBlock;
    for (int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride) o[ndx_offset(d, i)] = v;
}

template <typename U>
__global__ __launch_bounds__(kBlock) void k_copy_nd(U *o, NDX od, const U *s, NDX sd, int64_t n)
{
    const int64_t stride = int64_t(gridDim.x) * kBlock;
    for (int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride)
        o[ndx_offset(od, i)] = s[ndx_offset(sd, i)];
}

static int make_ndx(NDX &d, const int64_t *shape, const int64_t *bstride, int ndim, int es)
{
    if (ndim > 8) return set_error(NEURAL_ERR_DIM_MISMATCH);
    d.nd = ndim > 0 ? ndim : 1;
    if (ndim == 0) { d.shape[0] = 1; d.stride[0] = 0; return NEURAL_OK; }
    for (int i = 0; i < ndim; i++) {
        if (bstride[i] % es != 0) return set_error(NEURAL_ERR_INVALID_ARGUMENT);
        d.shape[i] = shape[i];
        d.stride[i] = bstride[i] / es;
    }
    return NEURAL_OK;
}

int launch_fill(void *dst, int dtype, int64_t n, double value)
{
    if (n <= 0) return NEURAL_OK;
    if (dtype == NEURAL_DTYPE_FLOAT32)
        NH_LAUNCH((k_fill<float>), dim3(flat_grid(n, 4, kUnroll)), dim3(kBlock), 0, stream(),
                           static_cast<float *>(dst), n, float(value));
    else
        NH_LAUNCH((k_fill<double>), dim3(flat_grid(n, 2, kUnroll)), dim3(kBlock), 0, stream(),
                           static_cast<double *>(dst), n, value);
    return check_launch();
}

int launch_fill_strided(void *dst, int dtype, const int64_t *shape, const int64_t *bstride, int ndim, double value)
{
    const int es = int(elem_size(dtype));
    NDX d;
    NH_TRY(make_ndx(d, shape, bstride, ndim, es));
    int64_t n = 1;
    for (int i = 0; i < ndim; i++) n *= shape[i];
    if (n <= 0) return NEURAL_OK;
    if (dtype == NEURAL_DTYPE_FLOAT32)
        NH_LAUNCH((k_fill_nd<float>), dim3(strided_grid(n)), dim3(kBlock), 0, stream(),
                           static_cast<float *>(dst), n, d, float(value));
    else
        NH_LAUNCH((k_fill_nd<double>), dim3(strided_grid(n)), dim3(kBlock), 0, stream(),
                           static_cast<double *>(dst), n, d, value);
    return check_launch();
}

int launch_copy_nd(void *dst, const int64_t *dshape, const int64_t *dstride, int dndim, const void *src,
                   const int64_t *sshape, const int64_t *sstride, int sndim, int es)
{
    NDX od, sd;
    NH_TRY(make_ndx(od, dshape, dstride, dndim, es));
    NH_TRY(make_ndx(sd, sshape, sstride, sndim, es));
    int64_t n = 1;
    for (int i = 0; i < dndim; i++) n *= dshape[i];
    if (n <= 0) return NEURAL_OK;
    if (es == 4)
        NH_LAUNCH((k_copy_nd<uint32_t>), dim3(strided_grid(n)), dim3(kBlock), 0, stream(),
                           static_cast<uint32_t *>(dst), od, static_cast<const uint32_t *>(src), sd, n);
    else
        NH_LAUNCH((k_copy_nd<uint64_t>), dim3(strided_grid(n)), dim3(kBlock), 0, stream(),
                           static_cast<uint64_t *>(dst), od, static_cast<const uint64_t *>(src), sd, n);
    return check_launch();
}

// ---- broadcast layout ---------------------------------------------------------------

int build_nd(const NeuralTensor *out, const NeuralTensor *a, const NeuralTensor *b, ND4 &d)
{
    constexpr int MAXD = 16;
    const int od = int(out->ndim);
    if (od > MAXD) return set_error(NEURAL_ERR_DIM_MISMATCH);
    const int64_t es = int64_t(elem_size(out->dtype));
    int64_t shp[MAXD], s[3][MAXD];
    for (int i = 0; i < od; i++) {
        shp[i] = out->shape[i];
        if (out->stride[i] % es) return set_error(NEURAL_ERR_INVALID_ARGUMENT);
        s[0][i] = out->stride[i] / es;
    }
    const NeuralTensor *ops[2] = {a, b};
    for (int k = 0; k < 2; k++) {
        const NeuralTensor *t = ops[k];
        int64_t *st = s[k + 1];
        if (!t) { for (int i = 0; i < od; i++) st[i] = 0; continue; }
        if (t->ndim > od) return set_error(NEURAL_ERR_SHAPE_MISMATCH);
        const int off = od - int(t->ndim);
        for (int i = 0; i < off; i++) st[i] = 0;
        for (int j = 0; j < int(t->ndim); j++) {
            const int i = off + j;
            if (t->stride[j] % es) return set_error(NEURAL_ERR_INVALID_ARGUMENT);
            if (t->shape[j] == shp[i]) st[i] = t->stride[j] / es;
            else if (t->shape[j] == 1) st[i] = 0;
            else return set_error(NEURAL_ERR_SHAPE_MISMATCH);
        }
    }
    // Drop unit dims, then merge neighbours whose strides chain for every
    // operand (outer stride == inner stride * inner extent).
    int64_t mshp[MAXD], ms[3][MAXD];
    int m = 0;
    for (int i = 0; i < od; i++) {
        if (shp[i] == 1) continue;
        if (m > 0) {
            bool merge = true;
            for (int k = 0; k < 3; k++)
                if (ms[k][m - 1] != s[k][i] * shp[i]) merge = false;
            if (merge) {
                mshp[m - 1] *= shp[i];
                for (int k = 0; k < 3; k++) ms[k][m - 1] = s[k][i];
                continue;
            }
        }
        mshp[m] = shp[i];
        for (int k = 0; k < 3; k++) ms[k][m] = s[k][i];
        m++;
    }
    if (m > 4) return set_error(NEURAL_ERR_DIM_MISMATCH);
    const int pad = 4 - m;
    for (int i = 0; i < 4; i++) {
        if (i < pad) {
            d.shape[i] = 1;
            d.so[i] = d.sa[i] = d.sb[i] = 0;
        } else {
            d.shape[i] = mshp[i - pad];
            d.so[i] = ms[0][i - pad];
            d.sa[i] = ms[1][i - pad];
            d.sb[i] = ms[2][i - pad];
        }
    }
    return NEURAL_OK;
}

// ---- raw-pointer f32 (simd.asm) --------------------------------------------------------

struct OpFma {
    NH_DEV float operator()(float x, float y, float z) const { return __builtin_fmaf(x, y, z); }
};

__global__ __launch_bounds__(kBlock) void k_fma_f32(const float *__restrict__ a, const float *__restrict__ b,
                                                    const float *__restrict__ c, float *__restrict__ o, int64_t n)
{
    const int64_t stride = int64_t(gridDim.x) * kBlock;
    for (int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride)
        o[i] = __builtin_fmaf(a[i], b[i], c[i]);
}

template <typename Op>
static int raw_binary_f32(float *dst, const float *a, const float *b, uint64_t n, Op op)
{
    NH_TRY(ensure_init());
    if (!dst || !a || !b) return set_error(NEURAL_ERR_NULL_POINTER);
    if (n == 0) return set_error(NEURAL_OK);
    if (n > kMaxRawCount) return set_error(NEURAL_ERR_TENSOR_TOO_LARGE);
    const size_t bytes = size_t(n) * 4;
    Staged sa, sb, so;
    NH_TRY(sa.open(a, bytes, true));
    NH_TRY(sb.open(b, bytes, true));
    NH_TRY(so.open(dst, bytes, false));
    NH_TRY(launch_map2_flat(static_cast<const float *>(sa.dev), static_cast<const float *>(sb.dev),
                            static_cast<float *>(so.dev), int64_t(n), op));
    NH_TRY(so.finish(true));
    NH_TRY(sa.finish(false));
    NH_TRY(sb.finish(false));
    return set_error(NEURAL_OK);
}

}  // namespace nh

using namespace nh;

extern "C" {

int neural_add(NeuralTensor *out, const NeuralTensor *a, const NeuralTensor *b) { return binary_api(out, a, b, OpAdd{}); }
int neural_sub(NeuralTensor *out, const NeuralTensor *a, const NeuralTensor *b) { return binary_api(out, a, b, OpSub{}); }
int neural_mul(NeuralTensor *out, const NeuralTensor *a, const NeuralTensor *b) { return binary_api(out, a, b, OpMul{}); }
int neural_div(NeuralTensor *out, const NeuralTensor *a, const NeuralTensor *b) { return binary_api(out, a, b, OpDiv{}); }
int neural_maximum(NeuralTensor *out, const NeuralTensor *a, const NeuralTensor *b) { return binary_api(out, a, b, OpMax{}); }

// Bias add of linear_forward_fn (nn_layers.asm:472-539): x [..., C] + bias [C].
int neural_bias_add(NeuralTensor *out, const NeuralTensor *x, const NeuralTensor *bias)
{
    if (!out || !x || !bias) return set_error(NEURAL_ERR_NULL_POINTER);
    if (bias->ndim < 1 || x->ndim < 1 || numel(bias) != x->shape[x->ndim - 1])
        return set_error(NEURAL_ERR_SHAPE_MISMATCH);
    for (int64_t i = 0; i < out->ndim || i < x->ndim; i++)
        if (out->ndim != x->ndim || out->shape[i] != x->shape[i]) return set_error(NEURAL_ERR_SHAPE_MISMATCH);
    return binary_api(out, x, bias, OpAdd{});
}

// out = relu(a + b) in one pass; b may broadcast like neural_add's operands
// (a [.., C] bias is the fused bias + ReLU).
int neural_add_relu(NeuralTensor *out, const NeuralTensor *a, const NeuralTensor *b)
{
    return binary_api(out, a, b, OpAddRelu{});
}

// vec_add_relu_fusion (fusion.asm:200-226): c[i] = max(0, a[i] + b[i]) over
// raw float pointers (host or device); nothing happens for length <= 0.
void vec_add_relu_fusion(const float *a, const float *b, float *c, int64_t n)
{
    if (n <= 0) return;
    (void)raw_binary_f32(c, a, b, uint64_t(n), OpAddRelu{});
}

int neural_scalar_add(NeuralTensor *out, const NeuralTensor *a, double s)
{
    FnScalarAdd f{float(s), s};
    return run_unary(out, a, f, f);
}

int neural_scalar_mul(NeuralTensor *out, const NeuralTensor *a, double s)
{
    FnScalarMul f{float(s), s};
    return run_unary(out, a, f, f);
}

int neural_neg(NeuralTensor *out, const NeuralTensor *a) { return run_unary(out, a, FnNeg{}, FnNeg{}); }

// neural_relu (neural_api.asm:1218-1274): the reference builds a node, computes
// into a fresh zeroed tensor and copies it out (three passes); one pass here.
int neural_relu(NeuralTensor *out, const NeuralTensor *in) { return run_unary(out, in, FnRelu{}, FnRelu{}); }

int simd_add_f32(float *dst, const float *a, const float *b, uint64_t n) { return raw_binary_f32(dst, a, b, n, OpAdd{}); }
int simd_mul_f32(float *dst, const float *a, const float *b, uint64_t n) { return raw_binary_f32(dst, a, b, n, OpMul{}); }

// simd_fma_f32 (simd.asm:436-540): dst = a*b + c, fused (the reference's
// vector body uses vfmadd213ps; its scalar tail rounds twice -- here every
// element is fused).
int simd_fma_f32(float *dst, const float *a, const float *b, const float *c, uint64_t n)
{
    NH_TRY(ensure_init());
    if (!dst || !a || !b || !c) return set_error(NEURAL_ERR_NULL_POINTER);
    if (n == 0) return set_error(NEURAL_OK);
    if (n > kMaxRawCount) return set_error(NEURAL_ERR_TENSOR_TOO_LARGE);
    const size_t bytes = size_t(n) * 4;
    Staged sa, sb, sc, so;
    NH_TRY(sa.open(a, bytes, true));
    NH_TRY(sb.open(b, bytes, true));
    NH_TRY(sc.open(c, bytes, true));
    NH_TRY(so.open(dst, bytes, false));
    NH_LAUNCH(k_fma_f32, dim3(strided_grid(int64_t(n))), dim3(kBlock), 0, stream(),
                       static_cast<const float *>(sa.dev), static_cast<const float *>(sb.dev),
                       static_cast<const float *>(sc.dev), static_cast<float *>(so.dev), int64_t(n));
    NH_TRY(check_launch());
    NH_TRY(so.finish(true));
    NH_TRY(sa.finish(false));
    NH_TRY(sb.finish(false));
    NH_TRY(sc.finish(false));
    return set_error(NEURAL_OK);
}

// neural_hip_stream_copy (NEW, no reference counterpart; a bandwidth
// reference for measurement): dst = src over `bytes` bytes of device memory
// through k_map1_flat (16-byte non-temporal loads and stores, the tiling of
// every flat streaming kernel).  Both pointers must be device pointers,
// 16-byte aligned, and bytes a multiple of 16.
int neural_hip_stream_copy(void *dst, const void *src, uint64_t bytes)
{
    NH_TRY(ensure_init());
    if (!dst || !src) return set_error(NEURAL_ERR_NULL_POINTER);
    if (bytes % 16 != 0 || !aligned16(dst) || !aligned16(src) || !is_device_ptr(dst) || !is_device_ptr(src))
        return set_error(NEURAL_ERR_INVALID_ARGUMENT);
    NH_TRY(launch_map1_flat(static_cast<const float *>(src), static_cast<float *>(dst), int64_t(bytes / 4),
                            FnCopy{}));
    return set_error(NEURAL_OK);
}

}  // extern "C"
