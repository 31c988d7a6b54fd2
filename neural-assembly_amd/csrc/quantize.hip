// quantize.hip -- INT8 calibration, quantization and dequantization.
//
// Reference: quantize.c:52-84 (calibrate_minmax), 144-158 (quantize_tensor),
// 163-174 (dequantize_tensor), 222-269 (quantization_error / _snr).
//   calibrate: mn = mx = d0; mn = d_i if d_i < mn; mx = d_i if d_i > mx, then
//              the scalar symmetric/affine epilogue.  Here: one grid reduction
//              of (min, max) that reproduces the loop's values and zero signs
//              (NaNs ignored unless d0 is NaN), and the epilogue evaluated on
//              the device by the last block with the same double expressions,
//              so params never round-trip through the host in the device
//              pipeline.
//   quantize:  q = (int32)round(x * (1.0/scale)) + zp, clamp [-128, 127].  The
//              int32 conversion reproduces x86 cvttsd2si (INT32_MIN for NaN and
//              out-of-range) and the wrap-around add of the reference build.
//   dequantize: ((double)q - (double)zp) * scale.
#include <cmath>

#include "reduce_impl.hpp"

namespace nh {

// cvttsd2si of an already-rounded double.
NH_DEV int32_t x86_cvt_i32(double r)
{
    if (!(r > -2147483649.0 && r < 2147483648.0)) return int32_t(0x80000000u);
    return int32_t(r);
}

NH_DEV int8_t quant_one(double x, double inv, int32_t zp)
{
    int32_t q = int32_t(uint32_t(x86_cvt_i32(round(x * inv))) + uint32_t(zp));
    q = q < -128 ? -128 : q;
    q = q > 127 ? 127 : q;
    return int8_t(q);
}

NH_DEV void minmax_epilogue(double mn, double mx, int symmetric, QuantParams *out)
{
    QuantParams p;
    p.zero_point = 0;
    if (symmetric) {
        double am = fmax(fabs(mn), fabs(mx));
        if (am < 1e-30) am = 1e-30;
        p.scale = am / 127.0;
        p.zero_point = 0;
        p.min_val = -am;
        p.max_val = am;
        p.symmetric = 1;
    } else {
        if (mn == mx) { mn -= 0.5; mx += 0.5; }
        p.scale = (mx - mn) / 255.0;
        if (p.scale < 1e-30) p.scale = 1e-30;
        int32_t zp = x86_cvt_i32(round(-128.0 - mn / p.scale));
        if (zp < -128) zp = -128;
        if (zp > 127) zp = 127;
        p.zero_point = zp;
        p.min_val = mn;
        p.max_val = mx;
        p.symmetric = 0;
    }
    *out = p;
}

// The sequential loop keeps, for each of min and max, the FIRST element
// holding the extreme value; values that compare equal only differ in the
// sign of zero.  Reduction state: NaN-ignoring min and max values and the
// index of the first zero (each lane walks increasing indices, so "first" is
// a one-time capture per lane and a min across lanes).  The epilogue re-reads
// that zero for its sign, and d0 for the NaN case (d0 NaN makes both NaN).
template <typename T>
struct RedMinMax {
    struct S { double mn, mx; int64_t zfirst; };
    static constexpr bool kSuffixPass = false;
    static constexpr int64_t kNone = INT64_MAX;
    int symmetric;
    const T *x;
    NH_DEV S init() const { return {__builtin_inf(), -__builtin_inf(), kNone}; }
    NH_DEV void acc(S &s, double v, int64_t i) const
    {
        s.mn = __builtin_fmin(s.mn, v);
        s.mx = __builtin_fmax(s.mx, v);
        s.zfirst = (v == 0.0 && s.zfirst == kNone) ? i : s.zfirst;
    }
    NH_DEV S comb(S a, S b) const
    {
        return {__builtin_fmin(a.mn, b.mn), __builtin_fmax(a.mx, b.mx), a.zfirst < b.zfirst ? a.zfirst : b.zfirst};
    }
    NH_DEV S shfl(S a, int off) const
    {
        return {__shfl_xor(a.mn, off, 64), __shfl_xor(a.mx, off, 64), __shfl_xor(a.zfirst, off, 64)};
    }
    NH_DEV void store(void *out, S s) const
    {
        double mn = s.mn, mx = s.mx;
        if (s.zfirst != kNone) {
            const double z = double(x[s.zfirst]);
            if (mn == 0.0) mn = z;
            if (mx == 0.0) mx = z;
        }
        const T first = x[0];
        if (first != first || mn > mx) mn = mx = __longlong_as_double(0x7ff8000000000000ll);
        minmax_epilogue(mn, mx, symmetric, static_cast<QuantParams *>(out));
    }
};

// Fused quantize -> dequantize -> squared error (and signal power).
struct RedQErr {
    struct S { double sig, noise; };
    static constexpr bool kSuffixPass = false;
    double inv, scale;
    int32_t zp;
    NH_DEV S init() const { return {0.0, 0.0}; }
    NH_DEV void acc(S &s, double x, int64_t) const
    {
        s.sig += x * x;
        const int8_t q = quant_one(x, inv, zp);
        const double rec = (double(q) - double(zp)) * scale;
        const double d = x - rec;
        s.noise += d * d;
    }
    NH_DEV S comb(S a, S b) const { return {a.sig + b.sig, a.noise + b.noise}; }
    NH_DEV S shfl(S a, int off) const { return {__shfl_xor(a.sig, off, 64), __shfl_xor(a.noise, off, 64)}; }
    NH_DEV void store(void *out, S s) const { *static_cast<S *>(out) = s; }
};

// Params either by value or from device memory (device pipeline).
struct QArgs {
    double scale;
    int32_t zp;
    const QuantParams *dev;
};

NH_DEV void load_q(const QArgs &a, double &inv, double &scale, int32_t &zp)
{
    if (a.dev) { scale = a.dev->scale; zp = a.dev->zero_point; }
    else { scale = a.scale; zp = a.zp; }
    inv = 1.0 / scale;
}

constexpr int kQBlock = 256;

// 16 elements per thread-step: four 4 x f32 (or eight 2 x f64) loads and one
// 16-byte store, all non-temporal.
template <typename T>
__global__ __launch_bounds__(kQBlock) void k_quantize(const T *__restrict__ x, int8_t *__restrict__ q, int64_t n,
                                                      QArgs qa)
{
    using V = typename Vec16<T>::type;
    constexpr int VN = Vec16<T>::n;
    constexpr int NV = 16 / VN;
    double inv, scale;
    int32_t zp;
    load_q(qa, inv, scale, zp);
    const int64_t n16 = n / 16;
    const int64_t stride = int64_t(gridDim.x) * kQBlock;
    for (int64_t i = int64_t(blockIdx.x) * kQBlock + threadIdx.x; i < n16; i += stride) {
        const V *xv = reinterpret_cast<const V *>(x + i * 16);
        V v[NV];
#pragma unroll
        for (int k = 0; k < NV; k++) v[k] = ld_nt(xv + k);
        i32x4 w;
#pragma unroll
        for (int word = 0; word < 4; word++) {
            uint32_t packed = 0;
#pragma unroll
            for (int b = 0; b < 4; b++) {
                const int e = word * 4 + b;
                packed |= uint32_t(uint8_t(quant_one(double(v[e / VN][e % VN]), inv, zp))) << (8 * b);
            }
            w[word] = int(packed);
        }
        st_nt(reinterpret_cast<i32x4 *>(q) + i, w);
    }
    if (blockIdx.x == 0) {
        const int64_t j = n16 * 16 + threadIdx.x;
        if (j < n) q[j] = quant_one(double(x[j]), inv, zp);
    }
}

template <typename T>
__global__ __launch_bounds__(kQBlock) void k_quantize_scalar(const T *x, int8_t *q, int64_t n, QArgs qa)
{
    double inv, scale;
    int32_t zp;
    load_q(qa, inv, scale, zp);
    const int64_t stride = int64_t(gridDim.x) * kQBlock;
    for (int64_t i = int64_t(blockIdx.x) * kQBlock + threadIdx.x; i < n; i += stride)
        q[i] = quant_one(double(x[i]), inv, zp);
}

template <typename T>
__global__ __launch_bounds__(kQBlock) void k_dequantize(const int8_t *__restrict__ q, T *__restrict__ y, int64_t n,
                                                        QArgs qa)
{
    using V = typename Vec16<T>::type;
    constexpr int VN = Vec16<T>::n;
    constexpr int NV = 16 / VN;
    double inv, scale;
    int32_t zp;
    load_q(qa, inv, scale, zp);
    const double dz = double(zp);
    const int64_t n16 = n / 16;
    const int64_t stride = int64_t(gridDim.x) * kQBlock;
    for (int64_t i = int64_t(blockIdx.x) * kQBlock + threadIdx.x; i < n16; i += stride) {
        const i32x4 w = ld_nt(reinterpret_cast<const i32x4 *>(q) + i);
        V *yv = reinterpret_cast<V *>(y + i * 16);
#pragma unroll
        for (int k = 0; k < NV; k++) {
            V o;
#pragma unroll
            for (int j = 0; j < VN; j++) {
                const int e = k * VN + j;
                const int8_t b = int8_t(uint32_t(w[e / 4]) >> (8 * (e % 4)));
                o[j] = T((double(b) - dz) * scale);
            }
            st_nt(yv + k, o);
        }
    }
    if (blockIdx.x == 0) {
        const int64_t j = n16 * 16 + threadIdx.x;
        if (j < n) y[j] = T((double(q[j]) - dz) * scale);
    }
}

template <typename T>
__global__ __launch_bounds__(kQBlock) void k_dequantize_scalar(const int8_t *q, T *y, int64_t n, QArgs qa)
{
    double inv, scale;
    int32_t zp;
    load_q(qa, inv, scale, zp);
    const int64_t stride = int64_t(gridDim.x) * kQBlock;
    for (int64_t i = int64_t(blockIdx.x) * kQBlock + threadIdx.x; i < n; i += stride)
        y[i] = T((double(q[i]) - double(zp)) * scale);
}

inline unsigned q_grid(int64_t work)
{
    int64_t g = ceil_div(work, kQBlock);
    const int64_t cap = int64_t(num_cus()) * 32;
    if (g > cap) g = cap;
    return unsigned(g < 1 ? 1 : g);
}

template <typename T>
static int launch_quantize(const T *x, int8_t *q, int64_t n, QArgs qa)
{
    const bool vec = ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(q)) & 15u) == 0;
    if (vec) hipLaunchKernelGGL((k_quantize<T>), dim3(q_grid(n / 16)), dim3(kQBlock), 0, stream(), x, q, n, qa);
    else hipLaunchKernelGGL((k_quantize_scalar<T>), dim3(q_grid(n)), dim3(kQBlock), 0, stream(), x, q, n, qa);
    return check_launch();
}

template <typename T>
static int launch_dequantize(const int8_t *q, T *y, int64_t n, QArgs qa)
{
    const bool vec = ((reinterpret_cast<uintptr_t>(y) | reinterpret_cast<uintptr_t>(q)) & 15u) == 0;
    if (vec) hipLaunchKernelGGL((k_dequantize<T>), dim3(q_grid(n / 16)), dim3(kQBlock), 0, stream(), q, y, n, qa);
    else hipLaunchKernelGGL((k_dequantize_scalar<T>), dim3(q_grid(n)), dim3(kQBlock), 0, stream(), q, y, n, qa);
    return check_launch();
}

// ---- host wrappers -------------------------------------------------------------------

template <typename T>
static int calibrate(const T *data, int64_t n, int symmetric, QuantParams *out, bool out_on_device)
{
    if (ensure_init() != NEURAL_OK) return -1;
    if (!data || n <= 0 || !out) return -1;
    Staged s;
    if (s.open(data, size_t(n) * sizeof(T), true) != NEURAL_OK) return -1;
    RedMinMax<T> red;
    red.symmetric = symmetric ? 1 : 0;
    red.x = static_cast<const T *>(s.dev);
    void *res = out_on_device ? static_cast<void *>(out) : workspace().result;
    if (launch_reduce_full(static_cast<const T *>(s.dev), n, red, res) != NEURAL_OK) return -1;
    if (!out_on_device && hipMemcpyAsync(out, res, sizeof(QuantParams), hipMemcpyDeviceToHost, stream()) != hipSuccess)
        return -1;
    if (s.finish(false) != NEURAL_OK || (!out_on_device && sync() != NEURAL_OK)) return -1;
    set_error(NEURAL_OK);
    return 0;
}

template <typename T>
static int quantize(const T *data, int8_t *out, int64_t n, const QuantParams *p, bool p_on_device)
{
    if (ensure_init() != NEURAL_OK) return -1;
    if (!data || !out || n <= 0 || !p) return -1;
    Staged si, so;
    if (si.open(data, size_t(n) * sizeof(T), true) != NEURAL_OK || so.open(out, size_t(n), false) != NEURAL_OK)
        return -1;
    QArgs qa{0.0, 0, nullptr};
    if (p_on_device) qa.dev = p;
    else { qa.scale = p->scale; qa.zp = p->zero_point; }
    if (launch_quantize(static_cast<const T *>(si.dev), static_cast<int8_t *>(so.dev), n, qa) != NEURAL_OK) return -1;
    if (so.finish(true) != NEURAL_OK || si.finish(false) != NEURAL_OK) return -1;
    set_error(NEURAL_OK);
    return 0;
}

template <typename T>
static int dequantize(const int8_t *data, T *out, int64_t n, const QuantParams *p, bool p_on_device)
{
    if (ensure_init() != NEURAL_OK) return -1;
    if (!data || !out || n <= 0 || !p) return -1;
    Staged si, so;
    if (si.open(data, size_t(n), true) != NEURAL_OK || so.open(out, size_t(n) * sizeof(T), false) != NEURAL_OK)
        return -1;
    QArgs qa{0.0, 0, nullptr};
    if (p_on_device) qa.dev = p;
    else { qa.scale = p->scale; qa.zp = p->zero_point; }
    if (launch_dequantize(static_cast<const int8_t *>(si.dev), static_cast<T *>(so.dev), n, qa) != NEURAL_OK) return -1;
    if (so.finish(true) != NEURAL_OK || si.finish(false) != NEURAL_OK) return -1;
    set_error(NEURAL_OK);
    return 0;
}

template <typename T>
static int qerr(const T *data, int64_t n, const QuantParams *p, double *sig, double *noise)
{
    if (ensure_init() != NEURAL_OK) return -1;
    Staged s;
    if (s.open(data, size_t(n) * sizeof(T), true) != NEURAL_OK) return -1;
    RedQErr red;
    red.scale = p->scale;
    red.inv = 1.0 / p->scale;
    red.zp = p->zero_point;
    RedQErr::S st;
    void *res = workspace().result;
    if (launch_reduce_full(static_cast<const T *>(s.dev), n, red, res) != NEURAL_OK) return -1;
    if (hipMemcpyAsync(&st, res, sizeof(st), hipMemcpyDeviceToHost, stream()) != hipSuccess) return -1;
    if (s.finish(false) != NEURAL_OK || sync() != NEURAL_OK) return -1;
    *sig = st.sig;
    *noise = st.noise;
    set_error(NEURAL_OK);
    return 0;
}

template <typename T>
static double quant_error(const T *d, int64_t n, const QuantParams *p)
{
    if (!d || n <= 0 || !p) return -1.0;
    double sig, noise;
    if (qerr(d, n, p, &sig, &noise) != 0) return -1.0;
    return noise / double(n);
}

template <typename T>
static double quant_snr(const T *d, int64_t n, const QuantParams *p)
{
    if (!d || n <= 0 || !p) return -1.0;
    double sig, noise;
    if (qerr(d, n, p, &sig, &noise) != 0) return -1.0;
    if (noise < 1e-30) return 999.0;
    return 10.0 * std::log10(sig / noise);
}

}  // namespace nh

using namespace nh;

static_assert(sizeof(QuantParams) == 40, "QuantParams must keep the reference's 40-byte layout");

extern "C" {

int calibrate_minmax(const double *d, int64_t n, int sym, QuantParams *o) { return calibrate(d, n, sym, o, false); }
int calibrate_minmax_f32(const float *d, int64_t n, int sym, QuantParams *o) { return calibrate(d, n, sym, o, false); }
int calibrate_minmax_f32_dev(const float *d, int64_t n, int sym, QuantParams *o) { return calibrate(d, n, sym, o, true); }

int quantize_tensor(const double *d, int8_t *o, int64_t n, const QuantParams *p) { return quantize(d, o, n, p, false); }
int quantize_tensor_f32(const float *d, int8_t *o, int64_t n, const QuantParams *p) { return quantize(d, o, n, p, false); }
int quantize_tensor_f32_dev(const float *d, int8_t *o, int64_t n, const QuantParams *p) { return quantize(d, o, n, p, true); }

int dequantize_tensor(const int8_t *d, double *o, int64_t n, const QuantParams *p) { return dequantize(d, o, n, p, false); }
int dequantize_tensor_f32(const int8_t *d, float *o, int64_t n, const QuantParams *p) { return dequantize(d, o, n, p, false); }
int dequantize_tensor_f32_dev(const int8_t *d, float *o, int64_t n, const QuantParams *p) { return dequantize(d, o, n, p, true); }

double quantization_error(const double *d, int64_t n, const QuantParams *p) { return quant_error(d, n, p); }
double quantization_snr(const double *d, int64_t n, const QuantParams *p) { return quant_snr(d, n, p); }
double quantization_error_f32(const float *d, int64_t n, const QuantParams *p) { return quant_error(d, n, p); }
double quantization_snr_f32(const float *d, int64_t n, const QuantParams *p) { return quant_snr(d, n, p); }

}  // extern "C"
