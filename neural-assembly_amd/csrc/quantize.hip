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
#include <cstdio>
#include <cstdlib>
#include <mutex>

#include "quant_common.hpp"
#include "reduce_impl.hpp"

namespace nh {

// q = clamp((int32)round(x * inv) + zp, -128, 127) with the reference build's
// x86 semantics.  For |x * inv| <= 2^30 (everything but NaN and huge
// outliers) round() is trunc plus a +-1 step decided by the exact remainder,
// and no int32 operation can overflow; otherwise cvttsd2si (INT32_MIN) and the
// wrapping add are reproduced.
NH_DEV int8_t quant_one(double x, double inv, int32_t zp)
{
    const double y = x * inv;
    int32_t q;
    if (__builtin_fabs(y) <= 0x1p30) {
        const double t = __builtin_trunc(y);
        const double d = y - t;  // exact
        q = int32_t(t) + (d >= 0.5 ? 1 : 0) - (d <= -0.5 ? 1 : 0) + zp;
    } else {
        q = int32_t(uint32_t(x86_cvt_i32(round(y))) + uint32_t(zp));
    }
    q = q < -128 ? -128 : q;
    q = q > 127 ? 127 : q;
    return int8_t(q);
}


// The sequential loop keeps, for each of min and max, the FIRST element
// holding the extreme value; values that compare equal only differ in the
// sign of zero.  Lanes keep NaN-ignoring min and max in the input's
// precision (exact); a segment whose min or max is zero rescans itself for
// its first zero and takes that zero's sign.  Segment summaries combine in
// index order with the loop's strict compares, so an earlier segment wins
// ties.  d0 NaN makes both NaN (no later compare succeeds against NaN).
template <typename T>
struct RedMinMax {
    struct L { T mn, mx; };
    struct B { double mn, mx; };
    int symmetric = 0;
    NH_DEV L linit() const { return {inf_t<T>(), -inf_t<T>()}; }
    NH_DEV void lacc(L &s, T x, int64_t) const
    {
        s.mn = fmin_nn(s.mn, x);
        s.mx = fmax_nn(s.mx, x);
    }
    NH_DEV L lcomb(L a, L b) const { return {fmin_nn(a.mn, b.mn), fmax_nn(a.mx, b.mx)}; }
    template <int TPR>
    NH_DEV B finish(L s, const T *row, int64_t lo, int64_t hi) const
    {
        using G = Grp<TPR>;
        B b{double(s.mn), double(s.mx)};
        if (s.mn == T(0) || s.mx == T(0)) {
            int64_t fz = INT64_MAX;
            for (int64_t j = lo + G::lane(); j < hi; j += TPR) fz = (fz == INT64_MAX && row[j] == T(0)) ? j : fz;
            fz = G::min_i64(fz);
            const double z = double(row[fz]);
            if (s.mn == T(0)) b.mn = z;
            if (s.mx == T(0)) b.mx = z;
        }
        return b;
    }
    NH_DEV B bident() const { return {__builtin_inf(), -__builtin_inf()}; }
    NH_DEV B bcomb(B a, B b) const { return {b.mn < a.mn ? b.mn : a.mn, b.mx > a.mx ? b.mx : a.mx}; }
    NH_DEV void store(void *out, int64_t, B b, const T *row, int64_t) const
    {
        double mn = b.mn, mx = b.mx;
        const T first = row[0];
        if (first != first || mn > mx) mn = mx = __longlong_as_double(0x7ff8000000000000ll);
        minmax_epilogue(mn, mx, symmetric, static_cast<QuantParams *>(out));
    }
};

// Fused quantize -> dequantize -> squared error (and signal power).
struct QErrOut { double sig, noise; };
template <typename T>
struct RedQErr {
    using L = QErrOut;
    using B = QErrOut;
    double inv, scale;
    int32_t zp;
    NH_DEV L linit() const { return {0.0, 0.0}; }
    NH_DEV void lacc(L &s, T xv, int64_t) const
    {
        const double x = double(xv);
        s.sig += x * x;
        const int8_t q = quant_one(x, inv, zp);
        const double rec = (double(q) - double(zp)) * scale;
        const double d = x - rec;
        s.noise += d * d;
    }
    NH_DEV L lcomb(L a, L b) const { return {a.sig + b.sig, a.noise + b.noise}; }
    template <int TPR>
    NH_DEV B finish(L s, const T *, int64_t, int64_t) const { return s; }
    NH_DEV B bident() const { return linit(); }
    NH_DEV B bcomb(B a, B b) const { return lcomb(a, b); }
    NH_DEV void store(void *out, int64_t, B b, const T *, int64_t) const { *static_cast<QErrOut *>(out) = b; }
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

// Four elements per lane-step: a 16-byte f32 load (two for f64) becomes one
// packed 4-byte store.  Consecutive lanes take consecutive 4-element units, so
// every load and store instruction of a wave covers one contiguous span
// (1 KiB read, 256 B written for f32).  Tiles of 256 lanes x U units, all
// loads of a tile issued before its stores; accesses are non-temporal.
constexpr int kQUnroll = 4;
// f32 / f64 -> i8 (k_quantize): 2 units per lane with each wave's 128 units
// contiguous (the flat streams' layout): quantize at 268M f32 210 us against
// 215-217 us for 4 units per lane strided by the block (the same for 4 units
// wave-contiguous), parity unchanged.
constexpr int kQUnrollQ = 2;

template <typename T>
struct Quad;  // 4 consecutive elements
template <> struct Quad<float> {
    f32x4 v;
    NH_DEV static Quad load(const float *p, int64_t u) { return {ld_nt(reinterpret_cast<const f32x4 *>(p) + u)}; }
    NH_DEV void store(float *p, int64_t u) const { st_nt(reinterpret_cast<f32x4 *>(p) + u, v); }
    NH_DEV double get(int k) const { return double(v[k]); }
    NH_DEV void set(int k, double x) { v[k] = float(x); }
};
template <> struct Quad<double> {
    f64x2 a, b;
    NH_DEV static Quad load(const double *p, int64_t u)
    {
        const f64x2 *q = reinterpret_cast<const f64x2 *>(p) + 2 * u;
        return {ld_nt(q), ld_nt(q + 1)};
    }
    NH_DEV void store(double *p, int64_t u) const
    {
        f64x2 *q = reinterpret_cast<f64x2 *>(p) + 2 * u;
        st_nt(q, a);
        st_nt(q + 1, b);
    }
    NH_DEV double get(int k) const { return k < 2 ? a[k] : b[k - 2]; }
    NH_DEV void set(int k, double x)
    {
        if (k < 2) a[k] = x;
        else b[k - 2] = x;
    }
};

template <typename T>
__global__ __launch_bounds__(kQBlock) void k_quantize(const T *__restrict__ x, int8_t *__restrict__ q, int64_t n,
                                                      QArgs qa)
{
    double inv, scale;
    int32_t zp;
    load_q(qa, inv, scale, zp);
    const int64_t n4 = n / 4;
    uint32_t *q4 = reinterpret_cast<uint32_t *>(q);
    const int64_t tile = int64_t(kQBlock) * kQUnrollQ;
    for (int64_t base = int64_t(blockIdx.x) * tile + (threadIdx.x >> 6) * (64 * kQUnrollQ) + (threadIdx.x & 63);
         base < n4; base += int64_t(gridDim.x) * tile) {
        Quad<T> v[kQUnrollQ];
#pragma unroll
        for (int u = 0; u < kQUnrollQ; u++) {
            const int64_t i = base + int64_t(u) * 64;
            if (i < n4) v[u] = Quad<T>::load(x, i);
        }
#pragma unroll
        for (int u = 0; u < kQUnrollQ; u++) {
            const int64_t i = base + int64_t(u) * 64;
            if (i < n4) {
                uint32_t packed = 0;
#pragma unroll
                for (int k = 0; k < 4; k++) packed |= uint32_t(uint8_t(quant_one(v[u].get(k), inv, zp))) << (8 * k);
                __builtin_nontemporal_store(packed, q4 + i);
            }
        }
    }
    if (blockIdx.x == 0) {
        const int64_t j = n4 * 4 + threadIdx.x;
        if (j < n) q[j] = quant_one(double(x[j]), inv, zp);
    }
}

// f64 -> i8 with every load instruction of a wave reading one contiguous
// 1 KiB: a wave's 64 units (256 doubles) arrive as two 16-byte loads per lane,
// lane l holding doubles 2l, 2l+1 (first load) and 128+2l, 128+2l+1 (second).
// Each lane quantizes its four doubles; two lane shuffles regroup the codes so
// that lane m stores the packed word of unit m.  The loop is uniform per wave
// (all lanes take part in the shuffles); lanes past the end load nothing and
// store nothing.
__global__ __launch_bounds__(kQBlock) void k_quantize_f64w(const double *__restrict__ x, int8_t *__restrict__ q,
                                                           int64_t n, QArgs qa)
{
    double inv, scale;
    int32_t zp;
    load_q(qa, inv, scale, zp);
    const int lane = int(threadIdx.x & 63);
    const int64_t n4 = n / 4;
    uint32_t *q4 = reinterpret_cast<uint32_t *>(q);
    const f64x2 *xv = reinterpret_cast<const f64x2 *>(x);
    const int64_t tile = int64_t(kQBlock) * kQUnroll;
    for (int64_t wb = int64_t(blockIdx.x) * tile + (threadIdx.x & ~63u); wb < n4; wb += int64_t(gridDim.x) * tile) {
        f64x2 a[kQUnroll], b[kQUnroll];
#pragma unroll
        for (int u = 0; u < kQUnroll; u++) {
            const int64_t ub = wb + int64_t(u) * kQBlock;  // the wave's first unit for this u
            const bool in_a = ub + (lane >> 1) < n4, in_b = ub + 32 + (lane >> 1) < n4;
            if (in_a) a[u] = ld_nt(xv + 2 * ub + lane);
            if (in_b) b[u] = ld_nt(xv + 2 * ub + 64 + lane);
        }
#pragma unroll
        for (int u = 0; u < kQUnroll; u++) {
            const int64_t ub = wb + int64_t(u) * kQBlock;
            if (ub >= n4) break;  // uniform over the wave
            const bool in_a = ub + (lane >> 1) < n4, in_b = ub + 32 + (lane >> 1) < n4;
            uint32_t h = 0;  // codes of this lane's doubles: bytes 0-1 from a, 2-3 from b
            if (in_a)
                h |= uint32_t(uint8_t(quant_one(a[u][0], inv, zp))) | uint32_t(uint8_t(quant_one(a[u][1], inv, zp))) << 8;
            if (in_b)
                h |= uint32_t(uint8_t(quant_one(b[u][0], inv, zp))) << 16 |
                     uint32_t(uint8_t(quant_one(b[u][1], inv, zp))) << 24;
            // unit m = 4 doubles = the pair of lane 2m mod 64 and the pair of lane 2m+1 mod 64
            const uint32_t p0 = uint32_t(__shfl(int(h), (2 * lane) & 63, 64));
            const uint32_t p1 = uint32_t(__shfl(int(h), (2 * lane + 1) & 63, 64));
            const uint32_t word = lane < 32 ? ((p0 & 0xffffu) | (p1 << 16)) : ((p0 >> 16) | (p1 & 0xffff0000u));
            if (ub + lane < n4) __builtin_nontemporal_store(word, q4 + ub + lane);
        }
    }
    if (blockIdx.x == 0) {
        const int64_t j = n4 * 4 + threadIdx.x;
        if (j < n) q[j] = quant_one(x[j], inv, zp);
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

// Units per lane per tile of the write-heavy dequantize streams.  Fewer bytes
// written per lane per block write HBM faster here (a plain 2 GiB fill: 6.72
// TB/s with one 16-byte store per lane per block, 5.72 TB/s with four).
// Measured at 268M codes with the output rotating over three buffers (so no
// cache absorbs a rewrite): i8 -> f32 228 / 216 / 245 us for 4 / 2 / 1 units,
// i8 -> f64 448 / 394 / 387 us.  The read-heavy quantize keeps more than one
// unit (one unit: 217 -> 257 us).  k_dequantize takes its U units per lane
// wave-contiguous (i8 -> f32 215 -> 209 us against the block-strided layout).
constexpr int kDqUnrollF32 = 2;
constexpr int kDqUnrollF64 = 1;

template <typename T, int U>
__global__ __launch_bounds__(kQBlock) void k_dequantize(const int8_t *__restrict__ q, T *__restrict__ y, int64_t n,
                                                        QArgs qa)
{
    double inv, scale;
    int32_t zp;
    load_q(qa, inv, scale, zp);
    const double dz = double(zp);
    const int64_t n4 = n / 4;
    const uint32_t *q4 = reinterpret_cast<const uint32_t *>(q);
    const int64_t tile = int64_t(kQBlock) * U;
    for (int64_t base = int64_t(blockIdx.x) * tile + (threadIdx.x >> 6) * (64 * U) + (threadIdx.x & 63); base < n4;
         base += int64_t(gridDim.x) * tile) {
        uint32_t w[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int64_t i = base + int64_t(u) * 64;
            if (i < n4) w[u] = __builtin_nontemporal_load(q4 + i);
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int64_t i = base + int64_t(u) * 64;
            if (i < n4) {
                Quad<T> o;
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const int8_t b = int8_t(w[u] >> (8 * k));
                    o.set(k, (double(b) - dz) * scale);
                }
                o.store(y, i);
            }
        }
    }
    if (blockIdx.x == 0) {
        const int64_t j = n4 * 4 + threadIdx.x;
        if (j < n) y[j] = T((double(q[j]) - dz) * scale);
    }
}

// i8 -> f64 with every store instruction of a wave writing one contiguous
// 1 KiB (a lane writing its own unit's 32 bytes as two 16-byte stores would
// leave every store instruction touching half of each 32-byte sector it
// covers: measured 2.6 TB/s).  Lane m loads the packed codes of unit m; two
// lane shuffles hand lane l the codes of doubles 2l, 2l+1 and 128+2l,
// 128+2l+1 of the wave's 256.  The loop is uniform per wave.
template <int U>
__global__ __launch_bounds__(kQBlock) void k_dequantize_f64w(const int8_t *__restrict__ q, double *__restrict__ y,
                                                             int64_t n, QArgs qa)
{
    double inv, scale;
    int32_t zp;
    load_q(qa, inv, scale, zp);
    const double dz = double(zp);
    const int lane = int(threadIdx.x & 63);
    const int sh = (lane & 1) * 16;
    const int64_t n4 = n / 4;
    const uint32_t *q4 = reinterpret_cast<const uint32_t *>(q);
    f64x2 *yv = reinterpret_cast<f64x2 *>(y);
    const int64_t tile = int64_t(kQBlock) * U;
    for (int64_t wb = int64_t(blockIdx.x) * tile + (threadIdx.x & ~63u); wb < n4; wb += int64_t(gridDim.x) * tile) {
        uint32_t w[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int64_t i = wb + int64_t(u) * kQBlock + lane;
            w[u] = i < n4 ? __builtin_nontemporal_load(q4 + i) : 0u;
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int64_t ub = wb + int64_t(u) * kQBlock;
            if (ub >= n4) break;  // uniform over the wave
            const uint32_t lo = uint32_t(__shfl(int(w[u]), lane >> 1, 64));
            const uint32_t hi = uint32_t(__shfl(int(w[u]), 32 + (lane >> 1), 64));
            f64x2 a, b;
            a[0] = (double(int8_t(lo >> sh)) - dz) * scale;
            a[1] = (double(int8_t(lo >> (sh + 8))) - dz) * scale;
            b[0] = (double(int8_t(hi >> sh)) - dz) * scale;
            b[1] = (double(int8_t(hi >> (sh + 8))) - dz) * scale;
            if (ub + (lane >> 1) < n4) st_nt(yv + 2 * ub + lane, a);
            if (ub + 32 + (lane >> 1) < n4) st_nt(yv + 2 * ub + 64 + lane, b);
        }
    }
    if (blockIdx.x == 0) {
        const int64_t j = n4 * 4 + threadIdx.x;
        if (j < n) y[j] = (double(q[j]) - dz) * scale;
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

// Enough tiles for the whole range, capped at 32 blocks per CU (the
// grid-stride loop covers the rest).
inline unsigned q_grid(int64_t units, int64_t per_block)
{
    int64_t g = ceil_div(units, per_block);
    const int64_t cap = kMaxGridBlocks;
    if (g > cap) g = cap;
    return unsigned(g < 1 ? 1 : g);
}

template <typename T>
static int launch_quantize(const T *x, int8_t *q, int64_t n, QArgs qa)
{
    const bool vec = (reinterpret_cast<uintptr_t>(x) & 15u) == 0 && (reinterpret_cast<uintptr_t>(q) & 3u) == 0;
    if (vec && sizeof(T) == 8)
        NH_LAUNCH(k_quantize_f64w, dim3(q_grid(n / 4, kQBlock * kQUnroll)), dim3(kQBlock), 0, stream(),
                  reinterpret_cast<const double *>(x), q, n, qa);
    else if (vec)
        NH_LAUNCH((k_quantize<T>), dim3(q_grid(n / 4, kQBlock * kQUnrollQ)), dim3(kQBlock), 0, stream(), x,
                           q, n, qa);
    else
        NH_LAUNCH((k_quantize_scalar<T>), dim3(q_grid(n, kQBlock)), dim3(kQBlock), 0, stream(), x, q, n, qa);
    return check_launch();
}

template <typename T>
static int launch_dequantize(const int8_t *q, T *y, int64_t n, QArgs qa)
{
    const bool vec = (reinterpret_cast<uintptr_t>(y) & 15u) == 0 && (reinterpret_cast<uintptr_t>(q) & 3u) == 0;
    if (vec && sizeof(T) == 8)
        NH_LAUNCH(k_dequantize_f64w<kDqUnrollF64>, dim3(q_grid(n / 4, kQBlock * kDqUnrollF64)), dim3(kQBlock), 0,
                  stream(), q, reinterpret_cast<double *>(y), n, qa);
    else if (vec)
        NH_LAUNCH((k_dequantize<T, kDqUnrollF32>), dim3(q_grid(n / 4, kQBlock * kDqUnrollF32)), dim3(kQBlock), 0,
                  stream(), q, y, n, qa);
    else
        NH_LAUNCH((k_dequantize_scalar<T>), dim3(q_grid(n, kQBlock)), dim3(kQBlock), 0, stream(), q, y, n,
                           qa);
    return check_launch();
}

// ---- host wrappers -------------------------------------------------------------------

template <typename T>
static int calibrate(const T *data, int64_t n, int symmetric, QuantParams *out, bool out_on_device)
{
    if (ensure_init() != NEURAL_OK) return -1;
    if (!data || n <= 0 || !out) return -1;
    Staged s;
    if (s.open_n(data, uint64_t(n), sizeof(T), true) != NEURAL_OK) return -1;
    RedMinMax<T> red;
    red.symmetric = symmetric ? 1 : 0;
    WsGuard wg;
    if (out_on_device) {
        if (launch_reduce_full(static_cast<const T *>(s.dev), n, red, out) != NEURAL_OK) return -1;
    } else if (reduce_full_to_host(static_cast<const T *>(s.dev), n, red, out, sizeof(QuantParams)) != NEURAL_OK) {
        return -1;
    }
    if (s.finish(false) != NEURAL_OK) return -1;
    set_error(NEURAL_OK);
    return 0;
}

template <typename T>
static int quantize(const T *data, int8_t *out, int64_t n, const QuantParams *p, bool p_on_device)
{
    if (ensure_init() != NEURAL_OK) return -1;
    if (!data || !out || n <= 0 || !p) return -1;
    Staged si, so;
    if (si.open_n(data, uint64_t(n), sizeof(T), true) != NEURAL_OK || so.open_n(out, uint64_t(n), 1, false) != NEURAL_OK)
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
    if (si.open_n(data, uint64_t(n), 1, true) != NEURAL_OK || so.open_n(out, uint64_t(n), sizeof(T), false) != NEURAL_OK)
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
    if (s.open_n(data, uint64_t(n), sizeof(T), true) != NEURAL_OK) return -1;
    RedQErr<T> red;
    red.scale = p->scale;
    red.inv = 1.0 / p->scale;
    red.zp = p->zero_point;
    WsGuard wg;
    QErrOut st;
    if (reduce_full_to_host(static_cast<const T *>(s.dev), n, red, &st, sizeof(st)) != NEURAL_OK) return -1;
    if (s.finish(false) != NEURAL_OK) return -1;
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

// ---- calibration without allocation ----------------------------------------------------

// Segment summaries of calibrate_minmax_f32_dev_noalloc live in this static
// device array, one copy per GPU, kept until the process ends.  Host code
// never passes the array's name to a kernel (on the host it is only a
// stand-in for the symbol); it uses the device address that
// hipGetSymbolAddress returned for that GPU at initialisation.
constexpr size_t kScratchBytes = size_t(64) << 10;  // 4096 summaries of 16 bytes: 16 per CU on 256 CUs
constexpr int kMaxScratchDevices = 64;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];
static void *g_scratch_ptr[kMaxScratchDevices];
static std::mutex g_scratch_mu;

int setup_static_scratch(int device)
{
    if (device < 0 || device >= kMaxScratchDevices) return NEURAL_ERR_INTERNAL;
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
        if (std::getenv("NEURAL_HIP_VERBOSE"))
            std::fprintf(stderr, "libneural_hip: hipGetSymbolAddress(scratch) failed: %s\n", hipGetErrorString(e));
        return NEURAL_ERR_INTERNAL;
    }
    g_scratch_ptr[device] = p;
    return NEURAL_OK;
}

static int calibrate_noalloc(const float *data, int64_t n, int symmetric, QuantParams *dev_params)
{
    if (!data || !dev_params) return set_error(NEURAL_ERR_NULL_POINTER);
    if (n <= 0) return set_error(NEURAL_ERR_INVALID_ARGUMENT);
    NH_TRY(ensure_ready());
    int dev = -1;
    NH_HIP(hipGetDevice(&dev));
    void *scr = (dev >= 0 && dev < kMaxScratchDevices) ? g_scratch_ptr[dev] : nullptr;
    if (!scr) return set_error(NEURAL_ERR_INVALID_CONFIG);
    // host buffers would need staging copies, i.e. an allocation
    if (!is_device_ptr(data) || !is_device_ptr(dev_params)) return set_error(NEURAL_ERR_INVALID_ARGUMENT);
    RedMinMax<float> red;
    red.symmetric = symmetric ? 1 : 0;
    // Held while the two launches are enqueued: later calls on the stream run
    // after this call's combine has read the summaries.
    std::lock_guard<std::mutex> g(g_scratch_mu);
    NH_TRY(launch_reduce(data, 1, n, n, red, dev_params, scr, kScratchBytes));
    return NEURAL_OK;
}

}  // namespace nh

using namespace nh;

static_assert(sizeof(QuantParams) == 40, "QuantParams must keep the reference's 40-byte layout");

extern "C" {

int calibrate_minmax(const double *d, int64_t n, int sym, QuantParams *o) { return calibrate(d, n, sym, o, false); }
int calibrate_minmax_f32(const float *d, int64_t n, int sym, QuantParams *o) { return calibrate(d, n, sym, o, false); }
int calibrate_minmax_f32_dev(const float *d, int64_t n, int sym, QuantParams *o) { return calibrate(d, n, sym, o, true); }
int calibrate_minmax_f32_dev_noalloc(const float *d, int64_t n, int sym, QuantParams *o)
{
    if (calibrate_noalloc(d, n, sym, o) != NEURAL_OK) return -1;
    set_error(NEURAL_OK);
    return 0;
}

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
