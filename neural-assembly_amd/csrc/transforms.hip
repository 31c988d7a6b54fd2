// transforms.hip -- per-feature statistics and affine transforms over
// [batch, features] float64 data (row-major).
//
// Reference: transforms.c:27-143 (declared at neural_api.h:1115-1126, bound by
// pyneural/transforms.py).  transform_compute_stats: per feature, sum and sum
// of squares in double; min / max start at +1e308 / -1e308 and take a value
// only when it is strictly smaller / larger (NaN never enters, the first of
// equal values stays, values beyond the start value leave it); mean = sum / b,
// var = sum2 / b - mean^2 clamped at 0, std = sqrt(var).  The three maps:
// (x - mean) / (std + eps), x * (std + eps) + mean, (x - min) / (max - min + eps).
//
// Statistics: a column reduction.  Stage 1 launches (feature groups of 64) x
// (row chunks) blocks; a wave covers 64 features of a row, or, for fewer than
// 64 features, 64 / F whole rows, so every wave load is one contiguous span;
// each lane keeps (sum, sum2, min, first-min row, max, first-max row) in
// registers, the block folds its lanes in LDS and writes one partial per
// (chunk, feature).  Stage 2, one block per feature, folds its chunks in a
// fixed tree order and finishes the statistics.  Sums are summed in a different order than the
// reference's single pass (results within rounding); min / max are exact,
// including which zero sign is "first".
//
// Maps: one flat pass over 16-byte vectors (8 B read + 8 B written per
// element); the feature index of each lane advances by constants mod F, so no
// division runs in the loop.
#include <cmath>

#include "common.hpp"
#include "kernels.hpp"
#include "reduce_impl.hpp"

namespace nh {

constexpr int kTBlock = 256;
constexpr int kTUnroll = 4;
// Pairs per lane of the per-feature maps, each wave's 64 x kTMapU pairs
// contiguous (normalize at [1M, 64] / [1M, 6] f64: 165 / 171 us against
// 170 / 180 us for 4 pairs per lane strided by the block).
constexpr int kTMapU = 2;

struct ColState {
    double sum, sum2, mnv, mxv;
    int64_t mni, mxi;  // row of the min / max; INT64_MAX for the start values
};

NH_DEV ColState cs_init()
{
    return {0.0, 0.0, 1e308, -1e308, INT64_MAX, INT64_MAX};
}

// Rows arrive in increasing order within a lane: strict compares keep the first.
NH_DEV void cs_acc(ColState &s, double v, int64_t r)
{
    s.sum += v;
    const double q = v * v;
    s.sum2 += q;
    if (v < s.mnv) { s.mnv = v; s.mni = r; }
    if (v > s.mxv) { s.mxv = v; s.mxi = r; }
}

// Fold b into a (a's rows and b's rows interleave: ties go to the earlier row).
NH_DEV void cs_comb(ColState &a, const ColState &b)
{
    a.sum += b.sum;
    a.sum2 += b.sum2;
    if (b.mnv < a.mnv || (b.mnv == a.mnv && b.mni < a.mni)) { a.mnv = b.mnv; a.mni = b.mni; }
    if (b.mxv > a.mxv || (b.mxv == a.mxv && b.mxi < a.mxi)) { a.mxv = b.mxv; a.mxi = b.mxi; }
}

// Feature group fg (64 features, or all F < 64 with 64 / F rows per wave
// step) over row chunk blockIdx.y.
NH_DEV void colstats_group(const double *__restrict__ x, int64_t b, int64_t F, int64_t chunk,
                           ColState *__restrict__ part, int64_t fg, ColState *sh)
{
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int Wf = F >= 64 ? 64 : int(F);
    const int R = 64 / Wf;  // rows per wave step
    const int ro = lane / Wf;
    const int64_t f = fg * 64 + lane % Wf;
    const bool active = ro < R && f < F;
    const int64_t r0 = int64_t(blockIdx.y) * chunk;
    const int64_t r1 = r0 + chunk < b ? r0 + chunk : b;
    const int64_t step = 4 * int64_t(R);
    ColState s = cs_init();
    if (active) {
        int64_t r = r0 + int64_t(w) * R + ro;
        for (; r + (kTUnroll - 1) * step < r1; r += kTUnroll * step) {
            double v[kTUnroll];
#pragma unroll
            for (int u = 0; u < kTUnroll; u++) v[u] = ld_nt(x + (r + u * step) * F + f);
#pragma unroll
            for (int u = 0; u < kTUnroll; u++) cs_acc(s, v[u], r + u * step);
        }
        for (; r < r1; r += step) cs_acc(s, x[r * F + f], r);
    }
    sh[threadIdx.x] = s;
    __syncthreads();
    if (threadIdx.x < Wf && f < F) {
        ColState t = sh[threadIdx.x];
        for (int ww = 0; ww < kTBlock / 64; ww++)
            for (int rr = 0; rr < R; rr++)
                if (ww | rr) cs_comb(t, sh[ww * 64 + rr * Wf + threadIdx.x]);
        part[f * int64_t(gridDim.y) + blockIdx.y] = t;  // chunks of one feature contiguous
    }
    __syncthreads();  // sh is rewritten by the block's next feature group
}

// Feature groups step by the grid's width (capped at kMaxGridBlocks).
__global__ __launch_bounds__(kTBlock) void k_colstats(const double *__restrict__ x, int64_t b, int64_t F,
                                                       int64_t chunk, ColState *__restrict__ part)
{
    __shared__ ColState sh[kTBlock];
    const int64_t fgroups = (F + 63) / 64;
    for (int64_t fg = blockIdx.x; fg < fgroups; fg += gridDim.x) colstats_group(x, b, F, chunk, part, fg, sh);
}

struct ColRed {
    using B = ColState;
    NH_DEV B bident() const { return cs_init(); }
    NH_DEV B bcomb(B a, const B &b) const
    {
        cs_comb(a, b);
        return a;
    }
};

// One block per feature folds its chunk partials (an ordered tree: loads
// issued together, not one dependent load per chunk); features step by the
// grid's width (capped at kMaxGridBlocks).
__global__ __launch_bounds__(kRBlock) void k_colstats_final(const ColState *__restrict__ part, int64_t nchunks,
                                                             int64_t b, int64_t F, double *mean, double *std,
                                                             double *mn, double *mx)
{
    for (int64_t f = blockIdx.x; f < F; f += gridDim.x) {
        const ColState t = ordered_combine(ColRed{}, part + f * nchunks, int(nchunks));
        if (threadIdx.x == 0) {
            const double m = t.sum / double(b);
            const double m2 = m * m;
            double var = t.sum2 / double(b) - m2;
            if (var < 0.0) var = 0.0;
            if (mean) mean[f] = m;
            if (std) std[f] = sqrt(var);
            if (mn) mn[f] = t.mnv;
            if (mx) mx[f] = t.mxv;
        }
        __syncthreads();  // the combine's LDS is reused by the next feature
    }
}

enum { MAP_NORMALIZE = 0, MAP_UNNORMALIZE = 1, MAP_MINMAX = 2 };

template <int MODE>
NH_DEV double feat_map(double v, double a, double c, double eps)
{
    if constexpr (MODE == MAP_NORMALIZE) {
        return (v - a) / (c + eps);
    } else if constexpr (MODE == MAP_UNNORMALIZE) {
        const double s = v * (c + eps);
        return s + a;
    } else {
        const double range = c - a + eps;
        return (v - a) / range;
    }
}

// Pairs of elements (F even, 16-byte aligned): pair p holds features f, f+1
// with f = 2p mod F.  f advances by d1 = 128 mod F between unrolled slots (64
// pairs apart) and by dS = 2 * stride mod F between grid-stride steps.  FIXED
// (d1 = dS = 0, e.g. F = 64): a lane meets the same two features throughout,
// so their parameters are loaded once instead of with every vector (four
// parameter loads per 16-byte data load otherwise).
template <int MODE, bool FIXED>
__global__ __launch_bounds__(kTBlock) void k_feat_map2(const f64x2 *__restrict__ x, f64x2 *__restrict__ o,
                                                        int64_t n2, int64_t F, const double *__restrict__ A,
                                                        const double *__restrict__ C, double eps, int64_t d1,
                                                        int64_t dS)
{
    const int64_t tile = int64_t(kTBlock) * kTMapU;
    int64_t base = int64_t(blockIdx.x) * tile + (threadIdx.x >> 6) * (64 * kTMapU) + (threadIdx.x & 63);
    int64_t fb = (2 * base) % F;
    if constexpr (FIXED) {
        const double a0 = A[fb], a1 = A[fb + 1], c0 = C[fb], c1 = C[fb + 1];
        for (; base < n2; base += int64_t(gridDim.x) * tile) {
            f64x2 v[kTMapU];
#pragma unroll
            for (int u = 0; u < kTMapU; u++) {
                const int64_t i = base + int64_t(u) * 64;
                if (i < n2) v[u] = ld_nt(x + i);
            }
#pragma unroll
            for (int u = 0; u < kTMapU; u++) {
                const int64_t i = base + int64_t(u) * 64;
                if (i < n2) {
                    f64x2 r;
                    r[0] = feat_map<MODE>(v[u][0], a0, c0, eps);
                    r[1] = feat_map<MODE>(v[u][1], a1, c1, eps);
                    st_nt(o + i, r);
                }
            }
        }
        return;
    }
    for (; base < n2; base += int64_t(gridDim.x) * tile) {
        f64x2 v[kTMapU];
        int64_t fu[kTMapU];
        int64_t fc = fb;
#pragma unroll
        for (int u = 0; u < kTMapU; u++) {
            const int64_t i = base + int64_t(u) * 64;
            fu[u] = fc;
            if (i < n2) v[u] = ld_nt(x + i);
            fc += d1;
            if (fc >= F) fc -= F;
        }
#pragma unroll
        for (int u = 0; u < kTMapU; u++) {
            const int64_t i = base + int64_t(u) * 64;
            if (i < n2) {
                const int64_t f = fu[u];
                f64x2 r;
                r[0] = feat_map<MODE>(v[u][0], A[f], C[f], eps);
                r[1] = feat_map<MODE>(v[u][1], A[f + 1], C[f + 1], eps);
                st_nt(o + i, r);
            }
        }
        fb += dS;
        if (fb >= F) fb -= F;
    }
}

// One element per lane (odd F or unaligned buffers).
template <int MODE>
__global__ __launch_bounds__(kTBlock) void k_feat_map1(const double *__restrict__ x, double *__restrict__ o,
                                                        int64_t n, int64_t F, const double *__restrict__ A,
                                                        const double *__restrict__ C, double eps, int64_t dS)
{
    int64_t e = int64_t(blockIdx.x) * kTBlock + threadIdx.x;
    int64_t f = e % F;
    for (; e < n; e += int64_t(gridDim.x) * kTBlock) {
        o[e] = feat_map<MODE>(x[e], A[f], C[f], eps);
        f += dS;
        if (f >= F) f -= F;
    }
}

inline unsigned t_grid(int64_t work)
{
    int64_t g = ceil_div(work, kTBlock);
    const int64_t cap = kMaxGridBlocks;
    if (g > cap) g = cap;
    return unsigned(g < 1 ? 1 : g);
}

static int stats(const double *data, int64_t b, int64_t F, double *mean, double *std, double *mn, double *mx)
{
    if (!data || b <= 0 || F <= 0) return -1;
    if (ensure_init() != NEURAL_OK) return -1;
    const int64_t fgroups = ceil_div(F, 64);
    const int64_t R = F >= 64 ? 1 : 64 / F;
    // about 4 blocks per CU, each chunk at least 16 wave steps of rows
    int64_t nchunks = ceil_div(int64_t(num_cus()) * 4, fgroups);
    const int64_t max_chunks = ceil_div(b, 16 * 4 * R);
    if (nchunks > max_chunks) nchunks = max_chunks;
    if (nchunks > 65535) nchunks = 65535;
    if (nchunks < 1) nchunks = 1;
    const int64_t chunk = ceil_div(b, nchunks);
    nchunks = ceil_div(b, chunk);
    Staged sx, so[4];
    int64_t bf;
    if (__builtin_mul_overflow(b, F, &bf)) return -1;
    if (sx.open_n(data, uint64_t(bf), sizeof(double), true) != NEURAL_OK) return -1;
    double *outs[4] = {mean, std, mn, mx};
    double *douts[4] = {nullptr, nullptr, nullptr, nullptr};
    for (int k = 0; k < 4; k++) {
        if (!outs[k]) continue;
        if (so[k].open_n(outs[k], uint64_t(F), sizeof(double), false) != NEURAL_OK) return -1;
        douts[k] = static_cast<double *>(so[k].dev);
    }
    ColState *part = static_cast<ColState *>(dev_alloc(size_t(nchunks * F) * sizeof(ColState)));
    if (!part) return -1;
    const unsigned gx = unsigned(fgroups < kMaxGridBlocks ? fgroups : kMaxGridBlocks);
    const unsigned gf = unsigned(F < kMaxGridBlocks ? F : kMaxGridBlocks);
    NH_LAUNCH(k_colstats, dim3(gx, unsigned(nchunks)), dim3(kTBlock), 0, stream(),
                       static_cast<const double *>(sx.dev), b, F, chunk, part);
    NH_LAUNCH(k_colstats_final, dim3(gf), dim3(kRBlock), 0, stream(), part, nchunks, b, F, douts[0],
                       douts[1], douts[2], douts[3]);
    const int rc = check_launch();
    dev_free(part);
    if (rc != NEURAL_OK) return -1;
    for (int k = 0; k < 4; k++)
        if (outs[k] && so[k].finish(true) != NEURAL_OK) return -1;
    if (sx.finish(false) != NEURAL_OK) return -1;
    return 0;
}

template <int MODE>
static int feat_apply(const double *data, double *out, int64_t b, int64_t F, const double *p0, const double *p1,
                      double eps)
{
    if (!data || !out || !p0 || !p1) return -1;
    if (b <= 0 || F <= 0) return -1;
    if (ensure_init() != NEURAL_OK) return -1;
    int64_t n;
    if (__builtin_mul_overflow(b, F, &n)) return -1;
    Staged sx, so, s0, s1;
    if (sx.open_n(data, uint64_t(n), sizeof(double), true) != NEURAL_OK ||
        so.open_n(out, uint64_t(n), sizeof(double), false) != NEURAL_OK ||
        s0.open_n(p0, uint64_t(F), sizeof(double), true) != NEURAL_OK ||
        s1.open_n(p1, uint64_t(F), sizeof(double), true) != NEURAL_OK)
        return -1;
    const double *X = static_cast<const double *>(sx.dev);
    double *O = static_cast<double *>(so.dev);
    const double *A = static_cast<const double *>(s0.dev), *C = static_cast<const double *>(s1.dev);
    const bool vec = (F % 2 == 0) && ((reinterpret_cast<uintptr_t>(X) | reinterpret_cast<uintptr_t>(O)) & 15u) == 0;
    if (vec) {
        const int64_t n2 = n / 2;
        const unsigned g = t_grid(ceil_div(n2, kTMapU));
        const int64_t stride = int64_t(g) * kTBlock * kTMapU;
        const int64_t d1 = 128 % F, dS = (2 * stride) % F;
        if (d1 == 0 && dS == 0)
            NH_LAUNCH((k_feat_map2<MODE, true>), dim3(g), dim3(kTBlock), 0, stream(),
                               reinterpret_cast<const f64x2 *>(X), reinterpret_cast<f64x2 *>(O), n2, F, A, C, eps, d1,
                               dS);
        else
            NH_LAUNCH((k_feat_map2<MODE, false>), dim3(g), dim3(kTBlock), 0, stream(),
                               reinterpret_cast<const f64x2 *>(X), reinterpret_cast<f64x2 *>(O), n2, F, A, C, eps, d1,
                               dS);
    } else {
        const unsigned g = t_grid(n);
        NH_LAUNCH(k_feat_map1<MODE>, dim3(g), dim3(kTBlock), 0, stream(), X, O, n, F, A, C, eps,
                           (int64_t(g) * kTBlock) % F);
    }
    if (check_launch() != NEURAL_OK) return -1;
    if (so.finish(true) != NEURAL_OK || sx.finish(false) != NEURAL_OK || s0.finish(false) != NEURAL_OK ||
        s1.finish(false) != NEURAL_OK)
        return -1;
    return 0;
}

}  // namespace nh

using namespace nh;

extern "C" {

int transform_compute_stats(const double *data, int64_t batch_size, int64_t num_features, double *mean_out,
                            double *std_out, double *min_out, double *max_out)
{
    return stats(data, batch_size, num_features, mean_out, std_out, min_out, max_out);
}

int transform_normalize(const double *data, double *output, int64_t batch_size, int64_t num_features,
                        const double *mean, const double *std, double eps)
{
    return feat_apply<MAP_NORMALIZE>(data, output, batch_size, num_features, mean, std, eps);
}

int transform_unnormalize(const double *data, double *output, int64_t batch_size, int64_t num_features,
                          const double *mean, const double *std, double eps)
{
    return feat_apply<MAP_UNNORMALIZE>(data, output, batch_size, num_features, mean, std, eps);
}

int transform_minmax(const double *data, double *output, int64_t batch_size, int64_t num_features,
                     const double *min_val, const double *max_val, double eps)
{
    return feat_apply<MAP_MINMAX>(data, output, batch_size, num_features, min_val, max_val, eps);
}

}  // extern "C"
