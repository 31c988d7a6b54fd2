// ew_impl.hpp -- streaming elementwise machinery for gfx950.
//
// Flat kernels move 128-bit vectors (4 x f32 / 2 x f64) with non-temporal
// loads and stores, grid-striding over tiles of 256*U vectors; block 0
// finishes the n % VN tail.  Inputs that are not 16-byte aligned take the
// scalar variant.  Strided / broadcast operands
// (up to 4 dims after merging) take the N-D kernel with per-element index
// decomposition.
#pragma once

#include <type_traits>

#include "common.hpp"

namespace nh {

constexpr int kBlock = 256;
constexpr int kUnroll = 4;
// Vectors per lane of the row-broadcast kernel: a [8192,4096] bias add between
// a log-softmax and four row reductions took 45.5 / 45.1 / 46.6 us with 4 / 2 /
// 1 (A/B in one run).
constexpr int kRowU = 2;
// Flat kernels: U vectors per lane per tile, and a wave's 64 U vectors are
// contiguous (lane l of wave w takes vectors w 64 U + u 64 + l): each wave
// streams one contiguous span.
constexpr int kFlatU = 2;

// First vector of the calling lane in the flat tile that starts at vector t0.
NH_DEV int64_t flat_lane0(int64_t t0) { return t0 + int64_t(threadIdx.x >> 6) * (64 * kFlatU) + (threadIdx.x & 63); }

inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ---- flat binary ----------------------------------------------------------
// Grid-stride over tiles of 256 * kFlatU vectors (flat_lane0 layout); per
// tile every lane issues its loads of both operands before any arithmetic or
// store.  All accesses are non-temporal.  Block 0 also finishes the n % VN
// tail.
template <typename T, typename Op>
__global__ __launch_bounds__(kBlock) void k_map2_flat(const T *__restrict__ a, const T *__restrict__ b,
                                                      T *__restrict__ o, int64_t n, Op op)
{
    using V = typename Vec16<T>::type;
    constexpr int VN = Vec16<T>::n;
    const int64_t nv = n / VN;
    const V *av = reinterpret_cast<const V *>(a);
    const V *bv = reinterpret_cast<const V *>(b);
    V *ov = reinterpret_cast<V *>(o);
    const int64_t step = int64_t(gridDim.x) * (kBlock * kFlatU);
    for (int64_t base = flat_lane0(int64_t(blockIdx.x) * (kBlock * kFlatU)); base < nv; base += step) {
        V ra[kFlatU], rb[kFlatU];
#pragma unroll
        for (int u = 0; u < kFlatU; u++) {
            const int64_t i = base + int64_t(u) * 64;
            if (i < nv) { ra[u] = ld_nt(av + i); rb[u] = ld_nt(bv + i); }
        }
#pragma unroll
        for (int u = 0; u < kFlatU; u++) {
            const int64_t i = base + int64_t(u) * 64;
            if (i < nv) {
                V r;
#pragma unroll
                for (int k = 0; k < VN; k++) r[k] = op(ra[u][k], rb[u][k]);
                st_nt(ov + i, r);
            }
        }
    }
    if (blockIdx.x == 0) {
        const int64_t j = nv * VN + threadIdx.x;
        if (j < n) o[j] = op(a[j], b[j]);
    }
}

template <typename T, typename Op>
__global__ __launch_bounds__(kBlock) void k_map2_flat_scalar(const T *a, const T *b, T *o, int64_t n, Op op)
{
    const int64_t stride = int64_t(gridDim.x) * kBlock;
    for (int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride) o[i] = op(a[i], b[i]);
}

// ---- flat unary (same element width in and out) ----------------------------
template <typename T, typename F>
__global__ __launch_bounds__(kBlock) void k_map1_flat(const T *__restrict__ a, T *__restrict__ o, int64_t n, F f)
{
    using V = typename Vec16<T>::type;
    constexpr int VN = Vec16<T>::n;
    const int64_t nv = n / VN;
    const V *av = reinterpret_cast<const V *>(a);
    V *ov = reinterpret_cast<V *>(o);
    const int64_t step = int64_t(gridDim.x) * (kBlock * kFlatU);
    for (int64_t base = flat_lane0(int64_t(blockIdx.x) * (kBlock * kFlatU)); base < nv; base += step) {
        V ra[kFlatU];
#pragma unroll
        for (int u = 0; u < kFlatU; u++) {
            const int64_t i = base + int64_t(u) * 64;
            if (i < nv) ra[u] = ld_nt(av + i);
        }
#pragma unroll
        for (int u = 0; u < kFlatU; u++) {
            const int64_t i = base + int64_t(u) * 64;
            if (i < nv) {
                V r;
#pragma unroll
                for (int k = 0; k < VN; k++) r[k] = f(ra[u][k]);
                st_nt(ov + i, r);
            }
        }
    }
    if (blockIdx.x == 0) {
        const int64_t j = nv * VN + threadIdx.x;
        if (j < n) o[j] = f(a[j]);
    }
}

template <typename T, typename F>
__global__ __launch_bounds__(kBlock) void k_map1_flat_scalar(const T *a, T *o, int64_t n, F f)
{
    const int64_t stride = int64_t(gridDim.x) * kBlock;
    for (int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride) o[i] = f(a[i]);
}

// ---- flat unary f32 with a rare expensive path ------------------------------
// F supplies head(x, need) -- the cheap evaluation, run for every element,
// which also says whether the element needs the expensive one -- and
// tail(x).  Per tile each lane keeps a bit mask of its elements that need the
// tail (no cross-lane work per element).  A wave with any such element counts
// them with five ballots (an exclusive prefix sum over the lanes via mbcnt),
// packs them into its LDS queue in (lane, element) order, runs tail() over the
// queue 64 at a time and puts the results back, so the tail costs one pass per
// 64 queued elements instead of one pass per element position that any lane
// needs.  The tile loop is block-uniform; the wave's queue holds a full tile.
// 16-byte vectors per lane per tile.  Measured on the cfg3 input: 2 (8
// elements per lane) beats 4, whose twice as many live values and the
// inlined double tail cut residency (gelu 87 -> 380 us, mish 82 -> 254 us).
constexpr int kTailUnroll = 2;

// Exclusive prefix sum over the wave of c in [0, 32), and the wave's total,
// from one ballot per bit of c.
NH_DEV int wave_excl_prefix_small(int c, int &total)
{
    int pre = 0;
    total = 0;
#pragma unroll
    for (int b = 0; b < 5; b++) {
        const uint64_t m = __ballot((c >> b) & 1);
        pre += int(__builtin_amdgcn_mbcnt_hi(uint32_t(m >> 32), __builtin_amdgcn_mbcnt_lo(uint32_t(m), 0u))) << b;
        total += __popcll(m) << b;
    }
    return pre;
}

// ROW: the input element is x + bias[column] in float (the rounding
// neural_bias_add does), [rows, ncv] vectors with the bias vector of `ncv`;
// a lane's column vector index is found once by a division and then advanced
// by d1 = 256 mod ncv per vector and dS = grid stride mod ncv per tile.
template <typename F, bool ROW = false>
__global__ __launch_bounds__(kBlock) void k_map1_f32_tail(const float *__restrict__ a, float *__restrict__ o,
                                                          int64_t n, F f, const float *__restrict__ bias = nullptr,
                                                          int64_t ncv = 1, int64_t d1 = 0, int64_t dS = 0)
{
    constexpr int U = kTailUnroll;
    constexpr int PL = U * 4;  // elements per lane per tile
    static_assert(PL < 32, "the per-lane count must fit wave_excl_prefix_small");
    __shared__ float queue[kBlock / 64][64 * PL];
    float *wq = queue[threadIdx.x >> 6];
    const int lane = threadIdx.x & 63;
    const int64_t nv = n / 4;
    const f32x4 *av = reinterpret_cast<const f32x4 *>(a);
    const f32x4 *bv = reinterpret_cast<const f32x4 *>(bias);
    f32x4 *ov = reinterpret_cast<f32x4 *>(o);
    const int64_t tile = int64_t(kBlock) * U;
    int64_t c = ROW ? (int64_t(blockIdx.x) * tile + threadIdx.x) % ncv : 0;
    for (int64_t t0 = int64_t(blockIdx.x) * tile; t0 < nv; t0 += int64_t(gridDim.x) * tile) {
        f32x4 x[U], r[U];
        int64_t cc = c;
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int64_t i = t0 + int64_t(u) * kBlock + threadIdx.x;
            x[u] = i < nv ? ld_nt(av + i) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            if constexpr (ROW) {
                if (i < nv) x[u] = x[u] + bv[cc];
                cc += d1;
                cc = cc >= ncv ? cc - ncv : cc;
            }
        }
        if constexpr (ROW) {
            c += dS;
            c = c >= ncv ? c - ncv : c;
        }
        uint32_t nm = 0;  // bit u*4+k: element k of vector u needs the tail
#pragma unroll
        for (int u = 0; u < U; u++) {
            const bool valid = t0 + int64_t(u) * kBlock + threadIdx.x < nv;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                bool need = false;
                r[u][k] = f.head(x[u][k], need);
                nm |= (need && valid) ? (1u << (u * 4 + k)) : 0u;
            }
        }
        if (__ballot(nm != 0u)) {  // wave-uniform
            int total;
            int pos = wave_excl_prefix_small(__popc(nm), total);
            const int first = pos;
#pragma unroll
            for (int e = 0; e < PL; e++)
                if ((nm >> e) & 1u) wq[pos++] = x[e / 4][e % 4];
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            __builtin_amdgcn_wave_barrier();
            for (int j = lane; j < total; j += 64) wq[j] = f.tail(wq[j]);
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            __builtin_amdgcn_wave_barrier();
            pos = first;
#pragma unroll
            for (int e = 0; e < PL; e++)
                if ((nm >> e) & 1u) r[e / 4][e % 4] = wq[pos++];
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            __builtin_amdgcn_wave_barrier();
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int64_t i = t0 + int64_t(u) * kBlock + threadIdx.x;
            if (i < nv) st_nt(ov + i, r[u]);
        }
    }
    if (blockIdx.x == 0) {
        const int64_t j = nv * 4 + threadIdx.x;
        if (j < n) {
            bool need = false;
            const float y = f.head(a[j], need);
            o[j] = need ? f.tail(a[j]) : y;
        }
    }
}

// ---- row broadcast: o[r, c] = op(a[r, c], b[c]) -----------------------------
// The [rows, ncv]-vector array is streamed like the flat kernel: grid-stride
// over tiles of 256 x U vectors, loads before stores.  A lane's column vector
// index is found once by a division and then advances by fixed amounts modulo
// the row width (d1 = 256 mod ncv per unrolled vector, dS = grid stride mod ncv
// per tile), so the loop has no division; the bias vector (a few KiB) is
// served from L1/L2.
template <typename T, typename Op, bool FIXED>
__global__ __launch_bounds__(kBlock) void k_rowbcast(const T *__restrict__ a, const T *__restrict__ b,
                                                     T *__restrict__ o, int64_t nv, int64_t ncv, int64_t d1,
                                                     int64_t dS, Op op)
{
    // FIXED: dS == 0, so a lane meets the same U bias vectors on every tile;
    // they are loaded once, before the loop.
    using V = typename Vec16<T>::type;
    constexpr int VN = Vec16<T>::n;
    const V *av = reinterpret_cast<const V *>(a);
    const V *bv = reinterpret_cast<const V *>(b);
    V *ov = reinterpret_cast<V *>(o);
    const int64_t tile = int64_t(kBlock) * kRowU;
    const int64_t stride = int64_t(gridDim.x) * tile;
    int64_t base = int64_t(blockIdx.x) * tile + threadIdx.x;
    int64_t c = base % ncv;
    V rb[kRowU];
    if (FIXED) {
        int64_t cc = c;
#pragma unroll
        for (int u = 0; u < kRowU; u++) {
            rb[u] = bv[cc];
            cc += d1;
            cc = cc >= ncv ? cc - ncv : cc;
        }
    }
    for (; base < nv; base += stride) {
        V ra[kRowU];
        int64_t cc = c;
#pragma unroll
        for (int u = 0; u < kRowU; u++) {
            const int64_t i = base + int64_t(u) * kBlock;
            if (i < nv) {
                ra[u] = ld_nt(av + i);
                if (!FIXED) rb[u] = bv[cc];
            }
            cc += d1;
            cc = cc >= ncv ? cc - ncv : cc;
        }
#pragma unroll
        for (int u = 0; u < kRowU; u++) {
            const int64_t i = base + int64_t(u) * kBlock;
            if (i < nv) {
                V res;
#pragma unroll
                for (int k = 0; k < VN; k++) res[k] = op(ra[u][k], rb[u][k]);
                // default-policy store: measured faster than a non-temporal
                // one here, and the row reductions that read the result next
                // run faster after it
                ov[i] = res;
            }
        }
        c += dS;
        c = c >= ncv ? c - ncv : c;
    }
}


// ---- N-D strided / broadcast (<= 4 dims, element strides) --------------------
struct ND4 {
    int64_t shape[4];
    int64_t so[4], sa[4], sb[4];
};

NH_DEV void nd_offsets(const ND4 &d, int64_t idx, int64_t &oo, int64_t &oa, int64_t &ob)
{
    int64_t i3 = idx % d.shape[3];
    int64_t r = idx / d.shape[3];
    int64_t i2 = r % d.shape[2];
    r /= d.shape[2];
    int64_t i1 = r % d.shape[1];
    int64_t i0 = r / d.shape[1];
    oo = i0 * d.so[0] + i1 * d.so[1] + i2 * d.so[2] + i3 * d.so[3];
    oa = i0 * d.sa[0] + i1 * d.sa[1] + i2 * d.sa[2] + i3 * d.sa[3];
    ob = i0 * d.sb[0] + i1 * d.sb[1] + i2 * d.sb[2] + i3 * d.sb[3];
}

template <typename T, typename Op>
__global__ __launch_bounds__(kBlock) void k_map2_nd(const T *a, const T *b, T *o, int64_t n, ND4 d, Op op)
{
    const int64_t stride = int64_t(gridDim.x) * kBlock;
    for (int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride) {
        int64_t oo, oa, ob;
        nd_offsets(d, i, oo, oa, ob);
        o[oo] = op(a[oa], b[ob]);
    }
}

template <typename T, typename F>
__global__ __launch_bounds__(kBlock) void k_map1_nd(const T *a, T *o, int64_t n, ND4 d, F f)
{
    const int64_t stride = int64_t(gridDim.x) * kBlock;
    for (int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride) {
        int64_t oo, oa, ob;
        nd_offsets(d, i, oo, oa, ob);
        o[oo] = f(a[oa]);
    }
}

// ---- host-side launch helpers ---------------------------------------------------

// One block per tile of u vectors per lane over the whole range
// (kMaxGridBlocks at most; the grid-stride loop covers the rest).
inline unsigned flat_grid(int64_t n, int vn, int u = kFlatU)
{
    const int64_t nv = n / vn;
    int64_t g = ceil_div(nv, int64_t(kBlock) * u);
    const int64_t cap = kMaxGridBlocks;
    if (g > cap) g = cap;
    return unsigned(g < 1 ? 1 : g);
}

inline unsigned strided_grid(int64_t n)
{
    int64_t g = ceil_div(n, kBlock);
    const int64_t cap = kMaxGridBlocks;
    if (g > cap) g = cap;
    return unsigned(g < 1 ? 1 : g);
}

template <typename T, typename Op>
int launch_rowbcast(const T *a, const T *b, T *o, int64_t rows, int64_t cols, Op op)
{
    constexpr int VN = Vec16<T>::n;
    const int64_t ncv = cols / VN;
    if (rows <= 0 || ncv <= 0) return NEURAL_OK;
    const int64_t nv = rows * ncv;
    const unsigned g = flat_grid(nv * VN, VN, kRowU);
    const int64_t d1 = int64_t(kBlock) % ncv;
    const int64_t dS = (int64_t(g) * kBlock * kRowU) % ncv;
    if (dS == 0)
        NH_LAUNCH((k_rowbcast<T, Op, true>), dim3(g), dim3(kBlock), 0, stream(), a, b, o, nv, ncv, d1, dS, op);
    else
        NH_LAUNCH((k_rowbcast<T, Op, false>), dim3(g), dim3(kBlock), 0, stream(), a, b, o, nv, ncv, d1, dS,
                           op);
    return check_launch();
}

template <typename T, typename Op>
int launch_map2_flat(const T *a, const T *b, T *o, int64_t n, Op op)
{
    if (n <= 0) return NEURAL_OK;
    if (aligned16(a) && aligned16(b) && aligned16(o))
        NH_LAUNCH((k_map2_flat<T, Op>), dim3(flat_grid(n, Vec16<T>::n)), dim3(kBlock), 0, stream(), a, b, o, n, op);
    else
        NH_LAUNCH((k_map2_flat_scalar<T, Op>), dim3(strided_grid(n)), dim3(kBlock), 0, stream(), a, b, o, n, op);
    return check_launch();
}

// f32 head/tail variant of launch_map1_flat (contiguous, 16-byte aligned).
template <typename F>
int launch_map1_f32_tail(const float *a, float *o, int64_t n, F f)
{
    if (n <= 0) return NEURAL_OK;
    int64_t g = ceil_div(n / 4, int64_t(kBlock) * kTailUnroll);
    const int64_t cap = kMaxGridBlocks;
    g = g > cap ? cap : (g < 1 ? 1 : g);
    NH_LAUNCH((k_map1_f32_tail<F>), dim3(unsigned(g)), dim3(kBlock), 0, stream(), a, o, n, f, nullptr,
              int64_t(1), int64_t(0), int64_t(0));
    return check_launch();
}

// The same over x [rows, cols] + bias [cols] (cols % 4 == 0, all 16-byte aligned):
// the fused bias add + activation for head/tail activations.
template <typename F>
int launch_rowbcast_f32_tail(const float *x, const float *bias, float *o, int64_t rows, int64_t cols, F f)
{
    const int64_t ncv = cols / 4;
    if (rows <= 0 || ncv <= 0) return NEURAL_OK;
    const int64_t n = rows * cols;
    int64_t g = ceil_div(n / 4, int64_t(kBlock) * kTailUnroll);
    const int64_t cap = kMaxGridBlocks;
    g = g > cap ? cap : (g < 1 ? 1 : g);
    const int64_t d1 = int64_t(kBlock) % ncv;
    const int64_t dS = (g * kBlock * kTailUnroll) % ncv;
    NH_LAUNCH((k_map1_f32_tail<F, true>), dim3(unsigned(g)), dim3(kBlock), 0, stream(), x, o, n, f, bias, ncv,
              d1, dS);
    return check_launch();
}

template <typename T, typename F>
int launch_map1_flat(const T *a, T *o, int64_t n, F f)
{
    if (n <= 0) return NEURAL_OK;
    if (aligned16(a) && aligned16(o))
        NH_LAUNCH((k_map1_flat<T, F>), dim3(flat_grid(n, Vec16<T>::n)), dim3(kBlock), 0, stream(), a, o, n, f);
    else
        NH_LAUNCH((k_map1_flat_scalar<T, F>), dim3(strided_grid(n)), dim3(kBlock), 0, stream(), a, o, n, f);
    return check_launch();
}

// Broadcast layout of up to three operands against the output shape.
// Returns NEURAL_OK and fills `d` (element strides, merged and left-padded to
// 4 dims), or SHAPE_MISMATCH / DIM_MISMATCH.
int build_nd(const NeuralTensor *out, const NeuralTensor *a, const NeuralTensor *b, ND4 &d);

// Unary op over tensors (contiguous fast path, else N-D); `in` and `out`
// must have the same dtype and element count.
// F32 functors that declare kHeadTail provide head()/tail() for k_map1_f32_tail.
template <typename F, typename = void> struct HasHeadTail : std::false_type {};
template <typename F> struct HasHeadTail<F, std::void_t<decltype(F::kHeadTail)>> : std::true_type {};

template <typename F32, typename F64>
int run_unary(NeuralTensor *out, const NeuralTensor *in, F32 f32, F64 f64)
{
    NH_TRY(ensure_init());
    if (!out || !in) return set_error(NEURAL_ERR_NULL_POINTER);
    NH_TRY(check_tensor(in));
    NH_TRY(check_tensor(out));
    if (in->dtype != out->dtype) return set_error(NEURAL_ERR_DTYPE_MISMATCH);
    const int64_t n = numel(in);
    if (numel(out) != n) return set_error(NEURAL_ERR_SHAPE_MISMATCH);
    if (n == 0) return set_error(NEURAL_OK);
    const void *src = nullptr;
    void *dst = nullptr;
    NH_TRY(dev_read(in, &src));
    const bool flat = is_contiguous(in) && is_contiguous(out);
    NH_TRY(dev_write(out, &dst, is_contiguous(out)));
    if (flat) {
        if (in->dtype == NEURAL_DTYPE_FLOAT32) {
            const float *fs = static_cast<const float *>(src);
            float *fd = static_cast<float *>(dst);
            if constexpr (HasHeadTail<F32>::value) {
                if (aligned16(fs) && aligned16(fd)) NH_TRY(launch_map1_f32_tail(fs, fd, n, f32));
                else NH_TRY(launch_map1_flat(fs, fd, n, f32));
            } else {
                NH_TRY(launch_map1_flat(fs, fd, n, f32));
            }
        } else
            NH_TRY(launch_map1_flat(static_cast<const double *>(src), static_cast<double *>(dst), n, f64));
    } else {
        ND4 d;
        NH_TRY(build_nd(out, in, nullptr, d));
        if (in->dtype == NEURAL_DTYPE_FLOAT32)
            NH_LAUNCH((k_map1_nd<float, F32>), dim3(strided_grid(n)), dim3(kBlock), 0, stream(),
                               static_cast<const float *>(src), static_cast<float *>(dst), n, d, f32);
        else
            NH_LAUNCH((k_map1_nd<double, F64>), dim3(strided_grid(n)), dim3(kBlock), 0, stream(),
                               static_cast<const double *>(src), static_cast<double *>(dst), n, d, f64);
        NH_TRY(check_launch());
    }
    NH_TRY(dev_written(out));
    return set_error(NEURAL_OK);
}

// Is `b` a [C] (or [1,..,1,C]) contiguous vector matching the last dim of a
// contiguous `a`/`out` pair of equal shape?
inline bool row_broadcast_case(const NeuralTensor *out, const NeuralTensor *a, const NeuralTensor *b)
{
    if (out->ndim < 1 || a->ndim != out->ndim || !is_contiguous(out) || !is_contiguous(a) || !is_contiguous(b))
        return false;
    for (int64_t i = 0; i < out->ndim; i++)
        if (a->shape[i] != out->shape[i]) return false;
    const int64_t C = out->shape[out->ndim - 1];
    if (b->ndim < 1 || b->shape[b->ndim - 1] != C) return false;
    for (int64_t i = 0; i + 1 < b->ndim; i++)
        if (b->shape[i] != 1) return false;
    const int64_t vn = out->dtype == NEURAL_DTYPE_FLOAT32 ? 4 : 2;
    return C % vn == 0;
}

// Binary ops that apply a head/tail f32 functor to a + b (the fused bias add +
// activation, whose f32 member declares kHeadTail) take the queued-tail kernel
// in the row-broadcast case.
template <typename Op, typename = void> struct RowHeadTail : std::false_type {};
template <typename Op> struct RowHeadTail<Op, std::void_t<decltype(Op::F32T::kHeadTail)>> : std::true_type {};

template <typename T, typename Op>
int launch_binary(NeuralTensor *out, const NeuralTensor *a, const NeuralTensor *b, const void *pa,
                         const void *pb, void *po, Op op)
{
    const int64_t n = numel(out);
    const T *A = static_cast<const T *>(pa);
    const T *B = static_cast<const T *>(pb);
    T *O = static_cast<T *>(po);
    if (numel(a) == n && numel(b) == n && is_contiguous(a) && is_contiguous(b) && is_contiguous(out))
        return launch_map2_flat(A, B, O, n, op);
    if (row_broadcast_case(out, a, b) && aligned16(A) && aligned16(B) && aligned16(O)) {
        const int64_t C = out->shape[out->ndim - 1];
        if constexpr (std::is_same<T, float>::value && RowHeadTail<Op>::value)
            return launch_rowbcast_f32_tail(A, B, O, n / C, C, op.f32);
        return launch_rowbcast(A, B, O, n / C, C, op);
    }
    ND4 d;
    NH_TRY(build_nd(out, a, b, d));
    NH_LAUNCH((k_map2_nd<T, Op>), dim3(strided_grid(n)), dim3(kBlock), 0, stream(), A, B, O, n, d, op);
    return check_launch();
}

// Binary op on tensors: flat when all three are contiguous and equal in size,
// the row-broadcast kernel for [.., C] (+) [C], else the strided N-D kernel.
template <typename Op>
int binary_api(NeuralTensor *out, const NeuralTensor *a, const NeuralTensor *b, Op op)
{
    NH_TRY(ensure_init());
    if (!out || !a || !b) return set_error(NEURAL_ERR_NULL_POINTER);
    NH_TRY(check_tensor(out));
    NH_TRY(check_tensor(a));
    NH_TRY(check_tensor(b));
    if (a->dtype != out->dtype || b->dtype != out->dtype) return set_error(NEURAL_ERR_DTYPE_MISMATCH);
    const int64_t n = numel(out);
    if (n == 0) return set_error(NEURAL_OK);
    const void *pa = nullptr, *pb = nullptr;
    void *po = nullptr;
    NH_TRY(dev_read(a, &pa));
    NH_TRY(dev_read(b, &pb));
    NH_TRY(dev_write(out, &po, is_contiguous(out)));
    if (out->dtype == NEURAL_DTYPE_FLOAT32) NH_TRY((launch_binary<float, Op>(out, a, b, pa, pb, po, op)));
    else NH_TRY((launch_binary<double, Op>(out, a, b, pa, pb, po, op)));
    NH_TRY(dev_written(out));
    return set_error(NEURAL_OK);
}

}  // namespace nh
