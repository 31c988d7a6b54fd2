// reduce_impl.hpp -- deterministic reductions for gfx950.
//
// Full-tensor reductions run in one launch: a fixed grid of G blocks walks
// the input in 128-bit vectors (grid-stride over tiles of 256*U vectors), each
// block reduces its lanes with a wave64 butterfly plus an LDS step, writes one
// partial, and the last block to arrive (device-scope counter) combines the G
// partials in a fixed order and stores the result.  G, the tile walk and the
// combine trees are fixed, so results are bitwise reproducible run to run.
//
// Row reductions give each row to one wave (short rows) or one 256-lane block
// (long rows) and reduce the same way without the cross-block step.
//
// A reducer `Red` supplies:  S (state, <= 64 bytes, trivially copyable),
// init(), acc(S&, double v, int64 idx), comb(S, S) (commutative), shfl(S, off).
#pragma once

#include "common.hpp"

namespace nh {

constexpr int kRBlock = 256;
constexpr int kRUnroll = 4;

template <class Red>
NH_DEV typename Red::S wave_reduce(const Red &red, typename Red::S s)
{
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) s = red.comb(s, red.shfl(s, off));
    return s;
}

// Block-wide reduce; the result is valid in every thread.
template <class Red>
NH_DEV typename Red::S block_reduce(const Red &red, typename Red::S s)
{
    __shared__ typename Red::S lds[kRBlock / 64];
    s = wave_reduce(red, s);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) lds[w] = s;
    __syncthreads();
    typename Red::S r = lds[0];
#pragma unroll
    for (int i = 1; i < kRBlock / 64; i++) r = red.comb(r, lds[i]);
    __syncthreads();
    return r;
}

template <typename T, class Red, bool VEC>
__global__ __launch_bounds__(kRBlock) void k_reduce_full(const T *__restrict__ x, int64_t n, Red red,
                                                         typename Red::S *partials, unsigned *counter,
                                                         void *result)
{
    using S = typename Red::S;
    S st = red.init();
    if (VEC) {
        using V = typename Vec16<T>::type;
        constexpr int VN = Vec16<T>::n;
        const V *xv = reinterpret_cast<const V *>(x);
        const int64_t nv = n / VN;
        const int64_t tile = int64_t(kRBlock) * kRUnroll;
        for (int64_t t0 = int64_t(blockIdx.x) * tile; t0 < nv; t0 += int64_t(gridDim.x) * tile) {
            V r[kRUnroll];
#pragma unroll
            for (int u = 0; u < kRUnroll; u++) {
                const int64_t i = t0 + int64_t(u) * kRBlock + threadIdx.x;
                if (i < nv) r[u] = ld_nt(xv + i);
            }
#pragma unroll
            for (int u = 0; u < kRUnroll; u++) {
                const int64_t i = t0 + int64_t(u) * kRBlock + threadIdx.x;
                if (i < nv) {
#pragma unroll
                    for (int k = 0; k < VN; k++) red.acc(st, double(r[u][k]), i * VN + k);
                }
            }
        }
        if (blockIdx.x == 0) {
            const int64_t j = nv * VN + threadIdx.x;
            if (j < n) red.acc(st, double(x[j]), j);
        }
    } else {
        const int64_t stride = int64_t(gridDim.x) * kRBlock;
        for (int64_t i = int64_t(blockIdx.x) * kRBlock + threadIdx.x; i < n; i += stride)
            red.acc(st, double(x[i]), i);
    }
    st = block_reduce(red, st);

    __shared__ bool s_last;
    if (threadIdx.x == 0) {
        partials[blockIdx.x] = st;
        __threadfence();
        const unsigned ticket = atomicAdd(counter, 1u);
        s_last = (ticket == gridDim.x - 1);
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    S acc = red.init();
    for (int i = threadIdx.x; i < int(gridDim.x); i += kRBlock) acc = red.comb(acc, partials[i]);
    acc = block_reduce(red, acc);
    if (threadIdx.x == 0) {
        red.store(result, acc);
        *counter = 0u;
    }
}

inline unsigned reduce_grid(int64_t n, int vn)
{
    const int64_t nv = n / vn;
    int64_t g = ceil_div(nv, int64_t(kRBlock) * kRUnroll);
    const int64_t cap = int64_t(num_cus()) * 4;
    if (g > cap) g = cap;
    if (g > kMaxPartials) g = kMaxPartials;
    return unsigned(g < 1 ? 1 : g);
}

// Launch a full reduction writing Red::store(...) into `dev_result` (device).
template <typename T, class Red>
int launch_reduce_full(const T *x, int64_t n, const Red &red, void *dev_result)
{
    static_assert(sizeof(typename Red::S) <= 64, "reduction state must fit a 64-byte partial slot");
    Workspace &ws = workspace();
    auto *partials = static_cast<typename Red::S *>(ws.partials);
    const bool vec = (reinterpret_cast<uintptr_t>(x) & 15u) == 0;
    if (vec)
        hipLaunchKernelGGL((k_reduce_full<T, Red, true>), dim3(reduce_grid(n, Vec16<T>::n)), dim3(kRBlock), 0,
                           stream(), x, n, red, partials, ws.counter, dev_result);
    else
        hipLaunchKernelGGL((k_reduce_full<T, Red, false>), dim3(reduce_grid(n, 1)), dim3(kRBlock), 0, stream(), x,
                           n, red, partials, ws.counter, dev_result);
    return check_launch();
}

// ---- row reductions -----------------------------------------------------------------
// TPR lanes per row (64: one wave, 256: one block); RPB = 256 / TPR rows per block.
// Red additionally supplies store_row_x(out, row, S, row_base, cols) and, for
// the running-max semantics, a second pass over the suffix after the row's
// last NaN (Red::kSuffixPass).

template <class Red>
NH_DEV typename Red::S row_group_reduce(const Red &red, typename Red::S s, int tpr)
{
    if (tpr == 64) return wave_reduce(red, s);
    return block_reduce(red, s);
}

template <typename T, class Red, int TPR>
NH_DEV typename Red::S row_scan(const Red &red, const T *xr, int64_t cols, int64_t from, bool vec)
{
    typename Red::S st = red.init();
    const int lane = threadIdx.x % TPR;
    if (vec && from == 0) {
        using V = typename Vec16<T>::type;
        constexpr int VN = Vec16<T>::n;
        const V *xv = reinterpret_cast<const V *>(xr);
        const int64_t nv = cols / VN;
        for (int64_t c = lane; c < nv; c += TPR) {
            const V v = ld_nt(xv + c);
#pragma unroll
            for (int k = 0; k < VN; k++) red.acc(st, double(v[k]), c * VN + k);
        }
        for (int64_t j = nv * VN + lane; j < cols; j += TPR) red.acc(st, double(xr[j]), j);
    } else {
        for (int64_t j = from + lane; j < cols; j += TPR) red.acc(st, double(xr[j]), j);
    }
    return st;
}

template <typename T, class Red, int TPR>
__global__ __launch_bounds__(kRBlock) void k_reduce_rows(const T *__restrict__ x, int64_t rows, int64_t cols,
                                                         Red red, void *out, bool vec)
{
    constexpr int RPB = kRBlock / TPR;
    const int64_t r = int64_t(blockIdx.x) * RPB + threadIdx.x / TPR;
    const bool valid = r < rows;
    const T *xr = x + (valid ? r : 0) * cols;
    typename Red::S st = valid ? row_scan<T, Red, TPR>(red, xr, cols, 0, vec) : red.init();
    st = row_group_reduce(red, st, TPR);
    if constexpr (Red::kSuffixPass) {
        // Running-max semantics: restart after the last NaN of the row.  The
        // branch is uniform per row group (a wave, or the whole block).
        const int64_t L = red.suffix_start(st);
        if (L >= 0) {
            typename Red::S s2 = valid ? row_scan<T, Red, TPR>(red, xr, cols, L + 1, false) : red.init();
            s2 = row_group_reduce(red, s2, TPR);
            st = red.suffix_result(st, s2, cols);
        }
    }
    if (valid && (threadIdx.x % TPR) == 0) red.store_row_x(out, r, st, xr, cols);
}

template <typename T, class Red>
int launch_reduce_rows(const T *x, int64_t rows, int64_t cols, const Red &red, void *out)
{
    if (rows <= 0) return NEURAL_OK;
    const bool vec = ((reinterpret_cast<uintptr_t>(x) & 15u) == 0) && (cols % Vec16<T>::n == 0);
    if (cols <= 1024) {
        const unsigned g = unsigned(ceil_div(rows, kRBlock / 64));
        hipLaunchKernelGGL((k_reduce_rows<T, Red, 64>), dim3(g), dim3(kRBlock), 0, stream(), x, rows, cols, red, out,
                           vec);
    } else {
        hipLaunchKernelGGL((k_reduce_rows<T, Red, 256>), dim3(unsigned(rows)), dim3(kRBlock), 0, stream(), x, rows,
                           cols, red, out, vec);
    }
    return check_launch();
}

}  // namespace nh
