// reduce_impl.hpp -- deterministic segmented reductions for gfx950.
//
// Every reduction here is a reduction of R rows of C elements (a whole tensor
// is one row).  A row is split into contiguous segments; each segment is
// reduced by one group of lanes (a wave64 or a 256-lane block):
//
//   lanes     walk the segment in 128-bit vectors (U vectors in flight per
//             lane), keeping a small lane state in the input's own precision
//             where that is exact (min / max / NaN tests) and in double where
//             it is not (sums);
//   group     combines lane states with a fixed butterfly (wave) and an LDS
//             step (block), then `finish` turns the result into an ORDERED
//             segment summary -- this is where rare cases (a NaN in a
//             running-max chain, a zero whose sign matters) rescan their own
//             segment, so the common case costs one or two VALU ops per element;
//   segments  of one row are combined in index order by a second launch
//             (one block per row, fixed sequential + ordered-tree combine).
//             Two launches instead of a last-block ticket: a device-scope
//             fence + atomic per block cost more than the whole stream at
//             thousands of blocks (measured on MI355X).
//
// Grid shapes are a pure function of (rows, cols, CU count), so results are
// bitwise reproducible run to run.
//
// A reducer `Red` for element type T supplies
//   L  lane state        L linit(); void lacc(L&, T x, int64_t i /*index in row*/);
//                        L lcomb(L, L)   (commutative)
//   B  segment summary   B finish<G>(L group_state, const T *row, int64_t lo, int64_t hi)
//                        B bident(); B bcomb(B earlier, B later)
//   store                void store(void *out, int64_t row, B, const T *row, int64_t cols)
// L and B are trivially copyable, a multiple of 4 bytes, B at most 64 bytes.
#pragma once

#include <type_traits>

#include "common.hpp"

namespace nh {

constexpr int kRBlock = 256;
constexpr int kRUnroll = 4;

// ---- generic cross-lane helpers ---------------------------------------------------------

template <typename S>
NH_DEV S shfl_xor_obj(const S &s, int off)
{
    static_assert(sizeof(S) % 4 == 0, "state must be a multiple of 4 bytes");
    constexpr int W = sizeof(S) / 4;
    int w[W];
    __builtin_memcpy(w, &s, sizeof(S));
#pragma unroll
    for (int k = 0; k < W; k++) w[k] = __shfl_xor(w[k], off, 64);
    S r;
    __builtin_memcpy(&r, w, sizeof(S));
    return r;
}

template <typename S>
NH_DEV S shfl_down_obj(const S &s, int off)
{
    constexpr int W = sizeof(S) / 4;
    int w[W];
    __builtin_memcpy(w, &s, sizeof(S));
#pragma unroll
    for (int k = 0; k < W; k++) w[k] = __shfl_down(w[k], off, 64);
    S r;
    __builtin_memcpy(&r, w, sizeof(S));
    return r;
}

template <int CTRL, typename S>
NH_DEV S dpp_obj(const S &s)
{
    constexpr int W = sizeof(S) / 4;
    int w[W];
    __builtin_memcpy(w, &s, sizeof(S));
#pragma unroll
    for (int k = 0; k < W; k++) w[k] = dpp_i<CTRL>(w[k]);
    S r;
    __builtin_memcpy(&r, w, sizeof(S));
    return r;
}

// Group of TPR lanes (64 = one wave, 256 = the whole block).  reduce() leaves
// the same value in every lane of the group: the pairs are fixed and each
// pair computes comb(a, b) and comb(b, a), equal for commutative comb.  Within
// a wave: quad swaps (xor 1, xor 2), the half-row and row mirrors as DPP
// operand moves (no LDS traffic), then lane exchanges across 16 and 32.
template <int TPR>
struct Grp {
    static_assert(TPR == 64 || TPR == kRBlock, "a group is one wave or one block");
    NH_DEV static int lane() { return int(threadIdx.x) % TPR; }
    template <typename S, typename C>
    NH_DEV static S reduce(S s, C comb)
    {
        s = comb(s, dpp_obj<kDppXor1>(s));
        s = comb(s, dpp_obj<kDppXor2>(s));
        s = comb(s, dpp_obj<kDppHalfMirror>(s));
        s = comb(s, dpp_obj<kDppMirror>(s));
        s = comb(s, shfl_xor_obj(s, 16));
        s = comb(s, shfl_xor_obj(s, 32));
        if constexpr (TPR == 64) {
            return s;
        } else {
            __shared__ S lds[kRBlock / 64];
            const int w = threadIdx.x >> 6;
            if ((threadIdx.x & 63) == 0) lds[w] = s;
            __syncthreads();
            S r = lds[0];
#pragma unroll
            for (int i = 1; i < kRBlock / 64; i++) r = comb(r, lds[i]);
            __syncthreads();
            return r;
        }
    }
    NH_DEV static int64_t max_i64(int64_t v)
    {
        return reduce(v, [](int64_t a, int64_t b) { return a > b ? a : b; });
    }
    NH_DEV static int64_t min_i64(int64_t v)
    {
        return reduce(v, [](int64_t a, int64_t b) { return a < b ? a : b; });
    }
};

// ---- the segment walk ---------------------------------------------------------------------

// Reducers that declare `static constexpr bool kRelIndex = true` receive the
// element's index relative to the segment start `lo` (it fits 32 bits: every
// launch checks that segments hold fewer than 2^31 elements), computed in
// 32-bit arithmetic; their finish() turns lane indices back into row indices.
// Others receive the index in the row.
template <class Red, typename = void> struct RelIndex { static constexpr bool value = false; };
template <class Red> struct RelIndex<Red, std::void_t<decltype(Red::kRelIndex)>> {
    static constexpr bool value = Red::kRelIndex;
};

// No prologue: the walked values are the row's own.  A prologue's load(i)
// fetches what vec() needs beside the row's vector i (the fused bias add: the
// bias vector); the walk issues those loads together with the row's loads,
// before it waits for any of them.
struct NoPre {
    static constexpr bool kActive = false;
    NH_DEV int load(int64_t) const { return 0; }
    template <typename V> NH_DEV V vec(const V &v, int, int64_t) const { return v; }
    template <typename T> NH_DEV T one(T x, int64_t) const { return x; }
};

// Walk row elements [lo, hi) with a group of TPR lanes and return the group's
// combined lane state (the same in every lane of the group).  `vec` promises
// that row is 16-byte aligned and lo is a multiple of the vector width.  NT:
// the vector loads are non-temporal.  A prologue `pre` (Pre::kActive) maps
// each loaded vector / element (by its index in the row) before it is reduced;
// the fused producers use it to compute and store a value and reduce it in the
// same pass.  The walk order does not depend on Red or Pre, so a fused
// reduction accumulates exactly what the stand-alone one does.
// `first` (optional) receives the first value the lane walked: for the
// group's lane 0 that is element lo (after the prologue).
template <typename T, class Red, int TPR, bool NT, class Pre = NoPre>
NH_DEV typename Red::L seg_walk(const Red &red, const T *__restrict__ row, int64_t lo, int64_t hi, bool vec,
                                const Pre &pre = Pre{}, T *first = nullptr)
{
    using L = typename Red::L;
    using G = Grp<TPR>;
    constexpr bool kRel = RelIndex<Red>::value;
    L st = red.linit();
    const int lane = G::lane();
    int64_t tail = lo;
    if (vec) {
        using V = typename Vec16<T>::type;
        constexpr int VN = Vec16<T>::n;
        const V *xv = reinterpret_cast<const V *>(row);
        const int64_t v0 = lo / VN, v1 = hi / VN;
        for (int64_t c = v0 + lane; c < v1; c += int64_t(TPR) * kRUnroll) {
            V r[kRUnroll];
            decltype(pre.load(0)) aux[kRUnroll];
#pragma unroll
            for (int u = 0; u < kRUnroll; u++) {
                const int64_t i = c + int64_t(u) * TPR;
                if (i < v1) r[u] = NT ? ld_nt(xv + i) : xv[i];
            }
            if constexpr (Pre::kActive) {
#pragma unroll
                for (int u = 0; u < kRUnroll; u++) {
                    const int64_t i = c + int64_t(u) * TPR;
                    if (i < v1) aux[u] = pre.load(i);
                }
#pragma unroll
                for (int u = 0; u < kRUnroll; u++) {
                    const int64_t i = c + int64_t(u) * TPR;
                    if (i < v1) r[u] = pre.vec(r[u], aux[u], i);
                }
            }
            if (first && c == v0 + lane) *first = r[0][0];
            const int32_t rb = kRel ? int32_t(c - v0) * VN : 0;  // lo is a multiple of VN here
#pragma unroll
            for (int u = 0; u < kRUnroll; u++) {
                const int64_t i = c + int64_t(u) * TPR;
                if (i < v1) {
#pragma unroll
                    for (int k = 0; k < VN; k++) {
                        if constexpr (kRel) red.lacc(st, r[u][k], rb + (u * TPR * VN + k));
                        else red.lacc(st, r[u][k], i * VN + k);
                    }
                }
            }
        }
        tail = v1 * VN > lo ? v1 * VN : lo;
    }
    for (int64_t j = tail + lane; j < hi; j += TPR) {
        const T x = pre.one(row[j], j);
        if (first && j == tail + lane && tail == lo) *first = x;
        red.lacc(st, x, kRel ? j - lo : j);
    }
    return G::reduce(st, [&](const L &a, const L &b) { return red.lcomb(a, b); });
}

// Reduce row elements [lo, hi) to the segment summary (`first`: see seg_walk).
template <typename T, class Red, int TPR, bool NT>
NH_DEV typename Red::B seg_reduce(const Red &red, const T *__restrict__ row, int64_t lo, int64_t hi, bool vec,
                                  T *first = nullptr)
{
    return red.template finish<TPR>(seg_walk<T, Red, TPR, NT>(red, row, lo, hi, vec, NoPre{}, first), row, lo, hi);
}

// Reducers whose store() reads only element 0 of the row (argmax: x0 NaN
// gives index 0) declare kStoreReadsFirst; the row kernels then hand them the
// value their lane 0 walked first instead of a pointer, so no lane waits on a
// load of row[0] after the reduction.
template <class Red, typename = void> struct StoreReadsFirst { static constexpr bool value = false; };
template <class Red> struct StoreReadsFirst<Red, std::void_t<decltype(Red::kStoreReadsFirst)>> {
    static constexpr bool value = Red::kStoreReadsFirst;
};
template <typename T>
struct FirstOnly {
    T v;
    NH_DEV T operator[](int64_t) const { return v; }
};

// Ordered combine of n segment summaries p[0..n) by one block; result valid
// in thread 0.  Each thread folds a contiguous run, then an ordered tree
// (lane l absorbs lane l+off) across the wave and the four waves in order.
template <class Red>
NH_DEV typename Red::B ordered_combine(const Red &red, const typename Red::B *p, int n)
{
    using B = typename Red::B;
    const int t = threadIdx.x;
    const int k = (n + kRBlock - 1) / kRBlock;
    B s = red.bident();
    const int a = t * k;
    const int e = a + k < n ? a + k : n;
    // loads of a batch issued together (the fold is sequential, the loads not)
    constexpr int kBatch = 4;
    for (int i0 = a; i0 < e; i0 += kBatch) {
        B buf[kBatch];
#pragma unroll
        for (int j = 0; j < kBatch; j++)
            if (i0 + j < e) buf[j] = p[i0 + j];
#pragma unroll
        for (int j = 0; j < kBatch; j++)
            if (i0 + j < e) s = red.bcomb(s, buf[j]);
    }
    const int lane = t & 63;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const B o = shfl_down_obj(s, off);
        if ((lane & (2 * off - 1)) == 0) s = red.bcomb(s, o);
    }
    __shared__ B lds[kRBlock / 64];
    if (lane == 0) lds[t >> 6] = s;
    __syncthreads();
    B r = lds[0];
#pragma unroll
    for (int i = 1; i < kRBlock / 64; i++) r = red.bcomb(r, lds[i]);
    return r;
}

// ---- kernels --------------------------------------------------------------------------------

// A result that only the host reads is stored into coherent host memory; the
// storing lane then writes the ticket after a system-scope fence, so a host
// that sees the ticket sees the result (host_result_wait).
NH_DEV void publish(const Ticket &tk)
{
    if (tk.slot) {
        __threadfence_system();
        __hip_atomic_store(tk.slot, tk.value, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
}

// One group (wave or block) per row; RPB = 256 / TPR rows per block.
template <typename T, class Red, int TPR>
__global__ __launch_bounds__(kRBlock) void k_reduce_rows(const T *__restrict__ x, int64_t rows, int64_t cols,
                                                         int64_t ld, Red red, void *out, bool vec, Ticket tk)
{
    constexpr int RPB = kRBlock / TPR;
    // rows past the grid (more than kMaxGridBlocks * RPB) are taken in further
    // rounds; r is uniform per group
    for (int64_t r = int64_t(blockIdx.x) * RPB + threadIdx.x / TPR; r < rows; r += int64_t(gridDim.x) * RPB) {
        const T *xr = x + r * ld;
        // default-policy loads: in a sequence (bias add, then several row
        // reductions of its result, then other streams) this measured faster
        // for the whole sequence than non-temporal ones
        if constexpr (StoreReadsFirst<Red>::value) {
            T x0 = T(0);
            const typename Red::B b = seg_reduce<T, Red, TPR, false>(red, xr, 0, cols, vec, &x0);
            if (Grp<TPR>::lane() == 0) {
                red.store(out, r, b, FirstOnly<T>{x0}, cols);
                publish(tk);  // tickets are used with a single row only
            }
        } else {
            const typename Red::B b = seg_reduce<T, Red, TPR, false>(red, xr, 0, cols, vec);
            if (Grp<TPR>::lane() == 0) {
                red.store(out, r, b, xr, cols);
                publish(tk);  // tickets are used with a single row only
            }
        }
    }
}

// gridDim.x blocks per row (blockIdx.y = row), each reducing one contiguous
// segment of `chunk` elements into its summary slot.  No fence or atomic: the
// kernel boundary before k_reduce_combine publishes the summaries.
template <typename T, class Red>
__global__ __launch_bounds__(kRBlock) void k_reduce_seg(const T *__restrict__ x, int64_t cols, int64_t ld,
                                                        int64_t chunk, Red red, typename Red::B *partials, bool vec)
{
    const int64_t r = blockIdx.y;
    const T *xr = x + r * ld;
    const int64_t lo = int64_t(blockIdx.x) * chunk;
    const int64_t hi = lo + chunk < cols ? lo + chunk : cols;
    const typename Red::B b = seg_reduce<T, Red, kRBlock, true>(red, xr, lo, hi, vec);
    if (threadIdx.x == 0) partials[r * int64_t(gridDim.x) + blockIdx.x] = b;
}

// One block per row: ordered combine of the row's gx summaries, then store.
template <typename T, class Red>
__global__ __launch_bounds__(kRBlock) void k_reduce_combine(const T *__restrict__ x, int64_t cols, int64_t ld,
                                                            int gx, Red red, const typename Red::B *partials,
                                                            void *out, Ticket tk)
{
    const int64_t r = blockIdx.x;
    const typename Red::B tot = ordered_combine(red, partials + r * gx, gx);
    if (threadIdx.x == 0) {
        red.store(out, r, tot, x + r * ld, cols);
        publish(tk);  // tickets are used with a single row only
    }
}

// ---- launch policy --------------------------------------------------------------------------

// Reduce `rows` rows of `cols` elements (row r at x + r*ld) and store through
// Red::store into `out` (device memory).  Many rows: one wave (cols <= 2048)
// or one block per row.  Few long rows: ~4 blocks per CU spread over the rows,
// each block one contiguous segment of a multiple of 16 KiB, then the
// one-block-per-row combine.
//
// The segment summaries go to the shared workspace (under WsGuard), or to
// `scratch` (scratch_bytes long) when the caller brings its own buffer; a
// grid whose summaries do not fit it returns NEURAL_ERR_TENSOR_TOO_LARGE.
// The grid of a reduction of `rows` rows of `cols` elements of T: gx segments
// of `chunk` elements per row (gx > 1: k_reduce_seg + k_reduce_combine), else
// one group per row of `tpr` lanes (k_reduce_rows).  A pure function of the
// shape and the CU count, shared by every reducer, so a fused reduction walks
// exactly the segments the stand-alone one does.
struct ReducePlan {
    int64_t gx, chunk;
    int tpr;
};

template <typename T>
ReducePlan reduce_plan(int64_t rows, int64_t cols)
{
    constexpr int VN = Vec16<T>::n;
    const int64_t want = int64_t(num_cus()) * 4;  // blocks that keep every CU streaming (measured: 4/CU >= 8/CU here)
    constexpr int64_t kGran = int64_t(kRBlock) * kRUnroll * VN;
    ReducePlan p{1, cols, cols <= 2048 ? 64 : kRBlock};
    // (a single block per row is slower even for a 512 KiB row: 18.7 us vs
    // 9.4 us for 32 segments + the combine launch, measured)
    if (rows < want && cols > 2 * kGran) {
        p.gx = ceil_div(want, rows);
        p.chunk = ceil_div(ceil_div(cols, p.gx), kGran) * kGran;
        p.gx = ceil_div(cols, p.chunk);
        const int64_t cap = kMaxPartials / rows;
        if (p.gx > cap) {
            p.gx = cap;
            p.chunk = ceil_div(ceil_div(cols, p.gx), kGran) * kGran;
            p.gx = ceil_div(cols, p.chunk);
        }
    }
    return p;
}

// Blocks of a row-per-group launch (rpb rows per block), capped at kMaxGridBlocks.
inline unsigned rows_grid(int64_t rows, int rpb)
{
    const int64_t g = ceil_div(rows, rpb);
    return unsigned(g < kMaxGridBlocks ? g : kMaxGridBlocks);
}

template <typename T, class Red>
int launch_reduce(const T *x, int64_t rows, int64_t cols, int64_t ld, const Red &red, void *out,
                  void *scratch = nullptr, size_t scratch_bytes = 0, Ticket tk = Ticket{})
{
    if (tk.slot && rows != 1) return set_error(NEURAL_ERR_INTERNAL);
    static_assert(sizeof(typename Red::B) <= 64, "segment summary must fit a 64-byte partial slot");
    if (rows <= 0 || cols <= 0) return NEURAL_OK;
    const bool vec = ((reinterpret_cast<uintptr_t>(x) & 15u) == 0) && ((ld * int64_t(sizeof(T))) % 16 == 0);
    const ReducePlan plan = reduce_plan<T>(rows, cols);
    const int64_t gx = plan.gx, chunk = plan.chunk;
    if (RelIndex<Red>::value && chunk >= (int64_t(1) << 31)) return set_error(NEURAL_ERR_TENSOR_TOO_LARGE);
    if (gx > 1) {
        if (scratch && size_t(gx * rows) * sizeof(typename Red::B) > scratch_bytes)
            return set_error(NEURAL_ERR_TENSOR_TOO_LARGE);
        std::unique_lock<std::recursive_mutex> wg(workspace_mutex(), std::defer_lock);
        if (!scratch) wg.lock();
        auto *part = static_cast<typename Red::B *>(scratch ? scratch : workspace().partials);
        const dim3 grid{unsigned(gx), unsigned(rows), 1u};
        NH_LAUNCH((k_reduce_seg<T, Red>), grid, dim3(kRBlock), 0, stream(), x, cols, ld, chunk, red, part,
                           vec);
        NH_LAUNCH((k_reduce_combine<T, Red>), dim3(unsigned(rows)), dim3(kRBlock), 0, stream(), x, cols, ld,
                           int(gx), red, part, out, tk);
    } else if (plan.tpr == 64) {
        NH_LAUNCH((k_reduce_rows<T, Red, 64>), dim3(rows_grid(rows, kRBlock / 64)), dim3(kRBlock), 0, stream(), x,
                  rows, cols, ld, red, out, vec, tk);
    } else {
        NH_LAUNCH((k_reduce_rows<T, Red, kRBlock>), dim3(rows_grid(rows, 1)), dim3(kRBlock), 0, stream(), x, rows,
                  cols, ld, red, out, vec, tk);
    }
    return check_launch();
}

// Whole contiguous array as one row.
template <typename T, class Red>
int launch_reduce_full(const T *x, int64_t n, const Red &red, void *out)
{
    return launch_reduce(x, 1, n, n, red, out);
}

// Whole contiguous array reduced into workspace().host_result, then the
// result copied to dst (bytes <= 248) once the storing kernel's ticket shows
// in host memory.  The caller holds WsGuard.
template <typename T, class Red>
int reduce_full_to_host(const T *x, int64_t n, const Red &red, void *dst, size_t bytes)
{
    const Ticket tk = next_ticket();
    NH_TRY(launch_reduce(x, 1, n, n, red, workspace().host_result_dev, nullptr, 0, tk));
    return host_result_wait(tk.value, dst, bytes);
}

// ---- shared reducers ---------------------------------------------------------------------

template <typename T> NH_DEV T fmax_nn(T a, T b);  // NaN-ignoring max
template <> NH_DEV float fmax_nn(float a, float b) { return __builtin_fmaxf(a, b); }
template <> NH_DEV double fmax_nn(double a, double b) { return __builtin_fmax(a, b); }
template <typename T> NH_DEV T fmin_nn(T a, T b);
template <> NH_DEV float fmin_nn(float a, float b) { return __builtin_fminf(a, b); }
template <> NH_DEV double fmin_nn(double a, double b) { return __builtin_fmin(a, b); }
template <typename T> NH_DEV T fma_t(T a, T b, T c);
template <> NH_DEV float fma_t(float a, float b, float c) { return __builtin_fmaf(a, b, c); }
template <> NH_DEV double fma_t(double a, double b, double c) { return __builtin_fma(a, b, c); }
template <typename T> NH_DEV T fabs_t(T a);
template <> NH_DEV float fabs_t(float a) { return __builtin_fabsf(a); }
template <> NH_DEV double fabs_t(double a) { return __builtin_fabs(a); }
template <typename T> NH_DEV T inf_t();
template <> NH_DEV float inf_t<float>() { return __builtin_inff(); }
template <> NH_DEV double inf_t<double>() { return __builtin_inf(); }
template <typename T> NH_DEV T qnan_t();
template <> NH_DEV float qnan_t<float>() { return __builtin_nanf(""); }
template <> NH_DEV double qnan_t<double>() { return __builtin_nan(""); }

// Sum accumulated in double; the store policy decides what is written.
//   OUT_T   : out[row] = T(sum / div)          (row sums / means, whole-tensor sum into a tensor)
//   OUT_F64 : ((double*)out)[row] = sum        (host-returned results)
enum { SUM_OUT_T = 0, SUM_OUT_F64 = 1 };
template <typename T, int MODE>
struct RedSum {
    using L = double;
    using B = double;
    int64_t div = 1;
    NH_DEV L linit() const { return 0.0; }
    NH_DEV void lacc(L &s, T x, int64_t) const { s += double(x); }
    NH_DEV L lcomb(L a, L b) const { return a + b; }
    template <int TPR> NH_DEV B finish(L s, const T *, int64_t, int64_t) const { return s; }
    NH_DEV B bident() const { return 0.0; }
    NH_DEV B bcomb(B a, B b) const { return a + b; }
    NH_DEV void store(void *out, int64_t r, B s, const T *, int64_t) const
    {
        if (MODE == SUM_OUT_F64) static_cast<double *>(out)[r] = s;
        else static_cast<T *>(out)[r] = T(div > 1 ? s / double(div) : s);
    }
};

}  // namespace nh
