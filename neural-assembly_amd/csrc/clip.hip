// clip.hip -- gradient clipping over a list of gradient tensors.
//
// Reference: clip_grad_norm_ (optimizers.asm:1370-1516) and clip_grad_value_
// (optimizers.asm:1527-1620), reached through neural_clip_grad_norm /
// neural_clip_grad_value (neural_api.asm:1677-1720, neural_api.h:731,741).
//
// clip_grad_norm_: total = sum over every gradient element of double(g)^2, one
// sequential double sum; norm = sqrt(total); when norm > max_norm (ordered
// compare, so a NaN norm clips nothing) every gradient is multiplied by
// scale = max_norm / norm computed in double; f32 gradients use that scale
// rounded to float and a float multiply.  clip_grad_value_: maxsd then minsd,
// t = g > lo ? g : lo, then t < hi ? t : hi (a NaN gradient becomes lo), with
// the bounds rounded to float for f32 gradients.
//
// Device layout: every gradient of the list (either dtype) is cut into chunks
// and one block takes one chunk.  A table of {pointer, length, dtype, first
// chunk} entries goes to the device with one small host-to-device copy, so a
// whole gradient set costs three launches however many tensors it holds:
//   k_clip_sumsq   chunk sums of squares -> partials (4 or 8 B/elem read)
//   k_clip_decide  one block: ordered sum of the partials, sqrt, the compare
//                  and the scale, stored on the device
//   k_clip_scale   reads the decision; exits at once when nothing is clipped,
//                  else g *= scale in place (8 or 16 B/elem)
// The read-only pass uses long chunks (few partials, long streams per block);
// the read-write passes use short ones (measured: the short chunks spread the
// last blocks evenly over the CUs).  No host round trip sits between the
// passes; the host reads the norm only when the caller asks for it.  The sum
// order differs from the reference's sequential one: all terms are >= 0, so
// the norm differs by a few ulps at most, and the scale -- hence every clipped
// gradient -- follows the computed norm exactly as in the reference.
#include <cmath>
#include <mutex>
#include <type_traits>
#include <vector>

#include "common.hpp"
#include "kernels.hpp"
#include "reduce_impl.hpp"

namespace nh {

constexpr int kCBlock = 256;
constexpr int kCUnroll = 4;                // 16-byte vectors in flight per lane
constexpr int64_t kChunkSum = 65536;       // elements per block, sum-of-squares pass (grows past kMaxPartials)
constexpr int64_t kChunkEw = 8192;         // elements per block, read-write passes

struct ClipEntry {
    const void *ptr;
    int64_t n;
    int32_t first_sum;  // first chunk of this tensor in the sum pass
    int32_t first_ew;   // first chunk of this tensor in the read-write passes
    int32_t dtype;
    int32_t pad;
};
static_assert(sizeof(ClipEntry) == 32, "table entry is 32 bytes");

// Decision of the norm pass, written by k_clip_decide.
struct ClipState {
    double total, norm, scale;
    int32_t clip, pad;
};

struct ChunkRef {
    int i;
    int64_t lo, hi;
};

// Lists of up to kInline tensors ride in the kernel arguments; longer ones in
// a device table uploaded per call.
constexpr int kInline = 32;
struct InlineTab {
    ClipEntry e[kInline];
};
NH_DEV const ClipEntry &entry(const InlineTab &t, int i) { return t.e[i]; }
NH_DEV const ClipEntry &entry(const ClipEntry *t, int i) { return t[i]; }

// Tensor and element range of chunk b: the last entry whose first chunk is <= b.
template <bool SUM, class Tab>
NH_DEV ChunkRef chunk_of(const Tab &tab, int count, int64_t chunk, int b)
{
    int lo = 0, hi = count - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        const int f = SUM ? entry(tab, mid).first_sum : entry(tab, mid).first_ew;
        if (f <= b) lo = mid;
        else hi = mid - 1;
    }
    const int f = SUM ? entry(tab, lo).first_sum : entry(tab, lo).first_ew;
    const int64_t s = int64_t(b - f) * chunk;
    const int64_t n = entry(tab, lo).n;
    return {lo, s, s + chunk < n ? s + chunk : n};
}

// s + (double)g * (double)g: the square of a float is exact in double, so the
// fused form equals the reference's mulsd + addsd; the f64 square is rounded
// on its own as in the reference.
NH_DEV double sq_acc(double s, float g)
{
    const double d = double(g);
    return __builtin_fma(d, d, s);
}
NH_DEV double sq_acc(double s, double g)
{
    const double q = g * g;
    return s + q;
}

template <typename T>
NH_DEV double chunk_sumsq(const T *__restrict__ x, int64_t lo, int64_t hi)
{
    using V = typename Vec16<T>::type;
    constexpr int VN = Vec16<T>::n;
    double s0 = 0.0, s1 = 0.0;
    int64_t tail = lo;
    if ((reinterpret_cast<uintptr_t>(x) & 15u) == 0) {  // lo is a multiple of the chunk, hence of VN
        const V *xv = reinterpret_cast<const V *>(x);
        const int64_t v0 = lo / VN, v1 = hi / VN;
        for (int64_t c = v0 + threadIdx.x; c < v1; c += int64_t(kCBlock) * kCUnroll) {
            V a[kCUnroll];
#pragma unroll
            for (int u = 0; u < kCUnroll; u++) {
                const int64_t i = c + int64_t(u) * kCBlock;
                if (i < v1) a[u] = ld_nt(xv + i);
            }
#pragma unroll
            for (int u = 0; u < kCUnroll; u++) {
                const int64_t i = c + int64_t(u) * kCBlock;
                if (i < v1) {
#pragma unroll
                    for (int k = 0; k < VN; k += 2) {
                        s0 = sq_acc(s0, a[u][k]);
                        s1 = sq_acc(s1, a[u][k + 1]);
                    }
                }
            }
        }
        tail = v1 * VN;
    }
    for (int64_t j = tail + threadIdx.x; j < hi; j += kCBlock) s0 = sq_acc(s0, x[j]);
    return s0 + s1;
}

template <class Tab>
__global__ __launch_bounds__(kCBlock) void k_clip_sumsq(Tab tab, int count, int64_t chunk, double *__restrict__ part)
{
    const ChunkRef r = chunk_of<true>(tab, count, chunk, int(blockIdx.x));
    const ClipEntry &e = entry(tab, r.i);
    const double s = e.dtype == NEURAL_DTYPE_FLOAT32
                         ? chunk_sumsq(static_cast<const float *>(e.ptr), r.lo, r.hi)
                         : chunk_sumsq(static_cast<const double *>(e.ptr), r.lo, r.hi);
    const double w = wave_dsum(s);
    __shared__ double lds[kCBlock / 64];
    if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = w;
    __syncthreads();
    if (threadIdx.x == 0) part[blockIdx.x] = (lds[0] + lds[1]) + (lds[2] + lds[3]);
}

struct SumD {
    using B = double;
    NH_DEV B bident() const { return 0.0; }
    NH_DEV B bcomb(B a, B b) const { return a + b; }
};

// The decision to st (device, read by the scale pass) and, with a ticket, to
// the mapped host result area, so the caller gets the norm without waiting
// for the scale pass.
__global__ __launch_bounds__(kRBlock) void k_clip_decide(const double *__restrict__ part, int nparts,
                                                          double max_norm, ClipState *st, ClipState *host_st,
                                                          Ticket tk)
{
    const double tot = ordered_combine(SumD{}, part, nparts);
    if (threadIdx.x == 0) {
        ClipState c;
        c.total = tot;
        c.norm = sqrt(tot);
        c.clip = c.norm > max_norm ? 1 : 0;
        c.scale = c.clip ? max_norm / c.norm : 1.0;
        c.pad = 0;
        *st = c;
        if (tk.slot) {
            *host_st = c;
            publish(tk);
        }
    }
}

// Elementwise in-place map over [lo, hi) of one tensor.
template <typename T, typename F>
NH_DEV void chunk_map(T *__restrict__ x, int64_t lo, int64_t hi, F f)
{
    using V = typename Vec16<T>::type;
    constexpr int VN = Vec16<T>::n;
    int64_t tail = lo;
    if ((reinterpret_cast<uintptr_t>(x) & 15u) == 0) {
        V *xv = reinterpret_cast<V *>(x);
        const int64_t v0 = lo / VN, v1 = hi / VN;
        // each wave's kCUnroll x 64 vectors contiguous (clip value at 100M f32:
        // 126 us against 128 us with the units strided by the block)
        for (int64_t c = v0 + (threadIdx.x >> 6) * (64 * kCUnroll) + (threadIdx.x & 63); c < v1;
             c += int64_t(kCBlock) * kCUnroll) {
            V a[kCUnroll];
#pragma unroll
            for (int u = 0; u < kCUnroll; u++) {
                const int64_t i = c + int64_t(u) * 64;
                if (i < v1) a[u] = ld_nt(xv + i);
            }
#pragma unroll
            for (int u = 0; u < kCUnroll; u++) {
                const int64_t i = c + int64_t(u) * 64;
                if (i < v1) {
#pragma unroll
                    for (int k = 0; k < VN; k++) a[u][k] = f(a[u][k]);
                    st_nt(xv + i, a[u]);
                }
            }
        }
        tail = v1 * VN;
    }
    for (int64_t j = tail + threadIdx.x; j < hi; j += kCBlock) x[j] = f(x[j]);
}

// g *= scale in place when the decision says so (f32: the scale rounded to
// float and a float multiply).  Blocks stride over the chunks, so the grid is
// one residency wave and a pass that clips nothing ends at once.
template <class Tab>
__global__ __launch_bounds__(kCBlock) void k_clip_scale(Tab tab, int count, int64_t chunk, int64_t blocks,
                                                         const ClipState *__restrict__ st)
{
    if (!st->clip) return;
    const double sd = st->scale;
    const float sf = float(sd);
    for (int64_t b = blockIdx.x; b < blocks; b += gridDim.x) {
        const ChunkRef r = chunk_of<false>(tab, count, chunk, int(b));
        const ClipEntry &e = entry(tab, r.i);
        if (e.dtype == NEURAL_DTYPE_FLOAT32)
            chunk_map(static_cast<float *>(const_cast<void *>(e.ptr)), r.lo, r.hi, [sf](float g) { return g * sf; });
        else
            chunk_map(static_cast<double *>(const_cast<void *>(e.ptr)), r.lo, r.hi, [sd](double g) { return g * sd; });
    }
}

template <typename T>
NH_DEV T clamp_sse(T g, T lo, T hi)
{
    const T t = g > lo ? g : lo;
    return t < hi ? t : hi;
}

template <class Tab>
__global__ __launch_bounds__(kCBlock) void k_clip_value(Tab tab, int count, int64_t chunk, int64_t blocks, double lo,
                                                         double hi)
{
    const float l = float(lo), h = float(hi);
    for (int64_t b = blockIdx.x; b < blocks; b += gridDim.x) {
        const ChunkRef r = chunk_of<false>(tab, count, chunk, int(b));
        const ClipEntry &e = entry(tab, r.i);
        if (e.dtype == NEURAL_DTYPE_FLOAT32)
            chunk_map(static_cast<float *>(const_cast<void *>(e.ptr)), r.lo, r.hi,
                      [l, h](float g) { return clamp_sse(g, l, h); });
        else
            chunk_map(static_cast<double *>(const_cast<void *>(e.ptr)), r.lo, r.hi,
                      [lo, hi](double g) { return clamp_sse(g, lo, hi); });
    }
}

// ---- host side ------------------------------------------------------------------------

// The entry table: a pinned host staging buffer and its device copy, both
// grow-only and kept for the process.  The event guards the staging buffer
// until the previous upload has left it.
struct TableBuf {
    std::mutex mu;
    ClipEntry *host = nullptr;
    ClipEntry *dev = nullptr;
    size_t cap = 0;
    hipEvent_t ev = nullptr;
};

static TableBuf &table_buf()
{
    static TableBuf *t = new TableBuf();  // never destroyed: kernels may outlive static dtors
    return *t;
}

struct GradRef {
    NeuralTensor *t;
    void *d;
    int64_t n;
    int dtype;
};

// Non-null, non-empty gradients with their device addresses (made current on
// the device for an in-place update).  NULL entries are skipped as the
// reference skips parameters without a gradient (optimizers.asm:1396-1403).
static int gather(NeuralTensor *const *grads, int64_t count, std::vector<GradRef> &out)
{
    if (count < 0) return set_error(NEURAL_ERR_INVALID_ARGUMENT);
    if (count > 0 && !grads) return set_error(NEURAL_ERR_NULL_POINTER);
    for (int64_t i = 0; i < count; i++) {
        NeuralTensor *t = grads[i];
        if (!t) continue;
        NH_TRY(check_tensor(t));
        if (!is_contiguous(t)) return set_error(NEURAL_ERR_INVALID_ARGUMENT);
        const int64_t n = numel(t);
        if (n == 0) continue;
        // more tensors than the sum pass has partials: refused before the
        // list grows further
        if (int64_t(out.size()) >= kMaxPartials) return set_error(NEURAL_ERR_INVALID_ARGUMENT);
        out.push_back({t, nullptr, n, t->dtype});
    }
    for (GradRef &g : out) NH_TRY(dev_write(g.t, &g.d, false));
    return NEURAL_OK;
}

struct Plan {
    InlineTab inl;          // the table when count <= kInline
    const ClipEntry *tab;   // else the device table
    int count;
    int64_t chunk_sum, chunk_ew;
    int64_t blocks_sum, blocks_ew;
    unsigned grid_ew;       // scale pass: one residency wave at most (it usually exits at once)
    unsigned grid_value;    // clamp pass: one block per chunk (it always works)
    template <class F>
    void with_tab(F f) const
    {
        if (count <= kInline) f(inl);
        else f(tab);
    }
};

// Chunk sizes, block counts and the uploaded table for a gradient list.
static int make_plan(const std::vector<GradRef> &g, Plan &p)
{
    int64_t cs = kChunkSum;
    for (;;) {
        int64_t c = 0;
        for (const GradRef &e : g) c += ceil_div(e.n, cs);
        if (c <= kMaxPartials) break;
        cs *= 2;
    }
    int64_t ce = kChunkEw, be = 0;
    for (;;) {
        be = 0;
        for (const GradRef &e : g) be += ceil_div(e.n, ce);
        if (be < (int64_t(1) << 31)) break;  // chunk indices are int32
        ce *= 2;
    }
    const size_t need = g.size();
    auto fill = [&](ClipEntry *out) {
        int64_t fs = 0, fe = 0;
        for (size_t i = 0; i < need; i++) {
            ClipEntry &e = out[i];
            e.ptr = g[i].d;
            e.n = g[i].n;
            e.first_sum = int32_t(fs);
            e.first_ew = int32_t(fe);
            e.dtype = g[i].dtype;
            e.pad = 0;
            fs += ceil_div(g[i].n, cs);
            fe += ceil_div(g[i].n, ce);
        }
        p.blocks_sum = fs;
        p.blocks_ew = fe;
    };
    p.count = int(need);
    p.chunk_sum = cs;
    p.chunk_ew = ce;
    p.tab = nullptr;
    if (need <= size_t(kInline)) {
        std::memset(&p.inl, 0, sizeof(p.inl));
        fill(p.inl.e);
    } else {
        TableBuf &tb = table_buf();
        std::lock_guard<std::mutex> lock(tb.mu);
        if (!tb.ev) NH_HIP(hipEventCreateWithFlags(&tb.ev, hipEventDisableTiming));
        NH_HIP(hipEventSynchronize(tb.ev));  // the previous upload has left the staging buffer
        if (need > tb.cap) {
            const size_t cap = need < 256 ? 256 : need;
            if (tb.host) NH_HIP(hipHostFree(tb.host));
            if (tb.dev) dev_free(tb.dev);
            tb.host = nullptr;
            tb.dev = nullptr;
            tb.cap = 0;
            NH_HIP(hipHostMalloc(reinterpret_cast<void **>(&tb.host), cap * sizeof(ClipEntry), hipHostMallocDefault));
            tb.dev = static_cast<ClipEntry *>(dev_alloc(cap * sizeof(ClipEntry)));
            if (!tb.dev) return set_error(NEURAL_ERR_OUT_OF_MEMORY);
            tb.cap = cap;
        }
        fill(tb.host);
        NH_HIP(hipMemcpyAsync(tb.dev, tb.host, need * sizeof(ClipEntry), hipMemcpyHostToDevice, stream()));
        NH_HIP(hipEventRecord(tb.ev, stream()));
        p.tab = tb.dev;
    }
    const int64_t wave = int64_t(num_cus()) * (2048 / kCBlock);  // resident 256-lane blocks per residency wave
    p.grid_ew = unsigned(p.blocks_ew < wave ? p.blocks_ew : wave);
    // measured at 100M f32: the clamp pass 135.5 -> 128.5 us with a block per
    // chunk; the scale pass keeps one residency wave, since a pass that clips
    // nothing (the common case) then costs ~3 us less per call
    p.grid_value = unsigned(p.blocks_ew < kMaxGridBlocks ? p.blocks_ew : kMaxGridBlocks);
    return NEURAL_OK;
}

static int written_all(const std::vector<GradRef> &g)
{
    for (const GradRef &e : g) NH_TRY(dev_written(e.t));
    return NEURAL_OK;
}

int clip_norm_list(NeuralTensor *const *grads, int64_t count, double max_norm, double *total_norm)
{
    NH_TRY(ensure_init());
    std::vector<GradRef> g;
    NH_TRY(gather(grads, count, g));
    if (g.empty()) {
        // sqrt(0) = 0 and nothing to scale.
        if (total_norm) *total_norm = 0.0;
        return set_error(NEURAL_OK);
    }
    Plan p;
    NH_TRY(make_plan(g, p));
    WsGuard wg;
    double *part = static_cast<double *>(workspace().partials);
    ClipState *st = static_cast<ClipState *>(workspace().result);
    p.with_tab([&](const auto &tab) {
        using Tab = std::decay_t<decltype(tab)>;
        NH_LAUNCH(k_clip_sumsq<Tab>, dim3(unsigned(p.blocks_sum)), dim3(kCBlock), 0, stream(), tab,
                           p.count, p.chunk_sum, part);
    });
    NH_TRY(check_launch());
    const Ticket tk = total_norm ? next_ticket() : Ticket{};
    NH_LAUNCH(k_clip_decide, dim3(1), dim3(kRBlock), 0, stream(), part, int(p.blocks_sum), max_norm, st,
              static_cast<ClipState *>(workspace().host_result_dev), tk);
    NH_TRY(check_launch());
    p.with_tab([&](const auto &tab) {
        using Tab = std::decay_t<decltype(tab)>;
        NH_LAUNCH(k_clip_scale<Tab>, dim3(p.grid_ew), dim3(kCBlock), 0, stream(), tab, p.count, p.chunk_ew,
                           p.blocks_ew, st);
    });
    NH_TRY(check_launch());
    if (total_norm) {
        // the scale pass may still run: later work on the stream (and any
        // host read of the tensors, which synchronises) comes after it
        ClipState h;
        NH_TRY(host_result_wait(tk.value, &h, sizeof(h)));
        *total_norm = h.norm;
    }
    NH_TRY(written_all(g));
    return set_error(NEURAL_OK);
}

int clip_value_list(NeuralTensor *const *grads, int64_t count, double lo, double hi)
{
    NH_TRY(ensure_init());
    std::vector<GradRef> g;
    NH_TRY(gather(grads, count, g));
    if (g.empty()) return set_error(NEURAL_OK);
    Plan p;
    NH_TRY(make_plan(g, p));
    p.with_tab([&](const auto &tab) {
        using Tab = std::decay_t<decltype(tab)>;
        NH_LAUNCH(k_clip_value<Tab>, dim3(p.grid_value), dim3(kCBlock), 0, stream(), tab, p.count, p.chunk_ew,
                           p.blocks_ew, lo, hi);
    });
    NH_TRY(check_launch());
    NH_TRY(written_all(g));
    return set_error(NEURAL_OK);
}

}  // namespace nh

using namespace nh;

extern "C" {

int neural_clip_grad_norm_list(NeuralTensor **grads, int64_t n, double max_norm, double *total_norm)
{
    return clip_norm_list(grads, n, max_norm, total_norm);
}

int neural_clip_grad_value_list(NeuralTensor **grads, int64_t n, double min_val, double max_val)
{
    return clip_value_list(grads, n, min_val, max_val);
}

}  // extern "C"
