// percentile.hip -- calibrate_percentile (quantize.c:89-132).
//
// The reference sorts a copy of the data with qsort and the comparator
// (a > b) - (a < b) (quantize.c:31-35, 99), takes clipped_min = sorted[lo],
// clipped_max = sorted[hi] with lo = (int64)(n p), hi = (int64)(n (1 - p))
// (clamped to [0, n - 1]; p outside [0, 0.5] taken as 0.01) and calibrates on
// that range with the same expressions as calibrate_minmax.
//
// Here the two order statistics are found by a radix select on the device,
// never sorting: each element maps to a 64-bit key that orders as the
// comparator does (-0 and +0 compare equal, so they share one key), and eight
// histogram passes -- 12 bits (sign and exponent), six of 8 bits, 4 bits; one
// histogram for each rank, counting only the elements that match the rank's
// prefix so far -- fix the keys digit by digit;
// once few elements match, their keys are copied out and the remaining
// passes read only those copies.  A one-block step after each pass picks the
// byte on the device, so the host waits once per call.
// Equal keys are equal doubles except for the zero key: the reference's qsort
// (glibc's merge sort, stable while its n * 8-byte copy fits in about a
// quarter of physical memory) keeps equal elements in input order, so a
// selected zero takes the sign of the j-th zero of the input, j the rank's
// position among the zeros; two more launches find it (zero counts per chunk,
// then one wave walks the chunk that holds it).  Beyond that size glibc falls
// back to an unstable in-place sort and the reference's zero sign no longer
// follows input order.  The parameter arithmetic then runs on the host in the
// reference's expressions.
//
// Divergences (the reference's behaviour is undefined there): a NaN
// percentile returns -1 (the reference indexes out of bounds); NaN data sort
// above +inf (the reference's comparator orders NaN inconsistently, so its
// result depends on the sort's internals).
#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>

#include "common.hpp"
#include "quant_common.hpp"

namespace nh {

namespace {

constexpr int kPB = 256;               // threads per block
constexpr int64_t kZChunk = 1 << 16;   // elements per zero-count chunk

// Key ordering doubles as the comparator does; NaN takes the largest key.
// Integer selects only (no branch), so that loads can be hoisted past it.
__device__ __forceinline__ uint64_t pct_key_bits(uint64_t b)
{
    const uint64_t mag = b & ~(uint64_t(1) << 63);
    b = mag == 0 ? 0 : b;  // -0 -> +0: they compare equal
    const uint64_t k = (b >> 63) ? ~b : (b | (uint64_t(1) << 63));
    return mag > 0x7FF0000000000000ull ? ~uint64_t(0) : k;
}

constexpr uint64_t kZeroKey = uint64_t(1) << 63;  // key of +0 and of -0

double key_value(uint64_t k)
{
    if (k == ~uint64_t(0)) return std::nan("");
    const uint64_t b = (k >> 63) ? (k & ~(uint64_t(1) << 63)) : ~k;
    double v;
    std::memcpy(&v, &b, 8);
    return v;
}

constexpr int kPU = 8;                // elements per thread per tile (loads in flight)
constexpr int kTile = kPB * kPU;      // elements per block tile
constexpr int64_t kRegion = 2 * kTile; // copied keys per block, at most
constexpr int kPasses = 8;
constexpr int kMaxBins = 4096;

// Digits: the first pass takes the top 12 bits (sign and exponent), so that
// for most data few elements match after it; then 8-bit digits, and 4 last.
__host__ __device__ constexpr int pass_bits(int p) { return p == 0 ? 12 : (p == kPasses - 1 ? 4 : 8); }
__host__ __device__ constexpr int pass_shift(int p) { return p == 0 ? 52 : (p == kPasses - 1 ? 0 : 52 - 8 * p); }
static_assert(pass_shift(kPasses - 2) == 4 && pass_bits(kPasses - 2) == 8, "digits must tile the 64-bit key");

// h[d] += 1 for every lane with m set.  The first three distinct bytes of the
// wave each take one atomic for all their lanes (the leading passes see few
// distinct bytes: sign and exponent bits), the rest one atomic per lane.
__device__ __forceinline__ void hist_add(unsigned *h, bool m, unsigned d)
{
    uint64_t rem = __ballot(m);
#pragma unroll
    for (int it = 0; it < 3; it++) {
        if (rem == 0) return;
        const int leader = __builtin_ctzll(rem);
        const unsigned dl = __builtin_amdgcn_readlane(d, leader);
        const uint64_t same = __ballot(m && d == dl);
        if (int(threadIdx.x & 63) == leader) atomicAdd(&h[dl], unsigned(__popcll(same)));
        m = m && d != dl;
        rem &= ~same;
    }
    if (m) atomicAdd(&h[d], 1u);
}

// Select state, in device memory, carried from pass to pass.
struct PctState {
    uint64_t pre[2];   // key prefixes of the two ranks (bytes fixed so far)
    uint64_t mask;     // bits of the key fixed so far
    int64_t rem[2];    // rank within the elements matching pre[q]
    int64_t matched;   // elements matching either prefix
    int cur;           // key buffer holding every matching element, -1: none
    int copy;          // this pass copies its matches into buffer dst
    int dst;
    int err;           // a rank fell outside its histogram (cannot happen)
};

// Fixed-size record the host reads at the end.
struct PctResult {
    uint64_t key[2];
    int64_t within[2];
    int err;
};

// The pass body.  KEYS = false: the doubles, block b taking tiles b, b + grid,
// ... of kTile elements.  KEYS = true: keys copied out by an earlier pass,
// block b reading its own region [b R, b R + cnt_in[b]).  h[0..nb) counts
// digit (key >> shift) & (nb - 1) of the elements whose key matches pre0
// under mask, h[nb..2 nb) likewise for pre1 (left at zero when pre1 == pre0:
// the two would be equal).  With out set, the elements matching either prefix are
// also copied to block b's region of out (slots below R) and cnt_out[b] is
// how many matched; above R only on a first copy from the doubles, which is
// then discarded.
template <bool KEYS>
__device__ __forceinline__ void pct_pass_body(const void *__restrict__ src, int64_t n,
                                              const unsigned *__restrict__ cnt_in, int64_t R, int shift,
                                              unsigned dmask, uint64_t mask, uint64_t pre0, uint64_t pre1, unsigned *h,
                                              unsigned &nout, uint64_t *__restrict__ out)
{
    const int lane = int(threadIdx.x & 63);
    const bool two = pre1 != pre0;
    int64_t t0, hi, step;
    if (KEYS) {
        t0 = int64_t(blockIdx.x) * R;
        hi = t0 + int64_t(cnt_in[blockIdx.x]);
        step = kTile;
    } else {
        t0 = int64_t(blockIdx.x) * kTile;
        hi = n;
        step = int64_t(gridDim.x) * kTile;
    }
    for (; t0 < hi; t0 += step) {
        uint64_t k[kPU];
        bool v[kPU];
        // Past the end a lane re-reads the last element (hi > t0 >= 0 here) and
        // is masked by v: unconditional loads stay in flight together.
#pragma unroll
        for (int u = 0; u < kPU; u++) {
            const int64_t i = t0 + u * kPB + int64_t(threadIdx.x);
            v[u] = i < hi;
            const int64_t ic = v[u] ? i : hi - 1;
            k[u] = KEYS ? static_cast<const uint64_t *>(src)[ic]
                        : __builtin_nontemporal_load(static_cast<const uint64_t *>(src) + ic);
        }
        if (!KEYS) {
#pragma unroll
            for (int u = 0; u < kPU; u++) k[u] = pct_key_bits(k[u]);
        }
        uint64_t bal[kPU];
#pragma unroll
        for (int u = 0; u < kPU; u++) {
            const bool m0 = v[u] && (k[u] & mask) == pre0;
            const bool m1 = v[u] && (k[u] & mask) == pre1;
            const unsigned d = unsigned(k[u] >> shift) & dmask;
            hist_add(h, m0, d);
            if (two) hist_add(h + dmask + 1, m1, d);
            bal[u] = __ballot(m0 || m1);
        }
        if (out) {
            // one slot reservation per wave and tile
            unsigned total = 0u;
#pragma unroll
            for (int u = 0; u < kPU; u++) total += unsigned(__popcll(bal[u]));
            if (total) {
                unsigned base = 0u;
                if (lane == 0) base = atomicAdd(&nout, total);
                base = __builtin_amdgcn_readfirstlane(base);
                const uint64_t below = (uint64_t(1) << lane) - 1;
#pragma unroll
                for (int u = 0; u < kPU; u++) {
                    const int64_t slot = int64_t(base) + __popcll(bal[u] & below);
                    if (((bal[u] >> lane) & 1) && slot < R) out[int64_t(blockIdx.x) * R + slot] = k[u];
                    base += unsigned(__popcll(bal[u]));
                }
            }
        }
    }
}

// One radix pass over the doubles or, once they exist, the copied keys; the
// prefixes and the copy decision come from the state the previous select
// step wrote.  Adds the block's counts into hist and, when copying, stores
// the block's match count into cnt[dst][b].
__global__ __launch_bounds__(kPB) void k_pct_pass(const double *__restrict__ x, int64_t n, int64_t R, int pass,
                                                   const PctState *__restrict__ st,
                                                   unsigned long long *__restrict__ hist, uint64_t *keys0,
                                                   uint64_t *keys1, unsigned *cnt0, unsigned *cnt1)
{
    __shared__ unsigned h[kMaxBins];
    __shared__ unsigned nout;
    const int shift = pass_shift(pass);
    const int nb = 1 << pass_bits(pass);
    const int nh = st->pre[1] != st->pre[0] ? 2 * nb : nb;
    for (int i = threadIdx.x; i < nh; i += kPB) h[i] = 0u;
    if (threadIdx.x == 0) nout = 0u;
    __syncthreads();
    const int cur = st->cur, dst = st->dst;
    uint64_t *out = st->copy ? (dst ? keys1 : keys0) : nullptr;
    if (cur >= 0)
        pct_pass_body<true>(cur ? keys1 : keys0, n, cur ? cnt1 : cnt0, R, shift, unsigned(nb - 1), st->mask,
                            st->pre[0], st->pre[1], h, nout, out);
    else
        pct_pass_body<false>(x, n, nullptr, R, shift, unsigned(nb - 1), st->mask, st->pre[0], st->pre[1], h, nout,
                             out);
    __syncthreads();
    for (int i = threadIdx.x; i < nh; i += kPB)
        if (h[i]) atomicAdd(&hist[i], (unsigned long long)h[i]);
    if (out && threadIdx.x == 0) (dst ? cnt1 : cnt0)[blockIdx.x] = nout;
}

// Initial state for ranks r0, r1 of n elements; clears the histogram.
__global__ __launch_bounds__(64) void k_pct_init(PctState *st, unsigned long long *hist, int64_t r0, int64_t r1,
                                                 int64_t n)
{
    for (int i = threadIdx.x; i < kMaxBins; i += 64) hist[i] = 0ull;
    if (threadIdx.x == 0) {
        PctState s;
        s.pre[0] = s.pre[1] = 0;
        s.mask = 0;
        s.rem[0] = r0;
        s.rem[1] = r1;
        s.matched = n;
        s.cur = -1;
        s.copy = 0;
        s.dst = 0;
        s.err = 0;
        *st = s;
    }
}

// After pass `pass`: fix each rank's digit from the histogram, take over the
// copied keys if every block's matches fitted its region, decide whether the
// next pass copies, clear the histogram.  One wave; lane l holds bins
// [l PER, (l + 1) PER) of each histogram in registers (PER = nb / 64, or 1 for
// the 16-bin last digit, lanes past the bins holding none); every lane
// computes the same new state from a scan over the lanes and lane 0 stores
// it.  The last pass also writes the result record (res, host-visible memory).
template <int PER>
__global__ __launch_bounds__(64) void k_pct_select(PctState *st, unsigned long long *hist, const unsigned *cnt0,
                                                   const unsigned *cnt1, int64_t g, int64_t R, int pass,
                                                   PctResult *res)
{
    const int lane = int(threadIdx.x);
    const int shift = pass_shift(pass), nb = 1 << pass_bits(pass);
    const bool mine = lane * PER < nb;  // this lane holds bins
    PctState s = *st;
    const bool same = s.pre[1] == s.pre[0];  // the pass built one histogram for both
    int64_t hb[2][PER];
#pragma unroll
    for (int q = 0; q < 2; q++) {
        const unsigned long long *hq = hist + (same ? 0 : nb * q) + lane * PER;
#pragma unroll
        for (int j = 0; j < PER; j++) hb[q][j] = mine ? int64_t(hq[j]) : 0;
    }
    // first copy from the doubles: did every block's matches fit its region?
    bool fits = true;
    if (s.copy && s.cur < 0) {
        const unsigned *c = s.dst ? cnt1 : cnt0;
        for (int64_t b = lane; b < g; b += 64) fits = fits && int64_t(c[b]) <= R;
        fits = __ballot(!fits) == 0;
    }
    if (mine) {
#pragma unroll
        for (int j = 0; j < PER; j++) {
            hist[lane * PER + j] = 0ull;
            if (!same) hist[nb + lane * PER + j] = 0ull;
        }
    }
    if (s.copy && fits) s.cur = s.dst;
    int64_t c[2] = {0, 0};
#pragma unroll
    for (int q = 0; q < 2; q++) {
        int64_t ls = 0;
#pragma unroll
        for (int j = 0; j < PER; j++) ls += hb[q][j];
        int64_t inc = ls;  // inclusive scan over the lanes
        for (int off = 1; off < 64; off <<= 1) {
            const int64_t t = __shfl_up(inc, off);
            if (lane >= off) inc += t;
        }
        const uint64_t hit = __ballot(s.rem[q] < inc);
        int d = 0;
        int64_t cnt = 0, below = 0;
        if (hit == 0) {
            s.err = 1;  // counts lost: cannot happen for a valid rank
        } else {
            // the first lane whose bins reach the rank holds it
            const int L = __builtin_ctzll(hit);
            below = inc - ls;
            int jj = PER - 1;
            bool found = false;
#pragma unroll
            for (int j = 0; j < PER; j++) {
                const bool here = !found && s.rem[q] < below + hb[q][j];
                if (here) {
                    jj = j;
                    cnt = hb[q][j];
                    found = true;
                }
                if (!found) below += hb[q][j];
            }
            d = __shfl(L * PER + jj, L);
            cnt = __shfl(cnt, L);
            below = __shfl(below, L);
        }
        c[q] = cnt;
        s.pre[q] |= uint64_t(d) << shift;
        s.rem[q] -= below;
    }
    s.matched = s.pre[0] == s.pre[1] ? c[0] : c[0] + c[1];
    s.mask |= uint64_t(nb - 1) << shift;
    // A run of consecutive matches of at most g R / 2 <= g kTile elements
    // covers at most g + 1 tiles, dealt round-robin: at most 2 tiles per
    // block, within a region of 2 (or, for small n, regions that hold a
    // block's whole share).
    s.copy = s.cur >= 0 || s.matched <= g * R / 2;
    s.dst = s.cur >= 0 ? 1 - s.cur : 0;
    if (lane != 0) return;
    *st = s;
    if (res) {
        PctResult r;
        for (int q = 0; q < 2; q++) {
            r.key[q] = s.pre[q];
            r.within[q] = s.rem[q];
        }
        r.err = s.err;
        *res = r;
    }
}

// counts[c] = zeros (either sign) in elements [c * kZChunk, (c + 1) * kZChunk).
__global__ __launch_bounds__(kPB) void k_pct_zero_count(const double *__restrict__ x, int64_t n,
                                                        unsigned *__restrict__ counts)
{
    const int64_t c0 = int64_t(blockIdx.x) * kZChunk;
    const int64_t c1 = c0 + kZChunk < n ? c0 + kZChunk : n;
    unsigned s = 0u;
    for (int64_t i = c0 + threadIdx.x; i < c1; i += kPB) s += x[i] == 0.0 ? 1u : 0u;
    __shared__ unsigned sh[kPB];
    sh[threadIdx.x] = s;
    __syncthreads();
    for (int off = kPB / 2; off > 0; off >>= 1) {
        if (int(threadIdx.x) < off) sh[threadIdx.x] += sh[threadIdx.x + off];
        __syncthreads();
    }
    if (threadIdx.x == 0) counts[blockIdx.x] = sh[0];
}

// One wave walks [c0, c1) in order and stores the sign bit (0 / 1) of its
// j-th zero into *sign (j < the chunk's zero count, so the walk finds it).
__global__ __launch_bounds__(64) void k_pct_zero_pick(const double *__restrict__ x, int64_t c0, int64_t c1,
                                                      unsigned j, int *__restrict__ sign)
{
    const int lane = threadIdx.x;
    for (int64_t base = c0; base < c1; base += 64) {
        const int64_t i = base + lane;
        const bool z = i < c1 && x[i] == 0.0;
        const uint64_t m = __ballot(z);
        const unsigned cnt = unsigned(__popcll(m));
        if (j < cnt) {
            // lane holding the j-th set bit of m
            const uint64_t below = lane == 0 ? 0 : (m & ((uint64_t(1) << lane) - 1));
            if (z && unsigned(__popcll(below)) == j) *sign = __builtin_signbit(x[i]) ? 1 : 0;
            return;
        }
        j -= cnt;
    }
}

}  // namespace

// Keys of the elements at ranks r[0], r[1] of the comparator's order, and the
// rank within its run of equal keys (rank - elements with a smaller key).
// Eight passes fix the keys a digit at a time, each followed by a one-block
// select step that updates the state on the device, so the host waits once.
// Once few enough elements match the two prefixes (at most half the copy
// area, so that a run of consecutive matches spread over the tiles fits every
// block's region), a pass also copies their keys out, and the later
// passes read only the copies, each copying its own matches on into the
// other buffer.
static int select_ranks(const double *x, int64_t n, const int64_t r[2], uint64_t key[2], int64_t within[2])
{
    const int64_t tiles = ceil_div(n, int64_t(kTile));
    int64_t g = int64_t(num_cus()) * 8;
    if (g > tiles) g = tiles;
    int64_t R = ceil_div(tiles, g) * kTile;
    if (R > kRegion) R = kRegion;
    // [state][hist kMaxBins x u64][counts 2 x g x u32][keys 2 x g x R x u64]
    const size_t st_b = 256, hist_b = kMaxBins * sizeof(unsigned long long), cnt_b = size_t(2 * g) * sizeof(unsigned);
    const size_t keys_off = (st_b + hist_b + cnt_b + 255) / 256 * 256;
    char *ws = static_cast<char *>(dev_alloc(keys_off + size_t(2 * g * R) * sizeof(uint64_t)));
    if (!ws) return set_error(NEURAL_ERR_OUT_OF_MEMORY);
    auto *st = reinterpret_cast<PctState *>(ws);
    auto *hist = reinterpret_cast<unsigned long long *>(ws + st_b);
    unsigned *cnt0 = reinterpret_cast<unsigned *>(ws + st_b + hist_b), *cnt1 = cnt0 + g;
    uint64_t *keys0 = reinterpret_cast<uint64_t *>(ws + keys_off), *keys1 = keys0 + g * R;
    static_assert(sizeof(PctResult) <= 256, "result record exceeds the host result area");
    WsGuard wg;
    auto *res = static_cast<PctResult *>(workspace().host_result_dev);
    NH_LAUNCH(k_pct_init, dim3(1), dim3(64), 0, stream(), st, hist, r[0], r[1], n);
    int rc = check_launch();
    for (int pass = 0; pass < kPasses && rc == NEURAL_OK; pass++) {
        NH_LAUNCH(k_pct_pass, dim3(unsigned(g)), dim3(kPB), 0, stream(), x, n, R, pass, st, hist, keys0,
                           keys1, cnt0, cnt1);
        rc = check_launch();
        if (rc != NEURAL_OK) break;
        PctResult *last = pass == kPasses - 1 ? res : nullptr;
        const int nb = 1 << pass_bits(pass);
        if (nb == 4096)
            NH_LAUNCH(k_pct_select<64>, dim3(1), dim3(64), 0, stream(), st, hist, cnt0, cnt1, g, R, pass, last);
        else if (nb == 256)
            NH_LAUNCH(k_pct_select<4>, dim3(1), dim3(64), 0, stream(), st, hist, cnt0, cnt1, g, R, pass, last);
        else
            NH_LAUNCH(k_pct_select<1>, dim3(1), dim3(64), 0, stream(), st, hist, cnt0, cnt1, g, R, pass, last);
        rc = check_launch();
    }
    PctResult out{};
    if (rc == NEURAL_OK) rc = host_result_fetch(&out, sizeof(out));
    dev_free(ws);
    if (rc != NEURAL_OK) return set_error(rc);
    if (out.err) return set_error(NEURAL_ERR_INTERNAL);  // counts lost: cannot happen for a valid rank
    for (int q = 0; q < 2; q++) {
        key[q] = out.key[q];
        within[q] = out.within[q];
    }
    return NEURAL_OK;
}

// Sign bit of the j-th zero of x in input order.
static int zero_sign(const double *x, int64_t n, int64_t j, int *sign_out)
{
    const int64_t nch = ceil_div(n, kZChunk);
    unsigned *counts = static_cast<unsigned *>(dev_alloc(size_t(nch) * sizeof(unsigned) + sizeof(int)));
    if (!counts) return set_error(NEURAL_ERR_OUT_OF_MEMORY);
    int *dsign = reinterpret_cast<int *>(counts + nch);
    std::vector<unsigned> c(static_cast<size_t>(nch));
    NH_LAUNCH(k_pct_zero_count, dim3(unsigned(nch)), dim3(kPB), 0, stream(), x, n, counts);
    int rc = check_launch();
    if (rc == NEURAL_OK &&
        hipMemcpyAsync(c.data(), counts, size_t(nch) * sizeof(unsigned), hipMemcpyDeviceToHost, stream()) != hipSuccess)
        rc = NEURAL_ERR_INTERNAL;
    if (rc == NEURAL_OK) rc = sync();
    int64_t ch = 0;
    if (rc == NEURAL_OK) {
        for (; ch < nch && j >= int64_t(c[size_t(ch)]); ch++) j -= int64_t(c[size_t(ch)]);
        if (ch == nch) rc = NEURAL_ERR_INTERNAL;
    }
    int sign = 0;
    if (rc == NEURAL_OK) {
        const int64_t c0 = ch * kZChunk, c1 = c0 + kZChunk < n ? c0 + kZChunk : n;
        NH_LAUNCH(k_pct_zero_pick, dim3(1), dim3(64), 0, stream(), x, c0, c1, unsigned(j), dsign);
        rc = check_launch();
        if (rc == NEURAL_OK && hipMemcpyAsync(&sign, dsign, sizeof(int), hipMemcpyDeviceToHost, stream()) != hipSuccess)
            rc = NEURAL_ERR_INTERNAL;
        if (rc == NEURAL_OK) rc = sync();
    }
    dev_free(counts);
    if (rc != NEURAL_OK) return set_error(rc);
    *sign_out = sign;
    return NEURAL_OK;
}

static int calibrate_pct(const double *data, int64_t n, double percentile, int symmetric, QuantParams *out)
{
    if (!data || n <= 0 || !out) return -1;
    if (percentile != percentile) return -1;
    if (percentile < 0.0 || percentile > 0.5) percentile = 0.01;
    if (ensure_init() != NEURAL_OK) return -1;
    int64_t lo_idx = int64_t(double(n) * percentile);
    int64_t hi_idx = int64_t(double(n) * (1.0 - percentile));
    if (lo_idx < 0) lo_idx = 0;
    if (hi_idx >= n) hi_idx = n - 1;
    Staged s;
    if (s.open_n(data, uint64_t(n), sizeof(double), true) != NEURAL_OK) return -1;
    const double *x = static_cast<const double *>(s.dev);
    const int64_t ranks[2] = {lo_idx, hi_idx};
    uint64_t key[2];
    int64_t within[2];
    if (select_ranks(x, n, ranks, key, within) != NEURAL_OK) return -1;
    double v[2];
    for (int q = 0; q < 2; q++) {
        v[q] = key_value(key[q]);
        if (key[q] == kZeroKey) {
            int sign = 0;
            if (zero_sign(x, n, within[q], &sign) != NEURAL_OK) return -1;
            v[q] = sign ? -0.0 : 0.0;
        }
    }
    if (s.finish(false) != NEURAL_OK) return -1;
    // quantize.c:112-129: the epilogue shared with calibrate_minmax
    minmax_epilogue(v[0], v[1], symmetric, out);
    set_error(NEURAL_OK);
    return 0;
}

}  // namespace nh

extern "C" int calibrate_percentile(const double *data, int64_t n, double percentile, int symmetric,
                                    QuantParams *out)
{
    return nh::calibrate_pct(data, n, percentile, symmetric, out);
}
