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
// passes of 8-bit histograms -- one for each rank, counting only the
// elements that match the rank's prefix so far -- fix the keys byte by byte.
// Equal keys are equal doubles except for the zero key: the reference's qsort
// (glibc's merge sort, which is stable) keeps equal elements in input order,
// so a selected zero takes the sign of the j-th zero of the input, j the
// rank's position among the zeros; two more launches find it (zero counts per
// chunk, then one wave walks the chunk that holds it).  The parameter
// arithmetic then runs on the host in the reference's expressions.
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
__device__ __forceinline__ uint64_t pct_key(double x)
{
    uint64_t b = uint64_t(__double_as_longlong(x));
    if (x != x) return ~uint64_t(0);
    if ((b << 1) == 0) b = 0;  // -0 -> +0: they compare equal
    return (b >> 63) ? ~b : (b | (uint64_t(1) << 63));
}

constexpr uint64_t kZeroKey = uint64_t(1) << 63;  // pct_key(+0) == pct_key(-0)

double key_value(uint64_t k)
{
    if (k == ~uint64_t(0)) return std::nan("");
    const uint64_t b = (k >> 63) ? (k & ~(uint64_t(1) << 63)) : ~k;
    double v;
    std::memcpy(&v, &b, 8);
    return v;
}

// Histograms of byte (key >> shift) & 255 over the elements whose key matches
// pre0 (counts 0..255) and pre1 (counts 256..511) under mask.
__global__ __launch_bounds__(kPB) void k_pct_hist(const double *__restrict__ x, int64_t n, int shift,
                                                   uint64_t mask, uint64_t pre0, uint64_t pre1,
                                                   unsigned long long *__restrict__ hist)
{
    __shared__ unsigned h[512];
    for (int i = threadIdx.x; i < 512; i += kPB) h[i] = 0u;
    __syncthreads();
    for (int64_t i = int64_t(blockIdx.x) * kPB + threadIdx.x; i < n; i += int64_t(gridDim.x) * kPB) {
        const uint64_t k = pct_key(x[i]);
        const unsigned d = unsigned(k >> shift) & 255u;
        if ((k & mask) == pre0) atomicAdd(&h[d], 1u);
        if ((k & mask) == pre1) atomicAdd(&h[256 + d], 1u);
    }
    __syncthreads();
    for (int i = threadIdx.x; i < 512; i += kPB)
        if (h[i]) atomicAdd(&hist[i], (unsigned long long)h[i]);
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
static int select_ranks(const double *x, int64_t n, const int64_t r[2], uint64_t key[2], int64_t within[2])
{
    auto *hist = static_cast<unsigned long long *>(dev_alloc(512 * sizeof(unsigned long long)));
    if (!hist) return set_error(NEURAL_ERR_OUT_OF_MEMORY);
    std::vector<unsigned long long> h(512);
    uint64_t pre[2] = {0, 0}, mask = 0;
    int64_t rem[2] = {r[0], r[1]};
    int64_t g = ceil_div(n, kPB);
    if (g > int64_t(num_cus()) * 4) g = int64_t(num_cus()) * 4;
    int rc = NEURAL_OK;
    for (int pass = 0; pass < 8 && rc == NEURAL_OK; pass++) {
        const int shift = 56 - 8 * pass;
        if (hipMemsetAsync(hist, 0, 512 * sizeof(unsigned long long), stream()) != hipSuccess) {
            rc = NEURAL_ERR_INTERNAL;
            break;
        }
        hipLaunchKernelGGL(k_pct_hist, dim3(unsigned(g)), dim3(kPB), 0, stream(), x, n, shift, mask, pre[0], pre[1],
                           hist);
        rc = check_launch();
        if (rc == NEURAL_OK && hipMemcpyAsync(h.data(), hist, 512 * sizeof(unsigned long long),
                                              hipMemcpyDeviceToHost, stream()) != hipSuccess)
            rc = NEURAL_ERR_INTERNAL;
        if (rc == NEURAL_OK) rc = sync();
        for (int q = 0; q < 2 && rc == NEURAL_OK; q++) {
            int64_t cum = 0;
            int d = 0;
            for (; d < 256; d++) {
                const int64_t c = int64_t(h[size_t(q) * 256 + size_t(d)]);
                if (rem[q] < cum + c) break;
                cum += c;
            }
            if (d == 256) rc = NEURAL_ERR_INTERNAL;  // counts lost: cannot happen for a valid rank
            pre[q] |= uint64_t(d) << shift;
            rem[q] -= cum;
        }
        mask |= uint64_t(255) << shift;
    }
    dev_free(hist);
    if (rc != NEURAL_OK) return set_error(rc);
    for (int q = 0; q < 2; q++) {
        key[q] = pre[q];
        within[q] = rem[q];
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
    hipLaunchKernelGGL(k_pct_zero_count, dim3(unsigned(nch)), dim3(kPB), 0, stream(), x, n, counts);
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
        hipLaunchKernelGGL(k_pct_zero_pick, dim3(1), dim3(64), 0, stream(), x, c0, c1, unsigned(j), dsign);
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
    if (s.open(data, size_t(n) * sizeof(double), true) != NEURAL_OK) return -1;
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
