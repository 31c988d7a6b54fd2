// losses.hip -- cross-entropy losses: label-smoothed CE forward / backward and
// a fused forward+backward, and the tensor cross-entropy loss.
//
// Reference: metrics_losses.c:28-125 (label_smoothing_ce_forward/backward,
// f64 logits, int64 targets):
//   m = max (strict compare from row[0]); lse = log(sum_c exp(x_c - m));
//   st_c = a/K + (c == t ? 1 - a : 0); loss_row = -sum_c st_c * ((x_c - m) - lse);
//   loss = sum_rows / B;   grad_c = (1/B) * (exp(x_c - m) / sum - st_c)
// and losses.asm:315-613 (cross_entropy_loss, intended semantics -- the C-ABI
// wrapper neural_api.asm:2546-2568 passes a Tensor* where a Node* is expected
// and never writes *loss): softmax per row, target index = truncation of the
// target tensor's value, loss = mean_rows(-log(p_target + 1e-7)); f32 rows
// keep the float roundings of e_j, of p_t and of each row's loss.
//
// One wave per row with the row in VGPRs (one HBM read; the gradient written
// once), rows wider than the register budget take a block per row with three
// passes.  Per-row losses land in a double buffer and are summed by the
// segmented reduction (fixed order, deterministic); the row sums of exp use a
// fixed wave tree instead of the reference's sequential order, so losses
// agree to a few ulps of the row terms, not bit for bit.  An invalid target
// sets a device flag and the call returns -1 (C API) / INVALID_ARGUMENT.
#include <cmath>

#include <type_traits>

#include "reduce_impl.hpp"

namespace nh {

enum { CE_LS_FWD = 1, CE_LS_BWD = 2, CE_LS_FUSED = 3, CE_ASM = 4 };

template <typename T>
NH_DEV bool loss_target(const int64_t *ti, const T *tv, int64_t r, int64_t cols, int64_t &t)
{
    if (ti) {
        t = ti[r];
        return t >= 0 && t < cols;
    }
    const T v = tv[r];
    if (!(v > T(-1) && v < T(cols))) return false;  // NaN fails too
    t = int64_t(v);                                  // truncation (cvttss2si / cvttsd2si)
    return true;
}

// e = exp(x - m) for one element: double exp for f64 rows; for f32 rows the
// hardware exp2 of (x - m) * log2(e) in float (m is the row's largest float,
// so float(m) is exact).  Relative error about (|x - m| + 1) * 1.2e-7 against
// the reference's float rounding of the exact value: the losses built on it
// stay within 2e-6 of the exact loss (the f32 bar), and the float gradients
// within 1e-5.  Exact-difference double range reduction was measured ~20%
// slower for the tensor loss kernel.
NH_DEV double row_exp_d(double x, double m) { return exp(x - m); }

// e^y for the one-wave-per-row forward's f64 rows, from a 64-entry table of
// 2^(j/64) that each block keeps in LDS: y = (64 k + j) ln2 / 64 + r with
// |r| <= ln2 / 128, e^r by its Taylor polynomial through r^5 (truncation
// below 4e-17 relative), scaled by 2^k with ldexp (exact, or rounded once
// into the denormal range).  About 3 ulp against the device library's ~1,
// in 17 instructions instead of ~24: the 1e-12 bars of the losses and
// gradients are 3e3 times wider.  y below -1100 is taken as -1100 (e^y is 0
// either way), +inf and overflow give +inf, a NaN stays NaN (through r).
constexpr double kLn2_64Hi = kLn2Hi / 64.0;  // n * kLn2_64Hi exact for |n| < 2^20
constexpr double kLn2_64Lo = kLn2Lo / 64.0;
NH_DEV double exp_tab(double y, const double *tab)
{
    y = y < -1100.0 ? -1100.0 : y;  // NaN compares false and stays
    const double n = __builtin_rint(y * 92.332482616893658);  // 64 / ln 2
    double r = __builtin_fma(-n, kLn2_64Hi, y);
    r = __builtin_fma(-n, kLn2_64Lo, r);
    const int ni = int(n);  // |n| <= 2^17 for finite y <= 1100; a NaN's r carries it
    double p = 1.0 / 120.0;
    p = __builtin_fma(p, r, 1.0 / 24.0);
    p = __builtin_fma(p, r, 1.0 / 6.0);
    p = __builtin_fma(p, r, 0.5);
    p = __builtin_fma(p, r, 1.0);
    p = __builtin_fma(p, r, 1.0);
    return __builtin_ldexp(tab[ni & 63] * p, ni >> 6);  // 2^floor(n / 64); beyond 2^1023: +inf
}
NH_DEV double row_exp_f(float x, double m)
{
    return double(__builtin_amdgcn_exp2f((x - float(m)) * 1.4426950408889634f));
}

struct CeArgs {
    const int64_t *tidx;   // int64 targets (label-smoothed API) or null
    const void *tval;      // target values of the logits' dtype (tensor API) or null
    int64_t rows, cols;
    double alpha, inv_n;
    double *row_loss;      // [rows] or null: p_t (tensor CE) or sum_c st_c (x_c - m) (label-smoothed)
    double *row_s;         // [rows] or null: sum_c exp(x_c - m) (label-smoothed forward)
    void *grad;            // [rows, cols] or null
    int *bad;              // set to 1 when a target is out of range
};

// Per-element work once m and s are known.  Returns the element's part of the
// row loss without the log term and without its weight (label-smoothed:
// x - m) and writes the gradient element.  The row loss is
// -sum_c st_c ((x_c - m) - lse) = lse * sum_c st_c - A with
// A = sum_c st_c (x_c - m) = st0 * sum_c (x_c - m) + (st1 - st0) (x_t - m)
// (st_c = st0 off the target, st1 on it): every term of the reference's sum
// has one sign (x_c - m <= 0, lse >= 0), and so have the two parts of A, so
// the regrouping changes only the last bits; the log moves out of the row
// kernel into the summing pass and the weights out of the element loop.
template <typename T, int MODE>
NH_DEV double ce_elem(T xv, int64_t c, int64_t t, double m, double rs, const CeArgs &a, T &g)
{
    const double x = double(xv);
    const double st = a.alpha / double(a.cols) + (c == t ? 1.0 - a.alpha : 0.0);
    double term = 0.0;
    if (MODE == CE_LS_FWD || MODE == CE_LS_FUSED) term = x - m;
    if (MODE == CE_LS_BWD || MODE == CE_LS_FUSED) {
        const double e = sizeof(T) == 8 ? row_exp_d(x, m) : row_exp_f(float(xv), m);
        g = T(a.inv_n * (e * rs - st));
    }
    return term;
}

template <typename T>
NH_DEV double wave_fmax_t(T v);
template <> NH_DEV double wave_fmax_t<float>(float v) { return double(wave_fmax(v)); }
template <> NH_DEV double wave_fmax_t<double>(double v)
{
    return Grp<64>::reduce(v, [](double a, double b) { return __builtin_fmax(a, b); });
}

// One wave per row, VPL 16-byte vectors per lane (<= 64 * VPL * VN values).
// FULL: the row is exactly 64 * VPL * VN values and 16-byte aligned, so no
// element needs a bounds check (per-element checks around the exp turn into
// exec-mask branches).
//
// WAVES: the minimum waves per SIMD the compiler must fit (1: its own
// choice).  The f64 forward with rows of up to 1024 values takes 5 (83-84
// VGPRs, no spills; 103 and 4 waves otherwise): 88.8-90.1 -> 82.9 us at
// [65536,1024] (A/B in one run).  The fused and backward forms keep every
// exp for the gradient and spill under that bound (fused f64 180 -> 331 us),
// as do rows of 2048 doubles.
template <typename T, int VPL, int MODE, bool FULL, int WAVES = 1>
__global__ __launch_bounds__(256, WAVES) void k_ce_wave(const T *__restrict__ x, CeArgs a, bool vec, int64_t r_base)
{
    using V = typename Vec16<T>::type;
    constexpr int VN = Vec16<T>::n;
    const int lane = threadIdx.x & 63;
    // The f64 forward takes exp_tab (2^(j/64) by the device library's exp2,
    // in LDS): 85-90 -> 84-87 us at [65536,1024] (A/B in one run).  The modes
    // that keep every e for the gradient keep the library's exp: with the
    // table their longer-lived registers made the fused pass 177 -> 182 us.
    constexpr bool kTab = sizeof(T) == 8 && MODE == CE_LS_FWD;
    __shared__ double etab[kTab ? 64 : 1];
    if constexpr (kTab) {
        if (threadIdx.x < 64) etab[threadIdx.x] = exp2(double(threadIdx.x) * (1.0 / 64.0));
        __syncthreads();
    }
    const int64_t r = r_base + int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (r >= a.rows) return;  // uniform per wave
    const int64_t cols = a.cols;
    const T *xr = x + r * cols;
    // the target first: its load overlaps the row's instead of following the reductions
    int64_t t = 0;
    const bool ok = loss_target(a.tidx, static_cast<const T *>(a.tval), r, cols, t);
    V v[VPL];
#pragma unroll
    for (int k = 0; k < VPL; k++) {
        const int64_t c0 = (int64_t(k) * 64 + lane) * VN;
        if (FULL || vec) {
            if (FULL || c0 < cols) v[k] = ld_nt(reinterpret_cast<const V *>(xr + c0));
        } else {
#pragma unroll
            for (int j = 0; j < VN; j++)
                if (FULL || c0 + j < cols) v[k][j] = xr[c0 + j];
        }
    }
    T mx = -inf_t<T>();
#pragma unroll
    for (int k = 0; k < VPL; k++) {
        const int64_t c0 = (int64_t(k) * 64 + lane) * VN;
#pragma unroll
        for (int j = 0; j < VN; j++)
            if (FULL || c0 + j < cols) mx = fmax_nn(mx, v[k][j]);
    }
    const double m = wave_fmax_t<T>(mx);
    // e_c = exp(x_c - m), kept for the gradient (the backward modes)
    constexpr bool KEEP = MODE == CE_LS_BWD || MODE == CE_LS_FUSED;
    V ev[KEEP ? VPL : 1];
    // Per-lane sums: double, except the f32 tensor loss, whose reference sums
    // its float e_c in float (a lane's 16 float partial sums stay far inside
    // that sum's own rounding); the wave sum is double either way.
    using Acc = typename std::conditional<MODE == CE_ASM && sizeof(T) == 4, float, double>::type;
    Acc sl = Acc(0);
    Acc et = Acc(0);  // CE_ASM: e at the target column, in the lane that holds it
#pragma unroll
    for (int k = 0; k < VPL; k++) {
        const int64_t c0 = (int64_t(k) * 64 + lane) * VN;
#pragma unroll
        for (int j = 0; j < VN; j++)
            if (FULL || c0 + j < cols) {
                const double e = kTab ? exp_tab(double(v[k][j]) - m, etab)
                                      : (sizeof(T) == 8 ? row_exp_d(double(v[k][j]), m) : row_exp_f(float(v[k][j]), m));
                if constexpr (KEEP) ev[k][j] = T(e);
                if constexpr (MODE == CE_ASM) et = c0 + j == t ? Acc(e) : et;
                sl += Acc(e);
            }
    }
    double s = wave_dsum(double(sl));
    if (!ok) {
        if (lane == 0) {
            __hip_atomic_store(a.bad, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (a.row_loss) a.row_loss[r] = __builtin_nan("");
        }
        return;
    }
    if (MODE == CE_ASM) {
        // p_t = e_t / sum (f32: e_t, sum and p_t rounded to float); the row's
        // loss -log(p_t + 1e-7) is taken in the summing pass (RedCeLoss), where
        // the double log runs on all lanes instead of on lane 0 of every row.
        // e_t comes from the lane that computed it (the same value the
        // reference's exp(x_t - m) gives), not from a second read of the row.
        const int owner = int((t / VN) % 64);
        const long long eb = __double_as_longlong(double(et));
        const int lo = __builtin_amdgcn_readlane(int(eb), owner);
        const int hi = __builtin_amdgcn_readlane(int(eb >> 32), owner);
        const double e_t = __longlong_as_double((static_cast<long long>(hi) << 32) | static_cast<unsigned int>(lo));
        if (lane == 0) a.row_loss[r] = sizeof(T) == 4 ? double(float(e_t) / float(s)) : e_t / s;
        return;
    }
    const double rs = 1.0 / s;
    const double st0 = a.alpha / double(cols), st1 = st0 + (1.0 - a.alpha);
    // f32 rows: the per-element terms in float (the gradient is a float and
    // each loss term needs ~1e-7 of itself); the loss still sums in double
    const float mf = float(m), rsf = float(rs), st0f = float(st0), st1f = float(st1), inf_ = float(a.inv_n);
    double acc = 0.0;
    T *gr = static_cast<T *>(a.grad) + r * cols;
#pragma unroll
    for (int k = 0; k < VPL; k++) {
        const int64_t c0 = (int64_t(k) * 64 + lane) * VN;
        V g;
#pragma unroll
        for (int j = 0; j < VN; j++)
            if (FULL || c0 + j < cols) {
                const bool at_t = c0 + j == t;
                if constexpr (sizeof(T) == 4) {
                    if (MODE == CE_LS_FWD || MODE == CE_LS_FUSED) acc += double(v[k][j] - mf);
                    if constexpr (KEEP) g[j] = inf_ * (ev[k][j] * rsf - (at_t ? st1f : st0f));
                } else {
                    if (MODE == CE_LS_FWD || MODE == CE_LS_FUSED) acc += double(v[k][j]) - m;
                    if constexpr (KEEP) g[j] = T(a.inv_n * (double(ev[k][j]) * rs - (at_t ? st1 : st0)));
                }
            }
        if (MODE == CE_LS_BWD || MODE == CE_LS_FUSED) {
            if (FULL || vec) {
                if (FULL || c0 < cols) st_nt(reinterpret_cast<V *>(gr + c0), g);
            } else {
#pragma unroll
                for (int j = 0; j < VN; j++)
                    if (FULL || c0 + j < cols) gr[c0 + j] = g[j];
            }
        }
    }
    if (MODE == CE_LS_FWD || MODE == CE_LS_FUSED) {
        acc = wave_dsum(acc);
        // x_t from the registers of the lane that holds it: its vector k and
        // slot j are the same for every lane, so the pick is a uniform select
        const int kt = int(t / (64 * VN)), jt = int(t % VN), owner = int((t / VN) % 64);
        T xl = T(0);
#pragma unroll
        for (int k = 0; k < VPL; k++)
#pragma unroll
            for (int j = 0; j < VN; j++)
                if (k == kt && j == jt) xl = v[k][j];
        double xv;
        if constexpr (sizeof(T) == 4) {
            xv = double(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(xl), owner)));
        } else {
            const long long xb = __double_as_longlong(double(xl));
            const int lo = __builtin_amdgcn_readlane(int(xb), owner);
            const int hi = __builtin_amdgcn_readlane(int(xb >> 32), owner);
            xv = __longlong_as_double((static_cast<long long>(hi) << 32) | static_cast<unsigned int>(lo));
        }
        if (lane == 0) {
            const double xt = sizeof(T) == 4 ? double(float(xv) - mf) : xv - m;
            a.row_loss[r] = st0 * acc + (st1 - st0) * xt;
            a.row_s[r] = s;
        }
    }
}

// Block per row (any width): max, sum of exp, then the outputs, each a pass
// over the row.
template <typename T, int MODE>
__global__ __launch_bounds__(256) void k_ce_block(const T *__restrict__ x, CeArgs a, int64_t r_base)
{
    using G = Grp<256>;
    const int64_t r = r_base + blockIdx.x;
    const int64_t cols = a.cols;
    const T *xr = x + r * cols;
    T mx = -inf_t<T>();
    for (int64_t c = threadIdx.x; c < cols; c += 256) mx = fmax_nn(mx, xr[c]);
    const double m = double(G::reduce(mx, [](T p, T q) { return fmax_nn(p, q); }));
    double s = 0.0;
    for (int64_t c = threadIdx.x; c < cols; c += 256)
        s += sizeof(T) == 8 ? row_exp_d(double(xr[c]), m) : row_exp_f(float(xr[c]), m);
    s = G::reduce(s, [](double p, double q) { return p + q; });
    int64_t t = 0;
    const bool ok = loss_target(a.tidx, static_cast<const T *>(a.tval), r, cols, t);
    if (!ok) {
        if (threadIdx.x == 0) {
            __hip_atomic_store(a.bad, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (a.row_loss) a.row_loss[r] = __builtin_nan("");
        }
        return;
    }
    if (MODE == CE_ASM) {
        if (threadIdx.x == 0) {
            if (sizeof(T) == 4) a.row_loss[r] = double(float(row_exp_f(float(xr[t]), m)) / float(s));
            else a.row_loss[r] = row_exp_d(double(xr[t]), m) / s;
        }
        return;
    }
    const double rs = 1.0 / s;
    double acc = 0.0;
    T *gr = static_cast<T *>(a.grad) + r * cols;
    for (int64_t c = threadIdx.x; c < cols; c += 256) {
        T g = T(0);
        acc += ce_elem<T, MODE>(xr[c], c, t, m, rs, a, g);
        if (MODE == CE_LS_BWD || MODE == CE_LS_FUSED) gr[c] = g;
    }
    if (MODE == CE_LS_FWD || MODE == CE_LS_FUSED) {
        acc = G::reduce(acc, [](double p, double q) { return p + q; });
        if (threadIdx.x == 0) {
            const double st0 = a.alpha / double(cols), st1 = st0 + (1.0 - a.alpha);
            const double xt = double(xr[t]) - m;  // as ce_elem forms the other terms
            a.row_loss[r] = st0 * acc + (st1 - st0) * xt;
            a.row_s[r] = s;
        }
    }
}

template <typename T, int MODE, int VPL>
static void launch_ce_wave(const T *x, const CeArgs &a, bool vec)
{
    constexpr int W = sizeof(T) == 8 && MODE == CE_LS_FWD && VPL <= 8 ? 5 : 1;
    for_row_launches(a.rows, 4, [&](unsigned g, int64_t base) {
        if (vec && a.cols == int64_t(64) * VPL * Vec16<T>::n)
            NH_LAUNCH((k_ce_wave<T, VPL, MODE, true, W>), dim3(g), dim3(256), 0, stream(), x, a, vec, base);
        else
            NH_LAUNCH((k_ce_wave<T, VPL, MODE, false, W>), dim3(g), dim3(256), 0, stream(), x, a, vec, base);
    });
}

template <typename T, int MODE>
static int launch_ce(const T *x, const CeArgs &a)
{
    constexpr int VN = Vec16<T>::n;
    const bool vec = (reinterpret_cast<uintptr_t>(x) & 15u) == 0 && a.cols % VN == 0 &&
                     (!a.grad || (reinterpret_cast<uintptr_t>(a.grad) & 15u) == 0);
    const int64_t per = ceil_div(a.cols, int64_t(64) * VN);  // vectors per lane
    if (per <= 1) launch_ce_wave<T, MODE, 1>(x, a, vec);
    else if (per <= 2) launch_ce_wave<T, MODE, 2>(x, a, vec);
    else if (per <= 4) launch_ce_wave<T, MODE, 4>(x, a, vec);
    else if (per <= 8) launch_ce_wave<T, MODE, 8>(x, a, vec);
    else if (per <= 16) launch_ce_wave<T, MODE, 16>(x, a, vec);
    else
        for_row_launches(a.rows, 1, [&](unsigned g, int64_t base) {
            NH_LAUNCH((k_ce_block<T, MODE>), dim3(g), dim3(256), 0, stream(), x, a, base);
        });
    return check_launch();
}

// Sum of the per-row losses of the tensor CE (losses.asm intended semantics):
// the rows hold p_t, the loss term is -log(p_t + 1e-7), rounded to float for
// f32 logits as the reference's float loss.  div != 0: the stored value is
// the sum / div (the mean, for a loss left in device memory), the division
// the host makes otherwise.
template <bool F32>
struct RedCeLoss {
    using L = double;
    using B = double;
    double div = 0.0;
    NH_DEV L linit() const { return 0.0; }
    NH_DEV void lacc(L &s, double p, int64_t) const
    {
        const double lt = -log(p + 1e-7);
        s += F32 ? double(float(lt)) : lt;
    }
    NH_DEV L lcomb(L a, L b) const { return a + b; }
    template <int TPR> NH_DEV B finish(L s, const double *, int64_t, int64_t) const { return s; }
    NH_DEV B bident() const { return 0.0; }
    NH_DEV B bcomb(B a, B b) const { return a + b; }
    NH_DEV void store(void *out, int64_t r, B s, const double *, int64_t) const
    {
        static_cast<double *>(out)[r] = div != 0.0 ? s / div : s;
    }
};

// Sum of the label-smoothed row losses: row r holds A_r = sum_c st_c (x_c - m)
// and s_r = sum_c exp(x_c - m); its loss is log(s_r) * S - A_r with
// S = sum_c st_c = st0 (cols - 1) + st1.  div as in RedCeLoss.
struct RedLsLoss {
    using L = double;
    using B = double;
    const double *s;
    double S;
    double div = 0.0;
    NH_DEV L linit() const { return 0.0; }
    NH_DEV void lacc(L &acc, double A, int64_t i) const
    {
        const double lse = log(s[i]);
        const double sl = lse * S;
        acc += sl - A;
    }
    NH_DEV L lcomb(L a, L b) const { return a + b; }
    template <int TPR> NH_DEV B finish(L v, const double *, int64_t, int64_t) const { return v; }
    NH_DEV B bident() const { return 0.0; }
    NH_DEV B bcomb(B a, B b) const { return a + b; }
    NH_DEV void store(void *out, int64_t r, B v, const double *, int64_t) const
    {
        static_cast<double *>(out)[r] = div != 0.0 ? v / div : v;
    }
};

// Runs MODE over [rows, cols] logits already on the device; sums the per-row
// losses into *loss_host (mean over rows) when wanted.  Returns NEURAL_OK,
// NEURAL_ERR_INVALID_ARGUMENT for a target out of range, or an error code.
// With loss_dev (device memory) instead, the mean loss is stored there by the
// last launch and the call returns once everything is enqueued: nothing is
// waited for, and a target out of range shows only as a NaN loss.
template <typename T, int MODE>
static int ce_run(const T *x, const int64_t *tidx, const T *tval, int64_t rows, int64_t cols, double alpha,
                  double *loss_host, T *grad_dev, double *loss_dev = nullptr)
{
    WsGuard wg;
    Workspace &ws = workspace();
    const bool on_dev = loss_dev != nullptr;
    const bool want_loss = MODE != CE_LS_BWD;
    constexpr bool kLs = MODE == CE_LS_FWD || MODE == CE_LS_FUSED;
    // The loss sum (word 0) and the out-of-range flag (int word 32) are stored
    // into the mapped host area.  The flag is zero at init and between calls
    // (a call that finds it set clears it on the host).  A call that leaves
    // its loss on the device points the flag at a spare word of its own row
    // buffer, which nothing reads.
    int *bad = static_cast<int *>(ws.host_result_dev) + 32;
    double *row_loss = nullptr, *row_s = nullptr;
    if (want_loss) {
        // one block: [rows] row values, then [rows] exp sums (label-smoothed),
        // then the spare flag word for a device-resident loss
        const size_t words = size_t(rows) * (kLs ? 2 : 1);
        row_loss = static_cast<double *>(dev_alloc((words + (on_dev ? 1 : 0)) * sizeof(double)));
        if (!row_loss) return set_error(NEURAL_ERR_OUT_OF_MEMORY);
        if (kLs) row_s = row_loss + rows;
        if (on_dev) bad = reinterpret_cast<int *>(row_loss + words);
    }
    CeArgs a{tidx, tval, rows, cols, alpha, 1.0 / double(rows), row_loss, row_s, grad_dev, bad};
    int rc = launch_ce<T, MODE>(x, a);
    // The loss sum's launch stores a ticket after the sum (and after the CE
    // kernel, earlier on the stream, has set the flag or not): the host waits
    // for the ticket instead of synchronising the stream.
    const Ticket tk = want_loss && !on_dev ? next_ticket() : Ticket{};
    if (rc == NEURAL_OK && want_loss) {
        void *dst = on_dev ? static_cast<void *>(loss_dev) : ws.host_result_dev;
        const double div = on_dev ? double(rows) : 0.0;
        if (MODE == CE_ASM) {
            rc = launch_reduce(row_loss, 1, rows, rows, RedCeLoss<sizeof(T) == 4>{div}, dst, nullptr, 0, tk);
        } else {
            const double st0 = alpha / double(cols), st1 = st0 + (1.0 - alpha);
            rc = launch_reduce(row_loss, 1, rows, rows, RedLsLoss{row_s, st0 * double(cols - 1) + st1, div}, dst,
                               nullptr, 0, tk);
        }
    }
    if (on_dev) {
        if (row_loss) dev_free(row_loss);  // reused only by work enqueued after these launches
        return rc;
    }
    struct { double sum; int pad[30]; int bad; } res;  // result area layout: sum at 0, flag at word 32
    static_assert(sizeof(res) == 136, "");
    if (rc == NEURAL_OK)
        rc = want_loss ? host_result_wait(tk.value, &res, sizeof(res)) : host_result_fetch(&res, sizeof(res));
    if (row_loss) dev_free(row_loss);
    if (rc != NEURAL_OK) return rc;
    if (res.bad) {
        // every launch of this call has finished writing the area (the
        // ticket, or the stream wait, comes after them)
        static_cast<int *>(ws.host_result)[32] = 0;
        return NEURAL_ERR_INVALID_ARGUMENT;
    }
    if (want_loss && loss_host) *loss_host = res.sum / double(rows);
    return NEURAL_OK;
}

// Raw-pointer label-smoothed CE (host or device pointers).
template <typename T, int MODE>
static int ls_ce(const T *logits, const int64_t *targets, int64_t batch, int64_t classes, double smoothing,
                 double *loss_out, T *grad_out)
{
    if (ensure_init() != NEURAL_OK) return -1;
    if (!logits || !targets) return -1;
    if ((MODE != CE_LS_BWD && !loss_out) || (MODE != CE_LS_FWD && !grad_out)) return -1;
    if (batch <= 0 || classes <= 0) return -1;
    if (!(smoothing >= 0.0 && smoothing <= 1.0)) return -1;
    int64_t n;
    if (__builtin_mul_overflow(batch, classes, &n)) return -1;
    Staged sx, st, sg;
    if (sx.open_n(logits, uint64_t(n), sizeof(T), true) != NEURAL_OK ||
        st.open_n(targets, uint64_t(batch), 8, true) != NEURAL_OK)
        return -1;
    if (MODE != CE_LS_FWD && sg.open_n(grad_out, uint64_t(n), sizeof(T), false) != NEURAL_OK) return -1;
    const int rc = ce_run<T, MODE>(static_cast<const T *>(sx.dev), static_cast<const int64_t *>(st.dev), nullptr,
                                   batch, classes, smoothing, loss_out, static_cast<T *>(sg.dev));
    if (rc != NEURAL_OK) return -1;
    if (MODE != CE_LS_FWD && sg.finish(true) != NEURAL_OK) return -1;
    set_error(NEURAL_OK);
    return 0;
}

// Label-smoothed CE on device pointers with the mean loss left in device
// memory (*loss_dev): every launch enqueued, nothing waited for.
template <typename T, int MODE>
static int ls_ce_dev(const T *logits, const int64_t *targets, int64_t batch, int64_t classes, double smoothing,
                     double *loss_dev, T *grad_dev)
{
    if (ensure_init() != NEURAL_OK) return -1;
    if (!logits || !targets || !loss_dev || (MODE == CE_LS_FUSED && !grad_dev)) {
        set_error(NEURAL_ERR_NULL_POINTER);
        return -1;
    }
    int64_t n;
    if (batch <= 0 || classes <= 0 || !(smoothing >= 0.0 && smoothing <= 1.0) ||
        __builtin_mul_overflow(batch, classes, &n) || uint64_t(n) > kMaxRawCount) {
        set_error(NEURAL_ERR_INVALID_ARGUMENT);
        return -1;
    }
    const auto misaligned = [](const void *p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) != 0; };
    if (!is_device_ptr(logits) || !is_device_ptr(targets) || !is_device_ptr(loss_dev) ||
        (grad_dev && !is_device_ptr(grad_dev)) || misaligned(logits, sizeof(T)) || misaligned(targets, 8) ||
        misaligned(loss_dev, 8) || (grad_dev && misaligned(grad_dev, sizeof(T)))) {
        set_error(NEURAL_ERR_INVALID_ARGUMENT);
        return -1;
    }
    if (ce_run<T, MODE>(logits, targets, nullptr, batch, classes, smoothing, nullptr, grad_dev, loss_dev) !=
        NEURAL_OK)
        return -1;
    set_error(NEURAL_OK);
    return 0;
}

}  // namespace nh

using namespace nh;

extern "C" {

int label_smoothing_ce_forward_dev(const double *logits, const int64_t *targets, int64_t batch_size,
                                   int64_t num_classes, double smoothing, double *loss_dev)
{
    return ls_ce_dev<double, CE_LS_FWD>(logits, targets, batch_size, num_classes, smoothing, loss_dev, nullptr);
}

int label_smoothing_ce_fused_dev(const double *logits, const int64_t *targets, int64_t batch_size,
                                 int64_t num_classes, double smoothing, double *loss_dev, double *grad_dev)
{
    return ls_ce_dev<double, CE_LS_FUSED>(logits, targets, batch_size, num_classes, smoothing, loss_dev, grad_dev);
}

int label_smoothing_ce_fused_f32_dev(const float *logits, const int64_t *targets, int64_t batch_size,
                                     int64_t num_classes, double smoothing, double *loss_dev, float *grad_dev)
{
    return ls_ce_dev<float, CE_LS_FUSED>(logits, targets, batch_size, num_classes, smoothing, loss_dev, grad_dev);
}

int label_smoothing_ce_forward(const double *logits, const int64_t *targets, int64_t batch_size,
                               int64_t num_classes, double smoothing, double *loss_out)
{
    return ls_ce<double, CE_LS_FWD>(logits, targets, batch_size, num_classes, smoothing, loss_out, nullptr);
}

int label_smoothing_ce_backward(const double *logits, const int64_t *targets, int64_t batch_size,
                                int64_t num_classes, double smoothing, double *grad_out)
{
    return ls_ce<double, CE_LS_BWD>(logits, targets, batch_size, num_classes, smoothing, nullptr, grad_out);
}

int label_smoothing_ce_fused(const double *logits, const int64_t *targets, int64_t batch_size, int64_t num_classes,
                             double smoothing, double *loss_out, double *grad_out)
{
    return ls_ce<double, CE_LS_FUSED>(logits, targets, batch_size, num_classes, smoothing, loss_out, grad_out);
}

int label_smoothing_ce_fused_f32(const float *logits, const int64_t *targets, int64_t batch_size,
                                 int64_t num_classes, double smoothing, double *loss_out, float *grad_out)
{
    return ls_ce<float, CE_LS_FUSED>(logits, targets, batch_size, num_classes, smoothing, loss_out, grad_out);
}

int neural_cross_entropy_loss(const NeuralTensor *prediction, const NeuralTensor *target, double *loss)
{
    NH_TRY(ensure_init());
    if (!prediction || !target || !loss) return set_error(NEURAL_ERR_NULL_POINTER);
    NH_TRY(check_tensor(prediction));
    NH_TRY(check_tensor(target));
    if (prediction->dtype != target->dtype) return set_error(NEURAL_ERR_DTYPE_MISMATCH);
    if (prediction->ndim != 2) return set_error(NEURAL_ERR_DIM_MISMATCH);
    const int64_t rows = prediction->shape[0], cols = prediction->shape[1];
    if (rows <= 0 || cols <= 0) return set_error(NEURAL_ERR_INVALID_ARGUMENT);
    if (numel(target) != rows) return set_error(NEURAL_ERR_SHAPE_MISMATCH);
    if (!is_contiguous(prediction) || !is_contiguous(target)) return set_error(NEURAL_ERR_INVALID_ARGUMENT);
    const void *px = nullptr, *pt = nullptr;
    NH_TRY(dev_read(prediction, &px));
    NH_TRY(dev_read(target, &pt));
    int rc;
    if (prediction->dtype == NEURAL_DTYPE_FLOAT32)
        rc = ce_run<float, CE_ASM>(static_cast<const float *>(px), nullptr, static_cast<const float *>(pt), rows, cols,
                                   0.0, loss, nullptr);
    else
        rc = ce_run<double, CE_ASM>(static_cast<const double *>(px), nullptr, static_cast<const double *>(pt), rows,
                                    cols, 0.0, loss, nullptr);
    return set_error(rc);
}

}  // extern "C"
