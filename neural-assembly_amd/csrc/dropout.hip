// dropout.hip -- inverted dropout forward / backward with the reference's
// random stream.
//
// Reference: dropout_forward / dropout_backward (training_ops.asm:717-858),
// exported as neural_dropout_forward / _backward (neural_api.asm:2797-2803,
// bound at pyneural/core.py:499-515).  Forward, per element i in order: one
// libc rand() draw; drop when (int64)rand() < threshold with
// threshold = cvtsd2si((double)p * 2147483647.0) (round to nearest even);
// dropped: mask 0, out +0.0f; kept: mask 1, out = x * scale with
// scale = (float)(1.0 / (1.0 - (double)p)).  Backward: grad_in = mask ?
// grad_out * scale : +0.0f.
//
// The random stream is glibc's rand() (the reference calls it through the
// PLT; glibc's default TYPE_3 generator, published e.g. in P. Selinger, "The
// GLIBC pseudo-random number generator"): srand(s) fills r[0..30] with the
// Park-Miller sequence r[i] = 16807 * r[i-1] mod (2^31 - 1) from r[0] = s
// (s = 0 taken as 1), sets r[31..33] = r[0..2], continues
// r[i] = r[i-31] + r[i-3] (mod 2^32), and rand() returns r[k + 344] >> 1
// for k = 0, 1, ...  The library keeps its own stream: neural_dropout_seed(s)
// positions it as srand(s) would (unseeded = srand(1), glibc's default), and
// every forward call consumes n draws, so masks equal the reference's when its
// process is at the same point of its rand() stream.
//
// Parallel generation on the device: the recurrence is linear, so for the
// anchor window W = r[A .. A+30] any later value is r[A + k] = sum_m c_m W[m]
// with c = x^k mod P(x), P(x) = x^31 - x^28 - 1, coefficients mod 2^32.
// The n draws of a call are cut into segments of L = 372 draws (12 periods
// of 31), 64 segments per wave.  Segment j = 64 w + l starts at
// A + jL; its starting window is reached in two linear steps: the 62 values
// G_w = r[A + 64 w L ..] from R = r[A .. A+92] and e_w = x^(64 w L) mod P (a
// device table, 128 bytes per wave), then w_j[t] = sum_m d_l[m] G_w[m + t]
// with d_l = x^(lL) mod P, the same 64 rows for every wave: a [64 x 32] x
// [32 x 32] product mod 2^32, done on the matrix cores (int8 MFMA over signed
// byte limbs, below).  Thread j then runs
// the recurrence for its 372 draws with the 31-value ring in registers and
// packs keep bits into 12 words.  A second, streaming kernel reads x in
// 16-byte vectors, the 4 keep bits of each vector, and writes out and the
// mask bytes (9 B per element).  The stream values after the call (r at
// A + n .. A + n + 92, the next call's R) are one more jump of R, by
// x^n and x^(n+31) mod P (made on the host, kept while n repeats).
#include <cmath>
#include <cstring>
#include <mutex>
#include <utility>
#include <vector>

#include "common.hpp"
#include "kernels.hpp"

namespace nh {

constexpr int kLag = 31;                       // r[i] = r[i-31] + r[i-3]
// Segments of 12 periods (a multiple of 4 draws, for the 4-draw vectors of
// the streaming pass): keep-bit kernel at 64 M draws with 4 / 8 / 12 / 16 /
// 24 periods 20.9 / 17.4 / 16.9 / 20.5 / 20.0 us (shorter segments pay more
// jumps, longer ones leave SIMDs with too few waves).
constexpr int kPeriods = 12;
constexpr int64_t kSegL = int64_t(kLag) * kPeriods;   // 372 draws per thread segment (a multiple of 4)
constexpr int kSegWords = int((kSegL + 31) / 32);      // keep-bit words per segment (12)
constexpr int kDBlock = 256;
// Stream values kept between calls: r[A .. A+92], the anchor window and the
// 62 values after it (the first jump step reads all 93).
constexpr int kWin = 3 * kLag;

// ---- polynomials mod P(x) = x^31 - x^28 - 1 over Z / 2^32 ------------------------------

// a * b mod P.  x^d for d >= 31 is x^(d-3) + x^(d-31).
NH_DEV void dpoly_mul(uint32_t (&a)[kLag], const uint32_t *__restrict__ b)
{
    uint32_t prod[2 * kLag - 1];
#pragma unroll
    for (int d = 0; d < 2 * kLag - 1; d++) prod[d] = 0u;
#pragma unroll
    for (int i = 0; i < kLag; i++) {
#pragma unroll
        for (int j = 0; j < kLag; j++) prod[i + j] += a[i] * b[j];
    }
#pragma unroll
    for (int d = 2 * kLag - 2; d >= kLag; d--) {
        prod[d - kLag] += prod[d];
        prod[d - 3] += prod[d];
    }
#pragma unroll
    for (int i = 0; i < kLag; i++) a[i] = prod[i];
}

// ---- the jump as an int8 matrix product ---------------------------------------------------
//
// A 32-bit value is split into balanced base-256 digits, v = sum_p l_p 256^p
// (mod 2^32) with l_p in [-128, 127], so that products of digits fit the
// signed int8 inputs of v_mfma_i32_32x32x32_i8.  For C (segments x m) and
// H (m x t): C H = sum_{p+q <= 3} 256^(p+q) C_p H_q (mod 2^32) -- the
// digit products with p + q >= 4 vanish mod 2^32.  Each D_s = sum_{p+q=s}
// C_p H_q is exact in int32 (32 (s+1) terms of magnitude <= 2^14).
// Operand layout: lane l holds row l % 32 of A and column l % 32 of B, 16
// bytes each; the tables below store them as two 8-byte halves, coefficient
// m = 16 c + 8 (l / 32) + b in byte b of half c (m = 31 is padding, 0).  A
// and B place the same m at the same (lane half, byte), so the product sums
// every m once.  The 16 results of lane l are D[8 (v/4) + 4 (l/32) + v % 4][l % 32].
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

// Two 8-byte operand halves as the 16-byte operand of the K = 32 form.
NH_DEV i32x4 pack_k32(uint64_t lo, uint64_t hi)
{
    return i32x4{int(uint32_t(lo)), int(uint32_t(lo >> 32)), int(uint32_t(hi)), int(uint32_t(hi >> 32))};
}

// Balanced base-256 digits of v, each as the low byte of l[p].
__host__ __device__ inline void limbs4(uint32_t v, uint32_t (&l)[4])
{
    uint32_t u = v;
#pragma unroll
    for (int p = 0; p < 4; p++) {
        const uint32_t b = u & 0xFFu;
        l[p] = b;
        const uint32_t sb = b >= 128u ? b - 256u : b;  // the digit, sign-extended mod 2^32
        u = (u - sb) >> 8;
    }
}

// Table layout: the A operands of segment j's row, wave block w = j / 64
// (1024 64-bit words): word w*1024 + T*512 + (p*2 + c)*64 + lane holds
// digit p of coefficients m = 16c + 8(lane/32) + b, b = 0..7, of segment
// 64w + 32T + lane % 32 (m = 31 is padding, 0).
constexpr int kTabWordsPerWave = 1024;

// c_j = x^(j*L) mod P for j in [j0, j1), stored as MFMA A-operand digits:
// square-and-multiply over the host-made powers B[k] = x^(L * 2^k) mod P.
__global__ __launch_bounds__(kDBlock) void k_jump_table(uint64_t *__restrict__ TL, int64_t j0, int64_t j1,
                                                         const uint32_t *__restrict__ B)
{
    const int64_t j = j0 + int64_t(blockIdx.x) * kDBlock + threadIdx.x;
    if (j >= j1) return;
    uint32_t c[kLag];
#pragma unroll
    for (int i = 0; i < kLag; i++) c[i] = i == 0 ? 1u : 0u;
    for (int k = 0; k < 63 && (j >> k) != 0; k++)
        if ((j >> k) & 1) dpoly_mul(c, B + k * kLag);
    uint64_t *row = TL + (j >> 6) * kTabWordsPerWave + ((j >> 5) & 1) * 512 + (j & 31);
#pragma unroll
    for (int h = 0; h < 2; h++) {
#pragma unroll
        for (int cc = 0; cc < 2; cc++) {
            uint64_t q[4] = {0u, 0u, 0u, 0u};
#pragma unroll
            for (int b = 0; b < 8; b++) {
                const int m = 16 * cc + 8 * h + b;
                uint32_t l[4];
                limbs4(m < kLag ? c[m] : 0u, l);
#pragma unroll
                for (int p = 0; p < 4; p++) q[p] |= uint64_t(l[p]) << (8 * b);
            }
#pragma unroll
            for (int p = 0; p < 4; p++) row[(p * 2 + cc) * 64 + 32 * h] = q[p];
        }
    }
}

// Generate the keep bits of one segment from its starting window w.
// keep = (r >> 1) >= thr = (r > 2 thr - 1) for
// thr in [1, 2^31] (ALL: thr = 0, every draw kept): one subtraction
// t2m1 - r whose borrow is the keep bit, and one add-with-carry kb + kb +
// borrow that shifts it into the period's word, first draw highest -- three
// instructions per draw with the recurrence add (a sign-bit and funnel-shift
// form, add + shift + subtract + v_alignbit_b32, measured 1.6x slower in a
// probe of the ring alone) -- and a bit reversal per period puts draw u at
// bit u.  The pair goes through VCC, written as inline assembly because the
// compiler turns the C form (kb + kb + (r > t2m1)) into a compare, a select
// and shifts.  One period of 31 draws
// is unrolled (ring slots are then registers) and the period loop is not:
// the fully unrolled segment is ~50 KB of straight-line code, and fetching it
// cold made the kernel instruction-fetch bound (measured 4x slower).
template <bool ALL>
NH_DEV void gen_segment(uint32_t (&w)[kLag], uint32_t t2m1, uint32_t *__restrict__ bits)
{
    uint64_t acc = 0u;  // pending keep bits; the low `have` are valid
    int have = 0;
    int word = 0;
#pragma unroll 1
    for (int per = 0; per < kPeriods; per++) {
        uint32_t kb = 0u;  // keep bit of draw u at bit 30 - u
#pragma unroll
        for (int u = 0; u < kLag; u++) {
            const uint32_t r = w[u] + w[(u + 28) % kLag];
            w[u] = r;
            if constexpr (ALL) {
                kb = (kb << 1) | 1u;
            } else {
                uint32_t diff;
                asm volatile("v_sub_co_u32 %1, vcc, %2, %3\n\tv_addc_co_u32 %0, vcc, %0, %0, vcc"
                             : "+v"(kb), "=&v"(diff)
                             : "s"(t2m1), "v"(r)
                             : "vcc");
            }
        }
        const uint32_t pb = __builtin_bitreverse32(kb) >> 1;  // draw u at bit u
        acc |= uint64_t(pb) << have;
        have += kLag;
        if (have >= 32) {
            bits[word++] = uint32_t(acc);
            acc >>= 32;
            have -= 32;
        }
    }
    if (have > 0) bits[word] = uint32_t(acc);  // only when L is not a multiple of 32
}

// x^(64 w L) mod P for w in [w0, w1): the jump of wave w's first segment,
// 32 words per wave (word 31 = 0), square-and-multiply over the host-made
// powers B[k] = x^(64 L 2^k) mod P.
__global__ __launch_bounds__(kDBlock) void k_wave_jumps(uint32_t *__restrict__ E, int64_t w0, int64_t w1,
                                                         const uint32_t *__restrict__ B)
{
    const int64_t w = w0 + int64_t(blockIdx.x) * kDBlock + threadIdx.x;
    if (w >= w1) return;
    uint32_t c[kLag];
#pragma unroll
    for (int i = 0; i < kLag; i++) c[i] = i == 0 ? 1u : 0u;
    for (int k = 0; k < 63 && (w >> k) != 0; k++)
        if ((w >> k) & 1) dpoly_mul(c, B + k * kLag);
    uint32_t *row = E + w * 32;
#pragma unroll
    for (int i = 0; i < kLag; i++) row[i] = c[i];
    row[kLag] = 0u;
}

// One thread per segment, 64 segments per wave, the jump in two steps:
//   1. wave w's base values G_w[i] = r[A + 64 w L + i], i < 62, from
//      R = r[A .. A+92] (W: the 93 values the previous call, or the seed,
//      left) and e_w = x^(64 w L) mod P (E, 128 bytes per wave):
//      G_w[i] = sum_m e_w[m] R[i + m], one lane per i;
//   2. lane l's window w[t] = r[A + (64 w + l) L + t] = sum_m d_l[m] G_w[m + t]
//      with d_l = x^(l L) mod P, the same 64 rows for every wave (D, digits in
//      the MFMA A-operand layout, 8 KB): a [64 x 32] x [32 x 32] product mod
//      2^32 on the matrix cores, B = the Hankel digits of G_w.
// The per-segment table reads of a single-step jump (128 bytes per segment)
// become 128 bytes per 64 segments; D is staged in LDS once per block.
// E covers every wave of the grid, so all
// waves run the jump and reach every barrier; threads past nseg stop before
// generating.
// x^n and x^(n+31) mod P for the call's n: the next call's 93 values are
// Wn[i] = r[A + n + i] = sum_m c0[m] R[i + m] (i < 62) and
// Wn[62 + q] = sum_m c1[m] R[31 + q + m] (q < 31), from R alone.
struct NextJump {
    uint32_t c0[kLag];
    uint32_t c1[kLag];
};

// The work of block `bid` of the keep-bit pass (a block-uniform index: every
// thread of the block reaches every barrier).
template <bool ALL>
NH_DEV void dropout_bits_block(unsigned bid, const uint64_t *__restrict__ D, const uint32_t *__restrict__ E,
                               const uint32_t *__restrict__ W, uint32_t *__restrict__ Wn, const NextJump &nj,
                               int64_t nseg, uint32_t t2m1, uint32_t *__restrict__ bits)
{
    __shared__ uint64_t sD[kTabWordsPerWave];           // the 64-row digit table
    __shared__ uint32_t sR[kWin];                        // r[A .. A+92]
    __shared__ uint32_t sGd[kDBlock / 64][4][16];       // per wave: byte i of row p = digit p of G_w[i]
    __shared__ uint32_t sX[kDBlock / 64][32 * kLag];  // per wave: one tile's 32 windows, row stride 31 (odd: no bank conflicts)
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    if (tid < kWin) sR[tid] = W[tid];
#pragma unroll
    for (int i = 0; i < kTabWordsPerWave / kDBlock; i++) sD[i * kDBlock + tid] = D[i * kDBlock + tid];
    __syncthreads();
    const int64_t wave = int64_t(bid) * (kDBlock / 64) + wv;
    if (bid == 0 && wv < 2) {
        // the next call's 93 values (block 0, two waves; coefficients uniform)
        uint32_t g = 0u;
        if (wv == 0) {
            if (lane < 2 * kLag) {
#pragma unroll
                for (int m = 0; m < kLag; m++) g += nj.c0[m] * sR[lane + m];
                Wn[lane] = g;
            }
        } else if (lane < kLag) {
#pragma unroll
            for (int m = 0; m < kLag; m++) g += nj.c1[m] * sR[kLag + lane + m];
            Wn[2 * kLag + lane] = g;
        }
    }
    {
        const uint32_t *e = E + wave * 32;  // uniform per wave
        uint32_t g = 0u;
        if (lane < 2 * kLag) {
#pragma unroll
            for (int m = 0; m < kLag; m++) g += e[m] * sR[lane + m];
        }
        // its balanced digits, one byte per lane in each digit row
        uint32_t l[4];
        limbs4(g, l);
        uint8_t *gd = reinterpret_cast<uint8_t *>(sGd[wv]);
#pragma unroll
        for (int p = 0; p < 4; p++) gd[p * 64 + lane] = uint8_t(l[p]);
    }
    __syncthreads();
    // B operands of this wave: digits of H[m][t] = G_w[m + t], m = 16 c +
    // 8 (lane / 32) + b: bytes o .. o + 7 of each digit row, o = 16 c +
    // 8 (lane / 32) + t (<= 55), gathered as two byte-aligned dword pairs
    uint64_t Bq[4][2];
    {
        const int t = lane & 31, h = lane >> 5;
#pragma unroll
        for (int cc = 0; cc < 2; cc++) {
            const int o = 16 * cc + 8 * h + t;
            const int qd = o >> 2, sh = o & 3;
#pragma unroll
            for (int p = 0; p < 4; p++) {
                const uint32_t *row = sGd[wv][p];
                const uint32_t d0 = row[qd], d1 = row[qd + 1], d2 = row[qd + 2];
                const uint32_t lo = __builtin_amdgcn_alignbyte(d1, d0, uint32_t(sh));
                const uint32_t hi = __builtin_amdgcn_alignbyte(d2, d1, uint32_t(sh));
                Bq[p][cc] = uint64_t(lo) | (uint64_t(hi) << 32);
            }
        }
    }
    uint32_t *X = sX[wv];
    // Two 32-segment tiles, transposed through LDS one at a time.
    uint32_t w[kLag];
#pragma unroll
    for (int T = 0; T < 2; T++) {
        // K = 32 per instruction: both 16-coefficient chunks in one operand
        // (bytes 0-7 chunk 0, bytes 8-15 chunk 1, the same for A and B, so
        // the product sums all 32 coefficients whatever the unit's k order)
        i32x4 A4[4], B4[4];
#pragma unroll
        for (int p = 0; p < 4; p++) {
            A4[p] = pack_k32(sD[T * 512 + (p * 2) * 64 + lane], sD[T * 512 + (p * 2 + 1) * 64 + lane]);
            B4[p] = pack_k32(Bq[p][0], Bq[p][1]);
        }
        // Horner over the digit weight, s = 3, 2, 1, 0: d = (d << 8) + D_s,
        // the shifted sum entering the next products as their accumulator
        // (int32 accumulation wraps mod 2^32)
        i32x16 d = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
        for (int s = 3; s >= 0; s--) {
            if (s < 3) {
#pragma unroll
                for (int v = 0; v < 16; v++) d[v] = int(uint32_t(d[v]) << 8);
            }
#pragma unroll
            for (int p = 0; p <= s; p++) d = __builtin_amdgcn_mfma_i32_32x32x32_i8(A4[p], B4[s - p], d, 0, 0, 0);
        }
        uint32_t out[16];
#pragma unroll
        for (int v = 0; v < 16; v++) out[v] = uint32_t(d[v]);
        // result (row, t) of lane l, value v: row 8(v/4) + 4(l/32) + v%4, t = l % 32 (t = 31 is padding)
        if ((lane & 31) < kLag) {
#pragma unroll
            for (int v = 0; v < 16; v++) X[(8 * (v >> 2) + 4 * (lane >> 5) + (v & 3)) * kLag + (lane & 31)] = out[v];
        }
        __syncthreads();
        if ((lane >> 5) == T) {
#pragma unroll
            for (int t = 0; t < kLag; t++) w[t] = X[(lane & 31) * kLag + t];
        }
        __syncthreads();
    }
    const int64_t j = wave * 64 + lane;
    if (j >= nseg) return;
    uint32_t *b = bits + j * kSegWords;
    gen_segment<ALL>(w, t2m1, b);
}

template <bool ALL>
__global__ __launch_bounds__(kDBlock) void k_dropout_bits(const uint64_t *__restrict__ D,
                                                           const uint32_t *__restrict__ E,
                                                           const uint32_t *__restrict__ W, uint32_t *__restrict__ Wn,
                                                           NextJump nj, int64_t nseg, uint32_t t2m1,
                                                           uint32_t *__restrict__ bits)
{
    dropout_bits_block<ALL>(blockIdx.x, D, E, W, Wn, nj, nseg, t2m1, bits);
}

constexpr int kDUnroll = 2;

// Keep bit of draw d: segment d / L, bit d % L of its words.  I = uint32_t
// when every index fits (a division by the constant L is then a multiply-high
// and a shift).
template <typename I>
NH_DEV uint32_t keep_bits(const uint32_t *__restrict__ bits, I d)
{
    const I seg = d / I(kSegL);
    const I bi = d - seg * I(kSegL);
    return bits[size_t(seg) * kSegWords + size_t(bi >> 5)] >> (bi & 31);
}

// out = keep ? x * scale : +0, mask = keep; 4 elements per lane-unit; block
// `a` of `na` blocks striding over the n4 vectors.
template <typename I>
NH_DEV void dropout_apply_block(unsigned a, unsigned na, const f32x4 *__restrict__ x, f32x4 *__restrict__ out,
                                uint32_t *__restrict__ mask, const uint32_t *__restrict__ bits, int64_t n4,
                                float scale)
{
    const int64_t tile = int64_t(kDBlock) * kDUnroll;
    for (int64_t base = int64_t(a) * tile + threadIdx.x; base < n4; base += int64_t(na) * tile) {
        f32x4 v[kDUnroll];
        uint32_t kb[kDUnroll];
#pragma unroll
        for (int u = 0; u < kDUnroll; u++) {
            const int64_t q = base + int64_t(u) * kDBlock;
            if (q < n4) {
                v[u] = ld_nt(x + q);
                kb[u] = keep_bits<I>(bits, I(q * 4)) & 0xFu;
            }
        }
#pragma unroll
        for (int u = 0; u < kDUnroll; u++) {
            const int64_t q = base + int64_t(u) * kDBlock;
            if (q < n4) {
                f32x4 o;
                uint32_t m = 0u;
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const bool keep = (kb[u] >> k) & 1u;
                    o[k] = keep ? v[u][k] * scale : 0.0f;
                    m |= uint32_t(keep) << (8 * k);
                }
                st_nt(out + q, o);
                st_nt(mask + q, m);
            }
        }
    }
}

template <typename I>
__global__ __launch_bounds__(kDBlock) void k_dropout_apply(const f32x4 *__restrict__ x, f32x4 *__restrict__ out,
                                                            uint32_t *__restrict__ mask, const uint32_t *__restrict__ bits,
                                                            int64_t n4, float scale)
{
    dropout_apply_block<I>(blockIdx.x, gridDim.x, x, out, mask, bits, n4, scale);
}

// The apply pass of this call with the keep-bit pass of the next call's
// draws folded in, for a caller that repeats (n, p) (a training loop): `nb`
// keep-bit blocks for the draws after this call's, at block indices 0,
// period, 2 period, ... so that their arithmetic spreads over the stream
// instead of running before it; the other `na` blocks stream.  The next
// call finds its keep bits ready and launches only this kernel again.
template <bool ALL, typename I>
__global__ __launch_bounds__(kDBlock) void k_dropout_apply_ahead(
    const f32x4 *__restrict__ x, f32x4 *__restrict__ out, uint32_t *__restrict__ mask,
    const uint32_t *__restrict__ bits, int64_t n4, float scale, unsigned na,
    const uint64_t *__restrict__ D, const uint32_t *__restrict__ E, const uint32_t *__restrict__ W,
    uint32_t *__restrict__ Wn, NextJump nj, int64_t nseg, uint32_t t2m1, uint32_t *__restrict__ next_bits,
    unsigned nb, unsigned period)
{
    const unsigned b = blockIdx.x, q = b / period, r = b - q * period;
    if (r == 0 && q < nb) {
        dropout_bits_block<ALL>(q, D, E, W, Wn, nj, nseg, t2m1, next_bits);
    } else {
        const unsigned before = q + 1 < nb ? q + 1 : nb;  // keep-bit blocks at indices <= b
        dropout_apply_block<I>(b - before, na, x, out, mask, bits, n4, scale);
    }
}

// Element-at-a-time form for unaligned buffers and the n % 4 tail.
__global__ __launch_bounds__(kDBlock) void k_dropout_apply1(const float *__restrict__ x, float *__restrict__ out,
                                                             uint8_t *__restrict__ mask,
                                                             const uint32_t *__restrict__ bits, int64_t d0, int64_t n,
                                                             float scale)
{
    for (int64_t d = d0 + int64_t(blockIdx.x) * kDBlock + threadIdx.x; d < n; d += int64_t(gridDim.x) * kDBlock) {
        const bool keep = keep_bits<int64_t>(bits, d) & 1u;
        out[d] = keep ? x[d] * scale : 0.0f;
        mask[d] = keep ? 1 : 0;
    }
}

// grad_in = mask ? grad_out * scale : +0 (any nonzero mask byte keeps).
__global__ __launch_bounds__(kDBlock) void k_dropout_bwd(const f32x4 *__restrict__ go, f32x4 *__restrict__ gi,
                                                          const uint32_t *__restrict__ mask, int64_t n4, float scale)
{
    const int64_t tile = int64_t(kDBlock) * kDUnroll;
    for (int64_t base = int64_t(blockIdx.x) * tile + threadIdx.x; base < n4; base += int64_t(gridDim.x) * tile) {
        f32x4 v[kDUnroll];
        uint32_t m[kDUnroll];
#pragma unroll
        for (int u = 0; u < kDUnroll; u++) {
            const int64_t q = base + int64_t(u) * kDBlock;
            if (q < n4) {
                v[u] = ld_nt(go + q);
                m[u] = ld_nt(mask + q);
            }
        }
#pragma unroll
        for (int u = 0; u < kDUnroll; u++) {
            const int64_t q = base + int64_t(u) * kDBlock;
            if (q < n4) {
                f32x4 o;
#pragma unroll
                for (int k = 0; k < 4; k++) o[k] = ((m[u] >> (8 * k)) & 0xFFu) ? v[u][k] * scale : 0.0f;
                st_nt(gi + q, o);
            }
        }
    }
}

__global__ __launch_bounds__(kDBlock) void k_dropout_bwd1(const float *__restrict__ go, float *__restrict__ gi,
                                                           const uint8_t *__restrict__ mask, int64_t d0, int64_t n,
                                                           float scale)
{
    for (int64_t d = d0 + int64_t(blockIdx.x) * kDBlock + threadIdx.x; d < n; d += int64_t(gridDim.x) * kDBlock)
        gi[d] = mask[d] ? go[d] * scale : 0.0f;
}

// ---- host side ------------------------------------------------------------------------

namespace {

using HPoly = std::vector<uint32_t>;  // kLag coefficients

HPoly hpoly_mul(const HPoly &a, const HPoly &b)
{
    uint32_t prod[2 * kLag - 1] = {0};
    for (int i = 0; i < kLag; i++)
        for (int j = 0; j < kLag; j++) prod[i + j] += a[size_t(i)] * b[size_t(j)];
    for (int d = 2 * kLag - 2; d >= kLag; d--) {
        prod[d - kLag] += prod[d];
        prod[d - 3] += prod[d];
    }
    return HPoly(prod, prod + kLag);
}

HPoly hpoly_xpow(uint64_t k)
{
    HPoly r(kLag, 0u), base(kLag, 0u);
    r[0] = 1u;
    base[1] = 1u;  // x
    while (k) {
        if (k & 1) r = hpoly_mul(r, base);
        base = hpoly_mul(base, base);
        k >>= 1;
    }
    return r;
}

// glibc srand(seed) followed by the 310 discarded values: r[313 .. 405], the
// window that precedes the first rand() output r[344] and the 62 values after
// it.
void seed_window(uint32_t seed, uint32_t *win)
{
    uint32_t r[344 + 2 * kLag];
    const uint32_t s = seed == 0 ? 1u : seed;
    r[0] = s;
    int32_t word = int32_t(s);
    for (int i = 1; i < kLag; i++) {
        // 16807 * word mod (2^31 - 1) without overflow (Schrage), as glibc does
        const int32_t hi = word / 127773, lo = word % 127773;
        word = 16807 * lo - 2836 * hi;
        if (word < 0) word += 2147483647;
        r[i] = uint32_t(word);
    }
    for (int i = kLag; i < 34; i++) r[i] = r[i - kLag];
    for (int i = 34; i < 344 + 2 * kLag; i++) r[i] = r[i - kLag] + r[i - 3];
    std::memcpy(win, r + 344 - kLag, kWin * sizeof(uint32_t));
}

struct Stream {
    std::mutex mu;
    bool ready = false;
    uint32_t *win[2] = {nullptr, nullptr};  // device stream values, kWin words (current, next)
    int cur = 0;
    uint64_t *dig = nullptr;                // d_l = x^(lL) mod P, l < 64, as MFMA digits (1024 words)
    uint32_t *ejump = nullptr;              // e_w = x^(64 w L) mod P, 32 words per wave
    int64_t ejump_n = 0;                    // waves covered (a power of two >= 1024)
    uint32_t *wpowers = nullptr;            // x^(64 L 2^k) mod P, k < 63
    uint32_t *bits = nullptr;
    size_t bits_cap = 0;
    uint64_t drawn = 0;                     // draws since the last seed
    NextJump nj{};                          // x^n, x^(n+31) mod P for n = nj_n
    int64_t nj_n = -1;
    // Keep bits made ahead by the previous call's apply pass for the draws
    // that follow it, valid for a call of ahead_n draws at threshold
    // ahead_t2m1 (ahead_all: every draw kept); the window after those draws
    // is then in win[cur ^ 1].
    uint32_t *ahead_bits = nullptr;
    size_t ahead_cap = 0;
    bool ahead_valid = false;
    int64_t ahead_n = -1;
    uint32_t ahead_t2m1 = 0;
    bool ahead_all = false;
    // (A change of the library's stream synchronises the old one first, so
    // calls on different streams never overlap on these buffers.)
    int64_t last_n = -1;                    // the previous call's draws and threshold
    uint32_t last_t2m1 = 0;
    bool last_all = false;
};

Stream &S()
{
    static Stream *s = new Stream();  // never destroyed: kernels may outlive static dtors
    return *s;
}

int set_seed_locked(Stream &s, uint32_t seed)
{
    uint32_t w[kWin];
    seed_window(seed, w);
    s.ahead_valid = false;
    NH_TRY(sync());
    NH_HIP(hipMemcpy(s.win[s.cur], w, sizeof(w), hipMemcpyHostToDevice));
    s.drawn = 0;
    s.last_n = -1;
    return NEURAL_OK;
}

int ensure_stream_locked(Stream &s)
{
    if (s.ready) return NEURAL_OK;
    for (int i = 0; i < 2; i++) {
        s.win[i] = static_cast<uint32_t *>(dev_alloc(kWin * sizeof(uint32_t)));
        if (!s.win[i]) return set_error(NEURAL_ERR_OUT_OF_MEMORY);
    }
    // x^(L 2^k) for the 64-row digit table, x^(64 L 2^k) for the wave jumps
    std::vector<uint32_t> B(size_t(63) * kLag), B64(size_t(63) * kLag);
    HPoly p = hpoly_xpow(uint64_t(kSegL)), p64 = hpoly_xpow(uint64_t(64 * kSegL));
    for (int k = 0; k < 63; k++) {
        std::memcpy(B.data() + size_t(k) * kLag, p.data(), kLag * sizeof(uint32_t));
        std::memcpy(B64.data() + size_t(k) * kLag, p64.data(), kLag * sizeof(uint32_t));
        p = hpoly_mul(p, p);
        p64 = hpoly_mul(p64, p64);
    }
    uint32_t *powers = static_cast<uint32_t *>(dev_alloc(B.size() * sizeof(uint32_t)));
    s.wpowers = static_cast<uint32_t *>(dev_alloc(B64.size() * sizeof(uint32_t)));
    s.dig = static_cast<uint64_t *>(dev_alloc(kTabWordsPerWave * sizeof(uint64_t)));
    if (!powers || !s.wpowers || !s.dig) return set_error(NEURAL_ERR_OUT_OF_MEMORY);
    NH_HIP(hipMemcpy(powers, B.data(), B.size() * sizeof(uint32_t), hipMemcpyHostToDevice));
    NH_HIP(hipMemcpy(s.wpowers, B64.data(), B64.size() * sizeof(uint32_t), hipMemcpyHostToDevice));
    NH_LAUNCH(k_jump_table, dim3(1), dim3(kDBlock), 0, stream(), s.dig, int64_t(0), int64_t(64), powers);
    NH_TRY(check_launch());
    dev_free(powers);  // stream-ordered: reused only by later work on the stream
    s.ready = true;
    return set_seed_locked(s, 1u);  // glibc's initial state is srand(1)
}

// Grow the wave-jump table to cover nwaves waves (doubling; old entries kept).
int ensure_jumps_locked(Stream &s, int64_t nwaves)
{
    if (nwaves <= s.ejump_n) return NEURAL_OK;
    int64_t cap = s.ejump_n > 0 ? s.ejump_n : 1024;
    while (cap < nwaves) cap *= 2;
    uint32_t *t = static_cast<uint32_t *>(dev_alloc(size_t(cap) * 32 * sizeof(uint32_t)));
    if (!t) return set_error(NEURAL_ERR_OUT_OF_MEMORY);
    if (s.ejump_n > 0)
        NH_HIP(hipMemcpyAsync(t, s.ejump, size_t(s.ejump_n) * 32 * sizeof(uint32_t), hipMemcpyDeviceToDevice,
                              stream()));
    const int64_t fresh = cap - s.ejump_n;
    NH_LAUNCH(k_wave_jumps, dim3(unsigned(ceil_div(fresh, kDBlock))), dim3(kDBlock), 0, stream(), t, s.ejump_n,
              cap, s.wpowers);
    NH_TRY(check_launch());
    if (s.ejump) dev_free(s.ejump);
    s.ejump = t;
    s.ejump_n = cap;
    return NEURAL_OK;
}

// cvtsd2si under the default rounding mode: nearest-even; NaN and values
// outside int64 give the "integer indefinite" INT64_MIN.
int64_t cvtsd2si(double v)
{
    if (!(v >= -0x1p63 && v < 0x1p63)) return INT64_MIN;
    return int64_t(std::nearbyint(v));
}

float drop_scale(float p) { return float(1.0 / (1.0 - double(p))); }

inline unsigned d_grid(int64_t work)
{
    int64_t g = ceil_div(work, kDBlock);
    const int64_t cap = kMaxGridBlocks;
    if (g > cap) g = cap;
    return unsigned(g < 1 ? 1 : g);
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

static int dropout_fwd(const float *in, float *out, uint8_t *mask, uint64_t n, float p)
{
    if (!in || !out || !mask) return set_error(NEURAL_ERR_NULL_POINTER);
    NH_TRY(ensure_init());
    if (n == 0) return set_error(NEURAL_OK);
    if (n > (uint64_t(1) << 40)) return set_error(NEURAL_ERR_TENSOR_TOO_LARGE);
    Stream &s = S();
    std::lock_guard<std::mutex> lock(s.mu);
    NH_TRY(ensure_stream_locked(s));
    const int64_t nn = int64_t(n);
    const int64_t nseg = ceil_div(nn, kSegL);
    // every wave of the grid (ceil(nseg / 256) blocks of 4) has a wave jump
    NH_TRY(ensure_jumps_locked(s, ceil_div(nseg, kDBlock) * (kDBlock / 64)));
    const size_t words = size_t(nseg) * kSegWords;
    const int64_t th = cvtsd2si(double(p) * 2147483647.0);
    const uint32_t thr = th <= 0 ? 0u : (th >= (int64_t(1) << 31) ? 0x80000000u : uint32_t(th));
    const float scale = drop_scale(p);
    // keep = r > 2 thr - 1 (thr >= 1), or every draw (thr = 0)
    const uint32_t t2m1 = uint32_t(2 * uint64_t(thr) - 1u);
    const bool all = thr == 0;
    const bool hit = s.ahead_valid && s.ahead_n == nn && s.ahead_t2m1 == t2m1 && s.ahead_all == all;
    s.ahead_valid = false;
    if (hit) {
        // this call's keep bits were made by the previous call's apply pass
        std::swap(s.bits, s.ahead_bits);
        std::swap(s.bits_cap, s.ahead_cap);
    }
    if (words > s.bits_cap) {
        if (s.bits) dev_free(s.bits);
        s.bits = static_cast<uint32_t *>(dev_alloc(words * sizeof(uint32_t)));
        s.bits_cap = s.bits ? words : 0;
        if (!s.bits) return set_error(NEURAL_ERR_OUT_OF_MEMORY);
    }

    Staged xi, xo, xm;
    NH_TRY(xi.open_n(in, n, 4, true));
    NH_TRY(xo.open_n(out, n, 4, false));
    NH_TRY(xm.open(mask, size_t(n), false));
    if (nn != s.nj_n) {
        // x^n and x^(n+31) mod P for the next call's values
        const HPoly c0 = hpoly_xpow(uint64_t(nn)), c1 = hpoly_mul(c0, hpoly_xpow(uint64_t(kLag)));
        std::memcpy(s.nj.c0, c0.data(), sizeof(s.nj.c0));
        std::memcpy(s.nj.c1, c1.data(), sizeof(s.nj.c1));
        s.nj_n = nn;
    }
    const unsigned nbits_blocks = unsigned(ceil_div(nseg, kDBlock));
    if (!hit) {
        uint32_t *W = s.win[s.cur], *Wn = s.win[s.cur ^ 1];
        if (all)
            NH_LAUNCH(k_dropout_bits<true>, dim3(nbits_blocks), dim3(kDBlock), 0, stream(), s.dig, s.ejump, W, Wn,
                      s.nj, nseg, t2m1, s.bits);
        else
            NH_LAUNCH(k_dropout_bits<false>, dim3(nbits_blocks), dim3(kDBlock), 0, stream(), s.dig, s.ejump, W, Wn,
                      s.nj, nseg, t2m1, s.bits);
        NH_TRY(check_launch());
    }
    // win[cur ^ 1] now holds (or, after a hit, already held) the window after
    // this call's draws
    s.cur ^= 1;
    s.drawn += n;
    const float *X = static_cast<const float *>(xi.dev);
    float *O = static_cast<float *>(xo.dev);
    uint8_t *M = static_cast<uint8_t *>(xm.dev);
    int64_t done = 0;
    if (aligned16(X) && aligned16(O) && (reinterpret_cast<uintptr_t>(M) & 3u) == 0) {
        const int64_t n4 = nn / 4;
        // A second call in a row with these draws and threshold: make the next
        // call's keep bits during this apply pass.
        bool ahead = n4 > 0 && nn == s.last_n && t2m1 == s.last_t2m1 && all == s.last_all &&
                     int64_t(d_grid(ceil_div(n4, kDUnroll))) + nbits_blocks < (int64_t(1) << 31);
        if (ahead && words > s.ahead_cap) {
            if (s.ahead_bits) dev_free(s.ahead_bits);
            s.ahead_bits = static_cast<uint32_t *>(dev_alloc(words * sizeof(uint32_t)));
            s.ahead_cap = s.ahead_bits ? words : 0;
            ahead = s.ahead_bits != nullptr;  // without the buffer, the plain pass
        }
        if (ahead) {
            const unsigned na = d_grid(ceil_div(n4, kDUnroll));
            const unsigned total = na + nbits_blocks;
            const unsigned period = total / nbits_blocks;
            uint32_t *W = s.win[s.cur], *Wn = s.win[s.cur ^ 1];
            const auto *xv = reinterpret_cast<const f32x4 *>(X);
            auto *ov = reinterpret_cast<f32x4 *>(O);
            auto *mv = reinterpret_cast<uint32_t *>(M);
            if (nn < (int64_t(1) << 32)) {
                if (all)
                    NH_LAUNCH((k_dropout_apply_ahead<true, uint32_t>), dim3(total), dim3(kDBlock), 0, stream(), xv,
                              ov, mv, s.bits, n4, scale, na, s.dig, s.ejump, W, Wn, s.nj, nseg, t2m1,
                              s.ahead_bits, nbits_blocks, period);
                else
                    NH_LAUNCH((k_dropout_apply_ahead<false, uint32_t>), dim3(total), dim3(kDBlock), 0, stream(), xv,
                              ov, mv, s.bits, n4, scale, na, s.dig, s.ejump, W, Wn, s.nj, nseg, t2m1,
                              s.ahead_bits, nbits_blocks, period);
            } else {
                if (all)
                    NH_LAUNCH((k_dropout_apply_ahead<true, int64_t>), dim3(total), dim3(kDBlock), 0, stream(), xv,
                              ov, mv, s.bits, n4, scale, na, s.dig, s.ejump, W, Wn, s.nj, nseg, t2m1,
                              s.ahead_bits, nbits_blocks, period);
                else
                    NH_LAUNCH((k_dropout_apply_ahead<false, int64_t>), dim3(total), dim3(kDBlock), 0, stream(), xv,
                              ov, mv, s.bits, n4, scale, na, s.dig, s.ejump, W, Wn, s.nj, nseg, t2m1,
                              s.ahead_bits, nbits_blocks, period);
            }
            NH_TRY(check_launch());
            s.ahead_valid = true;
            s.ahead_n = nn;
            s.ahead_t2m1 = t2m1;
            s.ahead_all = all;
        } else if (n4 > 0) {
            if (nn < (int64_t(1) << 32))
                NH_LAUNCH(k_dropout_apply<uint32_t>, dim3(d_grid(ceil_div(n4, kDUnroll))), dim3(kDBlock), 0,
                                   stream(), reinterpret_cast<const f32x4 *>(X), reinterpret_cast<f32x4 *>(O),
                                   reinterpret_cast<uint32_t *>(M), s.bits, n4, scale);
            else
                NH_LAUNCH(k_dropout_apply<int64_t>, dim3(d_grid(ceil_div(n4, kDUnroll))), dim3(kDBlock), 0,
                                   stream(), reinterpret_cast<const f32x4 *>(X), reinterpret_cast<f32x4 *>(O),
                                   reinterpret_cast<uint32_t *>(M), s.bits, n4, scale);
            NH_TRY(check_launch());
        }
        done = n4 * 4;
    }
    s.last_n = nn;
    s.last_t2m1 = t2m1;
    s.last_all = all;
    if (done < nn) {
        NH_LAUNCH(k_dropout_apply1, dim3(d_grid(nn - done)), dim3(kDBlock), 0, stream(), X, O, M, s.bits,
                           done, nn, scale);
        NH_TRY(check_launch());
    }
    NH_TRY(xo.finish(true));
    NH_TRY(xm.finish(true));
    NH_TRY(xi.finish(false));
    return set_error(NEURAL_OK);
}

static int dropout_bwd(const float *go, float *gi, const uint8_t *mask, uint64_t n, float p)
{
    if (!go || !gi || !mask) return set_error(NEURAL_ERR_NULL_POINTER);
    NH_TRY(ensure_init());
    if (n == 0) return set_error(NEURAL_OK);
    const int64_t nn = int64_t(n);
    const float scale = drop_scale(p);
    Staged sg, so, sm;
    NH_TRY(sg.open_n(go, n, 4, true));
    NH_TRY(sm.open(mask, size_t(n), true));
    NH_TRY(so.open_n(gi, n, 4, false));
    const float *G = static_cast<const float *>(sg.dev);
    float *O = static_cast<float *>(so.dev);
    const uint8_t *M = static_cast<const uint8_t *>(sm.dev);
    int64_t done = 0;
    if (aligned16(G) && aligned16(O) && (reinterpret_cast<uintptr_t>(M) & 3u) == 0) {
        const int64_t n4 = nn / 4;
        if (n4 > 0) {
            NH_LAUNCH(k_dropout_bwd, dim3(d_grid(ceil_div(n4, kDUnroll))), dim3(kDBlock), 0, stream(),
                               reinterpret_cast<const f32x4 *>(G), reinterpret_cast<f32x4 *>(O),
                               reinterpret_cast<const uint32_t *>(M), n4, scale);
            NH_TRY(check_launch());
        }
        done = n4 * 4;
    }
    if (done < nn) {
        NH_LAUNCH(k_dropout_bwd1, dim3(d_grid(nn - done)), dim3(kDBlock), 0, stream(), G, O, M, done, nn,
                           scale);
        NH_TRY(check_launch());
    }
    NH_TRY(so.finish(true));
    NH_TRY(sg.finish(false));
    NH_TRY(sm.finish(false));
    return set_error(NEURAL_OK);
}

}  // namespace nh

using namespace nh;

extern "C" {

int neural_dropout_forward(const float *input, float *output, uint8_t *mask, uint64_t num_elements, float p)
{
    return dropout_fwd(input, output, mask, num_elements, p);
}

int neural_dropout_backward(const float *grad_output, float *grad_input, const uint8_t *mask, uint64_t num_elements,
                            float p)
{
    return dropout_bwd(grad_output, grad_input, mask, num_elements, p);
}

int neural_dropout_seed(uint32_t seed)
{
    NH_TRY(ensure_init());
    Stream &s = S();
    std::lock_guard<std::mutex> lock(s.mu);
    NH_TRY(ensure_stream_locked(s));
    NH_TRY(set_seed_locked(s, seed));
    return set_error(NEURAL_OK);
}

uint64_t neural_dropout_draws(void)
{
    Stream &s = S();
    std::lock_guard<std::mutex> lock(s.mu);
    return s.drawn;
}

}  // extern "C"
