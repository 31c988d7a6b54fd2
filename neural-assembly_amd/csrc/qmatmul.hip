// qmatmul.hip -- quantized_matmul (quantize.c:191-214): C[M x N] (double) from
// int8 A[M x K] and B[K x N] with their QuantParams:
//   C[i][j] = (double)acc * (sa * sb),  acc = sum_k (A[i][k] - za) (B[k][j] - zb)
// with acc an int32 (the reference's loop; an overflowing sum wraps).
//
// On the matrix cores.  (A - za) and (B - zb) do not fit int8, so the sum is
// split (exactly, mod 2^32):
//   acc = sum_k A B - zb * rowA[i] - za * colB[j] + K za zb,
// rowA[i] = sum_k A[i][k], colB[j] = sum_k B[k][j].  sum_k A B is an int8 x
// int8 -> int32 product, v_mfma_i32_32x32x16_i8 (lane l holds row / column
// l % 32 and k = 8 (l / 32) + b of a 16-deep slice; result v of lane l is
// (row 8 (v/4) + 4 (l/32) + v % 4, column l % 32)).
//
// Two launches (one where A needs no padding): A copied into a zero-padded
// [Mp x Kp] buffer (rows of Kp bytes, Mp a multiple of 256, Kp of 64) unless
// A already is one (M a multiple of 256, K of 64, 16-byte aligned); B
// transposed into a zero-padded [Np x Kp] buffer (Np a multiple of 128; both
// operands k-contiguous); then the product in 256 x 128 blocks (4 waves of
// 128 x 64, 4 x 2 tiles of v_mfma_i32_32x32x32_i8 each: 6 fragment reads from
// LDS per 8 products), 64-deep K steps through two LDS buffers (the next
// step's global loads are in flight while the current step multiplies; one
// barrier per step).  The block also sums its rows of A and columns of B from
// the bytes it stages (v_dot4_i32_i8 against ones; the zero padding adds
// nothing) and applies the correction and scaling in the epilogue.  The K
// loop needs no bounds checks.
#include <cstdint>

#include "common.hpp"

namespace nh {

namespace {

typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

constexpr int kQLimitTile = 128;  // the API's row limit: 65535 tiles of 128 rows
constexpr int kQTM = 4, kQTN = 2;  // 32 x 32 tiles per wave: a wave computes 128 x 64
constexpr int kQBM = 64 * kQTM;    // block tile rows (2 x 2 waves)
constexpr int kQBN = 64 * kQTN;    // block tile columns
constexpr int kQK = 64;            // K step (bytes of a row per LDS stage)
constexpr int kQRow = 5;           // LDS row stride in 16-byte units (4 used): 8 lanes of a
                                   // 16-byte read cover all 32 four-byte banks once
constexpr int kQGroupRows = 2048;  // rows per group of the block order

// A [M x K] -> Ap [Mp x Kp] zero-padded.  Thread (i, u) copies bytes
// 16u .. 16u + 15 of row i: one 16-byte load where those bytes lie inside the
// row at a 16-byte aligned address, else byte by byte; rows M .. Mp - 1 are
// written as zeros.
__global__ __launch_bounds__(256) void k_qpad_a(const int8_t *__restrict__ A, int8_t *__restrict__ Ap, int64_t M,
                                                int64_t Mp, int64_t K, int64_t Kp, int64_t units)
{
    const int64_t g0 = int64_t(blockIdx.x) * 256 + threadIdx.x, stride = int64_t(gridDim.x) * 256;
    for (int64_t t = g0; t < Mp * units; t += stride) {
        const int64_t i = t / units, u = t - i * units;
        const int8_t *src = A + i * K + 16 * u;
        int4 v = int4{0, 0, 0, 0};
        if (i < M) {
            if (16 * u + 16 <= K && (reinterpret_cast<uintptr_t>(src) & 15) == 0) {
                v = *reinterpret_cast<const int4 *>(src);
            } else {
                int8_t b[16];
#pragma unroll
                for (int q = 0; q < 16; q++) b[q] = 16 * u + q < K ? src[q] : int8_t(0);
                __builtin_memcpy(&v, b, 16);
            }
        }
        *reinterpret_cast<int4 *>(Ap + i * Kp + 16 * u) = v;
    }
}

// B [K x N] -> Bt [Np x Kp] (row j = column j of B) zero-padded, rows
// N .. Np - 1 as zeros.  A thread transposes a 16 x 4 byte block: 16 rows
// k = 64 g + 16 (l % 4) + q of B times 4 columns 4 c .. 4 c + 3 (one 4-byte
// load per row where N is a multiple of 4 and B 4-byte aligned, else byte
// loads), into 16 bytes of each of 4 rows of Bt.  Lane l of a wave takes
// column group c = 16 (wave) + l / 4 within its block: its loads read 64
// contiguous bytes of 4 rows of B, and lanes 4 m .. 4 m + 3 write 64
// contiguous bytes of each of their rows of Bt.
__global__ __launch_bounds__(256) void k_qpad_bt(const int8_t *__restrict__ B, int8_t *__restrict__ Bt, int64_t K,
                                                 int64_t N, int64_t Np, int64_t Kp, int vec)
{
    const int64_t c = int64_t(blockIdx.x) * 64 + (threadIdx.x >> 2);  // column group
    if (4 * c >= Np) return;
    const int ul = threadIdx.x & 3;
    // 64-byte K groups blockIdx.y, blockIdx.y + gridDim.y, ... (gridDim.y <= 65535)
    for (int64_t g = blockIdx.y; g < Kp / 64; g += gridDim.y) {
        const int64_t k0 = 64 * g + 16 * ul;
        uint32_t w[16];
#pragma unroll
        for (int q = 0; q < 16; q++) {
            const int64_t k = k0 + q;
            w[q] = 0;
            if (k < K) {
                if (vec && 4 * c < N) {
                    w[q] = *reinterpret_cast<const uint32_t *>(B + k * N + 4 * c);
                } else {
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        if (4 * c + e < N) w[q] |= uint32_t(uint8_t(B[k * N + 4 * c + e])) << (8 * e);
                }
            }
        }
#pragma unroll
        for (int e = 0; e < 4; e++) {
            uint32_t o[4];
#pragma unroll
            for (int r = 0; r < 4; r++)
                o[r] = ((w[4 * r] >> (8 * e)) & 0xff) | (((w[4 * r + 1] >> (8 * e)) & 0xff) << 8) |
                       (((w[4 * r + 2] >> (8 * e)) & 0xff) << 16) | (((w[4 * r + 3] >> (8 * e)) & 0xff) << 24);
            *reinterpret_cast<uint4 *>(Bt + (4 * c + e) * Kp + k0) = uint4{o[0], o[1], o[2], o[3]};
        }
    }
}

// acc + the sum of the 16 signed bytes of v (v_dot4_i32_i8 against ones;
// wraps mod 2^32 like the reference's int32 sums).
__device__ __forceinline__ int32_t byte_sum4(i32x4 v, int32_t acc)
{
    acc = __builtin_amdgcn_sdot4(v.x, 0x01010101, acc, false);
    acc = __builtin_amdgcn_sdot4(v.y, 0x01010101, acc, false);
    acc = __builtin_amdgcn_sdot4(v.z, 0x01010101, acc, false);
    return __builtin_amdgcn_sdot4(v.w, 0x01010101, acc, false);
}

// Block order: the hardware hands block h to XCD h % 8 (each XCD has its own
// L2), so h is first renumbered to make each XCD's blocks consecutive, then
// taken in groups of kQGroupRows rows of tiles, column by column within a
// group: the blocks that share an XCD share few A row panels and B column
// panels.
__device__ __forceinline__ void qgemm_tile(int64_t &bi, int64_t &bj)
{
    constexpr int64_t G = kQGroupRows / kQBM;
    const int64_t nbx = gridDim.x, nby = gridDim.y, nb = nbx * nby;
    const int64_t h = int64_t(blockIdx.y) * nbx + blockIdx.x;
    const int64_t L = (nb & 7) == 0 ? (h & 7) * (nb >> 3) + (h >> 3) : h;
    const int64_t gsz = G * nbx, g = L / gsz, r = L - g * gsz;
    const int64_t first = g * G, rows = nby - first < G ? nby - first : G;
    bi = first + r % rows;
    bj = r / rows;
}

// C block (kQBM x kQBN) of tile (bi, bj).  Ap [Mp x Kp] and Bt [Np x Kp]
// zero-padded, Kp a multiple of kQK.
__global__ __launch_bounds__(256) void k_qgemm(const int8_t *__restrict__ Ap, const int8_t *__restrict__ Bt,
                                               double *__restrict__ C, int64_t M, int64_t N, int64_t K, int64_t Kp,
                                               int32_t za, int32_t zb, double cs)
{
    __shared__ i32x4 sA[2][kQBM * kQRow];
    __shared__ i32x4 sB[2][kQBN * kQRow];
    __shared__ int32_t sRow[kQBM], sCol[kQBN];  // sums of the block's rows of A, columns of B
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    int64_t bi, bj;
    qgemm_tile(bi, bj);
    const int64_t i0 = bi * kQBM, j0 = bj * kQBN;
    const int wr = 32 * kQTM * (w >> 1), wc = 32 * kQTN * (w & 1);  // the wave's quadrant
    i32x16 acc[kQTM][kQTN];
#pragma unroll
    for (int a = 0; a < kQTM; a++)
#pragma unroll
        for (int b = 0; b < kQTN; b++) acc[a][b] = i32x16{0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    // stage loads: thread t copies 16-byte unit t % 4 of rows t / 4 + 64 q
    const int lr = tid >> 2, lu = tid & 3;
    const int8_t *pa = Ap + (i0 + lr) * Kp + 16 * lu;
    const int8_t *pb = Bt + (j0 + lr) * Kp + 16 * lu;
    const int64_t far = 64 * Kp;
    i32x4 ra[kQTM], rb[kQTN];
#pragma unroll
    for (int q = 0; q < kQTM; q++) ra[q] = *reinterpret_cast<const i32x4 *>(pa + q * far);
#pragma unroll
    for (int q = 0; q < kQTN; q++) rb[q] = *reinterpret_cast<const i32x4 *>(pb + q * far);
    // partial sums of the thread's rows of A / columns of B over its units
    int32_t ha[kQTM], hb[kQTN];
    auto add_sums = [&]() {
#pragma unroll
        for (int q = 0; q < kQTM; q++) ha[q] = byte_sum4(ra[q], ha[q]);
#pragma unroll
        for (int q = 0; q < kQTN; q++) hb[q] = byte_sum4(rb[q], hb[q]);
    };
#pragma unroll
    for (int q = 0; q < kQTM; q++) ha[q] = 0;
#pragma unroll
    for (int q = 0; q < kQTN; q++) hb[q] = 0;
    add_sums();
    const int st = lr * kQRow + lu;
#pragma unroll
    for (int q = 0; q < kQTM; q++) sA[0][st + 64 * kQRow * q] = ra[q];
#pragma unroll
    for (int q = 0; q < kQTN; q++) sB[0][st + 64 * kQRow * q] = rb[q];
    __syncthreads();
    // fragment reads: lane l takes row (column) l % 32 of a 32 x 32 tile and
    // bytes 16 (l / 32) .. 16 (l / 32) + 15 of a 32-deep chunk, for A and B
    // alike, so every k meets its partner in the product
    const int fa = (wr + (lane & 31)) * kQRow + (lane >> 5);
    const int fb = (wc + (lane & 31)) * kQRow + (lane >> 5);
    const int64_t steps = Kp / kQK;
    for (int64_t s = 0; s < steps; s++) {
        const int cur = int(s & 1);
        // the next step's slice (the last step reloads its own: in bounds, and
        // its sum is taken out after the loop)
        const int64_t k1 = (s + 1 < steps ? s + 1 : s) * kQK;
#pragma unroll
        for (int q = 0; q < kQTM; q++) ra[q] = *reinterpret_cast<const i32x4 *>(pa + q * far + k1);
#pragma unroll
        for (int q = 0; q < kQTN; q++) rb[q] = *reinterpret_cast<const i32x4 *>(pb + q * far + k1);
        // keep the loads ahead of the products (the scheduler would sink them
        // next to their LDS stores and wait on them there)
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int c = 0; c < kQK / 32; c++) {
            i32x4 av[kQTM], bv[kQTN];
#pragma unroll
            for (int t = 0; t < kQTM; t++) av[t] = sA[cur][fa + t * 32 * kQRow + 2 * c];
#pragma unroll
            for (int t = 0; t < kQTN; t++) bv[t] = sB[cur][fb + t * 32 * kQRow + 2 * c];
#pragma unroll
            for (int a = 0; a < kQTM; a++)
#pragma unroll
                for (int b = 0; b < kQTN; b++) acc[a][b] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[a], bv[b], acc[a][b], 0, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
        add_sums();
        // the other buffer was last read in step s - 1, before the barrier
        // that ended it; after the last step nothing reads it
#pragma unroll
        for (int q = 0; q < kQTM; q++) sA[cur ^ 1][st + 64 * kQRow * q] = ra[q];
#pragma unroll
        for (int q = 0; q < kQTN; q++) sB[cur ^ 1][st + 64 * kQRow * q] = rb[q];
        __syncthreads();
    }
    // the last step's reload was summed twice: take it out once (exact mod
    // 2^32); then whole-row sums: lanes 4 m .. 4 m + 3 hold the four units
    // of a row
#pragma unroll
    for (int q = 0; q < kQTM; q++) ha[q] -= byte_sum4(ra[q], 0);
#pragma unroll
    for (int q = 0; q < kQTN; q++) hb[q] -= byte_sum4(rb[q], 0);
#pragma unroll
    for (int q = 0; q < kQTM; q++) {
        ha[q] += __shfl_xor(ha[q], 1, 64);
        ha[q] += __shfl_xor(ha[q], 2, 64);
        if (lu == 0) sRow[lr + 64 * q] = ha[q];
    }
#pragma unroll
    for (int q = 0; q < kQTN; q++) {
        hb[q] += __shfl_xor(hb[q], 1, 64);
        hb[q] += __shfl_xor(hb[q], 2, 64);
        if (lu == 0) sCol[lr + 64 * q] = hb[q];
    }
    __syncthreads();
    // result v of lane l is (row 8 (v / 4) + 4 (l / 32) + v % 4, column l % 32)
    // of the 32 x 32 tile
    const uint32_t kzz = uint32_t(K) * uint32_t(za) * uint32_t(zb);
#pragma unroll
    for (int a = 0; a < kQTM; a++)
#pragma unroll
        for (int b = 0; b < kQTN; b++) {
            const int64_t col = j0 + wc + 32 * b + (lane & 31);
            if (col >= N) continue;
            const uint32_t cterm = uint32_t(za) * uint32_t(sCol[wc + 32 * b + (lane & 31)]);
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int rl = wr + 32 * a + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
                const int64_t row = i0 + rl;
                if (row < M) {
                    const uint32_t s = uint32_t(acc[a][b][v]) - uint32_t(zb) * uint32_t(sRow[rl]) - cterm + kzz;
                    __builtin_nontemporal_store(double(int32_t(s)) * cs, C + row * N + col);
                }
            }
        }
}

inline int64_t round_up(int64_t v, int64_t m) { return (v + m - 1) / m * m; }

}  // namespace

// A, B, C: host or device pointers; params: host pointers.  Returns 0 / -1
// like the reference.
static int qmatmul(const int8_t *A, const int8_t *B, double *C, int64_t M, int64_t K, int64_t N,
                   const QuantParams *pa, const QuantParams *pb)
{
    if (!A || !B || !C || !pa || !pb) return -1;
    if (M <= 0 || K <= 0 || N <= 0) return -1;
    if (ensure_init() != NEURAL_OK) return -1;
    // the API's limit: 65535 tiles of 128 rows (M <= 8,388,480; the reference
    // has no such limit)
    if (round_up(M, kQLimitTile) / kQLimitTile > 65535) {
        set_error(NEURAL_ERR_TENSOR_TOO_LARGE);
        return -1;
    }
    const int64_t Mp = round_up(M, kQBM), Np = round_up(N, kQBN), Kp = round_up(K, kQK);
    Staged sa, sb, sc;
    if (sa.open(A, size_t(M * K), true) != NEURAL_OK || sb.open(B, size_t(K * N), true) != NEURAL_OK ||
        sc.open(C, size_t(M * N) * sizeof(double), false) != NEURAL_OK)
        return -1;
    // A serves as its own padded copy when it already has the padded shape
    const bool copyA = Mp != M || Kp != K || (reinterpret_cast<uintptr_t>(sa.dev) & 15) != 0;
    const size_t bytesA = copyA ? size_t(Mp * Kp) : 0, bytesB = size_t(Np * Kp);
    char *blk = static_cast<char *>(dev_alloc(bytesA + bytesB));
    if (!blk) {
        set_error(NEURAL_ERR_OUT_OF_MEMORY);
        return -1;
    }
    int8_t *Bt = reinterpret_cast<int8_t *>(blk) + bytesA;
    const int8_t *Ap = copyA ? reinterpret_cast<int8_t *>(blk) : static_cast<const int8_t *>(sa.dev);
    // The copies write every byte of Ap and Bt (padding rows and K padding
    // as zeros).
    if (copyA) {
        const int64_t units = Kp / 16;
        int64_t ga = ceil_div(Mp * units, 256);
        ga = ga > kMaxGridBlocks ? kMaxGridBlocks : ga;
        NH_LAUNCH(k_qpad_a, dim3(unsigned(ga)), dim3(256), 0, stream(), static_cast<const int8_t *>(sa.dev),
                  reinterpret_cast<int8_t *>(blk), M, Mp, K, Kp, units);
    }
    const int64_t groups = Kp / 64;
    const unsigned gy = unsigned(groups < 65535 ? groups : 65535);
    const int vec = (N & 3) == 0 && (reinterpret_cast<uintptr_t>(sb.dev) & 3) == 0;
    NH_LAUNCH(k_qpad_bt, dim3(unsigned(ceil_div(Np, 256)), gy), dim3(256), 0, stream(),
              static_cast<const int8_t *>(sb.dev), Bt, K, N, Np, Kp, vec);
    const double cs = pa->scale * pb->scale;  // combined_scale, quantize.c:198
    NH_LAUNCH(k_qgemm, dim3(unsigned(Np / kQBN), unsigned(Mp / kQBM)), dim3(256), 0, stream(), Ap, Bt,
              static_cast<double *>(sc.dev), M, N, K, Kp, pa->zero_point, pb->zero_point, cs);
    const int rc = check_launch();
    dev_free(blk);
    if (rc != NEURAL_OK) return -1;
    if (sc.finish(true) != NEURAL_OK || sa.finish(false) != NEURAL_OK || sb.finish(false) != NEURAL_OK) return -1;
    set_error(NEURAL_OK);
    return 0;
}

}  // namespace nh

extern "C" int quantized_matmul(const int8_t *A, const int8_t *B, double *C, int64_t M, int64_t K, int64_t N,
                                const QuantParams *params_a, const QuantParams *params_b)
{
    return nh::qmatmul(A, B, C, M, K, N, params_a, params_b);
}
