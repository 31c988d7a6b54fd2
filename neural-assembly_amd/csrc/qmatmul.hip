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
// Four launches: A copied into a zero-padded [Mp x Kp] buffer (rows of Kp
// bytes, Mp a multiple of 256, Kp of 64); its row sums, one wave per row; B
// transposed into a zero-padded [Np x Kp] buffer (Np a multiple of 128; both
// operands k-contiguous) with its column sums (integer atomics spread over the
// grid: the sums are exact and order-free); then the product in 256 x 128
// blocks (4 waves of 128 x 64, 4 x 2 tiles of v_mfma_i32_32x32x32_i8 each: 6
// fragment reads from LDS per 8 products), 64-deep K
// steps through two LDS buffers (the next step's global loads are in flight
// while the current step multiplies; one barrier per step), and the
// correction and scaling in the epilogue.  The zero padding adds nothing to
// the products, so the K loop needs no bounds checks.
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
// written as zeros.  The same launch zeroes colB[0 .. Np) for the B pass's
// atomics (that pass runs after this one on the stream).
__global__ __launch_bounds__(256) void k_qpad_a(const int8_t *__restrict__ A, int8_t *__restrict__ Ap, int64_t M,
                                                int64_t Mp, int64_t K, int64_t Kp, int64_t units,
                                                int32_t *__restrict__ colB, int64_t Np)
{
    const int64_t g0 = int64_t(blockIdx.x) * 256 + threadIdx.x, stride = int64_t(gridDim.x) * 256;
    for (int64_t j = g0; j < Np; j += stride) colB[j] = 0;
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

// Sum of the four signed bytes of w.
__device__ __forceinline__ int32_t byte_sum(int32_t w)
{
    return int32_t(int8_t(w)) + int32_t(int8_t(w >> 8)) + int32_t(int8_t(w >> 16)) + (w >> 24);
}

// rowA[i] = sum of row i of Ap (its padding is zero), one wave per row.
__global__ __launch_bounds__(256) void k_qrowsum(const int8_t *__restrict__ Ap, int32_t *__restrict__ rowA,
                                                 int64_t M, int64_t Kp)
{
    const int64_t i = (int64_t(blockIdx.x) * 256 + threadIdx.x) >> 6;
    const int lane = threadIdx.x & 63;
    if (i >= M) return;  // uniform per wave
    const int4 *row = reinterpret_cast<const int4 *>(Ap + i * Kp);
    int32_t s = 0;
    for (int64_t u = lane; u < Kp / 16; u += 64) {
        const int4 v = row[u];
        s += byte_sum(v.x) + byte_sum(v.y) + byte_sum(v.z) + byte_sum(v.w);
    }
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
    if (lane == 0) rowA[i] = s;
}

// B [K x N] -> Bt [Np x Kp] (row j = column j of B) zero-padded; colB[j] +=
// the thread's 16 bytes.  Threads of a wave take consecutive j, so each of the
// 16 reads is one contiguous span of B's row k.  Rows N .. Np - 1 of Bt are
// written as zeros.
__global__ __launch_bounds__(256) void k_qpad_bt(const int8_t *__restrict__ B, int8_t *__restrict__ Bt,
                                                 int32_t *__restrict__ colB, int64_t K, int64_t N, int64_t Np,
                                                 int64_t Kp)
{
    const int64_t j = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (j >= Np) return;
    // 16-byte K units blockIdx.y, blockIdx.y + gridDim.y, ... (gridDim.y <= 65535)
    for (int64_t u = blockIdx.y; u < Kp / 16; u += gridDim.y) {
        int8_t b[16];
        int32_t s = 0;
#pragma unroll
        for (int q = 0; q < 16; q++) {
            const int64_t k = 16 * u + q;
            b[q] = k < K && j < N ? B[k * N + j] : int8_t(0);
            s += b[q];
        }
        int4 v;
        __builtin_memcpy(&v, b, 16);
        *reinterpret_cast<int4 *>(Bt + j * Kp + 16 * u) = v;
        if (j < N) atomicAdd(colB + j, s);
    }
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
                                               double *__restrict__ C, const int32_t *__restrict__ rowA,
                                               const int32_t *__restrict__ colB, int64_t M, int64_t N, int64_t K,
                                               int64_t Kp, int32_t za, int32_t zb, double cs)
{
    __shared__ i32x4 sA[2][kQBM * kQRow];
    __shared__ i32x4 sB[2][kQBN * kQRow];
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
        // the next step's slice (the last step reloads its own: in bounds, unused)
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
        // the other buffer was last read in step s - 1, before the barrier
        // that ended it; after the last step nothing reads it
#pragma unroll
        for (int q = 0; q < kQTM; q++) sA[cur ^ 1][st + 64 * kQRow * q] = ra[q];
#pragma unroll
        for (int q = 0; q < kQTN; q++) sB[cur ^ 1][st + 64 * kQRow * q] = rb[q];
        __syncthreads();
    }
    // result v of lane l is (row 8 (v / 4) + 4 (l / 32) + v % 4, column l % 32)
    // of the 32 x 32 tile
    const uint32_t kzz = uint32_t(K) * uint32_t(za) * uint32_t(zb);
#pragma unroll
    for (int a = 0; a < kQTM; a++)
#pragma unroll
        for (int b = 0; b < kQTN; b++) {
            const int64_t col = j0 + wc + 32 * b + (lane & 31);
            if (col >= N) continue;
            const uint32_t cterm = uint32_t(za) * uint32_t(colB[col]);
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int64_t row = i0 + wr + 32 * a + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
                if (row < M) {
                    const uint32_t s = uint32_t(acc[a][b][v]) - uint32_t(zb) * uint32_t(rowA[row]) - cterm + kzz;
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
    const size_t bytesA = size_t(Mp * Kp), bytesB = size_t(Np * Kp);
    char *blk = static_cast<char *>(dev_alloc(bytesA + bytesB + size_t(Mp + Np) * sizeof(int32_t)));
    if (!blk) {
        set_error(NEURAL_ERR_OUT_OF_MEMORY);
        return -1;
    }
    int8_t *Ap = reinterpret_cast<int8_t *>(blk), *Bt = Ap + bytesA;
    int32_t *rowA = reinterpret_cast<int32_t *>(Bt + bytesB), *colB = rowA + Mp;
    // The copies write every byte of Ap and Bt (padding rows and K padding
    // as zeros) and the A pass zeroes colB; rowA is written for rows < M, the
    // only ones the product reads.
    const int64_t units = Kp / 16;
    int64_t ga = ceil_div(Mp * units, 256);
    ga = ga > kMaxGridBlocks ? kMaxGridBlocks : ga;
    NH_LAUNCH(k_qpad_a, dim3(unsigned(ga)), dim3(256), 0, stream(), static_cast<const int8_t *>(sa.dev), Ap, M, Mp,
              K, Kp, units, colB, Np);
    NH_LAUNCH(k_qrowsum, dim3(unsigned(ceil_div(M, 4))), dim3(256), 0, stream(), Ap, rowA, M, Kp);
    const unsigned gy = unsigned(units < 65535 ? units : 65535);
    NH_LAUNCH(k_qpad_bt, dim3(unsigned(ceil_div(Np, 256)), gy), dim3(256), 0, stream(),
              static_cast<const int8_t *>(sb.dev), Bt, colB, K, N, Np, Kp);
    const double cs = pa->scale * pb->scale;  // combined_scale, quantize.c:198
    NH_LAUNCH(k_qgemm, dim3(unsigned(Np / kQBN), unsigned(Mp / kQBM)), dim3(256), 0, stream(), Ap, Bt,
              static_cast<double *>(sc.dev), rowA, colB, M, N, K, Kp, pa->zero_point, pb->zero_point, cs);
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
