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
// bytes, Mp a multiple of 128, Kp of 32); its row sums, one wave per row; B
// transposed into a zero-padded [Np x Kp] buffer (so both operands are
// k-contiguous) with its column sums (integer atomics spread over the grid:
// the sums are exact and order-free); then the
// product in 128 x 128 blocks (4 waves of 64 x 64, 2 x 2 MFMA tiles each),
// 32-deep K steps through LDS, and the correction and scaling in the
// epilogue.  The zero padding adds nothing to the products, so the K loop
// needs no bounds checks.
#include <cstdint>

#include "common.hpp"

namespace nh {

namespace {

typedef int i32x16 __attribute__((ext_vector_type(16)));

constexpr int kQT = 128;     // block tile (rows and columns)
constexpr int kQK = 32;      // K step
constexpr int kQPad = 5;     // LDS row stride in 8-byte words (4 used): spreads rows over banks

// A [M x K] -> Ap [Mp x Kp] zero-padded.  Thread (i, u) copies bytes
// 16u .. 16u + 15 of row i.
__global__ __launch_bounds__(256) void k_qpad_a(const int8_t *__restrict__ A, int8_t *__restrict__ Ap, int64_t M,
                                                int64_t K, int64_t Kp, int64_t units)
{
    // grid-stride over the M * units 16-byte units of the real rows (rows
    // M .. Mp - 1 of Ap were zeroed by the caller)
    for (int64_t t = int64_t(blockIdx.x) * 256 + threadIdx.x; t < M * units; t += int64_t(gridDim.x) * 256) {
        const int64_t i = t / units, u = t - i * units;
        int8_t b[16];
#pragma unroll
        for (int q = 0; q < 16; q++) {
            const int64_t k = 16 * u + q;
            b[q] = k < K ? A[i * K + k] : int8_t(0);
        }
        int4 v;
        __builtin_memcpy(&v, b, 16);
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
// 16 reads is one contiguous span of B's row k.
__global__ __launch_bounds__(256) void k_qpad_bt(const int8_t *__restrict__ B, int8_t *__restrict__ Bt,
                                                 int32_t *__restrict__ colB, int64_t K, int64_t N, int64_t Kp)
{
    const int64_t j = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (j >= N) return;
    // 16-byte K units blockIdx.y, blockIdx.y + gridDim.y, ... (gridDim.y <= 65535)
    for (int64_t u = blockIdx.y; u < Kp / 16; u += gridDim.y) {
        int8_t b[16];
        int32_t s = 0;
#pragma unroll
        for (int q = 0; q < 16; q++) {
            const int64_t k = 16 * u + q;
            b[q] = k < K ? B[k * N + j] : int8_t(0);
            s += b[q];
        }
        int4 v;
        __builtin_memcpy(&v, b, 16);
        *reinterpret_cast<int4 *>(Bt + j * Kp + 16 * u) = v;
        atomicAdd(colB + j, s);
    }
}

__global__ __launch_bounds__(256) void k_qgemm(const int8_t *__restrict__ Ap, const int8_t *__restrict__ Bt,
                                               double *__restrict__ C, const int32_t *__restrict__ rowA,
                                               const int32_t *__restrict__ colB, int64_t M, int64_t N, int64_t K,
                                               int64_t Kp, int32_t za, int32_t zb, double cs)
{
    __shared__ long sA[kQT][kQPad];
    __shared__ long sB[kQT][kQPad];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int64_t i0 = int64_t(blockIdx.y) * kQT, j0 = int64_t(blockIdx.x) * kQT;
    const int wr = 64 * (w >> 1), wc = 64 * (w & 1);  // the wave's 64 x 64 quadrant
    i32x16 acc[2][2];
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int b = 0; b < 2; b++) acc[a][b] = i32x16{0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    // tile loads: thread t copies 16 bytes of row t / 2 (half t % 2) of each tile
    const int lr = tid >> 1, lh = tid & 1;
    const int8_t *pa = Ap + (i0 + lr) * Kp + 16 * lh;
    const int8_t *pb = Bt + (j0 + lr) * Kp + 16 * lh;
    for (int64_t k0 = 0; k0 < Kp; k0 += kQK) {
        const int4 va = *reinterpret_cast<const int4 *>(pa + k0);
        const int4 vb = *reinterpret_cast<const int4 *>(pb + k0);
        long a2[2], b2[2];
        __builtin_memcpy(a2, &va, 16);
        __builtin_memcpy(b2, &vb, 16);
        sA[lr][2 * lh] = a2[0];
        sA[lr][2 * lh + 1] = a2[1];
        sB[lr][2 * lh] = b2[0];
        sB[lr][2 * lh + 1] = b2[1];
        __syncthreads();
#pragma unroll
        for (int kc = 0; kc < kQK / 16; kc++) {
            long av[2], bv[2];
#pragma unroll
            for (int t = 0; t < 2; t++) {
                av[t] = sA[wr + 32 * t + (lane & 31)][2 * kc + (lane >> 5)];
                bv[t] = sB[wc + 32 * t + (lane & 31)][2 * kc + (lane >> 5)];
            }
#pragma unroll
            for (int a = 0; a < 2; a++)
#pragma unroll
                for (int b = 0; b < 2; b++) acc[a][b] = __builtin_amdgcn_mfma_i32_32x32x16_i8(av[a], bv[b], acc[a][b], 0, 0, 0);
        }
        __syncthreads();
    }
    const uint32_t kzz = uint32_t(K) * uint32_t(za) * uint32_t(zb);
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int b = 0; b < 2; b++) {
            const int64_t col = j0 + wc + 32 * b + (lane & 31);
            if (col >= N) continue;
            const uint32_t cterm = uint32_t(za) * uint32_t(colB[col]);
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int64_t row = i0 + wr + 32 * a + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
                if (row < M) {
                    const uint32_t s = uint32_t(acc[a][b][v]) - uint32_t(zb) * uint32_t(rowA[row]) - cterm + kzz;
                    C[row * N + col] = double(int32_t(s)) * cs;
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
    const int64_t Mp = round_up(M, kQT), Np = round_up(N, kQT), Kp = round_up(K, kQK);
    // grid limit: the product's row tiles run in grid y (M <= 65535 * 128 =
    // 8,388,480; the reference has no such limit)
    if (Mp / kQT > 65535) {
        set_error(NEURAL_ERR_TENSOR_TOO_LARGE);
        return -1;
    }
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
    int rc = NEURAL_OK;
    // Only the padding rows (A rows M .. Mp-1, Bt rows N .. Np-1) and the
    // row / column sums start at zero: the copies write every byte of the
    // real rows, K padding included.
    const size_t padA = size_t((Mp - M) * Kp), padB = size_t((Np - N) * Kp);
    if ((padA && hipMemsetAsync(Ap + M * Kp, 0, padA, stream()) != hipSuccess) ||
        (padB && hipMemsetAsync(Bt + N * Kp, 0, padB, stream()) != hipSuccess) ||
        hipMemsetAsync(rowA, 0, size_t(Mp + Np) * sizeof(int32_t), stream()) != hipSuccess)
        rc = NEURAL_ERR_INTERNAL;
    const int64_t units = Kp / 16;
    if (rc == NEURAL_OK) {
        int64_t ga = ceil_div(M * units, 256);
        ga = ga > kMaxGridBlocks ? kMaxGridBlocks : ga;
        NH_LAUNCH(k_qpad_a, dim3(unsigned(ga)), dim3(256), 0, stream(), static_cast<const int8_t *>(sa.dev), Ap, M,
                  K, Kp, units);
        NH_LAUNCH(k_qrowsum, dim3(unsigned(ceil_div(M, 4))), dim3(256), 0, stream(), Ap, rowA, M, Kp);
        const unsigned gy = unsigned(units < 65535 ? units : 65535);
        NH_LAUNCH(k_qpad_bt, dim3(unsigned(ceil_div(N, 256)), gy), dim3(256), 0, stream(),
                  static_cast<const int8_t *>(sb.dev), Bt, colB, K, N, Kp);
        const double cs = pa->scale * pb->scale;  // combined_scale, quantize.c:198
        NH_LAUNCH(k_qgemm, dim3(unsigned(Np / kQT), unsigned(Mp / kQT)), dim3(256), 0, stream(), Ap, Bt,
                           static_cast<double *>(sc.dev), rowA, colB, M, N, K, Kp, pa->zero_point, pb->zero_point, cs);
        rc = check_launch();
    }
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
