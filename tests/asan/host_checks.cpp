// Host-side memory checks of libneural_hip: this program is built with
// AddressSanitizer and UndefinedBehaviorSanitizer and linked against
// libneural_hip_asan.so (the library's host code instrumented for both, its
// device code as usual), then walks the C ABI
// through the paths whose host code handles caller memory: tensor
// descriptors, shapes and strides, host mirrors and raw pointers into them,
// staging of host buffers, the optimizer state blob (including corrupt
// blobs), gradient-list tables, the dropout stream state, the measurement
// hooks and the error paths.  Numerics are checked elsewhere; here every
// call must return what its arguments call for, and the sanitizer must stay
// silent.  Prints "host checks: N passed" and exits 0, or lists failures.

#include <hip/hip_runtime_api.h>

#include <atomic>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <thread>
#include <vector>

#include "neural_api.h"

namespace {

std::atomic<int> g_checks{0}, g_fail{0};

#define CHECK(cond)                                                                   \
    do {                                                                              \
        g_checks++;                                                                   \
        if (!(cond)) {                                                                \
            g_fail++;                                                                 \
            std::printf("FAIL %s:%d: %s (last error %d)\n", __FILE__, __LINE__, #cond, \
                        neural_get_last_error());                                     \
            std::fflush(stdout);                                                      \
        }                                                                             \
    } while (0)

void section(const char *name)
{
    std::printf("== %s\n", name);
    std::fflush(stdout);
}

NeuralTensor *make(std::initializer_list<uint64_t> shape, int dtype = NEURAL_DTYPE_FLOAT32)
{
    std::vector<uint64_t> s(shape);
    return neural_tensor_create(s.data(), s.size(), dtype);
}

// Deterministic values in [-2, 2).
void fill_host(float *p, size_t n, uint32_t seed)
{
    uint32_t x = seed * 2654435761u + 1u;
    for (size_t i = 0; i < n; i++) {
        x = x * 1664525u + 1013904223u;
        p[i] = float(x >> 8) * (4.0f / 16777216.0f) - 2.0f;
    }
}

void fill_host(double *p, size_t n, uint32_t seed)
{
    std::vector<float> f(n);
    fill_host(f.data(), n, seed);
    for (size_t i = 0; i < n; i++) p[i] = double(f[i]);
}

NeuralTensor *upload(std::initializer_list<uint64_t> shape, uint32_t seed, int dtype = NEURAL_DTYPE_FLOAT32)
{
    NeuralTensor *t = make(shape, dtype);
    if (!t) return nullptr;
    const uint64_t n = neural_tensor_numel(t);
    if (dtype == NEURAL_DTYPE_FLOAT32) {
        std::vector<float> h(n);
        fill_host(h.data(), n, seed);
        if (n && neural_tensor_upload(t, h.data(), n * 4) != 0) return nullptr;
    } else {
        std::vector<double> h(n);
        fill_host(h.data(), n, seed);
        if (n && neural_tensor_upload(t, h.data(), n * 8) != 0) return nullptr;
    }
    return t;
}

void check_tensors()
{
    section("tensors");
    const std::vector<std::vector<uint64_t>> shapes = {{0}, {1}, {7}, {3, 5}, {2, 3, 4}, {2, 1, 3, 1}, {4, 0, 3}, {1, 1, 1, 1, 5}};
    for (int dt = 0; dt < 2; dt++) {
        for (const auto &s : shapes) {
            NeuralTensor *a = neural_tensor_create(s.data(), s.size(), dt);
            NeuralTensor *z = neural_tensor_zeros(s.data(), s.size(), dt);
            NeuralTensor *o = neural_tensor_ones(s.data(), s.size(), dt);
            CHECK(a && z && o);
            if (!a || !z || !o) continue;
            const uint64_t n = neural_tensor_numel(a), es = dt ? 8 : 4;
            CHECK(neural_tensor_ndim(a) == s.size());
            CHECK(std::memcmp(neural_tensor_shape(a), s.data(), s.size() * 8) == 0);
            CHECK(neural_tensor_bytes(a) == n * es);
            CHECK(neural_tensor_dtype(a) == dt);
            CHECK(neural_tensor_is_contiguous(a) == 1);
            CHECK(neural_tensor_stride(a) != nullptr);
            CHECK(neural_tensor_fill(a, 2.5) == 0);
            CHECK(neural_tensor_copy(z, a) == 0);
            // the host mirror: read what the device holds, write it, and read it back through a kernel
            void *h = neural_tensor_data(z);
            CHECK(n == 0 || h != nullptr);
            if (n && h) {
                if (dt) {
                    CHECK(static_cast<double *>(h)[n - 1] == 2.5);
                    static_cast<double *>(h)[0] = -1.0;
                } else {
                    CHECK(static_cast<float *>(h)[n - 1] == 2.5f);
                    static_cast<float *>(h)[0] = -1.0f;
                }
                CHECK(neural_tensor_copy(o, z) == 0);
                std::vector<unsigned char> back(n * es);
                CHECK(neural_tensor_download(o, back.data(), back.size()) == 0);
                if (dt) CHECK(reinterpret_cast<double *>(back.data())[0] == -1.0);
                else CHECK(reinterpret_cast<float *>(back.data())[0] == -1.0f);
                CHECK(neural_tensor_upload(o, back.data(), back.size()) == 0);
                CHECK(neural_tensor_upload(o, back.data(), back.size() + es) != 0);  // more than the tensor
            }
            NeuralBufferInfo info;
            CHECK(neural_buffer_info(a, &info) == 0);
            CHECK(info.ndim == s.size() && info.itemsize == es);
            // reshape to the flat shape and back
            const uint64_t flat[1] = {n};
            NeuralTensor *r = neural_tensor_reshape(a, flat, 1);
            CHECK(r != nullptr);
            if (r) {
                NeuralTensor *r2 = neural_tensor_reshape(r, s.data(), s.size());
                CHECK(r2 != nullptr);
                neural_tensor_free(r2);
                neural_tensor_free(r);
            }
            const uint64_t wrong[1] = {n + 1};
            CHECK(neural_tensor_reshape(a, wrong, 1) == nullptr);
            // a contiguous tensor comes back as itself (neural_api.h:199-204)
            NeuralTensor *c = neural_tensor_make_contiguous(a);
            CHECK(c == a);
            if (c != a) neural_tensor_free(c);
            neural_tensor_free(a);
            neural_tensor_free(z);
            neural_tensor_free(o);
        }
    }
    // from_data copies the host values
    std::vector<float> v(12);
    fill_host(v.data(), v.size(), 1);
    const uint64_t s34[2] = {3, 4};
    NeuralTensor *fd = neural_tensor_from_data(v.data(), s34, 2, NEURAL_DTYPE_FLOAT32);
    CHECK(fd != nullptr);
    std::vector<float> back(12);
    CHECK(neural_tensor_download(fd, back.data(), 48) == 0);
    CHECK(back == v);
    // from_buffer over a host buffer: contiguous, then a transposed view (byte strides)
    NeuralTensor *hb = neural_tensor_from_buffer(v.data(), s34, 2, NEURAL_DTYPE_FLOAT32, nullptr);
    const uint64_t s43[2] = {4, 3};
    const int64_t tstr[2] = {4, 16};
    NeuralTensor *tv = neural_tensor_from_buffer(v.data(), s43, 2, NEURAL_DTYPE_FLOAT32, tstr);
    CHECK(hb && tv);
    CHECK(neural_tensor_is_contiguous(tv) == 0);
    NeuralTensor *tc = neural_tensor_make_contiguous(tv);
    CHECK(tc != nullptr);
    if (tc) {
        CHECK(neural_tensor_download(tc, back.data(), 48) == 0);
        CHECK(back[1] == v[4] && back[3] == v[1]);
    }
    NeuralTensor *neg = make({3, 4});
    CHECK(neural_neg(neg, hb) == 0);
    CHECK(neural_scalar_mul(hb, hb, 2.0) == 0);  // writes back into the caller's buffer
    fill_host(back.data(), 12, 1);
    CHECK(v[5] == 2.0f * back[5]);
    neural_tensor_free(tc);
    neural_tensor_free(neg);
    neural_tensor_free(tv);
    neural_tensor_free(hb);
    neural_tensor_free(fd);
    // from_buffer over device memory
    float *dbuf = nullptr;
    CHECK(hipMalloc(&dbuf, 64 * 4) == hipSuccess);
    const uint64_t s64[1] = {64};
    NeuralTensor *db = neural_tensor_from_buffer(dbuf, s64, 1, NEURAL_DTYPE_FLOAT32, nullptr);
    CHECK(db != nullptr);
    CHECK(neural_tensor_fill(db, 3.0) == 0);
    double sum = 0;
    CHECK(neural_sum(db, &sum) == 0 && sum == 192.0);
    neural_tensor_free(db);
    CHECK(hipFree(dbuf) == hipSuccess);
    // refused shapes and arguments
    const uint64_t huge[3] = {uint64_t(1) << 40, uint64_t(1) << 40, 4};
    CHECK(neural_tensor_create(huge, 3, NEURAL_DTYPE_FLOAT32) == nullptr);
    CHECK(neural_get_last_error() == NEURAL_ERR_TENSOR_TOO_LARGE);
    CHECK(neural_tensor_create(s34, 2, 7) == nullptr);
    CHECK(neural_tensor_create(nullptr, 2, 0) == nullptr);
    CHECK(neural_tensor_fill(nullptr, 1.0) != 0);
    CHECK(neural_tensor_copy(nullptr, nullptr) != 0);
    neural_tensor_free(nullptr);
    CHECK(neural_get_error_message(NEURAL_ERR_SHAPE_MISMATCH) != nullptr);
    CHECK(neural_get_error_message(12345) != nullptr);
    CHECK(neural_version() != nullptr);
}

void check_math()
{
    section("elementwise, broadcast, activations");
    for (int dt = 0; dt < 2; dt++) {
        NeuralTensor *a = upload({4, 1, 3}, 2, dt), *b = upload({1, 5, 3}, 3, dt), *o = make({4, 5, 3}, dt);
        NeuralTensor *x = upload({6, 10}, 4, dt), *y = make({6, 10}, dt), *bias = upload({10}, 5, dt);
        CHECK(a && b && o && x && y && bias);
        CHECK(neural_add(o, a, b) == 0);
        CHECK(neural_sub(o, a, b) == 0);
        CHECK(neural_mul(o, a, b) == 0);
        CHECK(neural_div(o, a, b) == 0);
        CHECK(neural_maximum(o, a, b) == 0);
        CHECK(neural_add_relu(o, a, b) == 0);
        CHECK(neural_add(y, x, bias) == 0);
        CHECK(neural_add(y, x, a) != 0);  // shapes that do not broadcast
        CHECK(neural_scalar_add(y, x, 0.5) == 0);
        CHECK(neural_bias_add(y, x, bias) == 0);
        CHECK(neural_bias_add(x, x, bias) == 0);  // in place
        for (int act = 0; act <= 12; act++) CHECK(neural_bias_add_act(y, x, bias, act, 0.1) == 0);
        CHECK(neural_relu(y, x) == 0);
        CHECK(neural_sigmoid(y, x) == 0);
        CHECK(neural_tanh(y, x) == 0);
        CHECK(neural_gelu(y, x) == 0);
        CHECK(neural_leaky_relu(y, x, 0.01) == 0);
        CHECK(neural_elu(y, x, 1.0) == 0);
        CHECK(neural_selu(y, x) == 0);
        CHECK(neural_swish(y, x) == 0);
        CHECK(neural_mish(y, x) == 0);
        CHECK(neural_hardswish(y, x) == 0);
        CHECK(neural_softplus(y, x) == 0);
        CHECK(neural_hardtanh(y, x) == 0);
        CHECK(act_tanh(y, x) == 0 && act_gelu(y, x) == 0 && act_leaky_relu(y, x, 0.2) == 0);
        CHECK(act_elu(y, x, 1.0) == 0 && act_selu(y, x) == 0 && act_swish(y, x) == 0 && act_mish(y, x) == 0);
        CHECK(act_hardswish(y, x) == 0 && act_softplus(y, x) == 0 && act_hardtanh(y, x) == 0);
        CHECK(act_tanh(nullptr, x) != 0);
        neural_tensor_free(a);
        neural_tensor_free(b);
        neural_tensor_free(o);
        neural_tensor_free(x);
        neural_tensor_free(y);
        neural_tensor_free(bias);
    }
    // raw-pointer SIMD entry points on host arrays (odd lengths)
    for (uint64_t n : {uint64_t(1), uint64_t(13), uint64_t(1000), uint64_t(4099)}) {
        std::vector<float> a(n), b(n), c(n), d(n);
        fill_host(a.data(), n, 6);
        fill_host(b.data(), n, 7);
        fill_host(c.data(), n, 8);
        CHECK(simd_add_f32(d.data(), a.data(), b.data(), n) == 0);
        CHECK(d[n - 1] == a[n - 1] + b[n - 1]);
        CHECK(simd_mul_f32(d.data(), a.data(), b.data(), n) == 0);
        CHECK(simd_fma_f32(d.data(), a.data(), b.data(), c.data(), n) == 0);
        CHECK(std::isfinite(simd_dot_f32(a.data(), b.data(), n)));
        CHECK(std::isfinite(simd_sum_f32(a.data(), n)));
        vec_add_relu_fusion(a.data(), b.data(), d.data(), int64_t(n));
        CHECK(d[0] == std::fmax(a[0] + b[0], 0.0f));
    }
}

void check_reductions()
{
    section("reductions, row statistics, softmax");
    for (int dt = 0; dt < 2; dt++) {
        for (auto dims : std::vector<std::pair<uint64_t, uint64_t>>{{1, 1}, {5, 7}, {33, 4096}, {3, 70000}, {2049, 3}}) {
            const uint64_t r = dims.first, c = dims.second;
            NeuralTensor *x = upload({r, c}, 9, dt), *rows = make({r}, dt), *cols = make({c}, dt), *one = make({1}, dt);
            NeuralTensor *y = make({r, c}, dt), *bias = upload({c}, 10, dt);
            CHECK(x && rows && cols && one && y && bias);
            double v = 0;
            int64_t idx = -1;
            CHECK(neural_sum(x, &v) == 0 && neural_mean(x, &v) == 0 && neural_max(x, &v) == 0);
            CHECK(neural_argmax(x, &idx) == 0 && idx >= 0 && uint64_t(idx) < r * c);
            CHECK(neural_reduce_sum(x, -1, one) == 0 && neural_reduce_sum(x, 1, rows) == 0);
            CHECK(neural_reduce_sum(x, 0, cols) == 0 && neural_reduce_mean(x, 0, cols) == 0);
            CHECK(neural_reduce_mean(x, 1, rows) == 0 && neural_reduce_max(x, 1, rows) == 0);
            CHECK(neural_reduce_max(x, -1, rows) == 0);  // -1: the last dim, as ndim - 1
            CHECK(neural_reduce_max(x, 0, cols) == NEURAL_ERR_DIM_MISMATCH);
            CHECK(neural_reduce_sum(x, 1, cols) != 0 || r == c);  // wrong output size
            std::vector<int64_t> am(r);
            CHECK(neural_reduce_argmax(x, 1, am.data()) == 0);
            CHECK(am[r - 1] >= 0 && uint64_t(am[r - 1]) < c);
            CHECK(neural_row_stats(x, rows, nullptr, nullptr, nullptr) == 0);
            CHECK(neural_row_stats(x, nullptr, rows, nullptr, am.data()) == 0);
            CHECK(neural_row_stats(x, nullptr, nullptr, nullptr, nullptr) != 0);
            NeuralTensor *m2 = make({r}, dt), *m3 = make({r}, dt);
            CHECK(neural_bias_add_row_stats(y, x, bias, rows, m2, m3, am.data()) == 0);
            CHECK(neural_bias_add_row_stats(x, x, bias, rows, nullptr, m3, am.data()) == 0);  // in place
            CHECK(neural_softmax(y, x) == 0 && neural_log_softmax(y, x) == 0);
            int hn = -1, hi = -1;
            double ss = -1;
            CHECK(neural_tensor_scan(x, &hn, &hi, &ss) == 0 && hn == 0 && hi == 0 && ss >= 0);
            neural_tensor_free(m2);
            neural_tensor_free(m3);
            neural_tensor_free(x);
            neural_tensor_free(rows);
            neural_tensor_free(cols);
            neural_tensor_free(one);
            neural_tensor_free(y);
            neural_tensor_free(bias);
        }
    }
}

void check_raw_pointers()
{
    section("raw pointers: scans, quantization, mirrors, device pipeline");
    const uint64_t n = 100003;
    std::vector<float> g(n);
    fill_host(g.data(), n, 11);
    CHECK(neural_tensor_has_nan(g.data(), n) == 0 && neural_tensor_has_inf(g.data(), n) == 0);
    g[n - 1] = NAN;
    CHECK(neural_tensor_has_nan(g.data(), n) == 1);
    g[n - 1] = 1.0f;
    CHECK(neural_tensor_grad_l2_norm(g.data(), n) > 0.0f);
    int hn = -1, hi = -1;
    double ss = 0;
    CHECK(neural_scan_nan_inf_l2(g.data(), n, &hn, &hi, &ss) == 0);
    CHECK(neural_tensor_has_nan(nullptr, n) == 0);
    // a pointer into a library tensor's mirror, at an offset, as the reference's Python passes it
    NeuralTensor *t = upload({n}, 12);
    float *m = static_cast<float *>(neural_tensor_data(t));
    CHECK(m != nullptr);
    if (m) {
        m[7] = INFINITY;
        CHECK(neural_tensor_has_inf(m + 5, n - 5) == 1);
        CHECK(neural_tensor_has_inf(m + 8, n - 8) == 0);
        CHECK(neural_tensor_grad_l2_norm(m + 8, 1000) > 0.0f);
        std::vector<int8_t> q(n - 8);
        QuantParams p;
        CHECK(calibrate_minmax_f32(m + 8, int64_t(n - 8), 1, &p) == 0);
        CHECK(quantize_tensor_f32(m + 8, q.data(), int64_t(n - 8), &p) == 0);
        CHECK(dequantize_tensor_f32(q.data(), m + 8, int64_t(n - 8), &p) == 0);  // output through the mirror
        CHECK(std::isfinite(m[9]));
    }
    neural_tensor_free(t);
    // the double API on host arrays
    std::vector<double> d(n);
    fill_host(d.data(), n, 13);
    QuantParams pa, pb;
    CHECK(calibrate_minmax(d.data(), int64_t(n), 0, &pa) == 0);
    CHECK(calibrate_percentile(d.data(), int64_t(n), 0.01, 1, &pb) == 0);
    std::vector<int8_t> q(n);
    std::vector<double> dq(n);
    CHECK(quantize_tensor(d.data(), q.data(), int64_t(n), &pa) == 0);
    CHECK(dequantize_tensor(q.data(), dq.data(), int64_t(n), &pa) == 0);
    CHECK(std::isfinite(quantization_error(d.data(), int64_t(n), &pa)));
    CHECK(std::isfinite(quantization_snr(d.data(), int64_t(n), &pa)));
    CHECK(std::isfinite(quantization_error_f32(g.data(), int64_t(n), &pa)));
    CHECK(calibrate_minmax(nullptr, int64_t(n), 0, &pa) == -1);
    CHECK(calibrate_minmax(d.data(), 0, 0, &pa) == -1);
    CHECK(quantize_tensor(d.data(), q.data(), -5, &pa) == -1);
    // int8 product, host arrays, odd shapes
    const int64_t M = 37, K = 70, N = 29;
    std::vector<int8_t> A(M * K), B(K * N);
    for (size_t i = 0; i < A.size(); i++) A[i] = int8_t(int(i * 7) % 255 - 127);
    for (size_t i = 0; i < B.size(); i++) B[i] = int8_t(int(i * 13) % 255 - 127);
    std::vector<double> C(M * N);
    CHECK(quantized_matmul(A.data(), B.data(), C.data(), M, K, N, &pa, &pb) == 0);
    CHECK(quantized_matmul(A.data(), B.data(), C.data(), 0, K, N, &pa, &pb) == -1);
    // the device-resident pipeline and the allocation-free calibration
    float *dx = nullptr;
    int8_t *dq8 = nullptr;
    QuantParams *dp = nullptr;
    CHECK(hipMalloc(&dx, n * 4) == hipSuccess && hipMalloc(&dq8, n) == hipSuccess &&
          hipMalloc(&dp, sizeof(QuantParams)) == hipSuccess);
    CHECK(hipMemcpy(dx, g.data(), n * 4, hipMemcpyHostToDevice) == hipSuccess);
    CHECK(calibrate_minmax_f32_dev(dx, int64_t(n), 0, dp) == 0);
    CHECK(calibrate_minmax_f32_dev_noalloc(dx, int64_t(n), 1, dp) == 0);
    CHECK(calibrate_minmax_f32_dev_noalloc(g.data(), int64_t(n), 1, dp) != 0);  // host pointers refused
    CHECK(quantize_tensor_f32_dev(dx, dq8, int64_t(n), dp) == 0);
    CHECK(dequantize_tensor_f32_dev(dq8, dx, int64_t(n), dp) == 0);
    CHECK(neural_hip_synchronize() == 0);
    CHECK(hipFree(dx) == hipSuccess && hipFree(dq8) == hipSuccess && hipFree(dp) == hipSuccess);
    // counts past the raw-pointer limit are refused before any staging
    CHECK(neural_tensor_has_nan(g.data(), uint64_t(1) << 62) != 1);
    CHECK(neural_get_last_error() == NEURAL_ERR_TENSOR_TOO_LARGE);
}

void check_host_modules()
{
    section("tensor_ops, transforms, losses");
    std::vector<double> a(6 * 4), b(6 * 5), out(6 * 9), oa(6 * 4), ob(6 * 5);
    fill_host(a.data(), a.size(), 14);
    fill_host(b.data(), b.size(), 15);
    int64_t r = 0, c = 0, r2 = 0, c2 = 0;
    CHECK(tensor_concat_2d(a.data(), b.data(), 6, 4, 6, 5, 1, out.data(), &r, &c) == 0 && r == 6 && c == 9);
    CHECK(tensor_concat_2d(a.data(), b.data(), 6, 4, 6, 5, 0, out.data(), &r, &c) == -1);
    CHECK(tensor_split_2d(out.data(), 6, 9, 1, 4, oa.data(), ob.data(), &r, &c, &r2, &c2) == 0);
    CHECK(oa == a && ob == b);
    std::vector<double> padded(9 * 7);
    CHECK(tensor_pad_2d(a.data(), 6, 4, 1, 2, 2, 1, -3.0, padded.data(), &r, &c) == 0 && r == 9 && c == 7);
    CHECK(padded[0] == -3.0 && padded[1 * 7 + 2] == a[0]);
    std::vector<double> tr(4 * 6);
    CHECK(tensor_transpose2d_array(a.data(), 6, 4, tr.data()) == 0 && tr[1] == a[4]);
    CHECK(tensor_transpose2d_array(a.data(), -1, 4, tr.data()) == -1);
    // per-feature transforms on a ragged [1000, 13]
    const int64_t B = 1000, F = 13;
    std::vector<double> x(B * F), y(B * F), mean(F), sd(F), mn(F), mx(F);
    fill_host(x.data(), x.size(), 16);
    CHECK(transform_compute_stats(x.data(), B, F, mean.data(), sd.data(), mn.data(), mx.data()) == 0);
    CHECK(transform_compute_stats(x.data(), B, F, mean.data(), nullptr, nullptr, nullptr) == 0);
    CHECK(transform_normalize(x.data(), y.data(), B, F, mean.data(), sd.data(), 1e-8) == 0);
    CHECK(transform_unnormalize(y.data(), y.data(), B, F, mean.data(), sd.data(), 1e-8) == 0);
    CHECK(transform_minmax(x.data(), y.data(), B, F, mn.data(), mx.data(), 1e-8) == 0);
    CHECK(transform_compute_stats(x.data(), 0, F, mean.data(), sd.data(), mn.data(), mx.data()) == -1);
    // label-smoothed CE on host arrays, both widths, and the tensor CE loss
    const int64_t rows = 300, k = 37;
    std::vector<double> lg(rows * k), gr(rows * k);
    std::vector<float> lg32(rows * k), gr32(rows * k);
    std::vector<int64_t> tg(rows);
    fill_host(lg.data(), lg.size(), 17);
    fill_host(lg32.data(), lg32.size(), 17);
    for (int64_t i = 0; i < rows; i++) tg[i] = (i * 5) % k;
    double loss = 0;
    CHECK(label_smoothing_ce_forward(lg.data(), tg.data(), rows, k, 0.1, &loss) == 0 && loss > 0);
    CHECK(label_smoothing_ce_backward(lg.data(), tg.data(), rows, k, 0.1, gr.data()) == 0);
    CHECK(label_smoothing_ce_fused(lg.data(), tg.data(), rows, k, 0.1, &loss, gr.data()) == 0);
    CHECK(label_smoothing_ce_fused_f32(lg32.data(), tg.data(), rows, k, 0.1, &loss, gr32.data()) == 0);
    tg[3] = k;  // out of range
    CHECK(label_smoothing_ce_forward(lg.data(), tg.data(), rows, k, 0.1, &loss) == -1);
    NeuralTensor *pred = upload({uint64_t(rows), uint64_t(k)}, 18), *tgt = make({uint64_t(rows)});
    CHECK(pred && tgt);
    CHECK(neural_tensor_fill(tgt, 2.0) == 0);
    CHECK(neural_cross_entropy_loss(pred, tgt, &loss) == 0 && loss > 0);
    neural_tensor_free(pred);
    neural_tensor_free(tgt);
}

void check_dropout()
{
    section("dropout");
    CHECK(neural_dropout_seed(42) == 0);
    for (uint64_t n : {uint64_t(1), uint64_t(371), uint64_t(372), uint64_t(100001)}) {
        std::vector<float> x(n), y(n), gx(n);
        std::vector<uint8_t> mask(n);
        fill_host(x.data(), n, 19);
        for (int rep = 0; rep < 3; rep++)  // repeated (n, p): the made-ahead path
            CHECK(neural_dropout_forward(x.data(), y.data(), mask.data(), n, 0.3f) == 0);
        CHECK(neural_dropout_backward(x.data(), gx.data(), mask.data(), n, 0.3f) == 0);
        // unaligned host buffers take the element-wise kernels
        if (n > 4) CHECK(neural_dropout_forward(x.data() + 1, y.data() + 1, mask.data() + 1, n - 1, 0.5f) == 0);
    }
    CHECK(neural_dropout_draws() > 0);
    CHECK(neural_dropout_forward(nullptr, nullptr, nullptr, 4, 0.5f) != 0);
}

void check_optimizers()
{
    section("optimizers, state blobs, clipping");
    std::vector<NeuralTensor *> ps, gs;
    for (uint64_t n : {uint64_t(5), uint64_t(1000), uint64_t(33)}) {
        ps.push_back(upload({n}, uint32_t(20 + n)));
        gs.push_back(upload({n}, uint32_t(30 + n)));
    }
    void *opts[3] = {opt_sgd_create(0.1, 0.9), opt_adam_create(1e-3, 0.9, 0.999, 1e-8),
                     opt_adamw_create(1e-3, 0.9, 0.999, 1e-8, 0.01)};
    for (void *o : opts) {
        CHECK(o != nullptr);
        if (!o) continue;
        void **P = reinterpret_cast<void **>(ps.data()), **G = reinterpret_cast<void **>(gs.data());
        for (int s = 0; s < 3; s++) CHECK(opt_step(o, P, G, 3) == 0);
        CHECK(opt_step(o, P, G, 2) != 0);  // another parameter count
        CHECK(neural_clip_grad_norm(o, 0.5) == 0);
        CHECK(neural_clip_grad_value(o, -0.1, 0.1) == 0);
        const int64_t bytes = opt_state_bytes(o);
        CHECK(bytes > 0);
        std::vector<unsigned char> blob(size_t(bytes > 0 ? bytes : 0));
        CHECK(opt_state_export(o, blob.data(), bytes) == 0);
        CHECK(opt_state_export(o, blob.data(), bytes - 1) != 0);
        CHECK(opt_state_import(o, blob.data(), bytes) == 0);
        CHECK(opt_step(o, P, G, 3) == 0);
        // corrupt blobs: truncated, bad magic, a huge parameter count
        CHECK(opt_state_import(o, blob.data(), bytes / 2) != 0);
        std::vector<unsigned char> bad = blob;
        bad[0] ^= 0xff;
        CHECK(opt_state_import(o, bad.data(), bytes) != 0);
        for (size_t off = 8; off + 8 <= 80 && off + 8 <= bad.size(); off += 8) {
            bad = blob;
            const uint64_t big = uint64_t(1) << 61;
            std::memcpy(bad.data() + off, &big, 8);
            (void)opt_state_import(o, bad.data(), bytes);  // any code; the sanitizer watches the reads
        }
        CHECK(opt_state_import(o, blob.data(), bytes) == 0);
        CHECK(opt_step(o, P, G, 3) == 0);
        opt_set_lr(o, 0.05);
        CHECK(opt_get_lr(o) == 0.05);
        opt_free(o);
    }
    // gradient lists: inline table, uploaded table (more than 32), NULL entries
    double norm = 0;
    CHECK(neural_clip_grad_norm_list(gs.data(), 3, 1.0, &norm) == 0 && norm > 0);
    CHECK(neural_clip_grad_value_list(gs.data(), 3, -0.5, 0.5) == 0);
    std::vector<NeuralTensor *> many;
    for (int i = 0; i < 70; i++) many.push_back(i % 9 == 4 ? nullptr : upload({uint64_t(17 + i * 31)}, uint32_t(40 + i)));
    CHECK(neural_clip_grad_norm_list(many.data(), int64_t(many.size()), 2.0, &norm) == 0 && norm > 0);
    CHECK(neural_clip_grad_value_list(many.data(), int64_t(many.size()), -1.0, 1.0) == 0);
    CHECK(neural_clip_grad_norm_list(nullptr, 3, 1.0, &norm) != 0);
    for (NeuralTensor *t : many) neural_tensor_free(t);
    for (NeuralTensor *t : ps) neural_tensor_free(t);
    for (NeuralTensor *t : gs) neural_tensor_free(t);
}

void check_hooks()
{
    section("streams and measurement hooks");
    hipStream_t s = nullptr;
    CHECK(hipStreamCreate(&s) == hipSuccess);
    CHECK(neural_hip_set_stream(s) == 0);
    CHECK(neural_hip_get_stream() == static_cast<void *>(s));
    NeuralTensor *x = upload({1 << 20}, 50), *one = make({1});
    hipEvent_t e0 = nullptr, e1 = nullptr;
    CHECK(hipEventCreate(&e0) == hipSuccess && hipEventCreate(&e1) == hipSuccess);
    const unsigned long long c0 = neural_hip_launch_count();
    CHECK(neural_hip_time_launches(e0, e1, 0, 2) == 0);
    double v = 0;
    CHECK(neural_sum(x, &v) == 0);
    CHECK(neural_hip_launch_count() > c0);
    CHECK(neural_hip_synchronize() == 0);
    float ms = 0;
    CHECK(hipEventElapsedTime(&ms, e0, e1) == hipSuccess && ms > 0);
    CHECK(neural_hip_time_next_launch(e0, e1, 0) == 0);
    CHECK(neural_hip_time_cancel() == 0);
    CHECK(neural_hip_time_launches(nullptr, e1, 0, 1) != 0);
    unsigned long long da = 0, hm = 0;
    CHECK(neural_hip_alloc_stats(&da, &hm) == 0 && da >= hm);
    float *d0 = nullptr, *d1 = nullptr;
    CHECK(hipMalloc(&d0, 1 << 20) == hipSuccess && hipMalloc(&d1, 1 << 20) == hipSuccess);
    CHECK(neural_hip_stream_copy(d1, d0, 1 << 20) == 0);
    CHECK(neural_hip_stream_copy(d1, d0, 12) != 0);
    CHECK(neural_reduce_sum(x, -1, one) == 0);
    CHECK(neural_hip_reset_stream() == 0);
    CHECK(neural_hip_synchronize() == 0);
    CHECK(hipFree(d0) == hipSuccess && hipFree(d1) == hipSuccess);
    CHECK(hipEventDestroy(e0) == hipSuccess && hipEventDestroy(e1) == hipSuccess);
    CHECK(hipStreamDestroy(s) == hipSuccess);
    int ord = -1, cus = 0;
    char name[64];
    CHECK(neural_hip_device_info(&ord, &cus, name, int(sizeof(name))) == 0 && cus > 0);
    neural_tensor_free(x);
    neural_tensor_free(one);
    CHECK(neural_hip_empty_cache() == 0);
    // entry points outside the path answer NOT_IMPLEMENTED
    CHECK(neural_linear_create(4, 4, 1) == nullptr);
    CHECK(neural_get_last_error() == NEURAL_ERR_NOT_IMPLEMENTED);
}

// Strided device views, device-side index outputs, and the edge sizes of
// the quantization and transform entry points.
void check_views_and_edges()
{
    section("views, device outputs, edge sizes");
    // a [6, 8] f32 device buffer viewed as its transpose [8, 6] (byte strides)
    float *d = nullptr;
    CHECK(hipMalloc(&d, 48 * 4) == hipSuccess);
    std::vector<float> h(48);
    fill_host(h.data(), 48, 60);
    CHECK(hipMemcpy(d, h.data(), 48 * 4, hipMemcpyHostToDevice) == hipSuccess);
    const uint64_t s86[2] = {8, 6}, s68[2] = {6, 8};
    const int64_t tstr[2] = {4, 32};
    NeuralTensor *tv = neural_tensor_from_buffer(d, s86, 2, NEURAL_DTYPE_FLOAT32, tstr);
    NeuralTensor *dv = neural_tensor_from_buffer(d, s68, 2, NEURAL_DTYPE_FLOAT32, nullptr);
    NeuralTensor *o = make({8, 6}), *row = make({6});
    CHECK(tv && dv && o && row);
    CHECK(neural_tensor_is_contiguous(tv) == 0);
    CHECK(neural_add(o, tv, tv) == 0);  // strided inputs through the N-D kernel
    std::vector<float> back(48);
    CHECK(neural_tensor_download(o, back.data(), 48 * 4) == 0);
    CHECK(back[1] == 2.0f * h[8] && back[6] == 2.0f * h[1]);
    NeuralTensor *c = neural_tensor_make_contiguous(tv);
    CHECK(c != nullptr && c != tv);
    if (c != tv) neural_tensor_free(c);
    CHECK(neural_softmax(o, tv) != 0);         // rows must be contiguous
    CHECK(neural_reduce_sum(tv, 0, row) == 0);  // a strided view is read through a contiguous copy
    int64_t *didx = nullptr;
    CHECK(hipMalloc(&didx, 6 * 8) == hipSuccess);
    CHECK(neural_reduce_argmax(dv, 1, didx) == 0);
    CHECK(neural_row_stats(dv, nullptr, nullptr, nullptr, didx) == 0);
    int64_t hidx[6];
    CHECK(neural_hip_synchronize() == 0 && hipMemcpy(hidx, didx, 48, hipMemcpyDeviceToHost) == hipSuccess);
    CHECK(hidx[0] >= 0 && hidx[0] < 8 && hidx[5] >= 0 && hidx[5] < 8);
    int hn = -1, hi = -1;
    double ss = 0;
    CHECK(neural_scan_nan_inf_l2(d, 48, &hn, &hi, &ss) == 0 && hn == 0 && hi == 0 && ss > 0);
    CHECK(neural_tensor_grad_l2_norm(d + 3, 45) > 0.0f);  // a device pointer at an offset
    neural_tensor_free(tv);
    neural_tensor_free(dv);
    neural_tensor_free(o);
    neural_tensor_free(row);
    CHECK(hipFree(didx) == hipSuccess && hipFree(d) == hipSuccess);
    // percentile: n = 1 and 2, ties, zeros of both signs at the selected ranks
    QuantParams p;
    const double one[1] = {3.0}, two[2] = {-1.0, 1.0};
    CHECK(calibrate_percentile(one, 1, 0.01, 0, &p) == 0);
    CHECK(calibrate_percentile(two, 2, 0.25, 1, &p) == 0);
    std::vector<double> z(1001, 0.0);
    for (size_t i = 0; i < z.size(); i += 3) z[i] = -0.0;
    z[500] = 7.0;
    CHECK(calibrate_percentile(z.data(), int64_t(z.size()), 0.1, 0, &p) == 0);
    CHECK(calibrate_percentile(z.data(), int64_t(z.size()), NAN, 0, &p) == -1);
    // the int8 product at 1 x 1 x 1 and with a long K
    QuantParams qa{0.5, 3, -1.0, 1.0, 0}, qb{0.25, -2, -1.0, 1.0, 0};
    const int8_t a1 = 5, b1 = -7;
    double c1 = 0;
    CHECK(quantized_matmul(&a1, &b1, &c1, 1, 1, 1, &qa, &qb) == 0 && c1 == double((5 - 3) * (-7 + 2)) * 0.125);
    std::vector<int8_t> A(3 * 40000, 1), B(40000 * 2, -1);
    std::vector<double> C(6);
    CHECK(quantized_matmul(A.data(), B.data(), C.data(), 3, 40000, 2, &qa, &qb) == 0);
    // transforms on device pointers, one feature and one row
    double *dx = nullptr, *dy = nullptr, *dm = nullptr, *ds = nullptr;
    CHECK(hipMalloc(&dx, 64 * 8) == hipSuccess && hipMalloc(&dy, 64 * 8) == hipSuccess &&
          hipMalloc(&dm, 64 * 8) == hipSuccess && hipMalloc(&ds, 64 * 8) == hipSuccess);
    std::vector<double> hx(64);
    fill_host(hx.data(), 64, 61);
    CHECK(hipMemcpy(dx, hx.data(), 64 * 8, hipMemcpyHostToDevice) == hipSuccess);
    CHECK(transform_compute_stats(dx, 64, 1, dm, ds, nullptr, nullptr) == 0);
    CHECK(transform_compute_stats(dx, 1, 64, dm, ds, nullptr, nullptr) == 0);
    CHECK(transform_normalize(dx, dy, 1, 64, dm, ds, 1e-8) == 0);
    CHECK(neural_hip_synchronize() == 0);
    CHECK(hipFree(dx) == hipSuccess && hipFree(dy) == hipSuccess && hipFree(dm) == hipSuccess &&
          hipFree(ds) == hipSuccess);
}

// One of several host threads on the library's one stream: it creates, uses
// and frees its own tensors, buffers and optimizer, and checks results it can
// predict exactly, so a mix-up between threads (a shared workspace, the
// allocator's cache, the mirror registry, the dropout stream) would show.
void thread_body(int tid, int iters)
{
    const float v = float(tid) + 1.5f;
    for (int it = 0; it < iters; it++) {
        const uint64_t n = 1000 + uint64_t(tid) * 4099 + uint64_t(it) * 37;
        NeuralTensor *a = make({n}), *b = make({n}), *o = make({n});
        CHECK(a && b && o);
        if (!a || !b || !o) continue;
        CHECK(neural_tensor_fill(a, double(v) - 0.5) == 0);
        CHECK(neural_tensor_fill(b, 0.5) == 0);
        CHECK(neural_add(o, a, b) == 0);
        double s = 0;
        CHECK(neural_sum(o, &s) == 0 && s == double(n) * double(v));
        float *m = static_cast<float *>(neural_tensor_data(o));
        CHECK(m != nullptr);
        if (m) {
            m[n / 2] = 100.0f;
            int64_t idx = -1;
            CHECK(neural_argmax(o, &idx) == 0 && idx == int64_t(n / 2));
            CHECK(neural_tensor_has_inf(m, n) == 0);  // a pointer into the mirror
        }
        std::vector<float> h(n);
        CHECK(neural_tensor_download(o, h.data(), n * 4) == 0);
        CHECK(h[0] == v && h[n / 2] == 100.0f && h[n - 1] == v);
        QuantParams qp;
        CHECK(calibrate_minmax_f32(h.data(), int64_t(n), 0, &qp) == 0 && qp.max_val == 100.0 && qp.min_val == double(v));
        std::vector<int8_t> q(n);
        CHECK(quantize_tensor_f32(h.data(), q.data(), int64_t(n), &qp) == 0 && q[n / 2] == 127);
        // row sums of a [rows, 64] tensor of one value
        const uint64_t rows = n / 64;
        NeuralTensor *x = make({rows, 64}), *rs = make({rows});
        CHECK(x && rs);
        if (x && rs) {
            CHECK(neural_tensor_fill(x, double(v)) == 0);
            CHECK(neural_reduce_sum(x, 1, rs) == 0);
            std::vector<float> r(rows);
            CHECK(neural_tensor_download(rs, r.data(), rows * 4) == 0);
            bool ok = true;
            for (float e : r) ok = ok && e == 64.0f * v;
            CHECK(ok);
        }
        neural_tensor_free(x);
        neural_tensor_free(rs);
        // the global norm of (a, b), then an optimizer of its own
        NeuralTensor *L[2] = {a, b};
        double norm = 0;
        CHECK(neural_clip_grad_norm_list(L, 2, 1e30, &norm) == 0);
        const double want = std::sqrt(double(n) * (double(v - 0.5f) * double(v - 0.5f) + 0.25));
        CHECK(std::fabs(norm - want) <= 1e-12 * want);
        void *opt = opt_adamw_create(1e-3, 0.9, 0.999, 1e-8, 0.01);
        void *P[1] = {a}, *G[1] = {b};
        CHECK(opt != nullptr && opt_step(opt, P, G, 1) == 0 && opt_step(opt, P, G, 1) == 0);
        opt_free(opt);
        // dropout draws from the one shared stream, under its lock
        std::vector<float> y(n);
        std::vector<uint8_t> mask(n);
        CHECK(neural_dropout_forward(h.data(), y.data(), mask.data(), n, 0.25f) == 0);
        bool ok = true;
        for (uint64_t i = 0; i < n; i++) ok = ok && (mask[i] ? y[i] == h[i] * (1.0f / 0.75f) : y[i] == 0.0f);
        CHECK(ok);
        neural_tensor_free(a);
        neural_tensor_free(b);
        neural_tensor_free(o);
    }
}

void check_threads()
{
    section("threads");
    std::vector<std::thread> ts;
    for (int t = 0; t < 4; t++) ts.emplace_back(thread_body, t, 25);
    for (auto &t : ts) t.join();
}

}  // namespace

int main()
{
    if (neural_init() != 0) {
        std::printf("neural_init failed: %d\n", neural_get_last_error());
        return 2;
    }
    check_tensors();
    check_math();
    check_reductions();
    check_raw_pointers();
    check_host_modules();
    check_dropout();
    check_optimizers();
    check_hooks();
    check_views_and_edges();
    check_threads();
    neural_shutdown();
    std::printf("host checks: %d passed, %d failed\n", g_checks - g_fail, g_fail.load());
    return g_fail ? 1 : 0;
}
