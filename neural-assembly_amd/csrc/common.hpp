// common.hpp -- shared runtime types and device helpers for libneural_hip.so.
//
// One process-wide runtime (device, stream, caching allocator, reduction
// workspace) plus the 64-byte NeuralTensor descriptor whose first 40 bytes keep
// the reference layout (tensor.asm:7-24).
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <cstring>
#include <mutex>

#include "../../include/neural_api.h"

// ---------------------------------------------------------------------------
// Tensor descriptor
// ---------------------------------------------------------------------------

// flags@36 keep the reference bits (tensor.asm:29-31).
enum : int32_t { NT_OWN_DATA = 1, NT_OWN_META = 2 };

// Where the authoritative bytes live.
enum : int32_t { ST_DEVICE = 0, ST_HOST = 1, ST_SYNCED = 2 };

// What the data pointer at offset 0 is.
//   KIND_OWNED     library allocation: device buffer + lazily synced host mirror
//   KIND_EXT_HOST  caller's host buffer (from_buffer): host is authoritative,
//                  a device shadow is refreshed before and written back after use
//   KIND_EXT_DEV   caller's device buffer (from_buffer): used in place
//   KIND_VIEW      reshape view of another tensor (shares its storage)
enum : int32_t { KIND_OWNED = 0, KIND_EXT_HOST = 1, KIND_EXT_DEV = 2, KIND_VIEW = 3 };

struct Storage;

struct NeuralTensor {
    void     *data;    // 0   host-visible pointer to element 0 (device address for KIND_EXT_DEV)
    int64_t   ndim;    // 8
    int64_t  *shape;   // 16
    int64_t  *stride;  // 24  byte strides
    int32_t   dtype;   // 32  0 f32, 1 f64
    int32_t   flags;   // 36
    void     *dev;     // 40  device address of element 0
    int32_t   kind;    // 48
    int32_t   rsv;     // 52
    Storage  *st;      // 56  shared storage record
};
static_assert(sizeof(NeuralTensor) == 64, "NeuralTensor must stay 64 bytes");
static_assert(offsetof(NeuralTensor, dtype) == 32, "dtype offset");
static_assert(offsetof(NeuralTensor, flags) == 36, "flags offset");

// Storage shared between a tensor and its reshape views.  Byte span [lo, hi)
// relative to element 0 covers every element the strides can reach.
struct Storage {
    int      refs;
    int32_t  state;      // ST_*
    int32_t  kind;       // KIND_OWNED / KIND_EXT_HOST / KIND_EXT_DEV
    void    *host;       // mirror (owned) or caller buffer at element 0
    void    *dev_block;  // device allocation (owned or shadow); null for EXT_DEV
    size_t   dev_bytes;
    int64_t  lo, hi;     // byte span relative to element 0
    bool     host_owned; // host mirror allocated by us
};

namespace nh {

// ---------------------------------------------------------------------------
// Runtime
// ---------------------------------------------------------------------------
int          ensure_init();              // NEURAL_OK or error code (lazy init)
// NEURAL_OK when the runtime was initialised earlier (makes its device
// current on this thread); NEURAL_ERR_INVALID_CONFIG otherwise.  Never
// initialises, so it allocates nothing.
int          ensure_ready();
// Per-device set-up of static device buffers, run by ensure_init with the
// device current (defined beside the buffer it resolves).
int          setup_static_scratch(int device);
hipStream_t  stream();                   // active stream
// A pair of events armed by neural_hip_time_launches on the calling thread:
// after `skip` launches, the next launch carries `start` and the launch
// `count` - 1 later carries `stop` (the same launch both when count is 1), so
// the pair spans those launches and the gaps between them (see NH_LAUNCH).
struct LaunchTimer {
    hipEvent_t start = nullptr, stop = nullptr;
    int skip = 0;
    int count = 1;
};
// Called once per launch: counts this thread's launches (launch_count) and
// the armed span down, and returns the events this launch records (either or
// both may be null).
LaunchTimer  take_launch_timer();
int          num_cus();
int          set_error(int code);        // stores thread-local last error, returns code
int          hip_fail(hipError_t e);     // maps a HIP error to NEURAL_ERR_* and records it

void        *dev_alloc(size_t bytes);    // caching allocator (stream-ordered reuse)
void         dev_free(void *p);

// Per-runtime device workspace for multi-block reductions: partial results
// plus a self-resetting completion counter (the last block sets it back to 0).
struct Workspace {
    void         *partials;    // kMaxPartials * 64 bytes
    unsigned int *counter;     // kCounters counters, all zero between calls
    void         *result;      // 256 bytes of small results
    void         *host_result; // 256 bytes of coherent pinned host memory (host address)
    void         *host_result_dev; // the same bytes as kernels address them
};
constexpr int kMaxPartials = 16384;
constexpr int kCounters = 1024;
Workspace   &workspace();

// The workspace is shared by every thread of the process.  An entry point
// that uses it holds WsGuard from its first launch that writes it until the
// last read of it: until the host has copied a host-returned result out of
// host_result, or, for results left in device memory, until the last kernel
// that reads the summaries has been enqueued (later users enqueue behind it
// on the same stream).  Recursive, so helpers may take it again.
std::recursive_mutex &workspace_mutex();
struct WsGuard {
    std::lock_guard<std::recursive_mutex> g{workspace_mutex()};
};

// Raw pointer classification for the pointer-taking entry points.
bool         is_device_ptr(const void *p);

// Stage a caller pointer into device memory.  For device pointers the
// pointer itself is used.  A host pointer into the host mirror of a live
// library tensor (what neural_tensor_data() returns) resolves to that
// tensor's device copy: made current first if the host copy is
// authoritative, so no temporary buffer and no second upload by the tensor's
// next kernel.  Other host pointers get a device block, filled when upload.
// finish() copies back to the host pointer (when download) and frees.
struct Staged {
    void    *dev = nullptr;
    void    *host = nullptr;
    size_t   bytes = 0;
    bool     owned = false;
    Storage *mirror = nullptr;  // the tensor storage whose mirror `host` lies in
    int    open(const void *p, size_t nbytes, bool upload);
    // count elements of es bytes; a count beyond kMaxRawCount (whose bytes
    // could wrap size_t) is NEURAL_ERR_TENSOR_TOO_LARGE
    int    open_n(const void *p, uint64_t count, size_t es, bool upload);
    int    finish(bool download);
    ~Staged();
};

// Largest element count a raw-pointer entry point accepts: 2^56 elements of
// up to 8 bytes stay far inside size_t.
constexpr uint64_t kMaxRawCount = uint64_t(1) << 56;

// Owned tensors' host mirrors, for Staged::open (registered at creation,
// removed when the storage is released).
void         mirror_register(Storage *s);
void         mirror_unregister(Storage *s);

// Tensor coherence
int64_t      numel(const NeuralTensor *t);
size_t       elem_size(int dtype);
bool         is_contiguous(const NeuralTensor *t);
// True when a and b may address the same bytes: one shared storage, or
// element spans (through the strides) whose addresses intersect.
bool         tensors_may_overlap(const NeuralTensor *a, const NeuralTensor *b);
int          check_tensor(const NeuralTensor *t);   // null / dtype validation
// Make the device copy current and return its element-0 address.
int          dev_read(const NeuralTensor *t, const void **p);
// Prepare for a write; `full` = every element will be overwritten.
int          dev_write(NeuralTensor *t, void **p, bool full);
// After kernels that wrote `t` were enqueued: mark/propagate.
int          dev_written(NeuralTensor *t);

// Launch helpers
inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
// Streaming kernels launch one block per tile of work up to this many blocks
// (blocks x 256 lanes stay below 2^32 work-items) and stride beyond it.
// Measured: a grid covering the data beats 16-32 blocks per CU striding over
// it (AdamW 825 -> 698 us, quantize 71 -> 78 % of HBM, dequantize 70 -> 74 %,
// f32 activations +2-6 %).
constexpr int64_t kMaxGridBlocks = (int64_t(1) << 24) - 1;
// Kernels that give each block (or wave) its own rows take `rows` in launches
// of at most kMaxGridBlocks blocks of `rpb` rows each: launch(blocks, first
// row) once per such range.  (A row loop inside those kernels raised their
// register counts, e.g. 62 -> 96 VGPRs for the f32 log-softmax over rows of
// 1024, so the loop is on the host.)
template <typename L>
void for_row_launches(int64_t rows, int64_t rpb, L launch)
{
    const int64_t per = kMaxGridBlocks * rpb;
    for (int64_t base = 0; base < rows; base += per) {
        const int64_t n = rows - base < per ? rows - base : per;
        launch(unsigned(ceil_div(n, rpb)), base);
    }
}
int          check_launch();                         // hipGetLastError -> error code
int          sync();                                 // synchronise the active stream
// Copy `bytes` (<= 256) of a device result to `dst` (host): one D2H copy into
// the pinned landing area, a stream sync, then a host memcpy.
int          result_to_host(void *dst, const void *dev_src, size_t bytes);
// Results that only the host reads are stored by the last kernel straight
// into workspace().host_result_dev (coherent pinned memory): a stream sync
// and a host memcpy, no copy command (measured: 14.9 -> 11.3 us for a
// launch-and-return round trip).
int          host_result_fetch(void *dst, size_t bytes);
// Ticketed variant: the storing kernel also writes a 64-bit ticket into the
// last 8 bytes of the host area (after a system-scope fence), and the host
// spins on it instead of synchronising the stream, then copies `bytes` (<=
// 248) of the result.  A ticket that has not shown after ~2 s falls back to a
// stream synchronisation (which reports any fault).  next_ticket() gives the
// slot and a fresh value; callers hold WsGuard.
struct Ticket {
    unsigned long long *slot = nullptr;  // device address of the host word; null: no ticket
    unsigned long long value = 0;
};
Ticket       next_ticket();
int          host_result_wait(unsigned long long ticket, void *dst, size_t bytes);

}  // namespace nh

// ---------------------------------------------------------------------------
// Device helpers
// ---------------------------------------------------------------------------

#define NH_DEV __device__ __forceinline__

// Wave64 butterfly reductions; fixed pairing, so results are deterministic.
template <typename T>
NH_DEV T wave_sum(T v)
{
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

template <typename T>
NH_DEV T wave_max_ignore_nan(T v)
{
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        T o = __shfl_xor(v, off, 64);
        v = (v != v) ? o : ((o != o) ? v : (o > v ? o : v));
    }
    return v;
}

// DPP-based wave64 all-reductions: quad xor-1 / xor-2 swaps, half-row and row
// mirrors make every 16-lane row uniform in four VALU steps, then two lane
// swizzles across rows (xor 16, xor 32).  Fixed pairing: deterministic, and
// every lane ends with the same value.
template <int CTRL>
NH_DEV int dpp_i(int v) { return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, true); }
template <int CTRL>
NH_DEV float dpp_f(float v) { return __int_as_float(dpp_i<CTRL>(__float_as_int(v))); }
template <int CTRL>
NH_DEV double dpp_d(double v)
{
    const long long b = __double_as_longlong(v);
    const int lo = dpp_i<CTRL>(int(b)), hi = dpp_i<CTRL>(int(b >> 32));
    return __longlong_as_double((static_cast<long long>(hi) << 32) | static_cast<unsigned int>(lo));
}
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140;

NH_DEV float wave_fmax(float v)  // NaN-ignoring max over the wave
{
    v = __builtin_fmaxf(v, dpp_f<kDppXor1>(v));
    v = __builtin_fmaxf(v, dpp_f<kDppXor2>(v));
    v = __builtin_fmaxf(v, dpp_f<kDppHalfMirror>(v));
    v = __builtin_fmaxf(v, dpp_f<kDppMirror>(v));
    v = __builtin_fmaxf(v, __shfl_xor(v, 16, 64));
    return __builtin_fmaxf(v, __shfl_xor(v, 32, 64));
}

NH_DEV double wave_dsum(double v)
{
    v += dpp_d<kDppXor1>(v);
    v += dpp_d<kDppXor2>(v);
    v += dpp_d<kDppHalfMirror>(v);
    v += dpp_d<kDppMirror>(v);
    v += __shfl_xor(v, 16, 64);
    return v + __shfl_xor(v, 32, 64);
}

// e^y as a float for a double argument y <= ~88.7: t = y * log2(e) = n + f with
// n = rint(t) and |f| <= 1/2 exact, 2^f from the hardware exp2 of float(f)
// (about 1 ulp), scaled by 2^n with ldexp (exact, or correctly rounded into
// the denormal range).  About 1.5e-7 relative in ~7 instructions.  t is clamped
// at -300 so exp(-inf) = 0; a NaN passes through.
NH_DEV float exp_d2f(double y)
{
    double t = y * 1.4426950408889634;
    t = t < -300.0 ? -300.0 : t;
    const double n = __builtin_rint(t);
    return __builtin_ldexpf(__builtin_amdgcn_exp2f(float(t - n)), int(n));
}

// ln 2 split so that k * kLn2Hi is exact for |k| < 2^20 (32 significant bits).
constexpr double kLn2Hi = 0x1.62e42fee00000p-1;
constexpr double kLn2Lo = 0x1.a39ef35793c76p-33;
constexpr double kSqrtHalf = 0x1.6a09e667f3bcdp-1;

// Natural log of u >= 1 (also +inf and NaN, returned unchanged) to about
// 3 ulp: u = m * 2^k with m in [sqrt(1/2), sqrt(2)), log m = 2 atanh(s),
// s = (m - 1) / (m + 1), |s| <= 0.1716, atanh by its odd power series through
// s^19 (truncation below 2.4e-17 relative).
NH_DEV double log_ge1(double u)
{
    int k;
    double m = frexp(u, &k);
    if (m < kSqrtHalf) {
        m += m;
        k -= 1;
    }
    const double f = m - 1.0;  // exact (Sterbenz)
    const double s = f / (m + 1.0);
    const double s2 = s * s;
    double q = 1.0 / 19.0;
    q = __builtin_fma(q, s2, 1.0 / 17.0);
    q = __builtin_fma(q, s2, 1.0 / 15.0);
    q = __builtin_fma(q, s2, 1.0 / 13.0);
    q = __builtin_fma(q, s2, 1.0 / 11.0);
    q = __builtin_fma(q, s2, 1.0 / 9.0);
    q = __builtin_fma(q, s2, 1.0 / 7.0);
    q = __builtin_fma(q, s2, 1.0 / 5.0);
    q = __builtin_fma(q, s2, 1.0 / 3.0);
    const double s_2 = s + s;
    const double lm = __builtin_fma(s_2 * s2, q, s_2);  // 2s (1 + s^2/3 + s^4/5 + ...)
    const double dk = double(k);
    const double r = __builtin_fma(dk, kLn2Hi, __builtin_fma(dk, kLn2Lo, lm));
    return (u < __builtin_inf()) ? r : u;
}

// 128-bit vector types (clang ext vectors: element access by index, and
// accepted by the non-temporal load/store builtins).
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef double f64x2 __attribute__((ext_vector_type(2)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

template <typename T> struct Vec16;
template <> struct Vec16<float>  { using type = f32x4; static constexpr int n = 4; };
template <> struct Vec16<double> { using type = f64x2; static constexpr int n = 2; };

template <typename V> NH_DEV auto vget(const V &v, int i) { return v[i]; }
template <typename V, typename S> NH_DEV void vset(V &v, int i, S x) { v[i] = x; }

// Streaming (non-temporal) global accesses: data that is read or written
// once per kernel does not displace reusable lines in L2 / MALL.  Measured on
// MI355X: +10-15 % bandwidth for pure streams.
template <typename T> NH_DEV T ld_nt(const T *p) { return __builtin_nontemporal_load(p); }
template <typename T> NH_DEV void st_nt(T *p, T v) { __builtin_nontemporal_store(v, p); }

// Every kernel launch goes through NH_LAUNCH.  When the calling thread has
// armed an event pair (neural_hip_time_launches), the launches that carry its
// start and stop events are made with hipExtLaunchKernelGGL, which records
// them at the start and the end of that kernel's own execution on its stream;
// every other launch is plain.
#define NH_LAUNCH(kernel, grid, block, shmem, strm, ...)                                            \
    do {                                                                                            \
        const nh::LaunchTimer t__ = nh::take_launch_timer();                                        \
        if (t__.start || t__.stop)                                                                  \
            hipExtLaunchKernelGGL(kernel, grid, block, shmem, strm, t__.start, t__.stop, 0, __VA_ARGS__); \
        else                                                                                        \
            hipLaunchKernelGGL(kernel, grid, block, shmem, strm, __VA_ARGS__);                      \
    } while (0)

// Error-return helper for host code.
#define NH_TRY(expr)                          \
    do {                                      \
        int rc__ = (expr);                    \
        if (rc__ != NEURAL_OK) return rc__;   \
    } while (0)
#define NH_HIP(expr)                                   \
    do {                                               \
        hipError_t e__ = (expr);                       \
        if (e__ != hipSuccess) return nh::hip_fail(e__); \
    } while (0)
