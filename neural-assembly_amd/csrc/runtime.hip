// runtime.hip -- device/stream/allocator runtime and the tensor C ABI.
//
// Replaces the reference's host runtime for this path: tensor.asm (descriptor,
// create/free/fill/copy/reshape), mem.asm (allocation), error.asm (codes and
// messages) and the tensor exports of neural_api.asm:297-967,2293-2426.
// Tensor bytes live in HBM; the host copy is a mirror synchronised at
// neural_tensor_data() (see the memory-model note in include/neural_api.h).
#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <map>
#include <mutex>
#include <new>
#include <unordered_map>
#include <vector>

#include "common.hpp"
#include "kernels.hpp"

namespace nh {

namespace {

struct Runtime {
    std::mutex mu;
    bool inited = false;
    int init_rc = NEURAL_OK;
    int device = 0;
    int cus = 0;
    char name[256] = {0};
    hipStream_t own = nullptr;
    hipStream_t active = nullptr;
    std::unordered_map<size_t, std::vector<void *>> cache;  // size class -> free blocks
    std::unordered_map<void *, size_t> live;                // block -> size class
    Workspace ws{};
};

Runtime &R()
{
    static Runtime *r = new Runtime();  // never destroyed: kernels may outlive static dtors
    return *r;
}

thread_local int t_last_error = NEURAL_OK;
thread_local bool t_device_set = false;

size_t size_class(size_t b)
{
    if (b <= 512) return 512;
    if (b < (size_t(1) << 20)) return (b + 4095) & ~size_t(4095);
    const size_t g = size_t(2) << 20;
    return (b + g - 1) & ~(g - 1);
}

void release_cache_locked(Runtime &r)
{
    for (auto &kv : r.cache)
        for (void *p : kv.second) (void)hipFree(p);
    r.cache.clear();
}

}  // namespace

int set_error(int code)
{
    t_last_error = code;
    return code;
}

int hip_fail(hipError_t e)
{
    if (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation) return set_error(NEURAL_ERR_OUT_OF_MEMORY);
    if (std::getenv("NEURAL_HIP_VERBOSE"))
        std::fprintf(stderr, "libneural_hip: HIP error %d (%s)\n", int(e), hipGetErrorString(e));
    return set_error(NEURAL_ERR_INTERNAL);
}

int ensure_init()
{
    Runtime &r = R();
    if (!r.inited) {
        std::lock_guard<std::mutex> g(r.mu);
        if (!r.inited) {
            int count = 0;
            hipError_t e = hipGetDeviceCount(&count);
            if (e != hipSuccess || count <= 0) {
                (void)hipGetLastError();
                std::fprintf(stderr, "libneural_hip: no HIP device available (%s)\n",
                             e == hipSuccess ? "device count 0" : hipGetErrorString(e));
                r.init_rc = NEURAL_ERR_INTERNAL;
                return set_error(r.init_rc);
            }
            const char *dv = std::getenv("NEURAL_HIP_DEVICE");
            r.device = dv ? std::atoi(dv) : 0;
            if (r.device < 0 || r.device >= count) r.device = 0;
            hipDeviceProp_t prop;
            if (hipSetDevice(r.device) != hipSuccess || hipGetDeviceProperties(&prop, r.device) != hipSuccess) {
                r.init_rc = NEURAL_ERR_INTERNAL;
                return set_error(r.init_rc);
            }
            r.cus = prop.multiProcessorCount;
            std::snprintf(r.name, sizeof(r.name), "%s", prop.gcnArchName);
            // A blocking stream: it orders implicitly with the legacy null
            // stream, which torch uses by default, so device buffers shared
            // with torch are written and read in program order without an
            // explicit sync on either side.
            if (hipStreamCreateWithFlags(&r.own, hipStreamDefault) != hipSuccess) {
                r.init_rc = NEURAL_ERR_INTERNAL;
                return set_error(r.init_rc);
            }
            r.active = r.own;
            // Reduction workspace; counters start at zero and every kernel that
            // uses one leaves it at zero.
            if (hipMalloc(&r.ws.partials, size_t(kMaxPartials) * 64) != hipSuccess ||
                hipMalloc((void **)&r.ws.counter, sizeof(unsigned) * kCounters) != hipSuccess ||
                hipMalloc(&r.ws.result, 256) != hipSuccess ||
                hipHostMalloc(&r.ws.host_result, 256, hipHostMallocCoherent | hipHostMallocMapped) != hipSuccess ||
                hipHostGetDevicePointer(&r.ws.host_result_dev, r.ws.host_result, 0) != hipSuccess ||
                std::memset(r.ws.host_result, 0, 256) == nullptr ||
                hipMemset(r.ws.counter, 0, sizeof(unsigned) * kCounters) != hipSuccess ||
                hipMemset(r.ws.result, 0, 256) != hipSuccess ||
                hipDeviceSynchronize() != hipSuccess) {
                r.init_rc = NEURAL_ERR_OUT_OF_MEMORY;
                return set_error(r.init_rc);
            }
            // A failure here only disables the allocation-free entry point
            // (it then reports NEURAL_ERR_INVALID_CONFIG); the rest works.
            if (setup_static_scratch(r.device) != NEURAL_OK) (void)hipGetLastError();
            r.inited = true;
            t_device_set = true;
        }
    }
    if (r.init_rc != NEURAL_OK) return set_error(r.init_rc);
    if (!t_device_set) {
        (void)hipSetDevice(r.device);
        t_device_set = true;
    }
    return NEURAL_OK;
}

int ensure_ready()
{
    Runtime &r = R();
    if (!r.inited) return set_error(NEURAL_ERR_INVALID_CONFIG);
    if (!t_device_set) {
        if (hipSetDevice(r.device) != hipSuccess) return set_error(NEURAL_ERR_INTERNAL);
        t_device_set = true;
    }
    return NEURAL_OK;
}

hipStream_t stream() { return R().active; }
int num_cus() { return R().cus; }
Workspace &workspace() { return R().ws; }

// Allocation counters for neural_hip_alloc_stats: every dev_alloc call, and
// the hipMalloc calls among them (cache misses).
static std::atomic<unsigned long long> g_dev_allocs{0}, g_hip_mallocs{0};

void *dev_alloc(size_t bytes)
{
    g_dev_allocs.fetch_add(1, std::memory_order_relaxed);
    Runtime &r = R();
    const size_t cls = size_class(bytes);
    std::lock_guard<std::mutex> g(r.mu);
    auto it = r.cache.find(cls);
    if (it != r.cache.end() && !it->second.empty()) {
        void *p = it->second.back();
        it->second.pop_back();
        r.live[p] = cls;
        return p;
    }
    void *p = nullptr;
    g_hip_mallocs.fetch_add(1, std::memory_order_relaxed);
    if (hipMalloc(&p, cls) != hipSuccess) {
        (void)hipGetLastError();
        // Give cached blocks back and retry once; outstanding work may still
        // read them, so drain the stream first.
        (void)hipStreamSynchronize(r.active);
        release_cache_locked(r);
        if (hipMalloc(&p, cls) != hipSuccess) {
            (void)hipGetLastError();
            return nullptr;
        }
    }
    r.live[p] = cls;
    return p;
}

void dev_free(void *p)
{
    if (!p) return;
    Runtime &r = R();
    std::lock_guard<std::mutex> g(r.mu);
    auto it = r.live.find(p);
    if (it == r.live.end()) return;
    // Stream-ordered reuse: every later use of this block is enqueued on the
    // same stream after the work that may still read it.
    r.cache[it->second].push_back(p);
    r.live.erase(it);
}

bool is_device_ptr(const void *p)
{
    if (!p) return false;
    hipPointerAttribute_t a;
    if (hipPointerGetAttributes(&a, p) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return a.type == hipMemoryTypeDevice || a.type == hipMemoryTypeManaged;
}

int check_launch()
{
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? NEURAL_OK : hip_fail(e);
}

int sync()
{
    NH_HIP(hipStreamSynchronize(stream()));
    return NEURAL_OK;
}

int host_result_fetch(void *dst, size_t bytes)
{
    WsGuard wg;
    if (bytes > 256) return set_error(NEURAL_ERR_INTERNAL);
    NH_TRY(sync());
    std::memcpy(dst, workspace().host_result, bytes);
    return NEURAL_OK;
}

namespace {
constexpr size_t kTicketOffset = 248;  // last 8 bytes of the 256-byte host result area
unsigned long long g_ticket = 0;       // last ticket handed out (under WsGuard)
}  // namespace

Ticket next_ticket()
{
    Ticket t;
    t.slot = reinterpret_cast<unsigned long long *>(static_cast<char *>(workspace().host_result_dev) + kTicketOffset);
    t.value = ++g_ticket;
    return t;
}

int host_result_wait(unsigned long long ticket, void *dst, size_t bytes)
{
    if (bytes > kTicketOffset) return set_error(NEURAL_ERR_INTERNAL);
    const char *area = static_cast<const char *>(workspace().host_result);
    const volatile unsigned long long *word =
        reinterpret_cast<const volatile unsigned long long *>(area + kTicketOffset);
    // Spin on the ticket for a while (a kernel that ends normally stores it
    // within microseconds of finishing), then fall back to the stream wait,
    // which also surfaces a fault.
    bool seen = false;
    for (long spins = 0; spins < (1L << 26); spins++) {
        if (__atomic_load_n(word, __ATOMIC_ACQUIRE) == ticket) {
            seen = true;
            break;
        }
        __builtin_ia32_pause();
    }
    if (!seen) {
        NH_TRY(sync());
        if (__atomic_load_n(word, __ATOMIC_ACQUIRE) != ticket) return set_error(NEURAL_ERR_INTERNAL);
    }
    std::memcpy(dst, area, bytes);
    return NEURAL_OK;
}

int result_to_host(void *dst, const void *dev_src, size_t bytes)
{
    WsGuard wg;
    Workspace &ws = workspace();
    if (bytes > 256) return set_error(NEURAL_ERR_INTERNAL);
    NH_HIP(hipMemcpyAsync(ws.host_result, dev_src, bytes, hipMemcpyDeviceToHost, stream()));
    NH_TRY(sync());
    std::memcpy(dst, ws.host_result, bytes);
    return NEURAL_OK;
}

// ---------------------------------------------------------------------------
// Staging of caller pointers
// ---------------------------------------------------------------------------

// Host mirrors of owned tensors by start address (the mirror of a storage
// covers [host, host + hi)), for Staged::open.
namespace {
std::mutex g_mirror_mu;
std::map<uintptr_t, Storage *> g_mirrors;
}  // namespace

void mirror_register(Storage *s)
{
    std::lock_guard<std::mutex> g(g_mirror_mu);
    g_mirrors[reinterpret_cast<uintptr_t>(s->host)] = s;
}

void mirror_unregister(Storage *s)
{
    std::lock_guard<std::mutex> g(g_mirror_mu);
    const auto it = g_mirrors.find(reinterpret_cast<uintptr_t>(s->host));
    if (it != g_mirrors.end() && it->second == s) g_mirrors.erase(it);
}

// The owned storage whose host mirror holds all of [p, p + nbytes), or null.
static Storage *mirror_lookup(const void *p, size_t nbytes)
{
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    std::lock_guard<std::mutex> g(g_mirror_mu);
    auto it = g_mirrors.upper_bound(a);
    if (it == g_mirrors.begin()) return nullptr;
    --it;
    Storage *s = it->second;
    const uintptr_t end = it->first + uintptr_t(s->hi);
    return (a >= it->first && a < end && nbytes <= end - a) ? s : nullptr;
}

int Staged::open(const void *p, size_t nbytes, bool upload)
{
    bytes = nbytes;
    host = const_cast<void *>(p);
    if (is_device_ptr(p)) {
        dev = const_cast<void *>(p);
        owned = false;
        return NEURAL_OK;
    }
    if (Storage *s = nbytes ? mirror_lookup(p, nbytes) : nullptr) {
        // The device copy serves both reads and writes; bytes outside
        // [p, p + nbytes) must be current on the device too, so a
        // host-authoritative mirror is uploaded whole (dev_read's rule).
        if (s->state == ST_HOST) {
            const int64_t span = s->hi - s->lo;
            if (span > 0) NH_HIP(hipMemcpyAsync(s->dev_block, s->host, size_t(span), hipMemcpyHostToDevice, stream()));
            s->state = ST_SYNCED;
        }
        dev = static_cast<char *>(s->dev_block) + (static_cast<const char *>(p) - static_cast<const char *>(s->host));
        mirror = s;
        owned = false;
        return NEURAL_OK;
    }
    dev = dev_alloc(nbytes ? nbytes : 1);
    if (!dev) return set_error(NEURAL_ERR_OUT_OF_MEMORY);
    owned = true;
    if (upload && nbytes) NH_HIP(hipMemcpyAsync(dev, p, nbytes, hipMemcpyHostToDevice, stream()));
    return NEURAL_OK;
}

int Staged::open_n(const void *p, uint64_t count, size_t es, bool upload)
{
    if (count > kMaxRawCount) return set_error(NEURAL_ERR_TENSOR_TOO_LARGE);
    return open(p, size_t(count) * es, upload);
}

int Staged::finish(bool download)
{
    // A mirror-backed output was written on the device; the caller may read
    // it through the host pointer, so the written range goes back there too
    // (the storage keeps its state: SYNCED stays in sync, DEVICE stays ahead).
    if ((owned || mirror) && download && bytes)
        NH_HIP(hipMemcpyAsync(host, dev, bytes, hipMemcpyDeviceToHost, stream()));
    if (mirror) {
        if (download && bytes) NH_TRY(sync());
        mirror = nullptr;
        dev = nullptr;
        return NEURAL_OK;
    }
    if (owned) {
        NH_TRY(sync());
        dev_free(dev);
        dev = nullptr;
        owned = false;
    }
    return NEURAL_OK;
}

Staged::~Staged()
{
    if (owned && dev) {
        (void)hipStreamSynchronize(stream());
        dev_free(dev);
    }
}

// ---------------------------------------------------------------------------
// Tensor helpers
// ---------------------------------------------------------------------------

size_t elem_size(int dtype) { return dtype == NEURAL_DTYPE_FLOAT64 ? 8 : 4; }

int64_t numel(const NeuralTensor *t)
{
    if (!t) return 0;
    int64_t n = 1;
    for (int64_t i = 0; i < t->ndim; i++) n *= t->shape[i];
    return n;
}

bool is_contiguous(const NeuralTensor *t)
{
    int64_t expect = int64_t(elem_size(t->dtype));
    for (int64_t i = t->ndim - 1; i >= 0; i--) {
        if (t->shape[i] != 1 && t->stride[i] != expect) return false;
        expect *= t->shape[i];
    }
    return true;
}

int check_tensor(const NeuralTensor *t)
{
    if (!t) return set_error(NEURAL_ERR_NULL_POINTER);
    if (t->dtype != NEURAL_DTYPE_FLOAT32 && t->dtype != NEURAL_DTYPE_FLOAT64)
        return set_error(NEURAL_ERR_INVALID_DTYPE);
    return NEURAL_OK;
}

static int upload_span(Storage *s, const NeuralTensor *t)
{
    const int64_t span = s->hi - s->lo;
    if (span <= 0) return NEURAL_OK;
    char *host0 = static_cast<char *>(s->host) + s->lo;
    NH_HIP(hipMemcpyAsync(s->dev_block, host0, size_t(span), hipMemcpyHostToDevice, stream()));
    (void)t;
    return NEURAL_OK;
}

static int download_span(Storage *s)
{
    const int64_t span = s->hi - s->lo;
    if (span <= 0) return NEURAL_OK;
    char *host0 = static_cast<char *>(s->host) + s->lo;
    NH_HIP(hipMemcpyAsync(host0, s->dev_block, size_t(span), hipMemcpyDeviceToHost, stream()));
    NH_TRY(sync());
    return NEURAL_OK;
}

int dev_read(const NeuralTensor *t, const void **p)
{
    Storage *s = t->st;
    if (s->kind == KIND_EXT_HOST || (s->kind == KIND_OWNED && s->state == ST_HOST)) {
        NH_TRY(upload_span(s, t));
        if (s->kind == KIND_OWNED) s->state = ST_SYNCED;
    }
    *p = t->dev;
    return NEURAL_OK;
}

int dev_write(NeuralTensor *t, void **p, bool full)
{
    Storage *s = t->st;
    const bool whole = full && (s->hi - s->lo) == int64_t(numel(t) * elem_size(t->dtype));
    if (s->kind == KIND_EXT_HOST || (s->kind == KIND_OWNED && s->state == ST_HOST)) {
        // Partial writes (or views that do not cover the storage) must keep
        // the bytes they do not touch.
        if (!whole) NH_TRY(upload_span(s, t));
    }
    *p = t->dev;
    return NEURAL_OK;
}

int dev_written(NeuralTensor *t)
{
    Storage *s = t->st;
    if (s->kind == KIND_OWNED) s->state = ST_DEVICE;
    else if (s->kind == KIND_EXT_HOST) NH_TRY(download_span(s));
    return NEURAL_OK;
}

// Make the host bytes current and hand them to the caller (map for host
// access): the next device use re-uploads them.
static void *host_map(NeuralTensor *t)
{
    Storage *s = t->st;
    if (s->kind == KIND_OWNED) {
        if (s->state == ST_DEVICE) {
            if (download_span(s) != NEURAL_OK) return nullptr;
        }
        s->state = ST_HOST;
    }
    return t->data;
}

thread_local LaunchTimer t_timer;
thread_local unsigned long long t_launches = 0;

LaunchTimer take_launch_timer()
{
    t_launches++;
    if (!t_timer.start && !t_timer.stop) return LaunchTimer{};
    if (t_timer.skip > 0) {
        t_timer.skip--;
        return LaunchTimer{};
    }
    LaunchTimer t;
    t.start = t_timer.start;  // null once the span's first launch has taken it
    t_timer.start = nullptr;
    if (--t_timer.count <= 0) {
        t.stop = t_timer.stop;
        t_timer = LaunchTimer{};
    }
    return t;
}

std::recursive_mutex &workspace_mutex()
{
    static std::recursive_mutex *m = new std::recursive_mutex();  // never destroyed, like the runtime
    return *m;
}

}  // namespace nh

using namespace nh;

// ---------------------------------------------------------------------------
// Tensor construction
// ---------------------------------------------------------------------------

namespace {

const char *k_messages[] = {
    "no error",
    "null pointer argument",
    "out of memory (device or host)",
    "invalid argument",
    "tensor shapes do not match",
    "tensor dtypes do not match",
    "file not found",
    "file read failed",
    "file write failed",
    "parse error",
    "invalid configuration",
    "tensor too large",
    "invalid dtype (expected 0=float32 or 1=float64)",
    "dimension mismatch (more than 4 broadcast dims, or bad axis)",
    "not implemented",
    "internal error (HIP runtime or kernel launch failed)",
    "gradient check failed",
    "NaN detected",
    "Inf detected",
};

void fill_contig_strides(NeuralTensor *t)
{
    int64_t s = int64_t(elem_size(t->dtype));
    for (int64_t i = t->ndim - 1; i >= 0; i--) {
        t->stride[i] = s;
        s *= t->shape[i];
    }
}

NeuralTensor *alloc_desc(int64_t ndim, int dtype)
{
    NeuralTensor *t = static_cast<NeuralTensor *>(std::calloc(1, sizeof(NeuralTensor)));
    if (!t) return nullptr;
    t->ndim = ndim;
    t->dtype = dtype;
    const int64_t nd = ndim > 0 ? ndim : 1;
    t->shape = static_cast<int64_t *>(std::calloc(size_t(nd), sizeof(int64_t)));
    t->stride = static_cast<int64_t *>(std::calloc(size_t(nd), sizeof(int64_t)));
    if (!t->shape || !t->stride) {
        std::free(t->shape);
        std::free(t->stride);
        std::free(t);
        return nullptr;
    }
    return t;
}

void free_desc(NeuralTensor *t)
{
    std::free(t->shape);
    std::free(t->stride);
    std::free(t);
}

void storage_release(Storage *s)
{
    if (!s || --s->refs > 0) return;
    // Stream-ordered reuse makes an immediate return to the cache safe.
    if (s->dev_block) dev_free(s->dev_block);
    if (s->host_owned) {
        mirror_unregister(s);
        std::free(s->host);
    }
    delete s;
}

// Byte span [lo, hi) reachable from element 0 through the strides.
// A caller's shape (and byte strides, when given) as the library can hold
// it: every dimension below 2^63, the element count and its bytes, and each
// dimension's byte extent and their sums (the storage span) all within
// int64 -- so no count, index or span computed later can wrap.
// NEURAL_ERR_TENSOR_TOO_LARGE otherwise.
static int check_shape(const uint64_t *shape, uint64_t ndim, int dtype, const int64_t *strides)
{
    int64_t n = 1, lo = 0, hi = 0;
    for (uint64_t i = 0; i < ndim; i++) {
        if (shape[i] > uint64_t(INT64_MAX)) return NEURAL_ERR_TENSOR_TOO_LARGE;
        if (__builtin_mul_overflow(n, int64_t(shape[i]), &n)) return NEURAL_ERR_TENSOR_TOO_LARGE;
        if (strides && shape[i] > 0) {
            int64_t ext;
            if (__builtin_mul_overflow(int64_t(shape[i]) - 1, strides[i], &ext)) return NEURAL_ERR_TENSOR_TOO_LARGE;
            if (ext < 0 ? __builtin_add_overflow(lo, ext, &lo) : __builtin_add_overflow(hi, ext, &hi))
                return NEURAL_ERR_TENSOR_TOO_LARGE;
        }
    }
    int64_t bytes;
    if (__builtin_mul_overflow(n, int64_t(elem_size(dtype)), &bytes)) return NEURAL_ERR_TENSOR_TOO_LARGE;
    if (strides && (__builtin_add_overflow(hi, int64_t(elem_size(dtype)), &hi) ||
                    __builtin_sub_overflow(hi, lo, &hi)))
        return NEURAL_ERR_TENSOR_TOO_LARGE;
    return NEURAL_OK;
}

void span_of(const NeuralTensor *t, int64_t *lo, int64_t *hi)
{
    int64_t a = 0, b = 0;
    for (int64_t i = 0; i < t->ndim; i++) {
        if (t->shape[i] == 0) { *lo = 0; *hi = 0; return; }
        const int64_t ext = (t->shape[i] - 1) * t->stride[i];
        if (ext < 0) a += ext; else b += ext;
    }
    *lo = a;
    *hi = b + int64_t(elem_size(t->dtype));
}

NeuralTensor *create_owned(const uint64_t *shape, uint64_t ndim, int dtype, bool zero)
{
    if (ensure_init() != NEURAL_OK) return nullptr;
    if (ndim > 0 && !shape) { set_error(NEURAL_ERR_NULL_POINTER); return nullptr; }
    if (dtype != NEURAL_DTYPE_FLOAT32 && dtype != NEURAL_DTYPE_FLOAT64) {
        set_error(NEURAL_ERR_INVALID_DTYPE);
        return nullptr;
    }
    if (const int rc = check_shape(shape, ndim, dtype, nullptr)) { set_error(rc); return nullptr; }
    NeuralTensor *t = alloc_desc(int64_t(ndim), dtype);
    if (!t) { set_error(NEURAL_ERR_OUT_OF_MEMORY); return nullptr; }
    int64_t n = 1;
    for (uint64_t i = 0; i < ndim; i++) {
        t->shape[i] = int64_t(shape[i]);
        n *= int64_t(shape[i]);
    }
    fill_contig_strides(t);
    const size_t bytes = size_t(n) * elem_size(dtype);
    Storage *s = new (std::nothrow) Storage();
    void *host = nullptr;
    if (s && posix_memalign(&host, 64, bytes ? bytes : 64) != 0) host = nullptr;
    void *dev = s ? dev_alloc(bytes ? bytes : 64) : nullptr;
    if (!s || !host || !dev) {
        std::free(host);
        dev_free(dev);
        delete s;
        free_desc(t);
        set_error(NEURAL_ERR_OUT_OF_MEMORY);
        return nullptr;
    }
    s->refs = 1;
    s->kind = KIND_OWNED;
    s->state = ST_DEVICE;
    s->host = host;
    s->host_owned = true;
    s->dev_block = dev;
    s->dev_bytes = bytes;
    s->lo = 0;
    s->hi = int64_t(bytes);
    t->data = host;
    t->dev = dev;
    t->kind = KIND_OWNED;
    t->flags = NT_OWN_DATA | NT_OWN_META;
    t->st = s;
    mirror_register(s);
    // tensor_create zero-fills every new tensor (tensor.asm:326-329); the
    // fill runs in HBM.
    (void)zero;
    if (bytes && launch_fill(dev, dtype, n, 0.0) != NEURAL_OK) {
        neural_tensor_free(t);
        return nullptr;
    }
    set_error(NEURAL_OK);
    return t;
}

}  // namespace

bool nh::tensors_may_overlap(const NeuralTensor *a, const NeuralTensor *b)
{
    if (!a || !b) return false;
    if (a->st == b->st) return true;
    int64_t alo, ahi, blo, bhi;
    span_of(a, &alo, &ahi);
    span_of(b, &blo, &bhi);
    if (ahi <= alo || bhi <= blo) return false;
    const uintptr_t a0 = reinterpret_cast<uintptr_t>(a->data) + uintptr_t(alo);
    const uintptr_t a1 = reinterpret_cast<uintptr_t>(a->data) + uintptr_t(ahi);
    const uintptr_t b0 = reinterpret_cast<uintptr_t>(b->data) + uintptr_t(blo);
    const uintptr_t b1 = reinterpret_cast<uintptr_t>(b->data) + uintptr_t(bhi);
    return a0 < b1 && b0 < a1;
}

extern "C" {

int neural_init(void) { return ensure_init(); }

void neural_shutdown(void)
{
    Runtime &r = R();
    if (!r.inited) return;
    (void)hipStreamSynchronize(r.active);
    std::lock_guard<std::mutex> g(r.mu);
    release_cache_locked(r);
}

const char *neural_version(void) { return "neural-hip 1.0 (gfx950)"; }

void neural_clear_error(void) { t_last_error = NEURAL_OK; }

int neural_get_last_error(void) { return t_last_error; }

const char *neural_get_error_message(int code)
{
    if (code < 0 || code > 18) return "unknown error";
    return k_messages[code];
}

NeuralTensor *neural_tensor_create(const uint64_t *shape, uint64_t ndim, int dtype)
{
    return create_owned(shape, ndim, dtype, true);
}

NeuralTensor *neural_tensor_zeros(const uint64_t *shape, uint64_t ndim, int dtype)
{
    return create_owned(shape, ndim, dtype, true);
}

// The reference passes 1.0f bits where a double is expected and so fills with
// ~0 (neural_api.asm:517-519); this fills with 1.0.
NeuralTensor *neural_tensor_ones(const uint64_t *shape, uint64_t ndim, int dtype)
{
    NeuralTensor *t = create_owned(shape, ndim, dtype, false);
    if (t && neural_tensor_fill(t, 1.0) != NEURAL_OK) {
        neural_tensor_free(t);
        return nullptr;
    }
    return t;
}

NeuralTensor *neural_tensor_from_data(const void *data, const uint64_t *shape, uint64_t ndim, int dtype)
{
    if (!data) { set_error(NEURAL_ERR_NULL_POINTER); return nullptr; }
    NeuralTensor *t = create_owned(shape, ndim, dtype, false);
    if (!t) return nullptr;
    const size_t bytes = size_t(numel(t)) * elem_size(dtype);
    Staged src;
    if (bytes && (src.open(data, bytes, true) != NEURAL_OK ||
                  hipMemcpyAsync(t->dev, src.dev, bytes, hipMemcpyDeviceToDevice, stream()) != hipSuccess ||
                  src.finish(false) != NEURAL_OK)) {
        neural_tensor_free(t);
        set_error(NEURAL_ERR_INTERNAL);
        return nullptr;
    }
    return t;
}

// Zero-copy wrap (neural_api.asm:2293-2426).  The reference marks the buffer
// FLAG_OWN_DATA (neural_api.asm:2393) and so frees the caller's memory in
// tensor_free; here the caller keeps ownership (flags = OWN_META only).
NeuralTensor *neural_tensor_from_buffer(void *buffer, const uint64_t *shape, uint64_t ndim, int dtype,
                                        const int64_t *strides)
{
    if (ensure_init() != NEURAL_OK) return nullptr;
    if (!buffer || !shape) { set_error(NEURAL_ERR_NULL_POINTER); return nullptr; }
    if (dtype != NEURAL_DTYPE_FLOAT32 && dtype != NEURAL_DTYPE_FLOAT64) {
        set_error(NEURAL_ERR_INVALID_DTYPE);
        return nullptr;
    }
    if (const int rc = check_shape(shape, ndim, dtype, strides)) { set_error(rc); return nullptr; }
    NeuralTensor *t = alloc_desc(int64_t(ndim), dtype);
    if (!t) { set_error(NEURAL_ERR_OUT_OF_MEMORY); return nullptr; }
    for (uint64_t i = 0; i < ndim; i++) t->shape[i] = int64_t(shape[i]);
    if (strides) for (uint64_t i = 0; i < ndim; i++) t->stride[i] = strides[i];
    else fill_contig_strides(t);
    Storage *s = new (std::nothrow) Storage();
    if (!s) { free_desc(t); set_error(NEURAL_ERR_OUT_OF_MEMORY); return nullptr; }
    s->refs = 1;
    s->host = buffer;
    s->host_owned = false;
    span_of(t, &s->lo, &s->hi);
    t->data = buffer;
    t->flags = NT_OWN_META;
    t->st = s;
    if (is_device_ptr(buffer)) {
        s->kind = KIND_EXT_DEV;
        s->state = ST_DEVICE;
        t->dev = buffer;
    } else {
        s->kind = KIND_EXT_HOST;
        s->state = ST_HOST;
        const int64_t span = s->hi - s->lo;
        s->dev_block = dev_alloc(size_t(span > 0 ? span : 64));
        s->dev_bytes = size_t(span > 0 ? span : 0);
        if (!s->dev_block) {
            delete s;
            free_desc(t);
            set_error(NEURAL_ERR_OUT_OF_MEMORY);
            return nullptr;
        }
        t->dev = static_cast<char *>(s->dev_block) - s->lo;
    }
    t->kind = s->kind;
    set_error(NEURAL_OK);
    return t;
}

const int64_t *neural_tensor_stride(NeuralTensor *t) { return t ? t->stride : nullptr; }

int neural_tensor_is_contiguous(NeuralTensor *t)
{
    if (!t) { set_error(NEURAL_ERR_NULL_POINTER); return -1; }
    return nh::is_contiguous(t) ? 1 : 0;
}

NeuralTensor *neural_tensor_make_contiguous(NeuralTensor *t)
{
    if (!t) { set_error(NEURAL_ERR_NULL_POINTER); return nullptr; }
    if (nh::is_contiguous(t)) return t;
    std::vector<uint64_t> shp(size_t(t->ndim));
    for (int64_t i = 0; i < t->ndim; i++) shp[size_t(i)] = uint64_t(t->shape[i]);
    NeuralTensor *o = neural_tensor_create(shp.data(), uint64_t(t->ndim), t->dtype);
    if (!o) return nullptr;
    if (neural_tensor_copy(o, t) != NEURAL_OK) {
        neural_tensor_free(o);
        return nullptr;
    }
    return o;
}

int neural_buffer_info(NeuralTensor *t, NeuralBufferInfo *info)
{
    if (!t || !info) return set_error(NEURAL_ERR_NULL_POINTER);
    void *p = host_map(t);
    if (!p && numel(t) > 0) return set_error(NEURAL_ERR_INTERNAL);
    std::memset(info, 0, sizeof(*info));
    info->data = p;
    info->itemsize = elem_size(t->dtype);
    info->ndim = uint64_t(t->ndim);
    info->shape = reinterpret_cast<const uint64_t *>(t->shape);
    info->strides = t->stride;
    info->readonly = 0;
    info->format[0] = t->dtype == NEURAL_DTYPE_FLOAT64 ? 'd' : 'f';
    return set_error(NEURAL_OK);
}

void neural_tensor_free(NeuralTensor *t)
{
    if (!t) return;
    storage_release(t->st);
    free_desc(t);
}

void *neural_tensor_data(NeuralTensor *t)
{
    if (!t) return nullptr;
    return host_map(t);
}

uint64_t neural_tensor_ndim(NeuralTensor *t) { return t ? uint64_t(t->ndim) : 0; }

const uint64_t *neural_tensor_shape(NeuralTensor *t)
{
    return t ? reinterpret_cast<const uint64_t *>(t->shape) : nullptr;
}

uint64_t neural_tensor_numel(NeuralTensor *t) { return t ? uint64_t(numel(t)) : 0; }

int neural_tensor_dtype(NeuralTensor *t) { return t ? t->dtype : -1; }

uint64_t neural_tensor_bytes(NeuralTensor *t)
{
    return t ? uint64_t(numel(t)) * elem_size(t->dtype) : 0;
}

// tensor_fill (tensor.asm:531-589): the double value is rounded to float once
// for f32 tensors.  Strided tensors fill every addressed element.
int neural_tensor_fill(NeuralTensor *t, double value)
{
    NH_TRY(ensure_init());
    NH_TRY(check_tensor(t));
    const int64_t n = numel(t);
    if (n == 0) return set_error(NEURAL_OK);
    void *d = nullptr;
    const bool contig = nh::is_contiguous(t);
    NH_TRY(dev_write(t, &d, contig));
    if (contig) {
        NH_TRY(launch_fill(d, t->dtype, n, value));
    } else {
        NH_TRY(launch_fill_strided(d, t->dtype, t->shape, t->stride, int(t->ndim), value));
    }
    NH_TRY(dev_written(t));
    return set_error(NEURAL_OK);
}

// neural_tensor_copy (neural_api.asm:905-967): dtype must match (5) and
// element counts must match (4); copies in logical (row-major) order.
int neural_tensor_copy(NeuralTensor *dst, const NeuralTensor *src)
{
    NH_TRY(ensure_init());
    if (!dst || !src) return set_error(NEURAL_ERR_NULL_POINTER);
    if (dst->dtype != src->dtype) return set_error(NEURAL_ERR_DTYPE_MISMATCH);
    const int64_t n = numel(dst);
    if (n != numel(src)) return set_error(NEURAL_ERR_SHAPE_MISMATCH);
    if (n == 0) return set_error(NEURAL_OK);
    const void *s = nullptr;
    void *d = nullptr;
    NH_TRY(dev_read(src, &s));
    const bool dc = nh::is_contiguous(dst), sc = nh::is_contiguous(src);
    NH_TRY(dev_write(dst, &d, dc));
    const size_t es = elem_size(dst->dtype);
    if (dc && sc) {
        NH_HIP(hipMemcpyAsync(d, s, size_t(n) * es, hipMemcpyDeviceToDevice, stream()));
    } else {
        NH_TRY(launch_copy_nd(d, dst->shape, dst->stride, int(dst->ndim), s, src->shape, src->stride,
                              int(src->ndim), int(es)));
    }
    NH_TRY(dev_written(dst));
    return set_error(NEURAL_OK);
}

// tensor_reshape (tensor.asm:600-680): element counts must match (4); the
// result is a view sharing storage (OWN_META only).  Non-contiguous inputs
// are rejected with 3 (the reference views them anyway and mislabels strides).
NeuralTensor *neural_tensor_reshape(NeuralTensor *t, const uint64_t *new_shape, uint64_t new_ndim)
{
    if (!t || (new_ndim > 0 && !new_shape)) { set_error(NEURAL_ERR_NULL_POINTER); return nullptr; }
    // a count that does not fit int64 cannot match the tensor's
    if (check_shape(new_shape, new_ndim, t->dtype, nullptr) != NEURAL_OK) {
        set_error(NEURAL_ERR_SHAPE_MISMATCH);
        return nullptr;
    }
    int64_t n = 1;
    for (uint64_t i = 0; i < new_ndim; i++) n *= int64_t(new_shape[i]);
    if (n != numel(t)) { set_error(NEURAL_ERR_SHAPE_MISMATCH); return nullptr; }
    if (!nh::is_contiguous(t)) { set_error(NEURAL_ERR_INVALID_ARGUMENT); return nullptr; }
    NeuralTensor *v = alloc_desc(int64_t(new_ndim), t->dtype);
    if (!v) { set_error(NEURAL_ERR_OUT_OF_MEMORY); return nullptr; }
    for (uint64_t i = 0; i < new_ndim; i++) v->shape[i] = int64_t(new_shape[i]);
    fill_contig_strides(v);
    v->data = t->data;
    v->dev = t->dev;
    v->kind = KIND_VIEW;
    v->flags = NT_OWN_META;
    v->st = t->st;
    t->st->refs++;
    set_error(NEURAL_OK);
    return v;
}

int neural_tensor_upload(NeuralTensor *t, const void *host_src, uint64_t bytes)
{
    NH_TRY(ensure_init());
    if (!t || !host_src) return set_error(NEURAL_ERR_NULL_POINTER);
    if (bytes != neural_tensor_bytes(t) || !nh::is_contiguous(t)) return set_error(NEURAL_ERR_SHAPE_MISMATCH);
    void *d = nullptr;
    NH_TRY(dev_write(t, &d, true));
    NH_HIP(hipMemcpyAsync(d, host_src, bytes, hipMemcpyHostToDevice, stream()));
    NH_TRY(sync());
    NH_TRY(dev_written(t));
    return set_error(NEURAL_OK);
}

int neural_tensor_download(NeuralTensor *t, void *host_dst, uint64_t bytes)
{
    NH_TRY(ensure_init());
    if (!t || !host_dst) return set_error(NEURAL_ERR_NULL_POINTER);
    if (bytes != neural_tensor_bytes(t) || !nh::is_contiguous(t)) return set_error(NEURAL_ERR_SHAPE_MISMATCH);
    const void *s = nullptr;
    NH_TRY(dev_read(t, &s));
    NH_HIP(hipMemcpyAsync(host_dst, s, bytes, hipMemcpyDeviceToHost, stream()));
    NH_TRY(sync());
    return set_error(NEURAL_OK);
}

void *neural_tensor_device_data(NeuralTensor *t)
{
    if (!t) return nullptr;
    const void *p = nullptr;
    if (dev_read(t, &p) != NEURAL_OK) return nullptr;
    // The caller may write through the device address: device copy is now
    // authoritative.
    if (t->st->kind == KIND_OWNED) t->st->state = ST_DEVICE;
    return const_cast<void *>(p);
}

int neural_hip_set_stream(void *s)
{
    NH_TRY(ensure_init());
    Runtime &r = R();
    hipStream_t next = static_cast<hipStream_t>(s);  // NULL = the HIP null stream
    if (next != r.active) {
        NH_HIP(hipStreamSynchronize(r.active));
        r.active = next;
    }
    return set_error(NEURAL_OK);
}

int neural_hip_reset_stream(void)
{
    NH_TRY(ensure_init());
    Runtime &r = R();
    if (r.active != r.own) {
        NH_HIP(hipStreamSynchronize(r.active));
        r.active = r.own;
    }
    return set_error(NEURAL_OK);
}

int neural_hip_time_launches(void *start_event, void *stop_event, int skip, int count)
{
    NH_TRY(ensure_init());
    if (!start_event || !stop_event) return set_error(NEURAL_ERR_NULL_POINTER);
    if (skip < 0 || count < 1) return set_error(NEURAL_ERR_INVALID_ARGUMENT);
    t_timer.start = static_cast<hipEvent_t>(start_event);
    t_timer.stop = static_cast<hipEvent_t>(stop_event);
    t_timer.skip = skip;
    t_timer.count = count;
    return set_error(NEURAL_OK);
}

int neural_hip_time_next_launch(void *start_event, void *stop_event, int skip)
{
    return neural_hip_time_launches(start_event, stop_event, skip, 1);
}

int neural_hip_time_cancel(void)
{
    t_timer = LaunchTimer{};
    return set_error(NEURAL_OK);
}

unsigned long long neural_hip_launch_count(void) { return t_launches; }

int neural_hip_alloc_stats(unsigned long long *dev_allocs, unsigned long long *hip_mallocs)
{
    if (dev_allocs) *dev_allocs = g_dev_allocs.load(std::memory_order_relaxed);
    if (hip_mallocs) *hip_mallocs = g_hip_mallocs.load(std::memory_order_relaxed);
    return set_error(NEURAL_OK);
}

void *neural_hip_get_stream(void)
{
    if (ensure_init() != NEURAL_OK) return nullptr;
    return static_cast<void *>(R().active);
}

int neural_hip_synchronize(void)
{
    NH_TRY(ensure_init());
    NH_TRY(sync());
    return set_error(NEURAL_OK);
}

int neural_hip_empty_cache(void)
{
    NH_TRY(ensure_init());
    Runtime &r = R();
    NH_HIP(hipStreamSynchronize(r.active));
    std::lock_guard<std::mutex> g(r.mu);
    release_cache_locked(r);
    return set_error(NEURAL_OK);
}

int neural_hip_device_info(int *ordinal, int *cus, char *name, int name_len)
{
    NH_TRY(ensure_init());
    Runtime &r = R();
    if (ordinal) *ordinal = r.device;
    if (cus) *cus = r.cus;
    if (name && name_len > 0) std::snprintf(name, size_t(name_len), "%s", r.name);
    return set_error(NEURAL_OK);
}

}  // extern "C"
