// tl_hip runtime: device/stream state, thread-local errors, stream-ordered caching
// allocator, tensor handles and event timing.
//
// The reference backends keep one global device, the null stream and a mutex buffer pool
// that synchronises the device on every allocation (tl_cuda buffer_pool.rs:85-100) and
// after every launch (ops/llm.rs:91).  Here all work is ordered on one non-null stream and
// nothing synchronises except calls that hand data back to the host.
#include "internal.h"
#include "block_cache.h"

#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <vector>

namespace tlhip {

static thread_local int tls_status = TL_HIP_OK;
static thread_local char tls_msg[512] = {0};

void set_error(int status, const char* fmt, ...) {
    tls_status = status;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(tls_msg, sizeof(tls_msg), fmt, ap);
    va_end(ap);
}

void clear_error() {
    tls_status = TL_HIP_OK;
    tls_msg[0] = 0;
}

int hip_fail(hipError_t e, const char* what) {
    set_error(TL_HIP_ERR_DEVICE, "DeviceError: %s failed: %s", what, hipGetErrorString(e));
    return TL_HIP_ERR_DEVICE;
}

static std::mutex g_init_mu;
static DeviceState g_state;
static bool g_ready = false;
static thread_local hipStream_t tls_stream_override = nullptr;

static int init_locked(int device) {
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n == 0) {
        set_error(TL_HIP_ERR_DEVICE, "DeviceError: no HIP device available (%s)",
                  e == hipSuccess ? "count 0" : hipGetErrorString(e));
        return TL_HIP_ERR_DEVICE;
    }
    if (device < 0 || device >= n) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: device %d out of range (count %d)", device, n);
        return TL_HIP_ERR_ARG;
    }
    TLH_CHECK_HIP(hipSetDevice(device));
    hipDeviceProp_t prop;
    TLH_CHECK_HIP(hipGetDeviceProperties(&prop, device));
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        set_error(TL_HIP_ERR_DEVICE, "DeviceError: tl_hip is built for gfx950, device is %s",
                  prop.gcnArchName);
        return TL_HIP_ERR_DEVICE;
    }
    // default priority (a non-default stream priority is never used)
    TLH_CHECK_HIP(hipStreamCreateWithFlags(&g_state.stream, hipStreamNonBlocking));
    g_state.device = device;
    g_state.num_cus = prop.multiProcessorCount;
    // the allocation-free GEMM's fixed scratch: its address is looked up here, once, so that
    // entry never does it inside a caller's graph capture
    if (int rc = noalloc_scratch_init(device)) return rc;
    g_ready = true;
    return TL_HIP_OK;
}

DeviceState* state() {
    if (g_ready) {
        return &g_state;
    }
    std::lock_guard<std::mutex> lk(g_init_mu);
    if (!g_ready && init_locked(0) != TL_HIP_OK) return nullptr;
    return &g_state;
}

hipStream_t cur_stream() {
    if (tls_stream_override) return tls_stream_override;
    DeviceState* s = state();
    return s ? s->stream : nullptr;
}

// ---- allocator ---------------------------------------------------------------------
// Size-class cache of freed blocks (block_cache.h).  While every call runs on the library
// stream, a freed block is reused by the next request with no synchronisation (stream order).
// Once work is seen on another stream (tl_hip_set_stream or a launcher's stream argument),
// each free also records an event on the freeing stream, and a request on a different stream
// takes the block only after that event has completed.
static std::mutex g_alloc_mu;
static BlockCache<hipStream_t, hipEvent_t> g_cache;
static std::map<void*, size_t> g_live;           // block -> class size
static std::vector<hipEvent_t> g_ev_pool;
static std::atomic<bool> g_multi{false};
static std::atomic<int64_t> g_fail_after{-1};    // fault injection: allocations until a failure

bool note_stream_syncs(hipStream_t s) {
    return s && !g_multi.load(std::memory_order_acquire) && state() && s != g_state.stream;
}

bool single_stream() { return !g_multi.load(std::memory_order_acquire); }

static std::atomic<bool> g_one_launch{true};
bool one_launch_merge() { return g_one_launch.load(std::memory_order_relaxed); }

void note_stream(hipStream_t s) {
    if (!s || g_multi.load(std::memory_order_acquire) || !state() || s == g_state.stream) return;
    std::lock_guard<std::mutex> lk(g_alloc_mu);
    if (g_multi.load()) return;
    // every block cached so far was used on the library stream only
    (void)hipStreamSynchronize(g_state.stream);
    g_cache.mark_all_idle();
    g_multi.store(true, std::memory_order_release);
}

static hipEvent_t pool_event_locked() {
    if (!g_ev_pool.empty()) {
        hipEvent_t ev = g_ev_pool.back();
        g_ev_pool.pop_back();
        return ev;
    }
    hipEvent_t ev = nullptr;
    if (hipEventCreateWithFlags(&ev, hipEventDisableTiming) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    return ev;
}

static void release_cache_locked() {
    (void)hipDeviceSynchronize();
    g_cache.drain([](void* p, hipEvent_t ev) {
        (void)hipFree(p);
        if (ev) g_ev_pool.push_back(ev);
    });
}

void* dev_alloc_on(size_t bytes, hipStream_t s) {
    if (!state()) return nullptr;
    const size_t c = block_size_class(bytes);
    std::lock_guard<std::mutex> lk(g_alloc_mu);
    const int64_t left = g_fail_after.load();
    if (left >= 0) {
        g_fail_after.store(left - 1);
        if (left == 0) {
            set_error(TL_HIP_ERR_ALLOC, "AllocationError: injected failure of a %zu-byte allocation", c);
            return nullptr;
        }
    }
    void* p = g_cache.take(
        c, s, [](hipEvent_t ev) { return hipEventQuery(ev) == hipSuccess; },
        [](hipEvent_t ev) { g_ev_pool.push_back(ev); });
    if (p) {
        g_live[p] = c;
        return p;
    }
    hipError_t e = hipMalloc(&p, c);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        // cached blocks may be what stands in the way: return them and retry once
        release_cache_locked();
        e = hipMalloc(&p, c);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            set_error(TL_HIP_ERR_ALLOC, "AllocationError: hipMalloc(%zu) failed: %s", c,
                      hipGetErrorString(e));
            return nullptr;
        }
    }
    g_live[p] = c;
    return p;
}

void dev_free_on(void* p, hipStream_t s) {
    if (!p) return;
    std::lock_guard<std::mutex> lk(g_alloc_mu);
    auto it = g_live.find(p);
    if (it == g_live.end()) return;
    hipEvent_t ev = nullptr;
    if (g_multi.load()) {
        ev = pool_event_locked();
        if (ev && hipEventRecord(ev, s) != hipSuccess) {
            (void)hipGetLastError();
            g_ev_pool.push_back(ev);
            ev = nullptr;  // then only work on s itself may reuse the block
        }
    }
    g_cache.put(p, it->second, s, ev);
    g_live.erase(it);
}

void* dev_alloc(size_t bytes) { return dev_alloc_on(bytes, cur_stream()); }
void dev_free(void* p) { dev_free_on(p, cur_stream()); }

size_t dtype_size(int dtype) { return dtype == TL_HIP_F16 ? 2 : 4; }

Tensor* tensor_alloc(const int64_t* shape, int rank, int dtype) {
    if (rank < 0 || rank > TL_HIP_MAX_RANK) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: rank %d outside 0..%d", rank, TL_HIP_MAX_RANK);
        return nullptr;
    }
    int64_t n = 1;
    for (int i = 0; i < rank; i++) {
        if (shape[i] < 0) {
            set_error(TL_HIP_ERR_SHAPE, "ShapeMismatch: negative dimension %lld",
                      (long long)shape[i]);
            return nullptr;
        }
        if (shape[i] && n > (INT64_MAX / 4) / shape[i]) {
            set_error(TL_HIP_ERR_ALLOC, "AllocationError: tensor of more than 2^61 elements");
            return nullptr;
        }
        n *= shape[i];
    }
    Tensor* t = new Tensor();
    t->rank = rank;
    for (int i = 0; i < rank; i++) t->shape[i] = shape[i];
    t->numel = n;
    t->dtype = dtype;
    t->data = dev_alloc(n * dtype_size(dtype));
    if (!t->data) {
        delete t;
        return nullptr;
    }
    return t;
}

void tensor_drop(Tensor* t) {
    if (!t) return;
    if (t->refs.fetch_sub(1) == 1) {
        if (t->owns) dev_free(t->data);
        delete t;
    }
}

}  // namespace tlhip

using namespace tlhip;

extern "C" {

const char* tl_hip_last_error(void) { return tls_msg; }
int tl_hip_last_status(void) { return tls_status; }
void tl_hip_clear_error(void) { clear_error(); }

int tl_hip_init(int device) {
    std::lock_guard<std::mutex> lk(g_init_mu);
    if (g_ready) {
        if (device == g_state.device) return TL_HIP_OK;
        set_error(TL_HIP_ERR_ARG, "ArgumentError: already initialised on device %d",
                  g_state.device);
        return TL_HIP_ERR_ARG;
    }
    return init_locked(device);
}

int tl_hip_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    return n;
}

void* tl_hip_stream(void) { return (void*)cur_stream(); }

int tl_hip_set_stream(void* s) {
    if (!state()) return tls_status;
    note_stream((hipStream_t)s);
    tls_stream_override = (hipStream_t)s;
    return TL_HIP_OK;
}

int tl_hip_debug_fail_alloc(int64_t after) {
    g_fail_after.store(after < 0 ? -1 : after);
    return TL_HIP_OK;
}

int tl_hip_debug_one_launch_merge(int on) {
    if (on < 0) return single_stream() && one_launch_merge() ? 1 : 0;
    return g_one_launch.exchange(on != 0) ? 1 : 0;
}

int tl_hip_synchronize(void) {
    if (!state()) return tls_status;
    TLH_CHECK_HIP(hipStreamSynchronize(cur_stream()));
    return TL_HIP_OK;
}

void* tl_hip_malloc(size_t bytes) {
    if (!state()) return nullptr;
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, bytes ? bytes : 1);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        set_error(TL_HIP_ERR_ALLOC, "AllocationError: hipMalloc(%zu) failed: %s", bytes,
                  hipGetErrorString(e));
        return nullptr;
    }
    return p;
}

int tl_hip_free(void* p) {
    if (!p) return TL_HIP_OK;
    TLH_CHECK_HIP(hipFree(p));
    return TL_HIP_OK;
}

int tl_hip_memcpy_h2d(void* dst, const void* src, size_t bytes) {
    if (!state()) return tls_status;
    TLH_CHECK_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, cur_stream()));
    TLH_CHECK_HIP(hipStreamSynchronize(cur_stream()));
    return TL_HIP_OK;
}

int tl_hip_memcpy_d2h(void* dst, const void* src, size_t bytes) {
    if (!state()) return tls_status;
    TLH_CHECK_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, cur_stream()));
    TLH_CHECK_HIP(hipStreamSynchronize(cur_stream()));
    return TL_HIP_OK;
}

int tl_hip_memcpy_d2d(void* dst, const void* src, size_t bytes) {
    if (!state()) return tls_status;
    TLH_CHECK_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, cur_stream()));
    return TL_HIP_OK;
}

void* tl_hip_event_create(void) {
    if (!state()) return nullptr;
    hipEvent_t ev;
    hipError_t e = hipEventCreate(&ev);
    if (e != hipSuccess) {
        hip_fail(e, "hipEventCreate");
        return nullptr;
    }
    return (void*)ev;
}

int tl_hip_event_record(void* ev) {
    if (!ev) {
        set_error(TL_HIP_ERR_NULL, "NullPointerError: event");
        return TL_HIP_ERR_NULL;
    }
    TLH_CHECK_HIP(hipEventRecord((hipEvent_t)ev, cur_stream()));
    return TL_HIP_OK;
}

int tl_hip_event_elapsed_ms(void* a, void* b, float* ms) {
    if (!a || !b || !ms) {
        set_error(TL_HIP_ERR_NULL, "NullPointerError: event or output");
        return TL_HIP_ERR_NULL;
    }
    TLH_CHECK_HIP(hipEventSynchronize((hipEvent_t)b));
    TLH_CHECK_HIP(hipEventElapsedTime(ms, (hipEvent_t)a, (hipEvent_t)b));
    return TL_HIP_OK;
}

// One wavefront that sleeps for `us` microseconds of the 100 MHz constant clock
// (s_memrealtime); the loop also stops after a fixed number of iterations, so it always ends.
__global__ void k_stall(uint64_t ticks) {
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    for (int i = 0; i < (1 << 22); i++) {
        if (__builtin_amdgcn_s_memrealtime() - t0 >= ticks) break;
        __builtin_amdgcn_s_sleep(32);
    }
}

int tl_hip_stall(uint32_t us) {
    if (!state()) return tls_status;
    if (us > 100000) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: stall of %u us exceeds 100 ms", us);
        return TL_HIP_ERR_ARG;
    }
    k_stall<<<1, 64, 0, cur_stream()>>>((uint64_t)us * 100);
    TLH_CHECK_HIP(hipGetLastError());
    return TL_HIP_OK;
}

int tl_hip_event_destroy(void* ev) {
    if (!ev) return TL_HIP_OK;
    TLH_CHECK_HIP(hipEventDestroy((hipEvent_t)ev));
    return TL_HIP_OK;
}

// ---- tensors ------------------------------------------------------------------------

static bool check_shape(const int64_t* shape, int rank) {
    if (rank > 0 && !shape) {
        set_error(TL_HIP_ERR_NULL, "NullPointerError: shape");
        return false;
    }
    return true;
}

tl_hip_tensor* tl_hip_tensor_new(const float* host, const int64_t* shape, int rank) {
    if (!check_shape(shape, rank)) return nullptr;
    Tensor* t = tensor_alloc(shape, rank, TL_HIP_F32);
    if (!t) return nullptr;
    if (t->numel && host) {
        hipError_t e = hipMemcpyAsync(t->data, host, t->numel * 4, hipMemcpyHostToDevice,
                                      cur_stream());
        if (e == hipSuccess) e = hipStreamSynchronize(cur_stream());
        if (e != hipSuccess) {
            hip_fail(e, "hipMemcpyAsync(H2D)");
            tensor_drop(t);
            return nullptr;
        }
    } else if (t->numel) {
        (void)hipMemsetAsync(t->data, 0, t->numel * 4, cur_stream());
    }
    return H(t);
}

tl_hip_tensor* tl_hip_tensor_new_f16(const uint16_t* host, const int64_t* shape, int rank) {
    if (!check_shape(shape, rank)) return nullptr;
    Tensor* t = tensor_alloc(shape, rank, TL_HIP_F16);
    if (!t) return nullptr;
    if (t->numel && host) {
        hipError_t e = hipMemcpyAsync(t->data, host, t->numel * 2, hipMemcpyHostToDevice,
                                      cur_stream());
        if (e == hipSuccess) e = hipStreamSynchronize(cur_stream());
        if (e != hipSuccess) {
            hip_fail(e, "hipMemcpyAsync(H2D)");
            tensor_drop(t);
            return nullptr;
        }
    } else if (t->numel) {
        (void)hipMemsetAsync(t->data, 0, t->numel * 2, cur_stream());
    }
    return H(t);
}

tl_hip_tensor* tl_hip_tensor_zeros(const int64_t* shape, int rank, int dtype) {
    if (!check_shape(shape, rank)) return nullptr;
    if (dtype != TL_HIP_F32 && dtype != TL_HIP_F16) {
        set_error(TL_HIP_ERR_TYPE, "TypeMismatch: dtype %d", dtype);
        return nullptr;
    }
    Tensor* t = tensor_alloc(shape, rank, dtype);
    if (!t) return nullptr;
    if (t->numel) {
        hipError_t e = hipMemsetAsync(t->data, 0, t->numel * dtype_size(dtype), cur_stream());
        if (e != hipSuccess) {
            hip_fail(e, "hipMemsetAsync");
            tensor_drop(t);
            return nullptr;
        }
    }
    return H(t);
}

int tl_hip_tensor_release(tl_hip_tensor* h) {
    if (!h) return TL_HIP_OK;  // releasing NULL is a no-op (memory_ffi.rs:190-206)
    tensor_drop(T(h));
    return TL_HIP_OK;
}

tl_hip_tensor* tl_hip_tensor_acquire(tl_hip_tensor* h) {
    if (!h) {
        set_error(TL_HIP_ERR_NULL, "NullPointerError: tensor");
        return nullptr;
    }
    T(h)->refs.fetch_add(1);
    return h;
}

__global__ void k_f16_to_f32(const __half* in, float* out, int64_t n) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = __half2float(in[i]);
}

int tl_hip_tensor_to_host(const tl_hip_tensor* h, float* out, int64_t numel) {
    if (!h || !out) {
        set_error(TL_HIP_ERR_NULL, "NullPointerError: tensor or output");
        return TL_HIP_ERR_NULL;
    }
    const Tensor* t = reinterpret_cast<const Tensor*>(h);
    if (numel < t->numel) {
        set_error(TL_HIP_ERR_SHAPE, "ShapeMismatch: output holds %lld, tensor has %lld",
                  (long long)numel, (long long)t->numel);
        return TL_HIP_ERR_SHAPE;
    }
    if (t->numel == 0) return TL_HIP_OK;
    hipStream_t s = cur_stream();
    if (t->dtype == TL_HIP_F32) {
        TLH_CHECK_HIP(hipMemcpyAsync(out, t->data, t->numel * 4, hipMemcpyDeviceToHost, s));
    } else {
        float* tmp = (float*)dev_alloc(t->numel * 4);
        if (!tmp) return TL_HIP_ERR_ALLOC;
        k_f16_to_f32<<<cdiv(t->numel, 256), 256, 0, s>>>((const __half*)t->data, tmp, t->numel);
        hipError_t e = hipMemcpyAsync(out, tmp, t->numel * 4, hipMemcpyDeviceToHost, s);
        dev_free(tmp);
        if (e != hipSuccess) return hip_fail(e, "hipMemcpyAsync(D2H)");
    }
    TLH_CHECK_HIP(hipStreamSynchronize(s));
    return TL_HIP_OK;
}

int tl_hip_tensor_rank(const tl_hip_tensor* h) {
    if (!h) {
        set_error(TL_HIP_ERR_NULL, "NullPointerError: tensor");
        return -1;
    }
    return reinterpret_cast<const Tensor*>(h)->rank;
}

int tl_hip_tensor_shape(const tl_hip_tensor* h, int64_t* shape_out) {
    if (!h || !shape_out) {
        set_error(TL_HIP_ERR_NULL, "NullPointerError: tensor or output");
        return TL_HIP_ERR_NULL;
    }
    const Tensor* t = reinterpret_cast<const Tensor*>(h);
    for (int i = 0; i < t->rank; i++) shape_out[i] = t->shape[i];
    return TL_HIP_OK;
}

int64_t tl_hip_tensor_numel(const tl_hip_tensor* h) {
    if (!h) {
        set_error(TL_HIP_ERR_NULL, "NullPointerError: tensor");
        return -1;
    }
    return reinterpret_cast<const Tensor*>(h)->numel;
}

int tl_hip_tensor_dtype(const tl_hip_tensor* h) {
    if (!h) {
        set_error(TL_HIP_ERR_NULL, "NullPointerError: tensor");
        return -1;
    }
    return reinterpret_cast<const Tensor*>(h)->dtype;
}

void* tl_hip_tensor_data(const tl_hip_tensor* h) {
    if (!h) {
        set_error(TL_HIP_ERR_NULL, "NullPointerError: tensor");
        return nullptr;
    }
    return reinterpret_cast<const Tensor*>(h)->data;
}

tl_hip_tensor* tl_hip_tensor_reshape(const tl_hip_tensor* h, const int64_t* shape, int rank) {
    if (!h) {
        set_error(TL_HIP_ERR_NULL, "NullPointerError: tensor");
        return nullptr;
    }
    if (!check_shape(shape, rank)) return nullptr;
    const Tensor* t = reinterpret_cast<const Tensor*>(h);
    int64_t n = 1;
    for (int i = 0; i < rank; i++) n *= shape[i];
    if (n != t->numel) {
        set_error(TL_HIP_ERR_SHAPE, "ShapeMismatch: reshape of %lld elements to %lld",
                  (long long)t->numel, (long long)n);
        return nullptr;
    }
    Tensor* o = tensor_alloc(shape, rank, t->dtype);
    if (!o) return nullptr;
    if (n) {
        hipError_t e = hipMemcpyAsync(o->data, t->data, n * dtype_size(t->dtype),
                                      hipMemcpyDeviceToDevice, cur_stream());
        if (e != hipSuccess) {
            hip_fail(e, "hipMemcpyAsync(D2D)");
            tensor_drop(o);
            return nullptr;
        }
    }
    return H(o);
}

}  // extern "C"
