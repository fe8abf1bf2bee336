// dh_backend.hip -- device init, status, memory pool, copies, timing, conversions
// and the row-softmax kernel of the HIP backend.
//
// Replaces runtime/backend/gpu.inc: initBackend (313-361), dream_gpu_available
// (271-273), gpu_dispatch_threshold (293-307), DeviceMemPool (372-420) and the
// HostBuf fp64<->fp32 staging (177-196), for one device per process.
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <unordered_map>
#include <vector>

#include "dh_common.hpp"

namespace dh {

namespace {

struct State {
    std::once_flag once;
    int status = DH_ERR_NO_DEVICE;
    hipStream_t own_stream = nullptr;
    hipStream_t user_stream = nullptr;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    hipDeviceProp_t prop{};
    int cus = 0;
    std::mutex pool_mu;
    std::map<size_t, std::vector<void*>> free_lists;     // exact-size buckets
    std::unordered_map<void*, size_t> live;              // pointer -> bytes
    std::map<size_t, std::vector<void*>> host_free;      // pinned host buffers, by size
    std::unordered_map<void*, size_t> host_live;
};

State& st() {
    static State s;
    return s;
}

thread_local char g_err[512] = "";

void do_init() {
    State& s = st();
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n <= 0) {
        set_error(DH_ERR_NO_DEVICE, "no HIP device (%s)",
                  e != hipSuccess ? hipGetErrorString(e) : "count = 0");
        std::fprintf(stderr, "warning: no HIP device -- GPU ops unavailable\n");
        return;
    }
    if ((e = hipSetDevice(0)) != hipSuccess ||
        (e = hipGetDeviceProperties(&s.prop, 0)) != hipSuccess ||
        (e = hipStreamCreateWithFlags(&s.own_stream, hipStreamNonBlocking)) != hipSuccess ||
        (e = hipEventCreate(&s.ev0)) != hipSuccess ||
        (e = hipEventCreate(&s.ev1)) != hipSuccess) {
        set_error(DH_ERR_NO_DEVICE, "HIP init failed: %s", hipGetErrorString(e));
        std::fprintf(stderr, "warning: HIP init failed (%s) -- GPU ops unavailable\n",
                     hipGetErrorString(e));
        return;
    }
    s.cus = s.prop.multiProcessorCount;
    s.status = DH_OK;
    std::fprintf(stderr, "[dream] backend: HIP  (device: %s%s%s, %d CUs)\n", s.prop.name,
                 s.prop.name[0] ? ", " : "", s.prop.gcnArchName, s.cus);
}

}  // namespace

int set_error(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

int ensure_init() {
    State& s = st();
    std::call_once(s.once, do_init);
    if (s.status != DH_OK)
        return set_error(DH_ERR_NO_DEVICE, "HIP backend unavailable (no usable device)");
    return DH_OK;
}

hipStream_t stream() {
    State& s = st();
    return s.user_stream ? s.user_stream : s.own_stream;
}

int num_cus() { return st().cus; }

int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(DH_ERR_HIP, "%s launch failed: %s", what,
                                          hipGetErrorString(e));
    return DH_OK;
}

// ---------------------------------------------------------------------------
// Conversion kernels: grid-stride loop, one element per thread per step.
// ---------------------------------------------------------------------------
template <typename S, typename D>
__device__ inline D cvt(S x);
template <> __device__ inline float cvt<double, float>(double x) { return (float)x; }
template <> __device__ inline double cvt<float, double>(float x) { return (double)x; }
template <> __device__ inline uint16_t cvt<double, uint16_t>(double x) {
    return f32_to_bf16_bits((float)x);
}
template <> __device__ inline uint16_t cvt<float, uint16_t>(float x) {
    return f32_to_bf16_bits(x);
}
template <> __device__ inline float cvt<uint16_t, float>(uint16_t x) {
    return bf16_bits_to_f32(x);
}
template <> __device__ inline float cvt<float, float>(float x) { return x; }

template <typename S, typename D>
__global__ void __launch_bounds__(256) convert_kernel(D* __restrict__ dst,
                                                      const S* __restrict__ src, size_t n) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        dst[i] = cvt<S, D>(src[i]);
}

template <typename S, typename D>
int launch_convert(void* dst, const void* src, size_t n) {
    if (n == 0) return DH_OK;
    size_t blocks = (n + 255) / 256;
    const size_t cap = (size_t)num_cus() * 16;
    if (blocks > cap) blocks = cap;
    convert_kernel<S, D><<<(unsigned)blocks, 256, 0, stream()>>>((D*)dst, (const S*)src, n);
    return check_launch("dh_convert");
}

// y += alpha x over n fp32 values (grid-stride).
__global__ void __launch_bounds__(256) axpy_kernel(float* __restrict__ y, const float* __restrict__ x,
                                                   float alpha, size_t n) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
        y[i] += alpha * x[i];
}

}  // namespace dh

using namespace dh;

extern "C" {

int dh_init(void) { return ensure_init(); }

int dh_available(void) { return ensure_init() == DH_OK ? 1 : 0; }

const char* dh_last_error(void) { return g_err; }

int dh_device_info(char* name, int name_len, int* cus, int* xcds, int* sclk_mhz,
                   long long* hbm_bytes) {
    DH_TRY(ensure_init());
    const hipDeviceProp_t& p = st().prop;
    // Some driver stacks leave the marketing name empty (no amdgpu.ids table): name the chip
    // by its architecture and CU count then.
    if (name && name_len > 0) {
        if (p.name[0]) std::snprintf(name, name_len, "%s (%s)", p.name, p.gcnArchName);
        else std::snprintf(name, name_len, "%s, %d CUs", p.gcnArchName, p.multiProcessorCount);
    }
    if (cus) *cus = p.multiProcessorCount;
    if (xcds) *xcds = std::strncmp(p.gcnArchName, "gfx95", 5) == 0 ||
                              std::strncmp(p.gcnArchName, "gfx94", 5) == 0 ? 8 : 1;
    if (sclk_mhz) *sclk_mhz = p.clockRate / 1000;
    if (hbm_bytes) *hbm_bytes = (long long)p.totalGlobalMem;
    return DH_OK;
}

size_t dh_dispatch_threshold(void) {
    // 512 x 512 default; DREAM_GPU_THRESHOLD (elements of M*N) overrides when it parses.
    static size_t cached = [] {
        size_t v = 262144;
        const char* env = std::getenv("DREAM_GPU_THRESHOLD");
        if (env && *env) {
            char* end = nullptr;
            unsigned long long x = std::strtoull(env, &end, 10);
            if (end != env) v = (size_t)x;
        }
        return v;
    }();
    return cached;
}

int dh_matmul_eligible(int M, int N) {
    return (size_t)M * (size_t)N >= dh_dispatch_threshold() ? 1 : 0;
}

int dh_flash_eligible(int B, int S, int dk) {
    return ((size_t)B * S * S >= 262144 && dk <= 128) ? 1 : 0;
}

void* dh_malloc(size_t bytes) {
    if (ensure_init() != DH_OK) return nullptr;
    if (bytes == 0) bytes = 1;
    State& s = st();
    {
        std::lock_guard<std::mutex> g(s.pool_mu);
        auto it = s.free_lists.find(bytes);
        if (it != s.free_lists.end() && !it->second.empty()) {
            void* p = it->second.back();
            it->second.pop_back();
            s.live[p] = bytes;
            return p;
        }
    }
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, bytes);
    if (e != hipSuccess) {
        // One retry after returning the cached buffers to the driver.
        dh_pool_release();
        e = hipMalloc(&p, bytes);
        if (e != hipSuccess) {
            set_error(DH_ERR_OOM, "hipMalloc(%zu) failed: %s", bytes, hipGetErrorString(e));
            return nullptr;
        }
    }
    std::lock_guard<std::mutex> g(s.pool_mu);
    s.live[p] = bytes;
    return p;
}

int dh_free(void* p) {
    if (!p) return DH_OK;
    State& s = st();
    std::lock_guard<std::mutex> g(s.pool_mu);
    auto it = s.live.find(p);
    if (it == s.live.end())
        return set_error(DH_ERR_INVALID, "dh_free: %p was not allocated by dh_malloc", p);
    const size_t bytes = it->second;
    s.live.erase(it);
    auto& v = s.free_lists[bytes];
    if (v.size() < 64) {
        v.push_back(p);
    } else {
        // The buffer may still be read by queued work: wait before handing it back.
        hipStreamSynchronize(stream());
        hipFree(p);
    }
    return DH_OK;
}

int dh_pool_release(void) {
    State& s = st();
    if (s.status != DH_OK) return DH_OK;
    hipDeviceSynchronize();
    std::lock_guard<std::mutex> g(s.pool_mu);
    for (auto& kv : s.free_lists)
        for (void* p : kv.second) hipFree(p);
    s.free_lists.clear();
    for (auto& kv : s.host_free)
        for (void* p : kv.second) hipHostFree(p);
    s.host_free.clear();
    return DH_OK;
}

static int copy(void* dst, const void* src, size_t bytes, hipMemcpyKind kind, const char* what) {
    DH_TRY(ensure_init());
    if (bytes == 0) return DH_OK;
    if (!dst || !src) return set_error(DH_ERR_INVALID, "%s: null pointer", what);
    hipError_t e = hipMemcpyAsync(dst, src, bytes, kind, stream());
    if (e != hipSuccess) return set_error(DH_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
    if (kind == hipMemcpyDeviceToHost) {
        e = hipStreamSynchronize(stream());
        if (e != hipSuccess) return set_error(DH_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
    }
    return DH_OK;
}

int dh_memcpy_h2d(void* d, const void* h, size_t n) {
    return copy(d, h, n, hipMemcpyHostToDevice, "dh_memcpy_h2d");
}
int dh_memcpy_d2h(void* h, const void* d, size_t n) {
    return copy(h, d, n, hipMemcpyDeviceToHost, "dh_memcpy_d2h");
}
void* dh_event_create(void) {
    if (ensure_init() != DH_OK) return nullptr;
    hipEvent_t ev = nullptr;
    hipError_t e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    if (e != hipSuccess) {
        set_error(DH_ERR_HIP, "dh_event_create: %s", hipGetErrorString(e));
        return nullptr;
    }
    return (void*)ev;
}
int dh_event_record(void* ev) {
    DH_TRY(ensure_init());
    if (!ev) return set_error(DH_ERR_INVALID, "dh_event_record: null event");
    hipError_t e = hipEventRecord((hipEvent_t)ev, stream());
    if (e != hipSuccess) return set_error(DH_ERR_HIP, "dh_event_record: %s", hipGetErrorString(e));
    return DH_OK;
}
int dh_event_wait(void* ev) {
    DH_TRY(ensure_init());
    if (!ev) return set_error(DH_ERR_INVALID, "dh_event_wait: null event");
    hipError_t e = hipEventSynchronize((hipEvent_t)ev);
    if (e != hipSuccess) return set_error(DH_ERR_HIP, "dh_event_wait: %s", hipGetErrorString(e));
    return DH_OK;
}
int dh_event_destroy(void* ev) {
    if (!ev) return DH_OK;
    hipError_t e = hipEventDestroy((hipEvent_t)ev);
    if (e != hipSuccess) return set_error(DH_ERR_HIP, "dh_event_destroy: %s", hipGetErrorString(e));
    return DH_OK;
}
int dh_memcpy_d2h_async(void* h, const void* d, size_t n) {
    DH_TRY(ensure_init());
    if (n == 0) return DH_OK;
    if (!h || !d) return set_error(DH_ERR_INVALID, "dh_memcpy_d2h_async: null pointer");
    hipError_t e = hipMemcpyAsync(h, d, n, hipMemcpyDeviceToHost, stream());
    if (e != hipSuccess)
        return set_error(DH_ERR_HIP, "dh_memcpy_d2h_async: %s", hipGetErrorString(e));
    return DH_OK;
}
int dh_memcpy_d2d(void* d, const void* s, size_t n) {
    return copy(d, s, n, hipMemcpyDeviceToDevice, "dh_memcpy_d2d");
}

int dh_memset(void* d, int value, size_t bytes) {
    DH_TRY(ensure_init());
    if (bytes == 0) return DH_OK;
    hipError_t e = hipMemsetAsync(d, value, bytes, stream());
    if (e != hipSuccess) return set_error(DH_ERR_HIP, "dh_memset: %s", hipGetErrorString(e));
    return DH_OK;
}

int dh_sync(void) {
    DH_TRY(ensure_init());
    hipError_t e = hipStreamSynchronize(stream());
    if (e != hipSuccess) return set_error(DH_ERR_HIP, "dh_sync: %s", hipGetErrorString(e));
    return DH_OK;
}

void* dh_get_stream(void) { return ensure_init() == DH_OK ? (void*)stream() : nullptr; }

int dh_set_stream(void* s) {
    DH_TRY(ensure_init());
    st().user_stream = (hipStream_t)s;
    return DH_OK;
}

int dh_timer_start(void) {
    DH_TRY(ensure_init());
    hipError_t e = hipEventRecord(st().ev0, stream());
    if (e != hipSuccess) return set_error(DH_ERR_HIP, "dh_timer_start: %s", hipGetErrorString(e));
    return DH_OK;
}

int dh_timer_stop(float* ms) {
    DH_TRY(ensure_init());
    hipError_t e = hipEventRecord(st().ev1, stream());
    if (e == hipSuccess) e = hipEventSynchronize(st().ev1);
    if (e == hipSuccess) e = hipEventElapsedTime(ms, st().ev0, st().ev1);
    if (e != hipSuccess) return set_error(DH_ERR_HIP, "dh_timer_stop: %s", hipGetErrorString(e));
    return DH_OK;
}

int dh_convert(void* dst, int dt, const void* src, int stype, size_t n) {
    DH_TRY(ensure_init());
    if (n && (!dst || !src)) return set_error(DH_ERR_INVALID, "dh_convert: null pointer");
    if (stype == DH_F64 && dt == DH_F32) return launch_convert<double, float>(dst, src, n);
    if (stype == DH_F32 && dt == DH_F64) return launch_convert<float, double>(dst, src, n);
    if (stype == DH_F64 && dt == DH_BF16) return launch_convert<double, uint16_t>(dst, src, n);
    if (stype == DH_F32 && dt == DH_BF16) return launch_convert<float, uint16_t>(dst, src, n);
    if (stype == DH_BF16 && dt == DH_F32) return launch_convert<uint16_t, float>(dst, src, n);
    if (stype == DH_F32 && dt == DH_F32) return launch_convert<float, float>(dst, src, n);
    return set_error(DH_ERR_UNSUPPORTED, "dh_convert: unsupported pair %d -> %d", stype, dt);
}


int dh_axpy(float* y, const float* x, float alpha, size_t n) {
    DH_TRY(ensure_init());
    if (n == 0) return DH_OK;
    if (!y || !x) return set_error(DH_ERR_INVALID, "dh_axpy: null pointer");
    size_t blocks = (n + 255) / 256;
    const size_t cap = (size_t)num_cus() * 16;
    if (blocks > cap) blocks = cap;
    axpy_kernel<<<(unsigned)blocks, 256, 0, stream()>>>(y, x, alpha, n);
    return check_launch("dh_axpy");
}

// Pinned host memory for staging tensors: hipHostMalloc'd, kept in exact-size buckets (at most
// 16 per size) so repeated tensors of one shape never re-pin.  A returned buffer may still be
// the source or target of queued copies, so the stream is drained before it can be handed out
// again.
void* dh_host_alloc(size_t bytes) {
    if (ensure_init() != DH_OK) return nullptr;
    if (bytes == 0) bytes = 1;
    State& s = st();
    {
        std::lock_guard<std::mutex> g(s.pool_mu);
        auto it = s.host_free.find(bytes);
        if (it != s.host_free.end() && !it->second.empty()) {
            void* p = it->second.back();
            it->second.pop_back();
            s.host_live[p] = bytes;
            return p;
        }
    }
    void* p = nullptr;
    if (hipHostMalloc(&p, bytes, hipHostMallocDefault) != hipSuccess) {
        set_error(DH_ERR_OOM, "hipHostMalloc(%zu) failed", bytes);
        return nullptr;
    }
    std::lock_guard<std::mutex> g(s.pool_mu);
    s.host_live[p] = bytes;
    return p;
}

int dh_host_free(void* p) {
    if (!p) return DH_OK;
    State& s = st();
    hipStreamSynchronize(stream());
    std::lock_guard<std::mutex> g(s.pool_mu);
    auto it = s.host_live.find(p);
    if (it == s.host_live.end())
        return set_error(DH_ERR_INVALID, "dh_host_free: %p was not allocated by dh_host_alloc", p);
    const size_t bytes = it->second;
    s.host_live.erase(it);
    auto& v = s.host_free[bytes];
    if (v.size() < 16) v.push_back(p);
    else hipHostFree(p);
    return DH_OK;
}

}  // extern "C"
