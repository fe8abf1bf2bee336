// dream_rt.cpp -- Dream runtime builtins of the dense-tensor hot path over the HIP C ABI.
//
// Mirrors the reference runtime's builtin interface (names, argument meaning, +1
// ownership, "RUNTIME ERROR in <op>" error behaviour); see include/dream_rt.h.  Every
// GEMM, attention and row-wise computation goes through include/dream_hip.h.
//
// Data model.  Tensors are host fp64 (`data`, `grad`; optionally an fp32 mirror), and
// generated code reads `data` directly, so every GPU result is copied home before the builtin
// returns -- the contract of the reference's GPU branch (HostBuf + cuBLAS/OpenCL,
// runtime/ops/elementwise.inc:1042-1212).  What stays on the device:
//   - `dev`, an fp32 copy of `data` (the result of the op that produced the tensor, or the
//     first upload), reused by every later GPU op while the tensor's `version` is unchanged,
//     so chained ops and the backward pass do not upload their operands again;
//   - `dgrad`, the gradient between GPU ops during backward(): a GPU backward op accumulates
//     into its inputs' device gradients, the next GPU op consumes them in place, and
//     backward() adds every device gradient into the host `grad` before it returns.
#include "../../include/dream_rt.h"

#include <algorithm>
#include <atomic>
#include <condition_variable>
#include <functional>
#include <mutex>
#include <chrono>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <system_error>
#include <thread>
#include <unordered_set>
#include <vector>

#include "../../include/dream_hip.h"

namespace {

bool g_bf16 = false;   // dream_enable_fp16(): reduced-precision `@`

std::mt19937& rng() {
    static std::mt19937 g(std::random_device{}());
    return g;
}

// Host worker threads for par_for, started on first use and kept for the process (creating
// threads per loop cost 10-50 us each, a large part of the short loops of a training step).
// A thread that cannot be created leaves the pool smaller; with none the caller does all.
class HostPool {
public:
    static HostPool& get() {
        static HostPool p;
        return p;
    }
    int workers() const { return (int)th_.size(); }
    // job(k) for k in [0, nk) on the workers and the calling thread; returns when all ran.
    // The job state is guarded by mu_, so a worker that wakes late simply finds no chunk left
    // (or helps with the next job).  Not reentrant: a job must not call run() itself.
    template <typename F>
    void run(size_t nk, const F& job) {
        {
            std::lock_guard<std::mutex> g(mu_);
            job_ = [&job](size_t k) { job(k); };
            nk_ = nk;
            next_ = 0;
            left_.store(nk, std::memory_order_relaxed);
            gen_.fetch_add(1, std::memory_order_release);
        }
        cv_.notify_all();
        work();
        while (left_.load(std::memory_order_acquire) != 0) cpu_relax();
        std::lock_guard<std::mutex> g(mu_);
        job_ = nullptr;
    }

private:
    static void cpu_relax() { __builtin_ia32_pause(); }
    HostPool() {
        const unsigned hw = std::thread::hardware_concurrency();
        const unsigned n = std::min(hw ? hw : 1u, 16u) - 1;
        for (unsigned k = 0; k < n; ++k) {
            try {
                th_.emplace_back([this] { loop(); });
            } catch (const std::system_error&) {
                break;
            }
        }
    }
    ~HostPool() {
        {
            std::lock_guard<std::mutex> g(mu_);
            stop_ = true;
            gen_.fetch_add(1, std::memory_order_release);
        }
        cv_.notify_all();
        for (auto& t : th_) t.join();
    }
    void work() {   // claim chunks until none is left
        for (;;) {
            std::function<void(size_t)>* job;
            size_t k;
            {
                std::lock_guard<std::mutex> g(mu_);
                if (next_ >= nk_) return;
                k = next_++;
                job = &job_;
            }
            (*job)(k);   // job_ stays set until every claimed chunk is done (left_ == 0)
            left_.fetch_sub(1, std::memory_order_acq_rel);
        }
    }
    void loop() {
        uint64_t seen = 0;
        for (;;) {
            // A training step issues many short loops back to back: spin for ~100 us before
            // sleeping, so the next one does not wait for a wake-up.
            const auto t0 = std::chrono::steady_clock::now();
            for (int it = 0; gen_.load(std::memory_order_acquire) == seen; ++it) {
                cpu_relax();
                if ((it & 255) == 255 &&
                    std::chrono::steady_clock::now() - t0 > std::chrono::microseconds(100)) {
                    std::unique_lock<std::mutex> lk(mu_);
                    cv_.wait(lk, [&] { return gen_.load(std::memory_order_acquire) != seen; });
                }
            }
            seen = gen_.load(std::memory_order_acquire);
            {
                std::lock_guard<std::mutex> g(mu_);
                if (stop_) return;
            }
            work();
        }
    }
    std::mutex mu_;
    std::condition_variable cv_;
    std::vector<std::thread> th_;
    std::function<void(size_t)> job_;
    size_t nk_ = 0, next_ = 0;
    std::atomic<size_t> left_{0};
    std::atomic<uint64_t> gen_{0};
    bool stop_ = false;
};

// body(i0, i1) over [0, n) in chunks on the host pool (up to 16 threads), for host loops
// over large tensors whose iterations are independent (each writes only its own elements),
// so the result does not depend on the split.  Small ranges run inline.
template <typename F>
void par_for(size_t n, F body) {
    constexpr size_t kMin = size_t(1) << 18;
    const size_t nt = std::min<size_t>(n / kMin, 16);
    if (nt <= 1 || HostPool::get().workers() == 0) {
        body(size_t(0), n);
        return;
    }
    const size_t chunks = nt * 2;   // a little slack for uneven thread start
    const size_t step = (n + chunks - 1) / chunks;
    HostPool::get().run(chunks, [&](size_t k) {
        const size_t i0 = std::min(n, k * step), i1 = std::min(n, (k + 1) * step);
        if (i0 < i1) body(i0, i1);
    });
}

void rt_error(const char* op, const char* fmt, ...) {
    std::fprintf(stderr, "RUNTIME ERROR in %s: ", op);
    va_list ap;
    va_start(ap, fmt);
    std::vfprintf(stderr, fmt, ap);
    va_end(ap);
    std::fprintf(stderr, "\n");
    std::fflush(stderr);
}

// DREAM_TRACE=1: host-side time between trace points inside the builtins, on stderr (where
// the time of a builtin goes besides its kernels and copies).
bool trace_on() {
    static const bool on = [] {
        const char* e = std::getenv("DREAM_TRACE");
        return e && *e && *e != '0';
    }();
    return on;
}
void tpoint(const char* what) {
    if (!trace_on()) return;
    static auto last = std::chrono::steady_clock::now();
    const auto now = std::chrono::steady_clock::now();
    std::fprintf(stderr, "[trace] %-24s %9.1f us\n", what,
                 std::chrono::duration<double, std::micro>(now - last).count());
    last = now;
}

// Device buffer from the backend pool, returned on scope exit unless released.
struct Dev {
    void* p = nullptr;
    explicit Dev(size_t bytes) : p(dh_malloc(bytes ? bytes : 1)) {}
    ~Dev() { if (p) dh_free(p); }
    Dev(const Dev&) = delete;
    Dev& operator=(const Dev&) = delete;
    bool ok() const { return p != nullptr; }
    float* f() const { return static_cast<float*>(p); }
    double* d() const { return static_cast<double*>(p); }
    uint16_t* h() const { return static_cast<uint16_t*>(p); }
    void* release() { void* q = p; p = nullptr; return q; }
};

struct Failure {};   // thrown internally by need(), caught at the builtin boundary

void need(int status) {
    if (status != DH_OK) throw Failure{};
}
void need_buf(const Dev& d) {
    if (!d.ok()) throw Failure{};
}

Tensor* incref(Tensor* t) {
    if (t) ++t->refcount;
    return t;
}

bool hip_ready(const char* op) {
    if (dh_available()) return true;
    rt_error(op, "HIP backend unavailable (%s)", dh_last_error());
    return false;
}

// ---- host buffers ----------------------------------------------------------------------
// Tensor buffers of 1 MB and more live in pinned host memory from the backend's pool, so the
// copies to and from the device run at full PCIe rate; smaller ones are plain calloc.  zero =
// false is only for outputs the device result overwrites entirely.
constexpr size_t PIN_MIN_BYTES = 1u << 20;

double* host_buffer(size_t n, bool zero, bool& pinned) {
    const size_t bytes = n * sizeof(double);
    pinned = false;
    if (bytes >= PIN_MIN_BYTES && dh_available()) {
        if (void* p = dh_host_alloc(bytes)) {
            if (zero) {
                double* d = static_cast<double*>(p);
                par_for(n, [=](size_t i0, size_t i1) { std::fill(d + i0, d + i1, 0.0); });
            }
            pinned = true;
            return static_cast<double*>(p);
        }
    }
    return static_cast<double*>(std::calloc(n, sizeof(double)));
}

void release_host(double* p, bool pinned) {
    if (pinned) dh_host_free(p);
    else std::free(p);
}

Tensor* new_tensor(int d0, int d1, int d2, int d3, bool zero_data);
Tensor* alloc_result(int d0, int d1, int d2, int d3);

// ---- transfers ---------------------------------------------------------------------------
// Every value crossing PCIe in fp32 form goes as fp32 (half the bytes of fp64): fp64 host
// values are rounded to fp32 on the host threads (the same round-to-nearest-even as the
// device conversion) into pinned staging memory and uploaded; fp32 device values come home
// into pinned staging and are widened (exactly) on the host threads.
struct Stage {   // pinned host staging of n floats from the backend's pool (else plain memory)
    float* p = nullptr;
    bool pinned = false;
    explicit Stage(size_t n) {
        // pinned at every size: a copy to or from pageable memory is staged synchronously by
        // the HIP runtime (~0.1 ms even for a few KB)
        p = static_cast<float*>(dh_host_alloc(std::max<size_t>(n, 1) * sizeof(float)));
        pinned = p != nullptr;
        if (!p) p = static_cast<float*>(std::malloc(std::max<size_t>(n, 1) * sizeof(float)));
        if (!p) throw Failure{};
    }
    ~Stage() {
        if (pinned) dh_host_free(p);
        else std::free(p);
    }
    Stage(const Stage&) = delete;
    Stage& operator=(const Stage&) = delete;
};

// device fp32 dst[0..n) = (float) host src[0..n)
void upload_as_f32(float* dst, const double* src, size_t n) {
    Stage st(n);
    float* sp = st.p;
    par_for(n, [=](size_t i0, size_t i1) {
        for (size_t i = i0; i < i1; ++i) sp[i] = (float)src[i];
    });
    need(dh_memcpy_h2d(dst, sp, n * sizeof(float)));
    need(dh_sync());   // the copy reads the staging memory asynchronously
}

// Events on the library stream, created once and reused (mark where one copy of several
// ends, so the host can widen it while the later ones are still in flight).
void* copy_event(size_t k) {
    static std::vector<void*> evs;
    while (evs.size() <= k) {
        void* e = dh_event_create();
        if (!e) throw Failure{};
        evs.push_back(e);
    }
    return evs[k];
}

// host dst[i] = (or +=) (double) src[i] for i in [i0, i1), on the host pool
void widen(double* dst, const float* src, size_t n, bool add) {
    if (add) {
        par_for(n, [=](size_t i0, size_t i1) {
            for (size_t i = i0; i < i1; ++i) dst[i] += (double)src[i];
        });
    } else {
        par_for(n, [=](size_t i0, size_t i1) {
            for (size_t i = i0; i < i1; ++i) dst[i] = (double)src[i];
        });
    }
}

// host dst[0..n) = (or +=) (double) device fp32 src[0..n).  The copy comes home in chunks
// of 32 MB, each widened on the host pool while the next ones are still being copied.
void download_f32(double* dst, const float* src, size_t n, bool add) {
    constexpr size_t kChunk = size_t(1) << 23;
    tpoint("download: entry");
    Stage st(n);
    tpoint("download: stage");
    const size_t nch = (n + kChunk - 1) / kChunk;
    for (size_t c = 0; c < nch; ++c) {
        const size_t off = c * kChunk, len = std::min(kChunk, n - off);
        need(dh_memcpy_d2h_async(st.p + off, src + off, len * sizeof(float)));
        need(dh_event_record(copy_event(c)));
    }
    tpoint("download: queued");
    for (size_t c = 0; c < nch; ++c) {
        const size_t off = c * kChunk, len = std::min(kChunk, n - off);
        need(dh_event_wait(copy_event(c)));
        tpoint("download: waited");
        widen(dst + off, st.p + off, len, add);
        tpoint("download: widened");
    }
}

// ---- device residency ------------------------------------------------------------------
// fp32 device copy of t->data (t->size values), uploaded only when there is none or `data`
// changed since (version).
const float* dev_data(Tensor* t) {
    if (t->dev && t->dev_version == t->version) return t->dev;
    const size_t n = (size_t)t->size;
    if (!t->dev) {
        t->dev = static_cast<float*>(dh_malloc(n * sizeof(float)));
        if (!t->dev) throw Failure{};
    }
    upload_as_f32(t->dev, t->data, n);
    t->dev_version = t->version;
    t->dev_exact = 0;
    return t->dev;
}

// fp64 device copy of t->data for the fp64 elementwise kernels: kept while `version` does
// not change; rebuilt on the device from the fp32 copy when data is exactly that copy
// widened (a GPU result), else uploaded.
const double* dev_data64(Tensor* t) {
    if (t->dev64 && t->dev64_version == t->version) return t->dev64;
    const size_t n = (size_t)t->size;
    if (!t->dev64) {
        t->dev64 = static_cast<double*>(dh_malloc(n * sizeof(double)));
        if (!t->dev64) throw Failure{};
    }
    if (t->dev && t->dev_version == t->version && t->dev_exact)
        need(dh_convert(t->dev64, DH_F64, t->dev, DH_F32, n));
    else
        need(dh_memcpy_h2d(t->dev64, t->data, n * sizeof(double)));
    t->dev64_version = t->version;
    return t->dev64;
}

// A device fp32 result holding t's values becomes t's device copy, and is copied home.
void adopt_result(Tensor* t, Dev& d) {
    const size_t n = (size_t)t->size;
    download_f32(t->data, d.f(), n, false);
    if (t->dev) dh_free(t->dev);
    t->dev = static_cast<float*>(d.release());
    t->dev_version = t->version;
    t->dev_exact = 1;
}

// bf16 operand built on the device from the fp32 copy (round to nearest even, the rule of
// dream_to_bf16, runtime/nn/training.inc:1969-1976).
void dev_bf16(Tensor* t, size_t n, Dev& out) {
    need(dh_convert(out.p, DH_BF16, dev_data(t), DH_F32, n));
}

// Device gradient accumulator of t (zero on first use).
float* dgrad(Tensor* t) {
    if (!t->dgrad) {
        const size_t bytes = (size_t)t->size * sizeof(float);
        t->dgrad = static_cast<float*>(dh_malloc(bytes));
        if (!t->dgrad) throw Failure{};
        need(dh_memset(t->dgrad, 0, bytes));
    }
    return t->dgrad;
}

// The complete incoming gradient of node t for a GPU backward op (every consumer of t has
// run), as a device fp32 buffer.  t->dgrad holds only device contributions and the host part
// stays in t->grad (fp64, as the reference keeps it); when there is a host part it is
// uploaded and, if t->dgrad exists too, added to a copy of it, and the final flush adds
// t->dgrad into the host part.  An op that rewrites the gradient in place (linear_relu's
// mask, which the reference applies to the node's own gradient) gets t->dgrad holding the
// whole gradient instead: the host part is moved over and cleared, and the flush writes the
// rewritten values back.
struct GradIn {
    Dev tmp{0};
    float* p = nullptr;
    GradIn(Tensor* t, bool in_place) {
        const size_t n = (size_t)t->size;
        if (t->grad_zero) {
            p = dgrad(t);
            return;
        }
        if (in_place) {
            p = dgrad(t);
            Dev f(n * sizeof(float));
            need_buf(f);
            upload_as_f32(f.f(), t->grad, n);
            need(dh_axpy(p, f.f(), 1.f, n));
            double* hg = t->grad;
            par_for(n, [=](size_t i0, size_t i1) { std::fill(hg + i0, hg + i1, 0.0); });
            t->grad_zero = 1;
            return;
        }
        Dev f(n * sizeof(float));
        need_buf(f);
        upload_as_f32(f.f(), t->grad, n);
        if (t->dgrad) need(dh_axpy(f.f(), t->dgrad, 1.f, n));
        p = f.f();
        std::swap(tmp.p, f.p);
    }
};

// Host grad += device grad, and the device grad is released (also makes t->grad complete for
// a host backward op).
void flush_dgrad(Tensor* t) {
    if (!t->dgrad) return;
    // host grad all zero: the widened device gradient is the result, else it is added
    download_f32(t->grad, t->dgrad, (size_t)t->size, !t->grad_zero);
    dh_free(t->dgrad);
    t->dgrad = nullptr;
    t->grad_zero = 0;
}

// flush_dgrad for every tensor of `order` holding a device gradient: all copies queued
// into one pinned staging buffer, each tensor widened (or added) on the host pool as soon as
// its own copy has landed, while the later copies are still in flight.
void flush_all(const std::vector<Tensor*>& order) {
    std::vector<Tensor*> fl;
    size_t total = 0;
    for (Tensor* t : order)
        if (t->dgrad) {
            fl.push_back(t);
            total += (size_t)t->size;
        }
    if (fl.empty()) return;
    Stage st(total);
    size_t off = 0;
    for (size_t k = 0; k < fl.size(); ++k) {
        need(dh_memcpy_d2h_async(st.p + off, fl[k]->dgrad, (size_t)fl[k]->size * sizeof(float)));
        need(dh_event_record(copy_event(k)));
        off += (size_t)fl[k]->size;
    }
    off = 0;
    for (size_t k = 0; k < fl.size(); ++k) {
        Tensor* t = fl[k];
        const size_t n = (size_t)t->size;
        need(dh_event_wait(copy_event(k)));
        widen(t->grad, st.p + off, n, !t->grad_zero);
        off += n;
        dh_free(t->dgrad);
        t->dgrad = nullptr;
        t->grad_zero = 0;
    }
}

void drop_device(Tensor* t) {
    if (t->dev) dh_free(t->dev);
    if (t->dgrad) dh_free(t->dgrad);
    if (t->dlse) dh_free(t->dlse);
    if (t->dev64) dh_free(t->dev64);
    t->dev = t->dgrad = t->dlse = nullptr;
    t->dev64 = nullptr;
}

void set_graph(Tensor* c, Tensor* l, Tensor* r, int op) {
    c->is_leaf = 0;
    c->op = op;
    c->lhs = incref(l);
    c->rhs = incref(r);
}

void set_parents(Tensor* c, Tensor* a, Tensor* b, Tensor* d) {
    c->parents[0] = incref(a);
    c->parents[1] = incref(b);
    c->parents[2] = incref(d);
    c->num_parents = 3;
}

int padded_dim(int dk) { return dk <= 32 ? 32 : dk <= 64 ? 64 : dk <= 128 ? 128 : -1; }

// (B*S, dk) fp64 rows -> (B*S, Dp) rows with zero padding, on the device as dt.
void upload_rows(const double* h, size_t rows, int dk, int Dp, int dt, const Dev& out) {
    std::vector<float> buf(rows * Dp, 0.f);
    for (size_t r = 0; r < rows; ++r)
        for (int k = 0; k < dk; ++k) buf[r * Dp + k] = (float)h[r * dk + k];
    if (dt == DH_F32) {
        need(dh_memcpy_h2d(out.p, buf.data(), buf.size() * sizeof(float)));
    } else {
        Dev tmp(buf.size() * sizeof(float));
        need_buf(tmp);
        need(dh_memcpy_h2d(tmp.p, buf.data(), buf.size() * sizeof(float)));
        need(dh_convert(out.p, dt, tmp.p, DH_F32, buf.size()));
    }
}

std::vector<float> download_rows_f32(const void* d, size_t rows, int Dp, int dt) {
    std::vector<float> buf(rows * Dp);
    if (dt == DH_F32) {
        need(dh_memcpy_d2h(buf.data(), d, buf.size() * sizeof(float)));
    } else {
        Dev tmp(buf.size() * sizeof(float));
        need_buf(tmp);
        need(dh_convert(tmp.p, DH_F32, d, dt, buf.size()));
        need(dh_memcpy_d2h(buf.data(), tmp.p, buf.size() * sizeof(float)));
    }
    return buf;
}

// ---- fp64 ----------------------------------------------------------------------------------
// The shapes the reference computes in fp64 (below its GPU thresholds) run on the fp64
// kernels from the host fp64 values, uploaded afresh on every call: these are the small
// products, and a fresh upload also sees a direct write through `data` that did not bump
// `version` (the reference's gradcheck perturbs leaves that way, training.inc:3886-3890).
void upload_f64(const double* h, size_t n, Dev& d) {
    need_buf(d);
    need(dh_memcpy_h2d(d.p, h, n * sizeof(double)));
}

// Host grad += the device fp64 gradient g (n values).
void add_grad_f64(Tensor* t, const Dev& g, size_t n) {
    std::vector<double> h(n);
    need(dh_memcpy_d2h(h.data(), g.p, n * sizeof(double)));
    for (size_t i = 0; i < n; ++i) t->grad[i] += h[i];
    t->grad_zero = 0;
}

// ---- attention ---------------------------------------------------------------------------
// Shapes under the reference's GPU rule (B*S*S >= 262144, dk <= 128) run on the FlashAttention
// kernels: head dims 32 / 64 / 128 on the tensors' device copies directly, other dk zero-padded
// to the next kernel size on the host (zero columns of Q, K leave Q K^T unchanged; zero columns
// of V give zero columns of O; the scale stays 1/sqrt(dk)).  Every other shape runs in fp64
// (dh_attention_f64_fwd), as the reference computes it.
Tensor* attention_impl(const char* name, int op, bool causal, Tensor* Q, Tensor* K, Tensor* V,
                       Tensor* bt, Tensor* st, Tensor* dt_) {
    if (!Q || !K || !V || !bt || !st || !dt_) return create_scalar(0.0);
    const int B = (int)bt->data[0], S = (int)st->data[0], dk = (int)dt_->data[0];
    if (B <= 0 || S <= 0 || dk <= 0 || Q->size != B * S * dk || K->size != Q->size ||
        V->size != Q->size) {
        rt_error(name, "Q/K/V must hold batch*seq*dk = %d*%d*%d values (got %d, %d, %d)", B, S,
                 dk, Q->size, K->size, V->size);
        return alloc_tensor(1, 1, 1, 1);
    }
    if (!hip_ready(name)) return alloc_tensor(1, 1, 1, 1);
    Tensor* out = alloc_result(B, S * dk, 1, 1);
    out->is_leaf = 0;
    out->op = op;
    set_parents(out, Q, K, V);
    out->attn_B = B;
    out->attn_S = S;
    out->attn_dk = dk;
    const size_t rows = (size_t)B * S, n = rows * dk;
    if (!dh_flash_eligible(B, S, dk)) {
        try {
            Dev q(n * 8), k(n * 8), v(n * 8), o(n * 8);
            upload_f64(Q->data, n, q);
            upload_f64(K->data, n, k);
            upload_f64(V->data, n, v);
            need_buf(o);
            need(dh_attention_f64_fwd(B, S, dk, 1.0 / std::sqrt((double)dk), causal ? 1 : 0,
                                      q.d(), k.d(), v.d(), o.d()));
            need(dh_memcpy_d2h(out->data, o.p, n * sizeof(double)));
            out->f64_node = 1;
        } catch (const Failure&) {
            rt_error(name, "%s", dh_last_error());
            tensor_decref(out);
            return alloc_tensor(1, 1, 1, 1);
        }
        return out;
    }
    const int Dp = padded_dim(dk);
    const int dt = g_bf16 ? DH_BF16 : DH_F32;
    const size_t esz = dt == DH_BF16 ? 2 : 4;
    const float scale = (float)(1.0 / std::sqrt((double)dk));
    try {
        Dev lse(rows * sizeof(float));
        need_buf(lse);
        if (Dp == dk) {
            Dev o(n * sizeof(float));
            need_buf(o);
            if (dt == DH_F32) {
                need(dh_flash_fwd(dt, B, S, dk, scale, causal ? 1 : 0, dev_data(Q), dev_data(K),
                                  dev_data(V), o.p, lse.f()));
            } else {
                Dev q(n * 2), k(n * 2), v(n * 2), ob(n * 2);
                need_buf(q), need_buf(k), need_buf(v), need_buf(ob);
                dev_bf16(Q, n, q);
                dev_bf16(K, n, k);
                dev_bf16(V, n, v);
                need(dh_flash_fwd(dt, B, S, dk, scale, causal ? 1 : 0, q.p, k.p, v.p, ob.p,
                                  lse.f()));
                need(dh_convert(o.p, DH_F32, ob.p, DH_BF16, n));
            }
            adopt_result(out, o);
        } else {
            Dev q(rows * Dp * esz), k(rows * Dp * esz), v(rows * Dp * esz), o(rows * Dp * esz);
            need_buf(q), need_buf(k), need_buf(v), need_buf(o);
            upload_rows(Q->data, rows, dk, Dp, dt, q);
            upload_rows(K->data, rows, dk, Dp, dt, k);
            upload_rows(V->data, rows, dk, Dp, dt, v);
            need(dh_flash_fwd(dt, B, S, Dp, scale, causal ? 1 : 0, q.p, k.p, v.p, o.p, lse.f()));
            std::vector<float> ob = download_rows_f32(o.p, rows, Dp, dt);
            for (size_t r = 0; r < rows; ++r)
                for (int c = 0; c < dk; ++c) out->data[r * dk + c] = (double)ob[r * Dp + c];
        }
        out->dlse = static_cast<float*>(lse.release());
    } catch (const Failure&) {
        rt_error(name, "%s", dh_last_error());
        tensor_decref(out);
        return alloc_tensor(1, 1, 1, 1);
    }
    return out;
}

void attention_backward(Tensor* t, bool causal) {
    Tensor *Q = t->parents[0], *K = t->parents[1], *V = t->parents[2];
    const int B = t->attn_B, S = t->attn_S, dk = t->attn_dk, Dp = padded_dim(dk);
    const size_t rows = (size_t)B * S, n = rows * dk;
    if (t->f64_node) {
        // fp64 forward: the fp64 backward (autograd.inc:675-778) from the host values, into
        // separate device gradients added to the host grads one by one (Q, K, V may be one
        // tensor, which then receives the sum, as the reference's "+=" leaves it).
        flush_dgrad(t);
        Dev q(n * 8), k(n * 8), v(n * 8), g(n * 8), dq(n * 8), dkk(n * 8), dv(n * 8);
        upload_f64(Q->data, n, q);
        upload_f64(K->data, n, k);
        upload_f64(V->data, n, v);
        upload_f64(t->grad, n, g);
        need_buf(dq), need_buf(dkk), need_buf(dv);
        need(dh_attention_f64_bwd(B, S, dk, 1.0 / std::sqrt((double)dk), causal ? 1 : 0, q.d(),
                                  k.d(), v.d(), g.d(), dq.d(), dkk.d(), dv.d(), 0));
        add_grad_f64(Q, dq, n);
        add_grad_f64(K, dkk, n);
        add_grad_f64(V, dv, n);
        return;
    }
    const int dt = g_bf16 ? DH_BF16 : DH_F32;
    const float scale = (float)(1.0 / std::sqrt((double)dk));
    if (Dp == dk) {
        // dO, O, Q, K, V as device copies; dQ, dK, dV accumulate into the device gradients.
        GradIn gi(t, false);
        const float* g = gi.p;
        if (dt == DH_F32) {
            need(dh_flash_bwd(dt, B, S, dk, scale, causal ? 1 : 0, dev_data(Q), dev_data(K),
                              dev_data(V), dev_data(t), g, t->dlse, dgrad(Q), dgrad(K), dgrad(V),
                              1));
        } else {
            Dev q(n * 2), k(n * 2), v(n * 2), o(n * 2), gb(n * 2);
            need_buf(q), need_buf(k), need_buf(v), need_buf(o), need_buf(gb);
            dev_bf16(Q, n, q);
            dev_bf16(K, n, k);
            dev_bf16(V, n, v);
            dev_bf16(t, n, o);
            need(dh_convert(gb.p, DH_BF16, g, DH_F32, n));
            need(dh_flash_bwd(dt, B, S, dk, scale, causal ? 1 : 0, q.p, k.p, v.p, o.p, gb.p,
                              t->dlse, dgrad(Q), dgrad(K), dgrad(V), 1));
        }
        return;
    }
    flush_dgrad(t);
    const size_t esz = dt == DH_BF16 ? 2 : 4;
    Dev q(rows * Dp * esz), k(rows * Dp * esz), v(rows * Dp * esz), o(rows * Dp * esz),
        g(rows * Dp * esz), dq(rows * Dp * 4), dkk(rows * Dp * 4), dv(rows * Dp * 4);
    need_buf(q), need_buf(k), need_buf(v), need_buf(o), need_buf(g), need_buf(dq), need_buf(dkk),
        need_buf(dv);
    upload_rows(Q->data, rows, dk, Dp, dt, q);
    upload_rows(K->data, rows, dk, Dp, dt, k);
    upload_rows(V->data, rows, dk, Dp, dt, v);
    upload_rows(t->data, rows, dk, Dp, dt, o);
    upload_rows(t->grad, rows, dk, Dp, dt, g);
    need(dh_flash_bwd(dt, B, S, Dp, scale, causal ? 1 : 0, q.p, k.p, v.p, o.p, g.p, t->dlse,
                      dq.f(), dkk.f(), dv.f(), 0));
    Tensor* dst[3] = {Q, K, V};
    const Dev* src[3] = {&dq, &dkk, &dv};
    for (int x = 0; x < 3; ++x) {
        flush_dgrad(dst[x]);
        std::vector<float> h = download_rows_f32(src[x]->p, rows, Dp, DH_F32);
        for (size_t r = 0; r < rows; ++r)
            for (int c = 0; c < dk; ++c) dst[x]->grad[r * dk + c] += (double)h[r * Dp + c];
        dst[x]->grad_zero = 0;
    }
}

// ---- GEMM-family backward ------------------------------------------------------------------
void matmul_backward(Tensor* t) {
    // dA += dY B^T (NT), dB += A^T dY (TN) (runtime/ops/autograd.inc:91-125): in fp64 from the
    // host values when the forward ran in fp64, else in fp32 on the device copies.
    Tensor *A = t->lhs, *B = t->rhs;
    const int M = A->d0, K = A->d1, N = B->d1;
    if (t->f64_node) {
        flush_dgrad(t);
        const size_t mk = (size_t)M * K, kn = (size_t)K * N, mn = (size_t)M * N;
        Dev a(mk * 8), b(kn * 8), g(mn * 8), da(mk * 8), db(kn * 8);
        upload_f64(A->data, mk, a);
        upload_f64(B->data, kn, b);
        upload_f64(t->grad, mn, g);
        need_buf(da), need_buf(db);
        need(dh_gemm_f64(0, 1, M, K, N, g.d(), N, b.d(), N, 0.0, da.d(), K));
        need(dh_gemm_f64(1, 0, K, N, M, a.d(), K, g.d(), N, 0.0, db.d(), N));
        add_grad_f64(A, da, mk);
        add_grad_f64(B, db, kn);
        return;
    }
    GradIn gi(t, false);
    const float* dy = gi.p;
    need(dh_gemm_f32(0, 1, M, K, N, dy, N, dev_data(B), N, 1.f, dgrad(A), K));
    need(dh_gemm_f32(1, 0, K, N, M, dev_data(A), K, dy, N, 1.f, dgrad(B), N));
}

void linear_backward(Tensor* t, bool relu) {
    // autograd.inc:156-205: (linear_relu) dY <- 0 where Y <= 0, in place; db += colsum(dY);
    // dX += dY W (NN); dW += dY^T X (TN).
    Tensor *x = t->parents[0], *W = t->parents[1], *b = t->parents[2];
    const int N = x->d0, in = x->d1, out = W->d0;
    GradIn gi(t, relu);   // linear_relu masks its node's gradient in place
    float* dy = gi.p;
    need(dh_linear_bias_grad(relu ? dev_data(t) : nullptr, dy, dgrad(b), N, out, relu ? 1 : 0, 1));
    need(dh_gemm_f32(0, 0, N, in, out, dy, out, dev_data(W), in, 1.f, dgrad(x), in));
    need(dh_gemm_f32(1, 0, out, in, N, dy, out, dev_data(x), in, 1.f, dgrad(W), in));
}

void bmm_backward(Tensor* t) {
    // autograd.inc:549-574: gA += G B^T, gB += A^T G per batch member.
    Tensor *a = t->lhs, *b = t->rhs;
    const int Bt = t->bmm_B, M = t->bmm_M, K = t->bmm_K, N = t->bmm_N;
    GradIn gi(t, false);
    const float* g = gi.p;
    need(dh_gemm_f32_ex(0, 1, M, K, N, g, N, (long long)M * N, dev_data(b), N, (long long)K * N,
                        1.f, dgrad(a), K, (long long)M * K, Bt, nullptr, 0));
    need(dh_gemm_f32_ex(1, 0, K, N, M, dev_data(a), K, (long long)M * K, g, N, (long long)M * N,
                        1.f, dgrad(b), N, (long long)K * N, Bt, nullptr, 0));
}

// Rows of the row-wise ops: softmax / layer norm take d0 rows of size/d0 (elementwise.inc:
// 346-347, builtins.inc:174-175), log_softmax d0 rows of d1 (elementwise.inc:1556).
void row_shape(const Tensor* t, int op, int& R, int& C) {
    if (op == DREAM_OP_LOG_SOFTMAX) {
        R = t->d0;
        C = t->d1;
    } else {
        R = t->d0 > 0 ? t->d0 : 1;
        C = t->size / R;
    }
}

void row_backward(Tensor* t) {
    Tensor* x = t->lhs;
    int R, C;
    row_shape(x, t->op, R, C);
    GradIn gi(t, false);
    const float* g = gi.p;
    if (t->op == DREAM_OP_LAYER_NORM)
        need(dh_layer_norm_bwd(dev_data(x), dev_data(t), g, dgrad(x), R, C, 1));
    else
        need(dh_row_softmax_bwd(dev_data(t), g, dgrad(x), R, C,
                                t->op == DREAM_OP_LOG_SOFTMAX ? 1 : 0, 1));
}

Tensor* row_op(const char* name, int op, Tensor* x) {
    if (!x) return create_scalar(0.0);
    int R, C;
    row_shape(x, op, R, C);
    if (!hip_ready(name)) return alloc_tensor(1, 1, 1, 1);
    Tensor* y = op == DREAM_OP_LOG_SOFTMAX ? alloc_result(x->d0, x->d1, 1, 1)
                                           : alloc_result(x->d0, x->d1, x->d2, x->d3);
    set_graph(y, x, nullptr, op);
    try {
        Dev d((size_t)y->size * sizeof(float));
        need_buf(d);
        if ((size_t)R * C < (size_t)y->size) need(dh_memset(d.p, 0, (size_t)y->size * sizeof(float)));
        if (op == DREAM_OP_LAYER_NORM)
            need(dh_layer_norm(dev_data(x), d.f(), R, C));
        else
            need(dh_row_softmax(dev_data(x), d.f(), R, C, op == DREAM_OP_LOG_SOFTMAX ? 1 : 0));
        adopt_result(y, d);
    } catch (const Failure&) {
        rt_error(name, "%s", dh_last_error());
        tensor_decref(y);
        return alloc_tensor(1, 1, 1, 1);
    }
    return y;
}

// ---- conv2d -------------------------------------------------------------------------------
struct ConvDims {
    int N, Cin, H, W, Cout, KH, KW, pad, stride, OH, OW;
    size_t K() const { return (size_t)Cin * KH * KW; }
    size_t P() const { return (size_t)OH * OW; }
};

ConvDims conv_dims(const Tensor* t) {
    const int* c = t->conv;
    ConvDims d{t->lhs->d0, c[4], c[0], c[1], c[5], c[2], c[3], c[6], c[7], 0, 0};
    d.OH = (d.H + 2 * d.pad - d.KH) / d.stride + 1;
    d.OW = (d.W + 2 * d.pad - d.KW) / d.stride + 1;
    return d;
}

void conv_backward(Tensor* t) {
    // autograd.inc:507-535 over all images at once: gK += sum_n go_n col_n^T as one implicit
    // GEMM (dh_conv2d_bwd_filter, col gathered in the loader); gX += col2im(K^T go'), which for
    // stride 1 (pad < kernel size) is one implicit-GEMM convolution of go with the flipped
    // kernel (dh_conv2d_bwd_data) and otherwise a TN GEMM into dcol + col2im (go' = the
    // gradient channel-first).
    const ConvDims d = conv_dims(t);
    Tensor *x = t->lhs, *k = t->rhs;
    const size_t K = d.K(), NP = (size_t)d.N * d.P();
    GradIn gi(t, false);
    const float* go = gi.p;
    need(dh_conv2d_bwd_filter(go, dev_data(x), dgrad(k), d.N, d.Cin, d.H, d.W, d.Cout, d.KH,
                              d.KW, d.pad, d.stride, 1));
    if (d.stride == 1 && d.pad <= d.KH - 1 && d.pad <= d.KW - 1) {
        need(dh_conv2d_bwd_data(go, dev_data(k), dgrad(x), d.N, d.Cin, d.H, d.W, d.Cout, d.KH,
                                d.KW, d.pad, 1, 1));
        return;
    }
    Dev gop((size_t)d.Cout * NP * 4), dcol(K * NP * 4);
    need_buf(gop), need_buf(dcol);
    need(dh_nct_to_cnt(go, gop.f(), d.N, d.Cout, d.P()));
    need(dh_gemm_f32(1, 0, (int)K, (int)NP, d.Cout, dev_data(k), (int)K, gop.f(), (int)NP, 0.f,
                     dcol.f(), (int)NP));
    need(dh_col2im(dcol.f(), dgrad(x), d.N, d.Cin, d.H, d.W, d.KH, d.KW, d.pad, d.stride, 1));
}

// Elementwise backward branches on the host, as in the reference (autograd.inc:58-90 with
// operands indexed j % size, not by the forward's broadcast strides; pow 491-506 over the
// base's elements).
void binary_backward(Tensor* t) {
    Tensor *A = t->lhs, *B = t->rhs;
    const int na = A->size, nb = B->size, n = t->size;
    const double *a = A->data, *b = B->data, *g = t->grad;
    double *ga = A->grad, *gb = B->grad;
    switch (t->op) {
        case DREAM_OP_ADD:
            for (int j = 0; j < n; ++j) ga[j % na] += g[j], gb[j % nb] += g[j];
            break;
        case DREAM_OP_SUB:
            for (int j = 0; j < n; ++j) ga[j % na] += g[j], gb[j % nb] -= g[j];
            break;
        case DREAM_OP_DIV:
            for (int j = 0; j < n; ++j) {
                const double r = b[j % nb];
                ga[j % na] += g[j] / r;
                gb[j % nb] -= g[j] * a[j % na] / (r * r);
            }
            break;
        case DREAM_OP_MINIMUM:
        case DREAM_OP_MAXIMUM: {
            const bool is_max = t->op == DREAM_OP_MAXIMUM;
            for (int j = 0; j < n; ++j) {   // ties go to the left operand
                const double av = a[j % na], bv = b[j % nb];
                if (is_max ? av >= bv : av <= bv) ga[j % na] += g[j];
                else gb[j % nb] += g[j];
            }
            break;
        }
        default: {   // DREAM_OP_POW
            const double* y = t->data;
            for (int j = 0; j < na; ++j) {
                const double x = a[j], e = b[j % nb], yy = y[j % n], gg = g[j % n];
                if (x != 0.0) ga[j] += gg * e * yy / x;
                if (x > 0.0) gb[j % nb] += gg * yy * std::log(x);
            }
            break;
        }
    }
}

void unary_backward(Tensor* t) {
    const int n = t->lhs->size;
    const double *x = t->lhs->data, *y = t->data, *g = t->grad;
    double* gx = t->lhs->grad;
    for (int j = 0; j < n; ++j) {
        double d;
        switch (t->op) {
            case DREAM_OP_RELU: d = x[j] > 0 ? 1.0 : 0.0; break;
            case DREAM_OP_EXP: d = y[j]; break;
            case DREAM_OP_LOG: gx[j] += g[j] / x[j]; continue;
            case DREAM_OP_SQRT: gx[j] += g[j] / (2.0 * y[j]); continue;
            case DREAM_OP_ABS: d = x[j] >= 0 ? 1.0 : -1.0; break;
            case DREAM_OP_SIGMOID: d = y[j] * (1 - y[j]); break;
            case DREAM_OP_TANH: d = 1 - y[j] * y[j]; break;
            case DREAM_OP_SIN: d = std::cos(x[j]); break;
            case DREAM_OP_COS: d = -std::sin(x[j]); break;
            case DREAM_OP_TAN: {
                const double c = std::cos(x[j]);
                gx[j] += g[j] / (c * c);
                continue;
            }
            default: gx[j] += g[j] / (1.0 + x[j] * x[j]); continue;   // DREAM_OP_ATAN
        }
        gx[j] += d * g[j];
    }
}

void topo_sort(Tensor* root, std::vector<Tensor*>& order) {
    // Iterative post-order DFS over lhs, rhs and parents (runtime/backend/gpu.inc:742-779).
    std::unordered_set<Tensor*> seen;
    std::vector<std::pair<Tensor*, int>> stack{{root, 0}};
    seen.insert(root);
    while (!stack.empty()) {
        auto& [t, i] = stack.back();
        Tensor* kids[5] = {t->lhs, t->rhs, t->parents[0], t->parents[1], t->parents[2]};
        if (i < 5) {
            Tensor* k = kids[i++];
            if (k && !seen.count(k)) {
                seen.insert(k);
                stack.push_back({k, 0});
            }
        } else {
            order.push_back(t);
            stack.pop_back();
        }
    }
}

// Naive fp64 references used by the selftests only.
void ref_gemm(const double* A, const double* B, double* C, int M, int K, int N) {
    for (int i = 0; i < M; ++i)
        for (int j = 0; j < N; ++j) {
            double s = 0.0;
            for (int k = 0; k < K; ++k) s += A[(size_t)i * K + k] * B[(size_t)k * N + j];
            C[(size_t)i * N + j] = s;
        }
}

void ref_causal_attention(const double* Q, const double* K, const double* V, double* O, int S,
                          int dk) {
    const double scale = 1.0 / std::sqrt((double)dk);
    std::vector<double> p(S);
    for (int i = 0; i < S; ++i) {
        double mx = -1e300, sum = 0.0;
        for (int j = 0; j <= i; ++j) {
            double s = 0.0;
            for (int k = 0; k < dk; ++k) s += Q[i * dk + k] * K[j * dk + k];
            p[j] = s * scale;
            mx = std::max(mx, p[j]);
        }
        for (int j = 0; j <= i; ++j) sum += (p[j] = std::exp(p[j] - mx));
        for (int k = 0; k < dk; ++k) {
            double s = 0.0;
            for (int j = 0; j <= i; ++j) s += p[j] * V[j * dk + k];
            O[i * dk + k] = s / sum;
        }
    }
}

}  // namespace

extern "C" {

// ----------------------------------------------------------------------------- tensors
}  // extern "C"

namespace {
Tensor* new_tensor(int d0, int d1, int d2, int d3, bool zero_data) {
    if (d0 < 0 || d1 < 0 || d2 < 0 || d3 < 0) {
        std::fprintf(stderr, "RUNTIME ERROR: negative tensor dimension (%d,%d,%d,%d)\n", d0, d1,
                     d2, d3);
        d0 = d1 = d2 = d3 = 1;
    }
    long long n = (long long)d0 * d1 * d2 * d3;
    if (n > 500000000LL) {
        std::fprintf(stderr, "RUNTIME ERROR: tensor too large (%lld elements)\n", n);
        d0 = d1 = d2 = d3 = 1;
        n = 1;
    }
    const int size = n <= 0 ? 1 : (int)n;
    Tensor* t = (Tensor*)std::calloc(1, sizeof(Tensor));
    bool pd, pg;
    t->data = host_buffer(size, zero_data, pd);
    tpoint("new_tensor: data");
    t->grad = host_buffer(size, true, pg);
    tpoint("new_tensor: grad");
    t->host_pinned = (pd ? 1 : 0) | (pg ? 2 : 0);
    t->size = size;
    t->d0 = d0;
    t->d1 = d1;
    t->d2 = d2;
    t->d3 = d3;
    t->refcount = 1;
    t->is_leaf = 1;
    t->grad_zero = 1;
    return t;
}

// Output tensor of a GPU op: its data is overwritten by the device result, so it is not zeroed.
Tensor* alloc_result(int d0, int d1, int d2, int d3) { return new_tensor(d0, d1, d2, d3, false); }
}  // namespace

extern "C" {

Tensor* alloc_tensor(int d0, int d1, int d2, int d3) { return new_tensor(d0, d1, d2, d3, true); }

Tensor* create_scalar(double v) {
    Tensor* t = alloc_tensor(1, 1, 1, 1);
    t->data[0] = v;
    return t;
}

Tensor* tensor_incref(Tensor* t) { return incref(t); }

Tensor* tensor_decref(Tensor* t) {
    if (!t || --t->refcount > 0) return nullptr;
    tensor_decref(t->lhs);
    tensor_decref(t->rhs);
    for (int i = 0; i < t->num_parents; ++i) tensor_decref(t->parents[i]);
    drop_device(t);
    release_host(t->data, t->host_pinned & 1);
    release_host(t->grad, t->host_pinned & 2);
    std::free(t->fdata);
    std::free(t->fgrad);
    std::free(t);
    return nullptr;
}

Tensor* ones(Tensor* d0, Tensor* d1) {
    Tensor* t = alloc_tensor((int)d0->data[0], (int)d1->data[0], 1, 1);
    std::fill(t->data, t->data + t->size, 1.0);
    return t;
}

Tensor* dream_set_seed(Tensor* s) {
    const unsigned seed = s ? (unsigned)s->data[0] : 42u;
    rng().seed(seed);
    std::fprintf(stderr, "[seed] RNG seeded with %u\n", seed);
    return create_scalar((double)seed);
}

Tensor* dream_randn(Tensor* d0, Tensor* d1) {
    Tensor* t = alloc_tensor((int)d0->data[0], (int)d1->data[0], 1, 1);
    std::normal_distribution<double> nd(0.0, 1.0);
    for (int i = 0; i < t->size; ++i) t->data[i] = nd(rng());
    return t;
}

// dropout(x, keep) (runtime/io/builtins.inc:151-163): one fp32 uniform draw on [0, 1) from the
// shared generator per element, in element order; a draw below keep keeps x / keep, else 0.
// Host op, like the reference's: the draws define the mask, so the stream must be the same.
Tensor* dream_dropout(Tensor* t, Tensor* keep_rate) {
    if (!t || !keep_rate) return create_scalar(0.0);
    const float rate = (float)keep_rate->data[0];
    Tensor* c = alloc_tensor(t->d0, t->d1, t->d2, t->d3);
    std::uniform_real_distribution<float> dist(0.f, 1.f);
    for (int i = 0; i < t->size; ++i) c->data[i] = dist(rng()) < rate ? t->data[i] / rate : 0.0;
    c->keep = (double)rate;
    set_graph(c, t, nullptr, DREAM_OP_DROPOUT);
    return c;
}

Tensor* sum(Tensor* a) {
    Tensor* c = alloc_tensor(1, 1, 1, 1);
    double s = 0.0;
    for (int i = 0; i < a->size; ++i) s += a->data[i];
    c->data[0] = s;
    set_graph(c, a, nullptr, DREAM_OP_SUM);
    return c;
}

// ---- elementwise builtins (elementwise.inc:276-336, 1254-1270; math_extra.inc:1-10;
// builtins.inc:85-87) over runGPU / runGPUUnary (backend/gpu.inc:637-716): outputs of at most
// 4194304 elements run on the host (the reference's CPU-first rule, gpu.inc:640, 691), larger
// ones on the GPU in fp64 (DREAM_ELEMWISE_CPU_MAX moves the bound; 0 sends every op to the
// GPU).  fp64 is Dream's number type: the GPU gives the host loop's values exactly for the
// IEEE-exact ops, and within an ulp or two for the transcendental ones.
static long long elemwise_cpu_max() {
    const char* e = std::getenv("DREAM_ELEMWISE_CPU_MAX");
    return e && *e ? std::atoll(e) : 4194304;
}

static double host_bin(int op, double a, double b) {
    switch (op) {
        case DH_BOP_ADD: return a + b;
        case DH_BOP_SUB: return a - b;
        case DH_BOP_MUL: return a * b;
        case DH_BOP_DIV: return a / b;
        case DH_BOP_MOD: return std::fmod(a, b);
        case DH_BOP_GT: return a > b ? 1.0 : 0.0;
        case DH_BOP_LT: return a < b ? 1.0 : 0.0;
        case DH_BOP_GE: return a >= b ? 1.0 : 0.0;
        case DH_BOP_LE: return a <= b ? 1.0 : 0.0;
        case DH_BOP_EQ: return std::fabs(a - b) < 1e-6 ? 1.0 : 0.0;
        case DH_BOP_NE: return std::fabs(a - b) >= 1e-6 ? 1.0 : 0.0;
        case DH_BOP_AND: return (a > 0 && b > 0) ? 1.0 : 0.0;
        case DH_BOP_OR: return (a > 0 || b > 0) ? 1.0 : 0.0;
        case DH_BOP_ATAN2: return std::atan2(a, b);
        case DH_BOP_POW: return std::pow(a, b);
        case DH_BOP_MIN: return a < b ? a : b;
        default: return a > b ? a : b;
    }
}

static double host_un(int op, double a, double lo, double hi) {
    switch (op) {
        case DH_UOP_RELU: return a > 0.0 ? a : 0.0;
        case DH_UOP_EXP: return std::exp(a);
        case DH_UOP_LOG: return std::log(a);
        case DH_UOP_SQRT: return std::sqrt(a);
        case DH_UOP_ABS: return std::fabs(a);
        case DH_UOP_SIGMOID: return 1.0 / (1.0 + std::exp(-a));
        case DH_UOP_TANH: return std::tanh(a);
        case DH_UOP_LNOT: return a == 0.0 ? 1.0 : 0.0;
        case DH_UOP_SIN: return std::sin(a);
        case DH_UOP_COS: return std::cos(a);
        case DH_UOP_TAN: return std::tan(a);
        case DH_UOP_ATAN: return std::atan(a);
        case DH_UOP_FLOOR: return std::floor(a);
        case DH_UOP_CEIL: return std::ceil(a);
        case DH_UOP_ROUND: return std::round(a);
        default: return std::fmax(lo, std::fmin(hi, a));
    }
}

// bcastStrides (gpu.inc:443-449): the operand's own contiguous strides, 0 on a dim of 1.
static void bcast_strides(const Tensor* t, int s[4]) {
    s[0] = t->d0 > 1 ? t->d1 * t->d2 * t->d3 : 0;
    s[1] = t->d1 > 1 ? t->d2 * t->d3 : 0;
    s[2] = t->d2 > 1 ? t->d3 : 0;
    s[3] = t->d3 > 1 ? 1 : 0;
}

// Largest element index the strides reach over C's dims.  The reference reads past an
// operand whose dims do not broadcast against C's (after its shape-mismatch warning); here
// such a pair is an error instead.
static long long reach(const int s[4], const int cd[4]) {
    long long r = 0;
    for (int k = 0; k < 4; ++k) r += (long long)(cd[k] - 1) * s[k];
    return r;
}

static int binop_node(int op) {
    switch (op) {
        case DH_BOP_ADD: return DREAM_OP_ADD;
        case DH_BOP_SUB: return DREAM_OP_SUB;
        case DH_BOP_MUL: return DREAM_OP_MUL;
        case DH_BOP_DIV: return DREAM_OP_DIV;
        case DH_BOP_MIN: return DREAM_OP_MINIMUM;
        case DH_BOP_MAX: return DREAM_OP_MAXIMUM;
        case DH_BOP_POW: return DREAM_OP_POW;
        default: return DREAM_OP_NO_GRAD;   // no backward branch in the reference
    }
}

static int unop_node(int op) {
    switch (op) {
        case DH_UOP_RELU: return DREAM_OP_RELU;
        case DH_UOP_EXP: return DREAM_OP_EXP;
        case DH_UOP_LOG: return DREAM_OP_LOG;
        case DH_UOP_SQRT: return DREAM_OP_SQRT;
        case DH_UOP_ABS: return DREAM_OP_ABS;
        case DH_UOP_SIGMOID: return DREAM_OP_SIGMOID;
        case DH_UOP_TANH: return DREAM_OP_TANH;
        case DH_UOP_SIN: return DREAM_OP_SIN;
        case DH_UOP_COS: return DREAM_OP_COS;
        case DH_UOP_TAN: return DREAM_OP_TAN;
        case DH_UOP_ATAN: return DREAM_OP_ATAN;
        default: return DREAM_OP_NO_GRAD;
    }
}

// The GPU result's fp32 rounding becomes c's device copy, like a GEMM result's.
static void keep_dev32(Tensor* c, Dev& d32) {
    if (c->dev) dh_free(c->dev);
    c->dev = static_cast<float*>(d32.release());
    c->dev_version = c->version;
    c->dev_exact = 0;
}

// ... and the fp64 result itself its fp64 device copy.
static void keep_dev64(Tensor* c, Dev& d64) {
    if (c->dev64) dh_free(c->dev64);
    c->dev64 = static_cast<double*>(d64.release());
    c->dev64_version = c->version;
}

// c = op(a, b) over c's dims; false (error printed) when the shapes do not broadcast or the
// GPU path fails.
static bool elementwise_binary(const char* name, int op, Tensor* a, Tensor* b, Tensor* c) {
    int as[4], bs[4];
    const int cd[4] = {c->d0, c->d1, c->d2, c->d3};
    bcast_strides(a, as);
    bcast_strides(b, bs);
    if (reach(as, cd) >= a->size || reach(bs, cd) >= b->size) {
        rt_error(name, "operands %dx%dx%dx%d and %dx%dx%dx%d do not broadcast", a->d0, a->d1,
                 a->d2, a->d3, b->d0, b->d1, b->d2, b->d3);
        return false;
    }
    const long long n = c->size;
    if (n <= elemwise_cpu_max()) {
        // Operands of C's own shape (index i) or single values (index 0) need no index
        // decomposition: the same elements as the general loop below.
        auto whole = [&](const Tensor* x) {
            return x->d0 == cd[0] && x->d1 == cd[1] && x->d2 == cd[2] && x->d3 == cd[3];
        };
        if ((whole(a) || a->size == 1) && (whole(b) || b->size == 1)) {
            const double *ad = a->data, *bd = b->data;
            const size_t sa = a->size == 1 && !whole(a) ? 0 : 1;
            const size_t sb = b->size == 1 && !whole(b) ? 0 : 1;
            double* cdat = c->data;
            par_for((size_t)n, [=](size_t i0, size_t i1) {
                for (size_t i = i0; i < i1; ++i) cdat[i] = host_bin(op, ad[i * sa], bd[i * sb]);
            });
            return true;
        }
        for (long long i = 0; i < n; ++i) {
            long long r = i, ia = 0, ib = 0;
            for (int k = 3; k >= 0; --k) {
                const long long x = r % cd[k];
                r /= cd[k];
                ia += x * as[k];
                ib += x * bs[k];
            }
            c->data[i] = host_bin(op, a->data[ia], b->data[ib]);
        }
        return true;
    }
    if (!hip_ready(name)) return false;
    try {
        Dev dc((size_t)n * 8), d32((size_t)n * 4);
        need_buf(dc), need_buf(d32);
        const double* da = dev_data64(a);
        const double* db = dev_data64(b);
        need(dh_binary(op, DH_F64, da, (size_t)a->size, as, db, (size_t)b->size, bs, dc.p, cd,
                       d32.f()));
        need(dh_memcpy_d2h(c->data, dc.p, (size_t)n * 8));
        keep_dev32(c, d32);
        keep_dev64(c, dc);
    } catch (const Failure&) {
        rt_error(name, "%s", dh_last_error());
        return false;
    }
    return true;
}

static bool elementwise_unary(const char* name, int op, Tensor* a, Tensor* c, double lo, double hi) {
    const long long n = a->size;
    if (n <= elemwise_cpu_max()) {
        const double* ad = a->data;
        double* cdat = c->data;
        par_for((size_t)n, [=](size_t i0, size_t i1) {
            for (size_t i = i0; i < i1; ++i) cdat[i] = host_un(op, ad[i], lo, hi);
        });
        return true;
    }
    if (!hip_ready(name)) return false;
    try {
        Dev dc((size_t)n * 8), d32((size_t)n * 4);
        need_buf(dc), need_buf(d32);
        need(dh_unary(op, DH_F64, dev_data64(a), dc.p, (size_t)n, lo, hi, d32.f()));
        need(dh_memcpy_d2h(c->data, dc.p, (size_t)n * 8));
        keep_dev32(c, d32);
        keep_dev64(c, dc);
    } catch (const Failure&) {
        rt_error(name, "%s", dh_last_error());
        return false;
    }
    return true;
}

// BINOP (elementwise.inc:284-288): null operand -> error and a 1x1 tensor; C's dims are the
// per-dim maxima (makeBinop, elementwise.inc:269-283).
static Tensor* binop(const char* name, int op, Tensor* a, Tensor* b) {
    if (!a || !b) {
        std::fprintf(stderr, "RUNTIME ERROR in '%s': null operand\n", name);
        return alloc_tensor(1, 1, 1, 1);
    }
    Tensor* c = alloc_result(std::max(a->d0, b->d0), std::max(a->d1, b->d1),
                             std::max(a->d2, b->d2), std::max(a->d3, b->d3));
    if (!elementwise_binary(name, op, a, b, c)) {
        tensor_decref(c);
        return alloc_tensor(1, 1, 1, 1);
    }
    set_graph(c, a, b, binop_node(op));
    return c;
}

// UNARY (elementwise.inc:313-318): null input -> error naming the op and a 1x1 tensor.
static Tensor* unop(const char* name, int op, Tensor* a, double lo = 0.0, double hi = 0.0) {
    if (!a) {
        std::fprintf(stderr, "RUNTIME ERROR in '%s': null input\n", name);
        return alloc_tensor(1, 1, 1, 1);
    }
    Tensor* c = alloc_result(a->d0, a->d1, a->d2, a->d3);
    if (!elementwise_unary(name, op, a, c, lo, hi)) {
        tensor_decref(c);
        return alloc_tensor(1, 1, 1, 1);
    }
    set_graph(c, a, nullptr, unop_node(op));
    return c;
}

Tensor* tensor_add(Tensor* a, Tensor* b) { return binop("+", DH_BOP_ADD, a, b); }
Tensor* tensor_sub(Tensor* a, Tensor* b) { return binop("-", DH_BOP_SUB, a, b); }
Tensor* tensor_mul(Tensor* a, Tensor* b) { return binop("*", DH_BOP_MUL, a, b); }
Tensor* tensor_div(Tensor* a, Tensor* b) { return binop("/", DH_BOP_DIV, a, b); }
Tensor* tensor_mod(Tensor* a, Tensor* b) { return binop("%", DH_BOP_MOD, a, b); }
Tensor* tensor_gt(Tensor* a, Tensor* b) { return binop(">", DH_BOP_GT, a, b); }
Tensor* tensor_lt(Tensor* a, Tensor* b) { return binop("<", DH_BOP_LT, a, b); }
Tensor* tensor_ge(Tensor* a, Tensor* b) { return binop(">=", DH_BOP_GE, a, b); }
Tensor* tensor_le(Tensor* a, Tensor* b) { return binop("<=", DH_BOP_LE, a, b); }
Tensor* tensor_eq(Tensor* a, Tensor* b) { return binop("==", DH_BOP_EQ, a, b); }
Tensor* tensor_ne(Tensor* a, Tensor* b) { return binop("!=", DH_BOP_NE, a, b); }
Tensor* tensor_and(Tensor* a, Tensor* b) { return binop("&&", DH_BOP_AND, a, b); }
Tensor* tensor_or(Tensor* a, Tensor* b) { return binop("||", DH_BOP_OR, a, b); }
Tensor* dream_minimum(Tensor* a, Tensor* b) { return binop("min", DH_BOP_MIN, a, b); }
Tensor* dream_maximum(Tensor* a, Tensor* b) { return binop("max", DH_BOP_MAX, a, b); }
Tensor* dream_atan2(Tensor* y, Tensor* x) { return binop("atan2", DH_BOP_ATAN2, y, x); }

// dream_pow (elementwise.inc:1254-1270): C is 2-D, (max d0, max d1).
Tensor* dream_pow(Tensor* base, Tensor* exp_t) {
    if (!base || !exp_t) {
        std::fprintf(stderr, "RUNTIME ERROR in '**': null operand\n");
        return alloc_tensor(1, 1, 1, 1);
    }
    Tensor* c = alloc_result(std::max(base->d0, exp_t->d0), std::max(base->d1, exp_t->d1), 1, 1);
    if (!elementwise_binary("**", DH_BOP_POW, base, exp_t, c)) {
        tensor_decref(c);
        return alloc_tensor(1, 1, 1, 1);
    }
    set_graph(c, base, exp_t, DREAM_OP_POW);
    return c;
}

Tensor* relu(Tensor* a) { return unop("relu", DH_UOP_RELU, a); }
Tensor* dream_exp(Tensor* a) { return unop("exp", DH_UOP_EXP, a); }
Tensor* dream_log(Tensor* a) { return unop("log", DH_UOP_LOG, a); }
Tensor* dream_sqrt(Tensor* a) { return unop("sqrt", DH_UOP_SQRT, a); }
Tensor* dream_abs(Tensor* a) { return unop("abs", DH_UOP_ABS, a); }
Tensor* dream_sigmoid(Tensor* a) { return unop("sigmoid", DH_UOP_SIGMOID, a); }
Tensor* dream_tanh(Tensor* a) { return unop("tanh", DH_UOP_TANH, a); }
Tensor* dream_logical_not(Tensor* a) { return unop("lnot", DH_UOP_LNOT, a); }
Tensor* dream_sin(Tensor* a) { return unop("sin", DH_UOP_SIN, a); }
Tensor* dream_cos(Tensor* a) { return unop("cos", DH_UOP_COS, a); }
Tensor* dream_tan(Tensor* a) { return unop("tan", DH_UOP_TAN, a); }
Tensor* dream_atan(Tensor* a) { return unop("atan", DH_UOP_ATAN, a); }
Tensor* dream_floor(Tensor* a) { return unop("floor", DH_UOP_FLOOR, a); }
Tensor* dream_ceil(Tensor* a) { return unop("ceil", DH_UOP_CEIL, a); }
Tensor* dream_round(Tensor* a) { return unop("round", DH_UOP_ROUND, a); }

// dream_clip (elementwise.inc:329-336): fmax(lo, fmin(hi, x)) with the bounds' first values.
Tensor* dream_clip(Tensor* a, Tensor* lo, Tensor* hi) {
    if (!lo || !hi || !lo->data || !hi->data) {
        std::fprintf(stderr, "RUNTIME ERROR in 'clip': null bound\n");
        return alloc_tensor(1, 1, 1, 1);
    }
    return unop("clip", DH_UOP_CLIP, a, lo->data[0], hi->data[0]);
}

Tensor* tensor_get_grad(Tensor* t) {
    if (!t) {
        rt_error("grad()", "argument is null");
        return alloc_tensor(1, 1, 1, 1);
    }
    Tensor* g = alloc_tensor(t->d0, t->d1, t->d2, t->d3);
    std::copy(t->grad, t->grad + t->size, g->data);
    return g;
}

Tensor* zero_grad(Tensor* t) {
    if (!t) {
        rt_error("zero_grad", "tensor is null");
        return nullptr;
    }
    if (!t->grad_zero) {   // else already all zero
        double* g = t->grad;
        par_for((size_t)t->size, [=](size_t i0, size_t i1) { std::fill(g + i0, g + i1, 0.0); });
    }
    if (t->dgrad) dh_free(t->dgrad);
    t->dgrad = nullptr;
    t->grad_zero = 1;
    Tensor *l = t->lhs, *r = t->rhs;
    t->lhs = t->rhs = nullptr;
    tensor_decref(l);
    tensor_decref(r);
    for (int i = 0; i < t->num_parents; ++i) tensor_decref(t->parents[i]);
    t->num_parents = 0;
    return incref(t);
}

Tensor* tensor_set_element(Tensor* t, Tensor* idx_t, Tensor* val) {
    // runtime/core/indexing.inc:50-94: a flat write for vectors and 1 x N tensors, else the
    // row idx along d0 (copying min(val.size, row) values); negative indices wrap.
    if (!t || !idx_t || !val) return t;
    int idx = (int)idx_t->data[0];
    const bool inner = t->d1 > 1 || t->d2 > 1 || t->d3 > 1;
    const int slice = t->d1 * t->d2 * t->d3;
    const int extent = !inner ? t->d0 : (t->d0 == 1 && idx != 0) ? slice : t->d0;
    if (idx < 0) idx += extent;
    if (idx < 0 || idx >= extent) {
        std::fprintf(stderr, "runtime error: set index %d out of bounds (size %d)\n",
                     (int)idx_t->data[0], extent);
        return t;
    }
    if (!inner || (t->d0 == 1 && (int)idx_t->data[0] != 0)) {
        t->data[idx] = val->data[0];
    } else {
        const int n = std::min(val->size, slice);
        std::copy(val->data, val->data + n, t->data + (size_t)idx * slice);
    }
    ++t->version;   // the device copy of `data` is stale from here on
    return t;
}

Tensor* tensor_set_element_2d(Tensor* t, Tensor* row_t, Tensor* col_t, Tensor* val) {
    // runtime/core/indexing.inc:97-113
    if (!t || !row_t || !col_t || !val) return t;
    int row = (int)row_t->data[0], col = (int)col_t->data[0];
    const int cols = t->d1;
    if (row < 0) row += t->d0;
    if (col < 0) col += cols;
    const long long flat = (long long)row * cols + col;
    if (flat < 0 || flat >= t->size) {
        std::fprintf(stderr, "runtime error: index [%d, %d] out of bounds\n", (int)row_t->data[0],
                     (int)col_t->data[0]);
        return t;
    }
    t->data[flat] = val->data[0];
    ++t->version;
    return t;
}

// ----------------------------------------------------------------------------- precision
Tensor* dream_set_precision(Tensor* t, int code) {
    if (!t) return nullptr;
    if (code == 1) {
        if (t->dtype != 1 || !t->fdata) {
            if (!t->fdata) t->fdata = (float*)std::calloc(t->size, sizeof(float));
            if (!t->fgrad) t->fgrad = (float*)std::calloc(t->size, sizeof(float));
            for (int i = 0; i < t->size; ++i) t->fdata[i] = (float)t->data[i];
            t->dtype = 1;
        }
    } else {
        if (t->dtype == 1 && t->fdata) {
            for (int i = 0; i < t->size; ++i) t->data[i] = (double)t->fdata[i];
            ++t->version;
        }
        t->dtype = 0;
    }
    return incref(t);
}

Tensor* dream_to_float32(Tensor* t) {
    if (!t || t->dtype == 1) return incref(t);
    if (!t->fdata) t->fdata = (float*)std::calloc(t->size, sizeof(float));
    if (!t->fgrad) t->fgrad = (float*)std::calloc(t->size, sizeof(float));
    for (int i = 0; i < t->size; ++i) {
        t->fdata[i] = (float)t->data[i];
        t->data[i] = (double)t->fdata[i];
        t->fgrad[i] = (float)t->grad[i];
    }
    t->dtype = 1;
    ++t->version;
    return incref(t);
}

Tensor* dream_enable_fp16(void) {
    g_bf16 = true;
    std::fprintf(stderr, "[dream] reduced-precision matmul enabled (bf16 operands, fp32 accumulate)\n");
    return create_scalar(1.0);
}

Tensor* dream_disable_fp16(void) {
    g_bf16 = false;
    return create_scalar(1.0);
}

// ----------------------------------------------------------------------------- hot path
Tensor* tensor_matmul(Tensor* a, Tensor* b) {
    if (!a || !b) {
        rt_error("matmul (@)", "null operand%s%s", a ? "" : " (left=null)", b ? "" : " (right=null)");
        return alloc_tensor(1, 1, 1, 1);
    }
    if (!a->data || !b->data) {
        rt_error("matmul (@)", "null data pointer left=%dx%d right=%dx%d", a->d0, a->d1, b->d0, b->d1);
        return alloc_tensor(1, 1, 1, 1);
    }
    if (a->d1 != b->d0) {
        rt_error("matmul (@)", "shape mismatch (%dx%d @ %dx%d) \xe2\x80\x94 inner dimensions must match",
                 a->d0, a->d1, b->d0, b->d1);
        return alloc_tensor(1, 1, 1, 1);
    }
    if (!hip_ready("matmul (@)")) return alloc_tensor(1, 1, 1, 1);
    const int M = a->d0, K = a->d1, N = b->d1;
    Tensor* c = alloc_result(M, N, 1, 1);
    set_graph(c, a, b, DREAM_OP_MATMUL);
    const bool f32 = a->dtype == 1 && b->dtype == 1 && a->fdata && b->fdata;
    try {
        const size_t mk = (size_t)M * K, kn = (size_t)K * N, mn = (size_t)M * N;
        if (!f32 && !dh_matmul_eligible(M, N)) {
            // below the dispatch threshold: the reference's fp64 dgemm (elementwise.inc:1033-1040)
            Dev da(mk * 8), db(kn * 8), dc(mn * 8);
            upload_f64(a->data, mk, da);
            upload_f64(b->data, kn, db);
            need_buf(dc);
            need(dh_gemm_f64(0, 0, M, N, K, da.d(), K, db.d(), N, 0.0, dc.d(), N));
            need(dh_memcpy_d2h(c->data, dc.p, mn * sizeof(double)));
            c->f64_node = 1;
            return c;
        }
        Dev dc(mn * 4);
        need_buf(dc);
        if (g_bf16 && !f32) {
            Dev da(mk * 2), db(kn * 2);
            need_buf(da), need_buf(db);
            dev_bf16(a, mk, da);
            dev_bf16(b, kn, db);
            need(dh_gemm_bf16(0, 0, M, N, K, da.h(), K, db.h(), N, 0.f, dc.f(), N));
        } else {
            need(dh_gemm_f32(0, 0, M, N, K, dev_data(a), K, dev_data(b), N, 0.f, dc.f(), N));
        }
        if (f32) {
            // fp32 result: fdata is the live copy, data its fp64 mirror (elementwise.inc:1000-1017)
            c->fdata = (float*)std::calloc(c->size, sizeof(float));
            c->fgrad = (float*)std::calloc(c->size, sizeof(float));
            c->dtype = 1;
            need(dh_memcpy_d2h(c->fdata, dc.p, mn * 4));
        }
        adopt_result(c, dc);
    } catch (const Failure&) {
        rt_error("matmul (@)", "%s", dh_last_error());
        tensor_decref(c);
        return alloc_tensor(1, 1, 1, 1);
    }
    return c;
}

Tensor* dream_flash_attention(Tensor* Q, Tensor* K, Tensor* V, Tensor* batch, Tensor* seq,
                              Tensor* dk, Tensor* block) {
    (void)block;   // the key-block size is a CPU tiling knob; the GPU kernels fix their own
    return attention_impl("flash_attention", DREAM_OP_FLASH, true, Q, K, V, batch, seq, dk);
}

Tensor* dream_attention(Tensor* Q, Tensor* K, Tensor* V, Tensor* batch, Tensor* seq, Tensor* dk) {
    return attention_impl("attention", DREAM_OP_ATTN, false, Q, K, V, batch, seq, dk);
}

Tensor* dream_attention_causal(Tensor* Q, Tensor* K, Tensor* V, Tensor* batch, Tensor* seq,
                               Tensor* dk) {
    return attention_impl("attention_causal", DREAM_OP_ATTN_CAUSAL, true, Q, K, V, batch, seq, dk);
}

static Tensor* linear_impl(Tensor* x, Tensor* W, Tensor* b, bool relu) {
    // elementwise.inc:1432-1516.  Both forms report errors as "linear", like the reference
    // (linear_relu calls linear and then relabels the node).
    if (!x || !W || !b) {
        std::fprintf(stderr, "RUNTIME ERROR in linear: null arg%s%s%s\n", x ? "" : " x=null",
                     W ? "" : " W=null", b ? "" : " b=null");
        std::fflush(stderr);
        return alloc_tensor(1, 1, 1, 1);
    }
    const int N = x->d0, in = x->d1, out = W->d0;
    if (in != W->d1) {
        rt_error("linear", "x.d1(%d) != W.d1(%d)", in, W->d1);
        return alloc_tensor(1, 1, 1, 1);
    }
    if (b->size < out) {
        rt_error("linear", "bias holds %d values for %d outputs", b->size, out);
        return alloc_tensor(1, 1, 1, 1);
    }
    if (!hip_ready("linear")) return alloc_tensor(1, 1, 1, 1);
    tpoint("linear: entry");
    Tensor* y = alloc_result(N, out, 1, 1);
    tpoint("linear: alloc");
    set_graph(y, x, W, relu ? DREAM_OP_LINEAR_RELU : DREAM_OP_LINEAR);
    set_parents(y, x, W, b);
    try {
        Dev d((size_t)N * out * sizeof(float));
        need_buf(d);
        need(dh_gemm_f32_ex(0, 1, N, out, in, dev_data(x), in, 0, dev_data(W), in, 0, 0.f, d.f(),
                            out, 0, 1, dev_data(b), relu ? DH_EPI_RELU : 0));
        tpoint("linear: launched");
        adopt_result(y, d);
        tpoint("linear: adopted");
    } catch (const Failure&) {
        rt_error("linear", "%s", dh_last_error());
        tensor_decref(y);
        return alloc_tensor(1, 1, 1, 1);
    }
    return y;
}

Tensor* dream_linear(Tensor* x, Tensor* W, Tensor* b) { return linear_impl(x, W, b, false); }
Tensor* dream_linear_relu(Tensor* x, Tensor* W, Tensor* b) { return linear_impl(x, W, b, true); }
Tensor* linear(Tensor* x, Tensor* W, Tensor* b) { return dream_linear(x, W, b); }
Tensor* linear_relu(Tensor* x, Tensor* W, Tensor* b) { return dream_linear_relu(x, W, b); }

Tensor* dream_bmm(Tensor* a, Tensor* b, Tensor* batch_t, Tensor* m_t, Tensor* k_t, Tensor* n_t) {
    // elementwise.inc:1218-1252: a (B, M*K) @ b (B, K*N) -> (B, M*N) per batch member.
    const int Bt = (int)batch_t->data[0], M = (int)m_t->data[0], K = (int)k_t->data[0],
              N = (int)n_t->data[0];
    if (a->size < Bt * M * K || b->size < Bt * K * N) {
        std::fprintf(stderr, "error: bmm size mismatch (a=%d need %d, b=%d need %d)\n", a->size,
                     Bt * M * K, b->size, Bt * K * N);
        std::fflush(stderr);
        return alloc_tensor(1, 1, 1, 1);
    }
    if (!hip_ready("bmm")) return alloc_tensor(1, 1, 1, 1);
    Tensor* c = alloc_result(Bt, M * N, 1, 1);
    set_graph(c, a, b, DREAM_OP_BMM);
    c->bmm_B = Bt;
    c->bmm_M = M;
    c->bmm_K = K;
    c->bmm_N = N;
    try {
        Dev d((size_t)c->size * sizeof(float));
        need_buf(d);
        need(dh_gemm_f32_ex(0, 0, M, N, K, dev_data(a), K, (long long)M * K, dev_data(b), N,
                            (long long)K * N, 0.f, d.f(), N, (long long)M * N, Bt, nullptr, 0));
        adopt_result(c, d);
    } catch (const Failure&) {
        rt_error("bmm", "%s", dh_last_error());
        tensor_decref(c);
        return alloc_tensor(1, 1, 1, 1);
    }
    return c;
}

Tensor* dream_softmax(Tensor* a) { return row_op("softmax", DREAM_OP_SOFTMAX, a); }
Tensor* dream_log_softmax(Tensor* x) { return row_op("log_softmax", DREAM_OP_LOG_SOFTMAX, x); }
Tensor* dream_layer_norm(Tensor* t) { return row_op("layer_norm", DREAM_OP_LAYER_NORM, t); }

static Tensor* conv_impl(Tensor* input, Tensor* kernel, Tensor* bias, Tensor* h_t, Tensor* w_t,
                         Tensor* kh_t, Tensor* kw_t, int pad, int stride, bool padded) {
    // conv.inc:12-55 / 119-178: N = input.d0, Cin = input.d1 / (H W) (at least 1),
    // Cout = kernel.d0; image n of the input starts at n*Cin*H*W.
    const int H = (int)h_t->data[0], W = (int)w_t->data[0], KH = (int)kh_t->data[0],
              KW = (int)kw_t->data[0];
    if (stride < 1) stride = 1;
    const int OH = (H + 2 * pad - KH) / stride + 1, OW = (W + 2 * pad - KW) / stride + 1;
    if (H + 2 * pad < KH || W + 2 * pad < KW || OH <= 0 || OW <= 0 || KH < 1 || KW < 1) {
        std::fprintf(stderr, padded ? "error: conv2d output size <= 0\n"
                                    : "error: conv2d kernel larger than input\n");
        std::fflush(stderr);
        return alloc_tensor(1, 1, 1, 1);
    }
    const int N = input->d0;
    int Cin = H * W > 0 ? input->d1 / (H * W) : 1;
    if (Cin < 1) Cin = 1;
    const int Cout = kernel->d0;
    const long long K = (long long)Cin * KH * KW, P = (long long)OH * OW;
    if ((long long)N * Cin * H * W > input->size || (long long)Cout * K > kernel->size) {
        rt_error("conv2d", "input holds %d values for %d x %d x %d x %d, kernel %d for %d x %lld",
                 input->size, N, Cin, H, W, kernel->size, Cout, K);
        return alloc_tensor(1, 1, 1, 1);
    }
    if (!hip_ready("conv2d")) return alloc_tensor(1, 1, 1, 1);
    Tensor* out = alloc_result(N, (int)(Cout * P), 1, 1);
    set_graph(out, input, kernel, DREAM_OP_CONV2D);
    const int geom[8] = {H, W, KH, KW, Cin, Cout, pad, stride};
    std::copy(geom, geom + 8, out->conv);
    try {
        Dev y((size_t)out->size * 4);
        need_buf(y);
        // The reference adds bias[co] for co < min(Cout, bias.size) (conv.inc:5-10).
        const float* db = nullptr;
        Dev bpad(bias ? (size_t)Cout * 4 : 4);
        if (bias) {
            if (bias->size >= Cout) {
                db = dev_data(bias);
            } else {
                need_buf(bpad);
                need(dh_memset(bpad.p, 0, (size_t)Cout * 4));
                need(dh_memcpy_d2d(bpad.p, dev_data(bias), (size_t)bias->size * 4));
                db = bpad.f();
            }
        }
        // one implicit-GEMM launch: the im2col matrix is gathered inside the GEMM, never stored
        need(dh_conv2d_fwd(dev_data(input), dev_data(kernel), db, y.f(), N, Cin, H, W, Cout, KH,
                           KW, pad, stride));
        adopt_result(out, y);
    } catch (const Failure&) {
        rt_error("conv2d", "%s", dh_last_error());
        tensor_decref(out);
        return alloc_tensor(1, 1, 1, 1);
    }
    return out;
}

Tensor* dream_conv2d(Tensor* input, Tensor* kernel, Tensor* bias, Tensor* h_t, Tensor* w_t,
                     Tensor* kh_t, Tensor* kw_t) {
    return conv_impl(input, kernel, bias, h_t, w_t, kh_t, kw_t, 0, 1, false);
}

Tensor* dream_conv2d_padded(Tensor* input, Tensor* kernel, Tensor* bias, Tensor* h_t, Tensor* w_t,
                            Tensor* kh_t, Tensor* kw_t, Tensor* pad_t, Tensor* stride_t) {
    // Backward: the exact gradient of the padded, strided convolution.  (The reference's node
    // reuses the unpadded shapes in its backward, autograd.inc:507-535, which is only correct
    // for pad 0 and stride 1.)
    return conv_impl(input, kernel, bias, h_t, w_t, kh_t, kw_t, pad_t ? (int)pad_t->data[0] : 0,
                     stride_t ? (int)stride_t->data[0] : 1, true);
}

Tensor* backward(Tensor* root) {
    if (!root) {
        std::fprintf(stderr, "error: backward(null)\n");
        return create_scalar(0);
    }
    std::fill(root->grad, root->grad + root->size, 1.0);
    root->grad_zero = 0;
    std::vector<Tensor*> order;
    topo_sort(root, order);
    // A host backward op first takes its node's device gradient (flush_dgrad); a GPU backward
    // op first moves the host part onto the device (grad_in).
    auto host_grad = [](Tensor* t) {
        flush_dgrad(t);
        if (t->lhs) t->lhs->grad_zero = 0;
        if (t->rhs) t->rhs->grad_zero = 0;
    };
    // DREAM_TRACE_BACKWARD=1: each node's op code, size and time (device work waited for)
    // on stderr.
    static const bool trace = [] {
        const char* e = std::getenv("DREAM_TRACE_BACKWARD");
        return e && *e && *e != '0';
    }();
    auto now = [] { return std::chrono::steady_clock::now(); };
    auto t_last = now();
    auto stamp = [&](const char* what, int op, int size) {
        if (!trace) return;
        if (dh_available()) dh_sync();
        const auto t1 = now();
        std::fprintf(stderr, "[backward] %-8s op %2d size %9d  %8.3f ms\n", what, op, size,
                     std::chrono::duration<double, std::milli>(t1 - t_last).count());
        t_last = t1;
    };
    stamp("start", 0, root->size);
    for (int x = (int)order.size() - 1; x >= 0; --x) {
        Tensor* t = order[x];
        try {
            switch (t->op) {
                case DREAM_OP_MATMUL:
                    if (hip_ready("backward(matmul)")) matmul_backward(t);
                    break;
                case DREAM_OP_LINEAR:
                case DREAM_OP_LINEAR_RELU:
                    if (hip_ready("backward(linear)")) linear_backward(t, t->op == DREAM_OP_LINEAR_RELU);
                    break;
                case DREAM_OP_BMM:
                    if (hip_ready("backward(bmm)")) bmm_backward(t);
                    break;
                case DREAM_OP_CONV2D:
                    if (hip_ready("backward(conv2d)")) conv_backward(t);
                    break;
                case DREAM_OP_SOFTMAX:
                case DREAM_OP_LOG_SOFTMAX:
                case DREAM_OP_LAYER_NORM:
                    if (hip_ready("backward(row op)")) row_backward(t);
                    break;
                case DREAM_OP_FLASH:
                case DREAM_OP_ATTN_CAUSAL:
                case DREAM_OP_ATTN:
                    if ((t->dlse || t->f64_node) && hip_ready("backward(attention)"))
                        attention_backward(t, t->op != DREAM_OP_ATTN);
                    break;
                case DREAM_OP_SUM: {
                    host_grad(t);
                    double* lg = t->lhs->grad;
                    const double g0 = t->grad[0];
                    par_for((size_t)t->lhs->size, [=](size_t j0, size_t j1) {
                        for (size_t j = j0; j < j1; ++j) lg[j] += g0;
                    });
                    break;
                }
                case DREAM_OP_MUL:
                    host_grad(t);
                    if (t->lhs->size == t->size && t->rhs->size == t->size && t->lhs != t->rhs) {
                        // same shapes, distinct operands: every j updates its own elements
                        double *lg = t->lhs->grad, *rg = t->rhs->grad;
                        const double *ld = t->lhs->data, *rd = t->rhs->data, *g = t->grad;
                        par_for((size_t)t->size, [=](size_t j0, size_t j1) {
                            for (size_t j = j0; j < j1; ++j) {
                                lg[j] += g[j] * rd[j];
                                rg[j] += g[j] * ld[j];
                            }
                        });
                        break;
                    }
                    for (int j = 0; j < t->size; ++j) {
                        const double g = t->grad[j];
                        t->lhs->grad[j % t->lhs->size] += g * t->rhs->data[j % t->rhs->size];
                        t->rhs->grad[j % t->rhs->size] += g * t->lhs->data[j % t->lhs->size];
                    }
                    break;
                case DREAM_OP_ADD:
                case DREAM_OP_SUB:
                case DREAM_OP_DIV:
                case DREAM_OP_MINIMUM:
                case DREAM_OP_MAXIMUM:
                case DREAM_OP_POW:
                    host_grad(t);
                    binary_backward(t);
                    break;
                case DREAM_OP_RELU:
                case DREAM_OP_EXP:
                case DREAM_OP_LOG:
                case DREAM_OP_SQRT:
                case DREAM_OP_ABS:
                case DREAM_OP_SIGMOID:
                case DREAM_OP_TANH:
                case DREAM_OP_SIN:
                case DREAM_OP_COS:
                case DREAM_OP_TAN:
                case DREAM_OP_ATAN:
                    host_grad(t);
                    unary_backward(t);
                    break;
                case DREAM_OP_DROPOUT: {   // autograd.inc:472-482: kept elements, times 1/keep
                    host_grad(t);
                    const double inv = (t->keep > 0.0 && t->keep <= 1.0) ? 1.0 / t->keep : 1.0;
                    for (int j = 0; j < t->lhs->size; ++j)
                        if (t->data[j] != 0.0) t->lhs->grad[j] += t->grad[j] * inv;
                    break;
                }
                default:
                    break;
            }
        } catch (const Failure&) {
            rt_error("backward", "%s", dh_last_error());
        }
        stamp("node", t->op, t->size);
    }
    // Every gradient back on the host (the reference's grad buffers are host memory): all
    // device gradients queued home into one pinned staging buffer, one wait, then widened
    // (or added) on the host threads.
    try {
        flush_all(order);
        stamp("flush", -1, 0);
    } catch (const Failure&) {
        rt_error("backward", "%s", dh_last_error());
        for (Tensor* t : order) {
            try {
                flush_dgrad(t);
            } catch (const Failure&) {
            }
        }
    }
    return create_scalar(1.0);
}

// ----------------------------------------------------------------------------- queries
int dream_gpu_available(void) { return 0; }

int dream_hip_available(void) { return dh_available(); }

Tensor* gpu_selftest(void) {
    // elementwise.inc:802-875.  The reference's shapes go through `@`, which at these sizes
    // (M*N below the default threshold) runs fp64; the point of this test is the GPU kernels,
    // so the fp32 matrix-core GEMM and the fp32 FlashAttention kernel are called directly on
    // the same draws, under the reference's GPU gate (absolute sqrt(K) 1e-4).
    if (!dh_available()) {
        std::printf("=== gpu_selftest: no HIP device -- skipped ===\n");
        std::printf("  GPU: SKIP (CPU-only host; GPU kernels not exercised)\n");
        return create_scalar(1.0);
    }
    rng().seed(20260708);
    std::printf("=== gpu_selftest: GPU kernels vs fp64 reference ===\n");
    std::uniform_real_distribution<double> dist(-1.0, 1.0);
    int pass = 0, total = 0;
    double worst = 0.0;
    auto to_dev32 = [](const std::vector<double>& h, Dev& d) {
        std::vector<float> f(h.begin(), h.end());
        need_buf(d);
        need(dh_memcpy_h2d(d.p, f.data(), f.size() * sizeof(float)));
    };
    auto report = [&](bool ok, double err) {
        worst = std::max(worst, err);
        ++total;
        pass += ok;
    };
    const int shapes[3][3] = {{256, 128, 256}, {300, 200, 257}, {512, 64, 300}};
    for (const auto& sh : shapes) {
        const int M = sh[0], K = sh[1], N = sh[2];
        std::vector<double> A((size_t)M * K), B((size_t)K * N), Cc((size_t)M * N);
        for (auto& v : A) v = dist(rng());
        for (auto& v : B) v = dist(rng());
        double max_abs = 1e30;
        try {
            Dev da(A.size() * 4), db(B.size() * 4), dc(Cc.size() * 4);
            to_dev32(A, da);
            to_dev32(B, db);
            need_buf(dc);
            need(dh_gemm_f32(0, 0, M, N, K, da.f(), K, db.f(), N, 0.f, dc.f(), N));
            std::vector<float> Cg(Cc.size());
            need(dh_memcpy_d2h(Cg.data(), dc.p, Cg.size() * 4));
            ref_gemm(A.data(), B.data(), Cc.data(), M, K, N);
            max_abs = 0.0;
            for (size_t i = 0; i < Cc.size(); ++i)
                max_abs = std::max(max_abs, std::fabs((double)Cg[i] - Cc[i]));
        } catch (const Failure&) {
            rt_error("gpu_selftest", "%s", dh_last_error());
        }
        const double tol = std::sqrt((double)K) * 1e-4;   // elementwise.inc:843-845
        const bool ok = max_abs < tol;
        std::printf("  matmul %dx%dx%d  max_abs=%.2e (tol %.1e)  %s\n", M, K, N, max_abs, tol,
                    ok ? "PASS" : "FAIL");
        report(ok, max_abs);
    }
    {   // causal flash attention on one slice, S=256, dk=64, against fp64
        const int S = 256, dkk = 64;
        const size_t n = (size_t)S * dkk;
        std::vector<double> Q(n), Kt(n), Vt(n), Oc(n);
        for (auto* t : {&Q, &Kt, &Vt})
            for (auto& v : *t) v = dist(rng());
        double max_abs = 1e30;
        try {
            Dev q(n * 4), k(n * 4), v(n * 4), o(n * 4), lse(S * 4);
            to_dev32(Q, q);
            to_dev32(Kt, k);
            to_dev32(Vt, v);
            need_buf(o), need_buf(lse);
            need(dh_flash_fwd(DH_F32, 1, S, dkk, 0.125f, 1, q.p, k.p, v.p, o.p, lse.f()));
            std::vector<float> Og(n);
            need(dh_memcpy_d2h(Og.data(), o.p, n * 4));
            ref_causal_attention(Q.data(), Kt.data(), Vt.data(), Oc.data(), S, dkk);
            max_abs = 0.0;
            for (size_t i = 0; i < n; ++i) max_abs = std::max(max_abs, std::fabs((double)Og[i] - Oc[i]));
        } catch (const Failure&) {
            rt_error("gpu_selftest", "%s", dh_last_error());
        }
        const bool ok = max_abs < 1e-4;
        std::printf("  flash_attention S=%d dk=%d  max_abs=%.2e (tol 1.0e-04)  %s\n", S, dkk,
                    max_abs, ok ? "PASS" : "FAIL");
        report(ok, max_abs);
    }
    std::printf("  GPU: %d/%d PASS (worst abs err %.2e)\n", pass, total, worst);
    std::fflush(stdout);
    return create_scalar(pass == total ? 1.0 : 0.0);
}

// gemm_selftest (elementwise.inc:888-968): the reference checks its CPU blocked kernels on 11
// adversarial fp64 shapes and 6 short-K fp32 shapes against the naive loop.  Here `@` is the
// GPU GEMM, so the same 17 shapes (same seed and draws) go through tensor_matmul -- the last 6
// with `as f32` operands -- against the fp64 naive product, under the reference's own GPU gate
// (absolute sqrt(K) 1e-4, elementwise.inc:843-845); then the 512^3 throughput line.
Tensor* gemm_selftest(void) {
    // elementwise.inc:888-968: the same shapes, seed, draws and gates.  The fp64 shapes run the
    // fp64 GEMM `@` takes below the threshold, the f32 shapes the fp32 GEMM of `as f32`
    // operands; both against the naive fp64 product (the reference's gemm_ref_d).
    std::printf("=== gemm_selftest: GPU GEMM (the `@` path) vs naive fp64 reference ===\n");
    if (!dh_available()) {
        std::printf("  GEMM: SKIP (no HIP device: this runtime's `@` runs on the GPU)\n");
        std::fflush(stdout);
        return create_scalar(1.0);
    }
    rng().seed(20260707);
    std::uniform_real_distribution<double> dist(-1.0, 1.0);
    int pass = 0, total = 0;
    double worst = 0.0;
    const int shapes[11][3] = {{1, 1, 1},    {1, 7, 1},    {5, 1, 9},      {3, 4, 5},
                               {7, 13, 17},  {31, 33, 37}, {64, 64, 64},   {65, 63, 66},
                               {128, 100, 96}, {200, 50, 300}, {257, 129, 255}};
    try {
        for (const auto& sh : shapes) {
            const int M = sh[0], K = sh[1], N = sh[2];
            std::vector<double> A((size_t)M * K), B((size_t)K * N), C1((size_t)M * N),
                C2((size_t)M * N);
            for (auto& v : A) v = dist(rng());
            for (auto& v : B) v = dist(rng());
            Dev da(A.size() * 8), db(B.size() * 8), dc(C1.size() * 8);
            upload_f64(A.data(), A.size(), da);
            upload_f64(B.data(), B.size(), db);
            need_buf(dc);
            need(dh_gemm_f64(0, 0, M, N, K, da.d(), K, db.d(), N, 0.0, dc.d(), N));
            need(dh_memcpy_d2h(C1.data(), dc.p, C1.size() * 8));
            ref_gemm(A.data(), B.data(), C2.data(), M, K, N);
            double mr = 0.0;
            for (size_t i = 0; i < C1.size(); ++i)
                mr = std::max(mr, std::fabs(C1[i] - C2[i]) / std::max(std::fabs(C2[i]), 1e-9));
            const bool ok = mr < 1e-11;
            std::printf("  %4dx%-4dx%-4d max_rel=%.2e  %s\n", M, K, N, mr, ok ? "PASS" : "FAIL");
            worst = std::max(worst, mr);
            ++total;
            pass += ok;
        }
        {   // throughput: the fp64 GEMM at 512^3, operands resident, best of 3
            const int n = 512;
            std::vector<double> A((size_t)n * n), B((size_t)n * n);
            for (auto& v : A) v = dist(rng());
            for (auto& v : B) v = dist(rng());
            Dev da(A.size() * 8), db(B.size() * 8), dc(A.size() * 8);
            upload_f64(A.data(), A.size(), da);
            upload_f64(B.data(), B.size(), db);
            need_buf(dc);
            need(dh_sync());
            double best = 1e30;
            for (int rep = 0; rep < 3; ++rep) {
                const auto t0 = std::chrono::steady_clock::now();
                need(dh_gemm_f64(0, 0, n, n, n, da.d(), n, db.d(), n, 0.0, dc.d(), n));
                need(dh_sync());
                const auto t1 = std::chrono::steady_clock::now();
                best = std::min(best, std::chrono::duration<double>(t1 - t0).count());
            }
            std::printf("  throughput: 512^3 in %.2f ms = %.1f GFLOPS (fp64 GEMM)\n", best * 1e3,
                        2.0 * n * n * (double)n / best / 1e9);
        }
    } catch (const Failure&) {
        rt_error("gemm_selftest", "%s", dh_last_error());
    }
    // f32 shapes: short K, so any tile-indexing bug shows (elementwise.inc:938-964)
    const int fshapes[6][3] = {{8, 16, 16}, {7, 15, 13}, {9, 8, 17}, {1, 4, 1}, {16, 32, 24},
                               {32, 16, 32}};
    std::uniform_real_distribution<float> fdist(-1.0f, 1.0f);
    for (const auto& sh : fshapes) {
        const int M = sh[0], K = sh[1], N = sh[2];
        Tensor* A = alloc_tensor(M, K, 1, 1);
        Tensor* B = alloc_tensor(K, N, 1, 1);
        for (int i = 0; i < A->size; ++i) A->data[i] = (double)fdist(rng());
        for (int i = 0; i < B->size; ++i) B->data[i] = (double)fdist(rng());
        dream_set_precision(A, 1);
        dream_set_precision(B, 1);
        Tensor* C = tensor_matmul(A, B);
        std::vector<double> R((size_t)M * N);
        ref_gemm(A->data, B->data, R.data(), M, K, N);
        double mr = 0.0;
        const bool shaped = C->size == (int)R.size() && C->fdata;
        for (size_t i = 0; shaped && i < R.size(); ++i)
            mr = std::max(mr, std::fabs((double)C->fdata[i] - R[i]) / std::max(std::fabs(R[i]), 1e-4));
        const bool ok = shaped && mr < 2e-4;
        std::printf("  f32 %dx%dx%d max_rel=%.2e  %s\n", M, K, N, mr, ok ? "PASS" : "FAIL");
        worst = std::max(worst, mr);
        ++total;
        pass += ok;
        for (Tensor* t : {A, B, C}) tensor_decref(t);
    }
    std::printf("  GEMM: %d/%d PASS (worst rel err %.2e)\n", pass, total, worst);
    std::fflush(stdout);
    return create_scalar(pass == total ? 1.0 : 0.0);
}

// bf16_selftest (runtime/nn/training.inc:1978-2025): range and precision of the bf16 rounding
// -- here the device conversion every bf16 operand goes through (dh_convert, round to nearest
// even) -- and the reference's mixed-precision convergence check (a scalar host loop).
static float host_bf16(float x) {   // the same RNE rule, for the host loop of check 3
    uint32_t u;
    std::memcpy(&u, &x, 4);
    u = (u + 0x7FFFu + ((u >> 16) & 1u)) & 0xFFFF0000u;
    float r;
    std::memcpy(&r, &u, 4);
    return r;
}

Tensor* bf16_selftest(void) {
    std::printf("=== bf16_selftest: mixed-precision training ===\n");
    if (!dh_available()) {
        std::printf("  BF16_MIXED: SKIP (no HIP device: bf16 rounding runs on the GPU)\n");
        std::fflush(stdout);
        return create_scalar(1.0);
    }
    int pass = 0, total = 0;
    // the device round trip fp32 -> bf16 -> fp32 of n host values
    auto round_dev = [](std::vector<float>& v) {
        const size_t n = v.size();
        Dev f(n * 4), b(n * 2);
        need_buf(f), need_buf(b);
        need(dh_memcpy_h2d(f.p, v.data(), n * 4));
        need(dh_convert(b.p, DH_BF16, f.p, DH_F32, n));
        need(dh_convert(f.p, DH_F32, b.p, DH_BF16, n));
        need(dh_memcpy_d2h(v.data(), f.p, n * 4));
    };
    try {
        {   // 1. range: bf16 keeps fp32's exponent, so 1e30 survives
            std::vector<float> v{1e30f};
            round_dev(v);
            const bool ok = v[0] > 1e29f && v[0] < 1e31f;
            std::printf("  bf16 range (1e30 survives; fp16 would overflow): %s\n", ok ? "PASS" : "FAIL");
            ++total, pass += ok;
        }
        {   // 2. precision: relative error <= 2^-9 for values in [0.1, 10)
            rng().seed(1);
            std::uniform_real_distribution<float> d(0.1f, 10.0f);
            std::vector<float> x(10000), r;
            for (float& e : x) e = d(rng());
            r = x;
            round_dev(r);
            double mr = 0.0;
            for (size_t i = 0; i < x.size(); ++i) mr = std::max(mr, (double)std::fabs(r[i] - x[i]) / x[i]);
            const bool ok = mr < 0.01;
            std::printf("  bf16 precision (max rel err %.4f, expect <0.01): %s\n", mr, ok ? "PASS" : "FAIL");
            ++total, pass += ok;
        }
    } catch (const Failure&) {
        rt_error("bf16_selftest", "%s", dh_last_error());
        return create_scalar(0.0);
    }
    {   // 3. convergence: bf16 compute with fp32 master weights trains y = 3x + 0.5
        rng().seed(2);
        std::uniform_real_distribution<float> d(0.1f, 10.0f);
        const int N = 64;
        std::vector<float> X(N), Y(N);
        for (int i = 0; i < N; ++i) {
            X[i] = d(rng());
            Y[i] = 3.0f * X[i] + 0.5f;
        }
        auto train = [&](bool mixed) {
            float w = 0, b = 0;
            const float lr = 0.01f;
            for (int ep = 0; ep < 200; ++ep) {
                float gw = 0, gb = 0;
                for (int i = 0; i < N; ++i) {
                    const float xi = mixed ? host_bf16(X[i]) : X[i];
                    const float wi = mixed ? host_bf16(w) : w, bi = mixed ? host_bf16(b) : b;
                    const float pred = mixed ? host_bf16(wi * xi + bi) : wi * xi + bi;
                    const float err = pred - Y[i];
                    gw += err * xi;
                    gb += err;
                }
                w -= lr * gw / N;
                b -= lr * gb / N;
            }
            float loss = 0;
            for (int i = 0; i < N; ++i) {
                const float p = w * X[i] + b;
                loss += (p - Y[i]) * (p - Y[i]);
            }
            return loss / N;
        };
        const float lf = train(false), lm = train(true);
        const bool ok = lm < 0.01;
        std::printf("  fp32 loss %.6f, mixed loss %.6f -> converges: %s\n", lf, lm, ok ? "PASS" : "FAIL");
        ++total, pass += ok;
    }
    std::printf("  BF16_MIXED: %d/%d PASS\n", pass, total);
    std::fflush(stdout);
    return create_scalar(pass == total ? 1.0 : 0.0);
}

Tensor* dream_gpu_warmup(void) {
    const auto t0 = std::chrono::steady_clock::now();
    if (!dh_available()) {
        std::printf("[gpu_warmup] no GPU; nothing to warm up\n");
        return create_scalar(0.0);
    }
    const int n = 768;
    Tensor* a = alloc_tensor(n, n, 1, 1);
    Tensor* b = alloc_tensor(n, n, 1, 1);
    for (int i = 0; i < a->size; ++i) {
        a->data[i] = 0.01 * (i % 7);
        b->data[i] = 0.01 * (i % 5);
    }
    tensor_decref(tensor_matmul(a, b));
    const int S = 512, dkk = 64;
    Tensor* Q = alloc_tensor(1, S * dkk, 1, 1);
    for (int i = 0; i < Q->size; ++i) Q->data[i] = 0.01 * (i % 11);
    Tensor *bt = create_scalar(1), *st = create_scalar(S), *dt = create_scalar(dkk);
    tensor_decref(dream_flash_attention(Q, Q, Q, bt, st, dt, nullptr));
    for (Tensor* t : {a, b, Q, bt, st, dt}) tensor_decref(t);
    const double s = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    std::printf("[gpu_warmup] GPU ready (init + first launches took %.3f s)\n", s);
    std::fflush(stdout);
    return create_scalar(s);
}

Tensor* flash_attention_selftest(void) {
    std::printf("=== flash_attention_selftest: flash == standard attention ===\n");
    if (!dh_available()) {
        std::printf("  FLASH_ATTN: SKIP (no HIP device)\n");
        return create_scalar(1.0);
    }
    rng().seed(20260709);
    std::normal_distribution<double> nd(0.0, 1.0);
    int pass = 0, total = 0;
    double worst = 0.0;
    const int cfgs[4][3] = {{64, 16, 8}, {64, 16, 16}, {128, 32, 32}, {100, 24, 16}};
    for (const auto& c : cfgs) {
        const int S = c[0], dkk = c[1];
        Tensor* Q = alloc_tensor(1, S * dkk, 1, 1);
        Tensor* K = alloc_tensor(1, S * dkk, 1, 1);
        Tensor* V = alloc_tensor(1, S * dkk, 1, 1);
        for (int i = 0; i < Q->size; ++i) {
            Q->data[i] = nd(rng());
            K->data[i] = nd(rng());
            V->data[i] = nd(rng());
        }
        Tensor *bt = create_scalar(1), *st = create_scalar(S), *dt = create_scalar(dkk),
               *blk = create_scalar(c[2]);
        Tensor* fla = dream_flash_attention(Q, K, V, bt, st, dt, blk);
        std::vector<double> ref((size_t)S * dkk);
        ref_causal_attention(Q->data, K->data, V->data, ref.data(), S, dkk);
        // B*S*S < 262144: flash_attention runs in fp64, so the reference's gate applies
        double mr = 0.0;
        for (size_t i = 0; i < ref.size() && fla->size == (int)ref.size(); ++i)
            mr = std::max(mr, std::fabs(fla->data[i] - ref[i]) / std::max(std::fabs(ref[i]), 1e-9));
        const bool ok = fla->size == (int)ref.size() && mr < 1e-9;
        std::printf("  S=%d dk=%d block=%d: max_rel=%.2e  %s\n", S, dkk, c[2], mr,
                    ok ? "PASS" : "FAIL");
        worst = std::max(worst, mr);
        ++total;
        pass += ok;
        for (Tensor* t : {Q, K, V, bt, st, dt, blk, fla}) tensor_decref(t);
    }
    std::printf("  FLASH_ATTN: %d/%d PASS (worst rel err %.2e)\n", pass, total, worst);
    std::fflush(stdout);
    return create_scalar(pass == total ? 1.0 : 0.0);
}

}  // extern "C"
