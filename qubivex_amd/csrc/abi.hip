// The C ABI of include/qvkv.h: device handle, memory, staging of host arguments, and
// the kernel entry points (device-pointer `_async` forms and host-memory forms).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "internal.h"
#include "qvkv.h"

using qvkv::Geometry;

namespace {

thread_local std::string g_err;
thread_local int g_err_code = QVKV_OK;
thread_local qvkv::OomDetail g_oom;

int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    g_err_code = code;
    if (code != QVKV_E_OOM) g_oom = qvkv::OomDetail{};
    return code;
}

}  // namespace

int qvkv::set_error(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    g_err_code = code;
    if (code != QVKV_E_OOM) g_oom = qvkv::OomDetail{};
    return code;
}

void qvkv::set_oom(uint64_t requested, uint64_t used, uint64_t capacity) {
    g_oom = qvkv::OomDetail{requested, used, capacity};
}

qvkv::OomDetail qvkv::last_oom() { return g_oom; }

namespace {

int hip_fail(hipError_t e, const char *what) {
    return fail(QVKV_E_DEVICE, "hip device error: %s: %s", what, hipGetErrorString(e));
}

}  // namespace

// What the library keeps per hipStream_t a caller launches on: the kernels' index-error
// flag and the attention workspace.  Each stream has its own, so a caller's qvkv_check
// reports only what its own stream's kernels latched, and split-context attention
// launches on different streams never share partials.  Created on the first launch on
// the stream; freed by qvkv_close.
struct StreamState {
    hipStream_t stream = nullptr;
    int *d_err = nullptr;  // [0]: latched bits (ERR_*), [1]: taken by the last check
    void *ws = nullptr;    // attention workspace (partials of context chunks)
    uint64_t ws_bytes = 0;
    std::mutex check_mu;   // one check at a time per stream
    // The attention launches of this stream, one at a time: the workspace is grown (which
    // waits for this stream to drain) and handed to the launch under it.  Other streams'
    // calls never wait for it.
    std::mutex ws_mu;
};

struct qvkv_dev {
    int device = 0;
    hipStream_t stream = nullptr;  // the host-memory entry points' own stream
    StreamState *own = nullptr;    // its state
    std::vector<StreamState *> streams;  // every stream seen (guarded by mu)
    void *stage = nullptr;       // device staging for the host-memory entry points
    uint64_t stage_bytes = 0;
    hipEvent_t order_ev = nullptr;  // orders pool copies after a caller's stream
    hipEvent_t t0 = nullptr, t1 = nullptr;  // GPU time of a synchronous call
    // host_mu: the host-memory entry points, one at a time (the staging buffer and the
    // device stream's state are theirs); mu: the list of stream states (held briefly, never
    // across a wait).  Order: host_mu, then mu, then a stream's ws_mu.
    std::mutex host_mu, mu;
    std::atomic<uint64_t> used{0}, peak{0}, refused{0};
    std::atomic<uint64_t> uploads{0}, upload_bytes{0}, downloads{0}, download_bytes{0};
    std::atomic<uint64_t> submissions{0}, wait_ns{0}, timed{0}, gpu_ns{0}, last_gpu_ns{0};
    std::atomic<uint64_t> stream_waits{0};
    // TransferStats' remaining fields: activations_in / _out (bytes the host-memory entry
    // points stage in and copy back), transfer_ns (their copies' GPU time from events, plus
    // the synchronous write / read calls), fence_waits (host waits for completion),
    // submit_ns (host time in the library's calls outside those waits).
    std::atomic<uint64_t> act_in{0}, act_out{0}, transfer_ns{0}, fence_waits{0}, submit_ns{0};
    hipEvent_t c0 = nullptr, c1 = nullptr, d0 = nullptr, d1 = nullptr;  // copy intervals
    bool up_open = false, down_open = false;  // under host_mu: this call's copies recorded
    uint8_t *scratch = nullptr;  // this device's copy of `scratch` (allocation-free entry)
    int *scratch_err = nullptr;  // its error flag (the first 256 bytes)
    char name[256] = {0};
    // The caller's handle plus one per live buffer: a buffer may be freed after
    // qvkv_close (in any teardown order), and the struct goes with the last of them.
    std::atomic<int> refs{1};
    std::atomic<bool> closed{false};
};

namespace {
// The last reference (the caller's handle or a live buffer) also takes the device's stream
// and events: a buffer freed while, or after, the device closes still synchronizes on a
// valid (idle) stream.
void release(qvkv_dev *dev) {
    if (dev->refs.fetch_sub(1) != 1) return;
    (void)hipSetDevice(dev->device);
    if (dev->order_ev) (void)hipEventDestroy(dev->order_ev);
    for (hipEvent_t ev : {dev->c0, dev->c1, dev->d0, dev->d1})
        if (ev) (void)hipEventDestroy(ev);
    if (dev->t0) (void)hipEventDestroy(dev->t0);
    if (dev->t1) (void)hipEventDestroy(dev->t1);
    if (dev->stream) (void)hipStreamDestroy(dev->stream);
    delete dev;
}
}  // namespace

struct qvkv_buf {
    qvkv_dev *dev;
    void *ptr;
    size_t len;
};

// Scratch of the allocation-free attention entry point: the error flag of its kernels
// (the first 256 bytes) and the partial results of split-context launches.  Each GPU
// holds its own copy for the life of the process; host code reaches it only through
// the address hipGetSymbolAddress returns for the device (qvkv_dev::scratch).
static __device__ __align__(256) uint8_t scratch[QVKV_NOALLOC_SCRATCH_BYTES + 256];

namespace {

int set_device(qvkv_dev *dev) {
    hipError_t e = hipSetDevice(dev->device);
    return e == hipSuccess ? QVKV_OK : hip_fail(e, "hipSetDevice");
}

void account_alloc(qvkv_dev *dev, uint64_t n) {
    uint64_t u = dev->used.fetch_add(n) + n;
    uint64_t p = dev->peak.load();
    while (u > p && !dev->peak.compare_exchange_weak(p, u)) {
    }
}

int dev_malloc(qvkv_dev *dev, void **p, uint64_t n) {
    hipError_t e = hipMalloc(p, n ? n : 1);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        dev->refused.fetch_add(1);
        size_t fr = 0, tot = 0;
        (void)hipMemGetInfo(&fr, &tot);
        qvkv::set_oom(n, tot - fr, tot);
        return fail(QVKV_E_OOM,
                    "hip device is out of memory: %llu bytes requested, %llu of %llu in use",
                    (unsigned long long)n, (unsigned long long)(tot - fr),
                    (unsigned long long)tot);
    }
    account_alloc(dev, n);
    return QVKV_OK;
}

void dev_free(qvkv_dev *dev, void *p, uint64_t n) {
    if (!p) return;
    (void)hipFree(p);
    dev->used.fetch_sub(n);
}

// Grows a device buffer used only on stream `s` to at least `need` bytes (contents not
// kept).  Waits for `s` first, so no enqueued work still reads the old buffer.
int ensure(qvkv_dev *dev, hipStream_t s, void **buf, uint64_t *have, uint64_t need) {
    if (*have >= need) return QVKV_OK;
    hipError_t e = hipStreamSynchronize(s);
    if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
    dev_free(dev, *buf, *have);
    *buf = nullptr;
    *have = 0;
    uint64_t sz = std::max<uint64_t>(need, 1 << 20);
    sz = (sz + 4095) & ~4095ull;
    int rc = dev_malloc(dev, buf, sz);
    if (rc) return rc;
    *have = sz;
    return QVKV_OK;
}

// The attention workspace of a stream grown for a plan (partials of context chunks).
int ensure_attention(qvkv_dev *dev, StreamState *st, const qvkv::AttnPlan &p) {
    if (!p.ws_bytes) return QVKV_OK;
    return ensure(dev, st->stream, &st->ws, &st->ws_bytes, p.ws_bytes);
}

// The state of `stream`, created on first use.  Caller holds dev->mu.
int state_locked(qvkv_dev *dev, hipStream_t stream, StreamState **out) {
    for (StreamState *st : dev->streams)
        if (st->stream == stream) {
            *out = st;
            return QVKV_OK;
        }
    auto *st = new StreamState();
    st->stream = stream;
    if (int rc = dev_malloc(dev, (void **)&st->d_err, 256)) {
        delete st;
        return rc;
    }
    const int zero[64] = {};
    hipError_t e = hipMemcpy(st->d_err, zero, sizeof zero, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        dev_free(dev, st->d_err, 256);
        delete st;
        return hip_fail(e, "hipMemcpy (error flag)");
    }
    dev->streams.push_back(st);
    *out = st;
    return QVKV_OK;
}

int state_of(qvkv_dev *dev, void *stream, StreamState **out) {
    std::lock_guard<std::mutex> lk(dev->mu);
    return state_locked(dev, (hipStream_t)stream, out);
}

}  // namespace

int qvkv::use_device(qvkv_dev *dev) { return set_device(dev); }

namespace {

int geometry(const qvkv_layout *l, Geometry *g) {
    const char *why = "";
    int rc = qvkv::make_geometry(l, g, &why);
    return rc ? fail(rc, "shape mismatch in kv layout: %s", why) : QVKV_OK;
}

// Stages host arrays into the device staging buffer (16-byte aligned pieces).
struct Stager {
    struct Piece {
        const void *src;
        uint64_t len;
        uint64_t off;
    };
    std::vector<Piece> pieces;
    uint64_t total = 0;
    uint64_t add(const void *src, uint64_t len) {
        uint64_t off = total;
        pieces.push_back({src, len, off});
        total += (len + 255) & ~255ull;
        return off;
    }
    uint64_t reserve(uint64_t len) { return add(nullptr, len); }
    int upload(qvkv_dev *dev) {
        int rc = ensure(dev, dev->stream, &dev->stage, &dev->stage_bytes, total);
        if (rc) return rc;
        (void)hipEventRecord(dev->c0, dev->stream);
        for (auto &p : pieces) {
            if (!p.src || !p.len) continue;
            hipError_t e = hipMemcpyAsync((char *)dev->stage + p.off, p.src, p.len,
                                          hipMemcpyHostToDevice, dev->stream);
            if (e != hipSuccess) return hip_fail(e, "hipMemcpyAsync (upload)");
            dev->uploads.fetch_add(1);
            dev->upload_bytes.fetch_add(p.len);
            dev->act_in.fetch_add(p.len);
        }
        (void)hipEventRecord(dev->c1, dev->stream);
        dev->up_open = true;
        return QVKV_OK;
    }
    template <class T>
    T *at(qvkv_dev *dev, uint64_t off) {
        return (T *)((char *)dev->stage + off);
    }
};

// A copy back on the device's stream (caller holds host_mu); the call's copies back are
// timed from before the first to after the last.
int download(qvkv_dev *dev, void *host, const void *devp, uint64_t len, bool output = true) {
    if (!len) return QVKV_OK;
    if (output) dev->act_out.fetch_add(len);
    if (!dev->down_open) (void)hipEventRecord(dev->d0, dev->stream);
    hipError_t e = hipMemcpyAsync(host, devp, len, hipMemcpyDeviceToHost, dev->stream);
    if (e != hipSuccess) return hip_fail(e, "hipMemcpyAsync (download)");
    (void)hipEventRecord(dev->d1, dev->stream);
    dev->down_open = true;
    dev->downloads.fetch_add(1);
    dev->download_bytes.fetch_add(len);
    return QVKV_OK;
}

// After the device's stream has drained: the GPU time of this call's copies into
// transfer_ns (caller holds host_mu).
void take_copy_time(qvkv_dev *dev) {
    float ms = 0.f;
    if (dev->up_open && hipEventElapsedTime(&ms, dev->c0, dev->c1) == hipSuccess)
        dev->transfer_ns.fetch_add((uint64_t)((double)ms * 1e6));
    if (dev->down_open && hipEventElapsedTime(&ms, dev->d0, dev->d1) == hipSuccess)
        dev->transfer_ns.fetch_add((uint64_t)((double)ms * 1e6));
    (void)hipGetLastError();
    dev->up_open = dev->down_open = false;
}

// Host time waiting for the device on this thread (finish, write, read): a call's
// submit time is its host time less this.
thread_local uint64_t t_wait_ns = 0;

uint64_t now_ns() {
    return (uint64_t)std::chrono::duration_cast<std::chrono::nanoseconds>(
               std::chrono::steady_clock::now().time_since_epoch())
        .count();
}

// Adds the host time of one library call, less its waits, to submit_ns.
struct SubmitTimer {
    qvkv_dev *dev;
    uint64_t t0, w0;
    explicit SubmitTimer(qvkv_dev *d) : dev(d), t0(now_ns()), w0(t_wait_ns) {}
    ~SubmitTimer() {
        if (!dev) return;
        const uint64_t spent = now_ns() - t0, waited = t_wait_ns - w0;
        dev->submit_ns.fetch_add(spent > waited ? spent - waited : 0);
    }
};

// A host wait for the device: counted in fence_waits and wait_ns.
hipError_t fence_wait(qvkv_dev *dev, hipStream_t s) {
    const uint64_t t0 = now_ns();
    hipError_t e = hipStreamSynchronize(s);
    const uint64_t dt = now_ns() - t0;
    t_wait_ns += dt;
    dev->wait_ns.fetch_add(dt);
    dev->fence_waits.fetch_add(1);
    return e;
}

// Takes latched error bits: one thread exchanges each flag with 0 (so bits a kernel
// latches meanwhile are never lost) and leaves what they held in the calling stream's own
// flag[1].  `other` is the device-wide flag of the allocation-free entry point (may be
// null): what it held goes to this stream's slot too, never to a slot another stream's
// check also writes.
__global__ void k_take_error(int *flag, int *other) {
    if (threadIdx.x == 0) flag[1] = atomicExch(&flag[0], 0) | (other ? atomicExch(&other[0], 0) : 0);
}

// The status a set of latched bits stands for.
int status_of(int bits) {
    if (!bits) return QVKV_OK;
    if (bits == 16)
        return fail(QVKV_E_UNSUPPORTED,
                    "q8_0 prefill: a value scale above 512 (dequantised values past the f16 "
                    "range of the MFMA prefill; the knob prefill_q8_fast=0 selects the form "
                    "without that limit)");
    return fail(QVKV_E_SHAPE, "shape mismatch in kv kernel: %s%s%s%s%s",
                (bits & 1) ? "a block id past the pool; " : "",
                (bits & 2) ? "a block table shorter than its positions; " : "",
                (bits & 4) ? "a position past max_pos; " : "",
                (bits & 8) ? "an output or query range past its bound (out_positions, q_rows); " : "",
                (bits & 16) ? "a q8_0 value scale past the f16 prefill's range; " : "");
}

// Waits for the stream's work and turns the index errors its kernels latched into
// QVKV_E_SHAPE (clearing them).
int finish(qvkv_dev *dev, StreamState *st) {
    std::lock_guard<std::mutex> lk(st->check_mu);
    int *other = dev->scratch_err;
    hipLaunchKernelGGL(k_take_error, dim3(1), dim3(64), 0, st->stream, st->d_err, other);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, "error flag launch");
    int bits = 0;
    e = hipMemcpyAsync(&bits, st->d_err + 1, sizeof bits, hipMemcpyDeviceToHost, st->stream);
    if (e != hipSuccess) return hip_fail(e, "hipMemcpyAsync (error flag)");
    e = fence_wait(dev, st->stream);
    if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
    return status_of(bits);
}

int launched(qvkv_dev *dev, hipError_t e, const char *what) {
    if (e != hipSuccess) return hip_fail(e, what);
    dev->submissions.fetch_add(1);
    return QVKV_OK;
}

// GPU time of a synchronous call: events on the device's stream around its kernels
// (time_start before the first launch, time_stop after the last, time_take once done).
void time_start(qvkv_dev *dev) { (void)hipEventRecord(dev->t0, dev->stream); }
void time_stop(qvkv_dev *dev) { (void)hipEventRecord(dev->t1, dev->stream); }
void time_take(qvkv_dev *dev);

// finish() of the device's own stream after a timed synchronous call.
int finish_timed(qvkv_dev *dev) {
    const int rc = finish(dev, dev->own);
    if (rc == QVKV_OK) time_take(dev);
    take_copy_time(dev);
    return rc;
}

void time_take(qvkv_dev *dev) {
    float ms = 0.f;
    if (hipEventElapsedTime(&ms, dev->t0, dev->t1) != hipSuccess) {
        (void)hipGetLastError();
        return;
    }
    const uint64_t ns = (uint64_t)((double)ms * 1e6);
    dev->last_gpu_ns.store(ns);
    dev->gpu_ns.fetch_add(ns);
    dev->timed.fetch_add(1);
}

}  // namespace

extern "C" {

int qvkv_last_error(char *buf, size_t len) {
    if (buf && len) {
        size_t n = std::min(len - 1, g_err.size());
        memcpy(buf, g_err.data(), n);
        buf[n] = 0;
    }
    return g_err_code;
}

int qvkv_last_oom(uint64_t *requested, uint64_t *used, uint64_t *capacity) {
    const qvkv::OomDetail d = qvkv::last_oom();
    if (requested) *requested = d.requested;
    if (used) *used = d.used;
    if (capacity) *capacity = d.capacity;
    return QVKV_OK;
}

int qvkv_open(int device, qvkv_dev **out) {
    if (!out) return fail(QVKV_E_SHAPE, "null output handle");
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count <= device || device < 0)
        return fail(QVKV_E_DEVICE, "hip device error: no device %d (%d present)", device, count);
    auto *d = new qvkv_dev();
    d->device = device;
    if (int rc = set_device(d)) { delete d; return rc; }
    hipDeviceProp_t prop;
    if ((e = hipGetDeviceProperties(&prop, device)) != hipSuccess) {
        delete d;
        return hip_fail(e, "hipGetDeviceProperties");
    }
    snprintf(d->name, sizeof d->name, "hip:%d %s (%s, %d CUs, %.1f GiB)", device, prop.name,
             prop.gcnArchName, prop.multiProcessorCount, prop.totalGlobalMem / 1073741824.0);
    if ((e = hipStreamCreateWithFlags(&d->stream, hipStreamNonBlocking)) != hipSuccess) {
        delete d;
        return hip_fail(e, "hipStreamCreate");
    }
    if ((e = hipEventCreateWithFlags(&d->order_ev, hipEventDisableTiming)) != hipSuccess ||
        (e = hipEventCreate(&d->t0)) != hipSuccess || (e = hipEventCreate(&d->t1)) != hipSuccess ||
        (e = hipEventCreate(&d->c0)) != hipSuccess || (e = hipEventCreate(&d->c1)) != hipSuccess ||
        (e = hipEventCreate(&d->d0)) != hipSuccess || (e = hipEventCreate(&d->d1)) != hipSuccess) {
        qvkv_close(d);
        return hip_fail(e, "hipEventCreate");
    }
    {
        std::lock_guard<std::mutex> lk(d->mu);
        if (int rc = state_locked(d, d->stream, &d->own)) {
            qvkv_close(d);
            return rc;
        }
    }
    // This device's copy of the scratch array (device `device` is current), with its
    // error flag cleared.
    if ((e = hipGetSymbolAddress((void **)&d->scratch, HIP_SYMBOL(scratch))) != hipSuccess) {
        d->scratch = nullptr;
        qvkv_close(d);
        return hip_fail(e, "hipGetSymbolAddress (scratch)");
    }
    {
        const int zero[64] = {};
        if ((e = hipMemcpy(d->scratch, zero, sizeof zero, hipMemcpyHostToDevice)) != hipSuccess) {
            qvkv_close(d);
            return hip_fail(e, "hipMemcpy (scratch error flag)");
        }
        d->scratch_err = (int *)d->scratch;
    }
    *out = d;
    return QVKV_OK;
}

void qvkv_close(qvkv_dev *dev) {
    if (!dev) return;
    (void)hipSetDevice(dev->device);
    // Work may still be in flight on any stream the device's states belong to.
    (void)hipDeviceSynchronize();
    for (StreamState *st : dev->streams) {
        dev_free(dev, st->ws, st->ws_bytes);
        dev_free(dev, st->d_err, 256);
        delete st;
    }
    dev->streams.clear();
    dev_free(dev, dev->stage, dev->stage_bytes);
    dev->stage = nullptr;
    dev->stage_bytes = 0;
    dev->closed.store(true);
    release(dev);  // the stream and events go with the last reference
}

int qvkv_describe(const qvkv_dev *dev, char *buf, size_t len) {
    if (!dev) return fail(QVKV_E_SHAPE, "null device");
    if (buf && len) snprintf(buf, len, "%s", dev->name);
    return QVKV_OK;
}

int qvkv_usage(const qvkv_dev *dev, qvkv_usage_t *out) {
    if (!dev || !out) return fail(QVKV_E_SHAPE, "null argument");
    size_t fr = 0, tot = 0;
    (void)hipSetDevice(dev->device);
    hipError_t e = hipMemGetInfo(&fr, &tot);
    if (e != hipSuccess) return hip_fail(e, "hipMemGetInfo");
    out->capacity = tot;
    out->used = dev->used.load();
    out->peak = dev->peak.load();
    out->refused = dev->refused.load();
    return QVKV_OK;
}

int qvkv_max_arena(const qvkv_dev *dev, uint64_t *out) {
    if (!dev || !out) return fail(QVKV_E_SHAPE, "null argument");
    size_t fr = 0, tot = 0;
    (void)hipSetDevice(dev->device);
    hipError_t e = hipMemGetInfo(&fr, &tot);
    if (e != hipSuccess) return hip_fail(e, "hipMemGetInfo");
    *out = tot;
    return QVKV_OK;
}

int qvkv_tune(const char *name, int value) { return qvkv::set_tune(name, value); }
int qvkv_tune_get(const char *name, int *value) { return qvkv::get_tune(name, value); }
void qvkv_tune_reset(void) { qvkv::reset_tune(); }

int qvkv_transfers(const qvkv_dev *dev, qvkv_transfers_t *out) {
    if (!dev || !out) return fail(QVKV_E_SHAPE, "null argument");
    out->uploads = dev->uploads.load();
    out->upload_bytes = dev->upload_bytes.load();
    out->downloads = dev->downloads.load();
    out->download_bytes = dev->download_bytes.load();
    out->submissions = dev->submissions.load();
    out->wait_ns = dev->wait_ns.load();
    out->timed = dev->timed.load();
    out->gpu_ns = dev->gpu_ns.load();
    out->stream_waits = dev->stream_waits.load();
    out->activations_in = dev->act_in.load();
    out->activations_out = dev->act_out.load();
    out->transfer_ns = dev->transfer_ns.load();
    out->fence_waits = dev->fence_waits.load();
    out->submit_ns = dev->submit_ns.load();
    // the timed calls run one at a time on the device's own stream (host_mu): their GPU
    // intervals never overlap, so their union is their sum
    out->gpu_busy_ns = dev->gpu_ns.load();
    return QVKV_OK;
}

int qvkv_timing(const qvkv_dev *dev, uint64_t *gpu_ns) {
    if (!dev || !gpu_ns) return fail(QVKV_E_SHAPE, "null argument");
    *gpu_ns = dev->last_gpu_ns.load();
    return QVKV_OK;
}

void *qvkv_stream(const qvkv_dev *dev) { return dev ? (void *)dev->stream : nullptr; }

int qvkv_alloc(qvkv_dev *dev, size_t len, qvkv_buf **out) {
    if (!dev || !out) return fail(QVKV_E_SHAPE, "null argument");
    if (int rc = set_device(dev)) return rc;
    void *p = nullptr;
    if (int rc = dev_malloc(dev, &p, len)) return rc;
    dev->refs.fetch_add(1);
    *out = new qvkv_buf{dev, p, len};
    return QVKV_OK;
}

void qvkv_free(qvkv_buf *buf) {
    if (!buf) return;
    qvkv_dev *dev = buf->dev;
    (void)hipSetDevice(dev->device);
    // In-flight work on the device's stream may still read the buffer (a closed device
    // was synchronized by qvkv_close; its stream stays valid while this buffer holds it).
    if (!dev->closed.load()) (void)hipStreamSynchronize(dev->stream);
    dev_free(dev, buf->ptr, buf->len);
    delete buf;
    release(dev);
}

void *qvkv_buf_ptr(const qvkv_buf *buf) { return buf ? buf->ptr : nullptr; }
size_t qvkv_buf_len(const qvkv_buf *buf) { return buf ? buf->len : 0; }

int qvkv_write(qvkv_dev *dev, qvkv_buf *buf, size_t offset, const void *host, size_t len) {
    if (!dev || !buf || (!host && len)) return fail(QVKV_E_SHAPE, "null argument");
    if (buf->dev != dev) return fail(QVKV_E_DEVICE, "hip device error: a buffer of another device");
    if (offset > buf->len || len > buf->len - offset)
        return fail(QVKV_E_DEVICE, "hip device error: write of %zu bytes at %zu past a %zu-byte buffer",
                    len, offset, buf->len);
    SubmitTimer timer(dev);
    std::lock_guard<std::mutex> lk(dev->host_mu);
    if (int rc = set_device(dev)) return rc;
    const uint64_t t0 = now_ns();
    hipError_t e = hipMemcpyAsync((char *)buf->ptr + offset, host, len, hipMemcpyHostToDevice,
                                  dev->stream);
    if (e != hipSuccess) return hip_fail(e, "hipMemcpyAsync (write)");
    dev->uploads.fetch_add(1);
    dev->upload_bytes.fetch_add(len);
    e = fence_wait(dev, dev->stream);
    dev->transfer_ns.fetch_add(now_ns() - t0);
    return e == hipSuccess ? QVKV_OK : hip_fail(e, "hipStreamSynchronize");
}

int qvkv_read(qvkv_dev *dev, const qvkv_buf *buf, size_t offset, void *host, size_t len) {
    if (!dev || !buf || (!host && len)) return fail(QVKV_E_SHAPE, "null argument");
    if (buf->dev != dev) return fail(QVKV_E_DEVICE, "hip device error: a buffer of another device");
    if (offset > buf->len || len > buf->len - offset)
        return fail(QVKV_E_DEVICE, "hip device error: read of %zu bytes at %zu past a %zu-byte buffer",
                    len, offset, buf->len);
    SubmitTimer timer(dev);
    std::lock_guard<std::mutex> lk(dev->host_mu);
    if (int rc = set_device(dev)) return rc;
    if (int rc = download(dev, host, (const char *)buf->ptr + offset, len, false)) return rc;
    hipError_t e = fence_wait(dev, dev->stream);
    take_copy_time(dev);
    return e == hipSuccess ? QVKV_OK : hip_fail(e, "hipStreamSynchronize");
}

int qvkv_check(qvkv_dev *dev, void *stream) {
    if (!dev) return fail(QVKV_E_SHAPE, "null device");
    if (int rc = set_device(dev)) return rc;
    StreamState *st;
    if (int rc = state_of(dev, stream, &st)) return rc;
    return finish(dev, st);
}

int qvkv_block_bytes(const qvkv_layout *layout, uint64_t *out) {
    Geometry g;
    if (int rc = geometry(layout, &g)) return rc;
    if (out) *out = g.block_bytes;
    return QVKV_OK;
}

// ---------------------------------------------------------------------------------
// device-pointer forms
// ---------------------------------------------------------------------------------

int qvkv_append_async(qvkv_dev *dev, const qvkv_layout *layout, void *pool,
                      uint64_t pool_blocks, const float *k, const float *v,
                      const uint32_t *slots, uint32_t n, void *stream) {
    if (!dev) return fail(QVKV_E_SHAPE, "null device");
    SubmitTimer timer(dev);
    Geometry g;
    if (int rc = geometry(layout, &g)) return rc;
    if (n == 0) return QVKV_OK;
    if (!pool || !k || !v || !slots) return fail(QVKV_E_SHAPE, "shape mismatch in append: null pointer");
    if (int rc = set_device(dev)) return rc;
    StreamState *st;
    if (int rc = state_of(dev, stream, &st)) return rc;
    return launched(dev, qvkv::launch_append(g, pool, pool_blocks, k, v, slots, n, st->d_err,
                                             st->stream),
                    "append launch");
}

int qvkv_gather_async(qvkv_dev *dev, const qvkv_layout *layout, const void *pool,
                      uint64_t pool_blocks, const uint32_t *blocks, uint64_t n_table,
                      const uint32_t *table_at, const uint32_t *lens, const uint64_t *out_at,
                      uint32_t n_items, uint32_t max_len, uint32_t out_dtype,
                      uint64_t out_positions, void *out_k, void *out_v, void *stream) {
    if (!dev) return fail(QVKV_E_SHAPE, "null device");
    SubmitTimer timer(dev);
    Geometry g;
    if (int rc = geometry(layout, &g)) return rc;
    if (out_dtype != QVKV_F32 && !(out_dtype == QVKV_F16 && g.dtype == QVKV_F16))
        return fail(QVKV_E_UNSUPPORTED, "hip backend has no gather kernel for this output dtype");
    if (n_items == 0 || max_len == 0) return QVKV_OK;
    if (!pool || !blocks || !table_at || !lens || !out_at || !out_k || !out_v)
        return fail(QVKV_E_SHAPE, "shape mismatch in gather: null pointer");
    if (int rc = set_device(dev)) return rc;
    StreamState *st;
    if (int rc = state_of(dev, stream, &st)) return rc;
    return launched(dev, qvkv::launch_gather(g, pool, pool_blocks, blocks, n_table, table_at,
                                             lens, out_at, n_items, max_len, (int)out_dtype,
                                             out_positions, out_k, out_v, st->d_err, st->stream),
                    "gather launch");
}

int qvkv_attention_async(qvkv_dev *dev, const qvkv_layout *layout, const void *pool,
                         uint64_t pool_blocks, const float *q, const uint32_t *blocks,
                         uint64_t n_table, const uint32_t *table_at, const uint32_t *pos,
                         uint32_t n_items, uint32_t heads, uint32_t max_pos, float *out,
                         void *stream) {
    if (!dev) return fail(QVKV_E_SHAPE, "null device");
    SubmitTimer timer(dev);
    Geometry g;
    if (int rc = geometry(layout, &g)) return rc;
    qvkv::AttnPlan p;
    const char *why = "";
    if (int rc = qvkv::plan_attention(g, n_items, heads, max_pos, &p, &why))
        return fail(rc, "shape mismatch in attention: %s", why);
    if (n_items == 0) return QVKV_OK;
    if (!pool || !q || !blocks || !table_at || !pos || !out)
        return fail(QVKV_E_SHAPE, "shape mismatch in attention: null pointer");
    if (int rc = set_device(dev)) return rc;
    // The stream's workspace is grown and handed to the launch under that stream's own
    // lock, so no other thread frees it in between; launches on one stream use it in turn,
    // and a growth that waits for this stream to drain holds up no other stream's calls.
    // The device's own stream is also the host-memory entry points': take their lock too.
    std::unique_lock<std::mutex> host_lk(dev->host_mu, std::defer_lock);
    if ((hipStream_t)stream == dev->stream) host_lk.lock();
    StreamState *st;
    if (int rc = state_of(dev, stream, &st)) return rc;
    std::lock_guard<std::mutex> wl(st->ws_mu);
    if (int rc = ensure_attention(dev, st, p)) return rc;
    return launched(dev, qvkv::launch_attention(g, p, pool, pool_blocks, q, blocks, n_table,
                                                table_at, pos, n_items, heads, max_pos, out,
                                                st->ws, st->d_err, st->stream),
                    "attention launch");
}

int qvkv_append_attention_async(qvkv_dev *dev, const qvkv_layout *layout, void *pool,
                                uint64_t pool_blocks, const float *q, const float *k_new,
                                const float *v_new, const uint32_t *blocks, uint64_t n_table,
                                const uint32_t *table_at, const uint32_t *pos, uint32_t n_items,
                                uint32_t heads, uint32_t max_pos, float *out, void *stream) {
    if (!dev) return fail(QVKV_E_SHAPE, "null device");
    SubmitTimer timer(dev);
    Geometry g;
    if (int rc = geometry(layout, &g)) return rc;
    qvkv::AttnPlan p;
    const char *why = "";
    if (int rc = qvkv::plan_attention(g, n_items, heads, max_pos, &p, &why))
        return fail(rc, "shape mismatch in attention: %s", why);
    if (n_items == 0) return QVKV_OK;
    if (!pool || !q || !k_new || !v_new || !blocks || !table_at || !pos || !out)
        return fail(QVKV_E_SHAPE, "shape mismatch in attention: null pointer");
    if (int rc = set_device(dev)) return rc;
    std::unique_lock<std::mutex> host_lk(dev->host_mu, std::defer_lock);
    if ((hipStream_t)stream == dev->stream) host_lk.lock();
    StreamState *st;
    if (int rc = state_of(dev, stream, &st)) return rc;
    std::lock_guard<std::mutex> wl(st->ws_mu);
    const bool fused = qvkv::fused_append_attention(g);
    // unfused: the items' slots after the attention workspace, then append + attention
    const uint64_t slots_at = (p.ws_bytes + 255) / 256 * 256;
    qvkv::AttnPlan pw = p;
    if (!fused) pw.ws_bytes = slots_at + (uint64_t)n_items * 4;
    if (int rc = ensure_attention(dev, st, pw)) return rc;
    if (fused) {
        qvkv::NewRows nr;
        nr.k = k_new;
        nr.v = v_new;
        return launched(dev, qvkv::launch_attention(g, p, pool, pool_blocks, q, blocks, n_table,
                                                    table_at, pos, n_items, heads, max_pos, out,
                                                    st->ws, st->d_err, st->stream, nr),
                        "append + attention launch");
    }
    uint32_t *slots = (uint32_t *)((uint8_t *)st->ws + slots_at);
    hipError_t e = qvkv::launch_slots_at(g, blocks, n_table, table_at, pos, n_items, max_pos,
                                         slots, st->d_err, st->stream);
    if (e == hipSuccess)
        e = qvkv::launch_append(g, pool, pool_blocks, k_new, v_new, slots, n_items, st->d_err,
                                st->stream);
    if (e == hipSuccess)
        e = qvkv::launch_attention(g, p, pool, pool_blocks, q, blocks, n_table, table_at, pos,
                                   n_items, heads, max_pos, out, st->ws, st->d_err, st->stream);
    return launched(dev, e, "append + attention launch");
}

int qvkv_attention_noalloc_async(qvkv_dev *dev, const qvkv_layout *layout, const void *pool,
                                 uint64_t pool_blocks, const float *q, const uint32_t *blocks,
                                 uint64_t n_table, const uint32_t *table_at, const uint32_t *pos,
                                 uint32_t n_items, uint32_t heads, uint32_t max_pos, float *out,
                                 void *stream) {
    if (!dev) return fail(QVKV_E_SHAPE, "null device");
    SubmitTimer timer(dev);
    Geometry g;
    if (int rc = geometry(layout, &g)) return rc;
    qvkv::AttnPlan p;
    const char *why = "";
    if (int rc = qvkv::plan_attention(g, n_items, heads, max_pos, &p, &why))
        return fail(rc, "shape mismatch in attention: %s", why);
    if (p.ws_bytes > QVKV_NOALLOC_SCRATCH_BYTES)
        return fail(QVKV_E_SHAPE,
                    "shape mismatch in attention: the launch needs %llu bytes of scratch for its "
                    "context-chunk partials, past the allocation-free form's %llu",
                    (unsigned long long)p.ws_bytes,
                    (unsigned long long)QVKV_NOALLOC_SCRATCH_BYTES);
    if (n_items == 0) return QVKV_OK;
    if (!pool || !q || !blocks || !table_at || !pos || !out)
        return fail(QVKV_E_SHAPE, "shape mismatch in attention: null pointer");
    if (!dev->scratch) return fail(QVKV_E_DEVICE, "hip device error: no scratch address");
    if (int rc = set_device(dev)) return rc;
    return launched(dev, qvkv::launch_attention(g, p, pool, pool_blocks, q, blocks, n_table,
                                                table_at, pos, n_items, heads, max_pos, out,
                                                dev->scratch + 256, dev->scratch_err,
                                                (hipStream_t)stream),
                    "attention launch");
}

int qvkv_prefill_attention_async(qvkv_dev *dev, const qvkv_layout *layout, const void *pool,
                                 uint64_t pool_blocks, const float *q, uint64_t q_rows,
                                 const uint32_t *blocks, uint64_t n_table,
                                 const uint32_t *table_at, const uint32_t *pos0,
                                 const uint32_t *q_at, const uint32_t *n_tok, uint32_t n_seg,
                                 uint32_t heads, uint32_t max_pos, uint32_t max_tok, float *out,
                                 void *stream) {
    if (!dev) return fail(QVKV_E_SHAPE, "null device");
    SubmitTimer timer(dev);
    Geometry g;
    if (int rc = geometry(layout, &g)) return rc;
    const char *why = "";
    if (int rc = qvkv::check_prefill(g, n_seg, heads, max_tok, &why))
        return fail(rc, "shape mismatch in prefill attention: %s", why);
    if (n_seg == 0 || max_tok == 0) return QVKV_OK;
    if (!pool || !q || !blocks || !table_at || !pos0 || !q_at || !n_tok || !out)
        return fail(QVKV_E_SHAPE, "shape mismatch in prefill attention: null pointer");
    if (int rc = set_device(dev)) return rc;
    StreamState *st;
    if (int rc = state_of(dev, stream, &st)) return rc;
    return launched(dev, qvkv::launch_prefill(g, pool, pool_blocks, q, blocks, n_table, table_at,
                                              pos0, q_at, n_tok, n_seg, heads, max_pos, max_tok,
                                              q_rows, out, st->d_err, st->stream),
                    "prefill attention launch");
}

int qvkv_block_copy_async(qvkv_dev *dev, const qvkv_layout *layout, void *pool,
                          uint64_t pool_blocks, const uint32_t *src, const uint32_t *dst,
                          uint32_t n, void *stream) {
    if (!dev) return fail(QVKV_E_SHAPE, "null device");
    SubmitTimer timer(dev);
    Geometry g;
    if (int rc = geometry(layout, &g)) return rc;
    if (n == 0) return QVKV_OK;
    if (!pool || !src || !dst) return fail(QVKV_E_SHAPE, "shape mismatch in block copy: null pointer");
    if (int rc = set_device(dev)) return rc;
    StreamState *st;
    if (int rc = state_of(dev, stream, &st)) return rc;
    return launched(dev, qvkv::launch_block_copy(g, pool, pool_blocks, src, dst, n, st->d_err,
                                                 st->stream),
                    "block copy launch");
}

// ---------------------------------------------------------------------------------
// host-memory forms (synchronous)
// ---------------------------------------------------------------------------------

static int pool_of(const qvkv_dev *dev, const qvkv_buf *pool, const Geometry &g, uint64_t *blocks) {
    if (!pool) return fail(QVKV_E_SHAPE, "shape mismatch: null pool");
    if (pool->dev != dev) return fail(QVKV_E_DEVICE, "hip device error: a pool of another device");
    *blocks = pool->len / g.block_bytes;
    return QVKV_OK;
}

int qvkv_append(qvkv_dev *dev, const qvkv_layout *layout, qvkv_buf *pool, const float *k,
                const float *v, const uint32_t *slots, uint32_t n) {
    if (!dev) return fail(QVKV_E_SHAPE, "null device");
    SubmitTimer timer(dev);
    Geometry g;
    if (int rc = geometry(layout, &g)) return rc;
    uint64_t held;
    if (int rc = pool_of(dev, pool, g, &held)) return rc;
    if (n == 0) return QVKV_OK;
    if (!k || !v || !slots) return fail(QVKV_E_SHAPE, "shape mismatch in append: null pointer");
    for (uint32_t r = 0; r < n; r++)
        if (slots[r] / g.B >= held)
            return fail(QVKV_E_SHAPE, "shape mismatch in append: slot %u is in a block past the pool's %llu",
                        slots[r], (unsigned long long)held);
    std::lock_guard<std::mutex> lk(dev->host_mu);
    if (int rc = set_device(dev)) return rc;
    Stager st;
    const uint64_t rowb = g.kv_out * 4;
    uint64_t ko = st.add(k, n * rowb), vo = st.add(v, n * rowb), so = st.add(slots, n * 4ull);
    if (int rc = st.upload(dev)) return rc;
    time_start(dev);
    if (int rc = launched(dev, qvkv::launch_append(g, pool->ptr, held, st.at<float>(dev, ko),
                                                   st.at<float>(dev, vo),
                                                   st.at<uint32_t>(dev, so), n, dev->own->d_err,
                                                   dev->stream),
                          "append launch"))
        return rc;
    time_stop(dev);
    return finish_timed(dev);
}

int qvkv_gather(qvkv_dev *dev, const qvkv_layout *layout, const qvkv_buf *pool,
                const uint32_t *blocks, uint64_t n_table, const uint32_t *table_at,
                const uint32_t *lens, const uint64_t *out_at, uint32_t n_items,
                uint32_t out_dtype, uint64_t out_positions, void *out_k, void *out_v) {
    if (!dev) return fail(QVKV_E_SHAPE, "null device");
    SubmitTimer timer(dev);
    Geometry g;
    if (int rc = geometry(layout, &g)) return rc;
    uint64_t held;
    if (int rc = pool_of(dev, pool, g, &held)) return rc;
    if (out_dtype != QVKV_F32 && !(out_dtype == QVKV_F16 && g.dtype == QVKV_F16))
        return fail(QVKV_E_UNSUPPORTED, "hip backend has no gather kernel for this output dtype");
    if (n_items == 0) return QVKV_OK;
    if (!blocks || !table_at || !lens || !out_at || !out_k || !out_v)
        return fail(QVKV_E_SHAPE, "shape mismatch in gather: null pointer");
    uint32_t max_len = 0;
    for (uint32_t t = 0; t < n_items; t++) {
        max_len = std::max(max_len, lens[t]);
        const uint64_t nb = ((uint64_t)lens[t] + g.B - 1) / g.B;
        if ((uint64_t)table_at[t] + nb > n_table)
            return fail(QVKV_E_SHAPE, "shape mismatch in gather: item %u has no block for its positions", t);
        for (uint64_t b = 0; b < nb; b++)
            if (blocks[table_at[t] + b] >= held)
                return fail(QVKV_E_SHAPE, "shape mismatch in gather: a block past the pool's %llu",
                            (unsigned long long)held);
        if (out_at[t] + lens[t] > out_positions)
            return fail(QVKV_E_SHAPE, "shape mismatch in gather: item %u past out_positions", t);
    }
    std::lock_guard<std::mutex> lk(dev->host_mu);
    if (int rc = set_device(dev)) return rc;
    const uint64_t esz = out_dtype == QVKV_F16 ? 2 : 4;
    const uint64_t ob = out_positions * g.kv_out * esz;
    Stager st;
    uint64_t bo = st.add(blocks, n_table * 4), to = st.add(table_at, n_items * 4ull),
             lo = st.add(lens, n_items * 4ull), oo = st.add(out_at, n_items * 8ull);
    uint64_t ko = st.reserve(ob), vo = st.reserve(ob);
    if (int rc = st.upload(dev)) return rc;
    time_start(dev);
    if (int rc = launched(dev, qvkv::launch_gather(g, pool->ptr, held, st.at<uint32_t>(dev, bo),
                                                   n_table, st.at<uint32_t>(dev, to),
                                                   st.at<uint32_t>(dev, lo),
                                                   st.at<uint64_t>(dev, oo), n_items, max_len,
                                                   (int)out_dtype, out_positions,
                                                   st.at<void>(dev, ko), st.at<void>(dev, vo),
                                                   dev->own->d_err, dev->stream),
                          "gather launch"))
        return rc;
    time_stop(dev);
    if (int rc = download(dev, out_k, st.at<void>(dev, ko), ob)) return rc;
    if (int rc = download(dev, out_v, st.at<void>(dev, vo), ob)) return rc;
    return finish_timed(dev);
}

int qvkv_block_copy(qvkv_dev *dev, const qvkv_layout *layout, qvkv_buf *pool,
                    const uint32_t *src, const uint32_t *dst, uint32_t n) {
    SubmitTimer timer(dev);
    return qvkv::block_copy_after(dev, layout, pool, src, dst, n, false, nullptr);
}

}  // extern "C"

namespace {

// Runs of consecutive tokens that share a block table and have consecutive positions:
// a prefill chunk of one sequence is one run, a decode batch is runs of one token.
struct Segments {
    std::vector<uint32_t> table_at, pos0, q_at, n_tok;
    uint32_t max_tok = 0;
};

Segments segments_of(const uint32_t *table_at, const uint32_t *pos, uint32_t s) {
    Segments r;
    for (uint32_t t = 0; t < s;) {
        uint32_t e = t + 1;
        while (e < s && table_at[e] == table_at[t] && pos[e - 1] != UINT32_MAX &&
               pos[e] == pos[e - 1] + 1)
            e++;
        r.table_at.push_back(table_at[t]);
        r.pos0.push_back(pos[t]);
        r.q_at.push_back(t);
        r.n_tok.push_back(e - t);
        r.max_tok = std::max(r.max_tok, e - t);
        t = e;
    }
    return r;
}

// Device copies of a Segments, staged with the call's other inputs.
struct StagedSegments {
    uint64_t ta = 0, p0 = 0, qa = 0, nt = 0;
    void add(Stager &st, const Segments &sg) {
        const uint64_t b = sg.n_tok.size() * 4ull;
        ta = st.add(sg.table_at.data(), b);
        p0 = st.add(sg.pos0.data(), b);
        qa = st.add(sg.q_at.data(), b);
        nt = st.add(sg.n_tok.data(), b);
    }
};

// Attention of s stored tokens: the prefill kernel when some run has two or more tokens
// (every token then reads its table once per 32 query columns instead of once per token),
// else the decode kernel.
hipError_t attend_tokens(qvkv_dev *dev, const Geometry &g, const qvkv::AttnPlan &plan,
                         const Segments &sg, const StagedSegments &ss, Stager &st,
                         const void *pool, uint64_t held, const float *dq, const uint32_t *dblocks,
                         uint64_t n_table, const uint32_t *dtable_at, const uint32_t *dpos,
                         uint32_t s, uint32_t heads, uint32_t max_pos, float *dout,
                         bool f16_values = true) {
    if (sg.max_tok >= 2)
        return qvkv::launch_prefill(g, pool, held, dq, dblocks, n_table,
                                    st.at<uint32_t>(dev, ss.ta), st.at<uint32_t>(dev, ss.p0),
                                    st.at<uint32_t>(dev, ss.qa), st.at<uint32_t>(dev, ss.nt),
                                    (uint32_t)sg.n_tok.size(), heads, max_pos, sg.max_tok, s,
                                    dout, dev->own->d_err, dev->stream, f16_values);
    return qvkv::launch_attention(g, plan, pool, held, dq, dblocks, n_table, dtable_at, dpos, s,
                                  heads, max_pos, dout, dev->own->ws, dev->own->d_err, dev->stream);
}

}  // namespace

extern "C" {

int qvkv_decode_attention(qvkv_dev *dev, const qvkv_layout *layout, qvkv_buf *pool,
                          const float *q, uint32_t heads, const uint32_t *pos, uint32_t s,
                          const uint32_t *blocks, uint64_t n_table, const uint32_t *table_at,
                          const float *sync, const uint32_t *sync_to, uint32_t n_sync,
                          const float *k_new, const float *v_new, float *out) {
    if (!dev) return fail(QVKV_E_SHAPE, "null device");
    SubmitTimer timer(dev);
    Geometry g;
    if (int rc = geometry(layout, &g)) return rc;
    uint64_t held;
    if (int rc = pool_of(dev, pool, g, &held)) return rc;
    qvkv::AttnPlan p;
    const char *why = "";
    if (s && (!q || !pos || !blocks || !table_at || !out || (n_sync && (!sync || !sync_to)) ||
              !k_new || !v_new))
        return fail(QVKV_E_SHAPE, "shape mismatch in routed moe attention: null pointer");
    uint32_t max_pos = 0;
    for (uint32_t t = 0; t < s; t++) max_pos = std::max(max_pos, pos[t]);
    if (int rc = qvkv::plan_attention(g, s, heads, max_pos, &p, &why))
        return fail(rc, "shape mismatch in routed moe attention: %s", why);
    if (s == 0) return QVKV_OK;
    const Segments sg = segments_of(table_at, pos, s);
    if (int rc = qvkv::check_prefill(g, (uint32_t)sg.n_tok.size(), heads, sg.max_tok, &why))
        return fail(rc, "shape mismatch in routed moe attention: %s", why);
    // The checks of SimDevice::attention (sim.rs:377-381): every block and sync target
    // inside the pool, every token with a block for each of its positions.
    for (uint64_t i = 0; i < n_table; i++)
        if (blocks[i] >= held)
            return fail(QVKV_E_SHAPE, "shape mismatch in routed moe attention: a block past the pool's %llu",
                        (unsigned long long)held);
    for (uint32_t i = 0; i < n_sync; i++)
        if (sync_to[i] / g.B >= held)
            return fail(QVKV_E_SHAPE, "shape mismatch in routed moe attention: a block past the pool's %llu",
                        (unsigned long long)held);
    std::vector<uint32_t> slots(s);
    for (uint32_t t = 0; t < s; t++) {
        const uint64_t i = (uint64_t)table_at[t] + pos[t] / g.B;
        if ((uint64_t)table_at[t] + pos[t] / g.B + 1 > n_table)
            return fail(QVKV_E_SHAPE, "shape mismatch in routed moe attention: token %u has no block for position %u",
                        t, pos[t]);
        slots[t] = blocks[i] * g.B + pos[t] % g.B;
    }
    // sync rows are [key row | value row]; the append takes separate key and value rows
    std::vector<float> sk((uint64_t)n_sync * g.kv_out), sv((uint64_t)n_sync * g.kv_out);
    for (uint32_t r = 0; r < n_sync; r++) {
        memcpy(&sk[(uint64_t)r * g.kv_out], sync + (uint64_t)r * 2 * g.kv_out, g.kv_out * 4);
        memcpy(&sv[(uint64_t)r * g.kv_out], sync + ((uint64_t)r * 2 + 1) * g.kv_out, g.kv_out * 4);
    }
    std::lock_guard<std::mutex> lk(dev->host_mu);
    if (int rc = set_device(dev)) return rc;
    if (int rc = ensure_attention(dev, dev->own, p)) return rc;
    const uint64_t rowb = g.kv_out * 4, qb = (uint64_t)s * heads * g.D * 4;
    Stager st;
    uint64_t sko = st.add(sk.data(), n_sync * rowb), svo = st.add(sv.data(), n_sync * rowb),
             sto = st.add(sync_to, n_sync * 4ull), kno = st.add(k_new, s * rowb),
             vno = st.add(v_new, s * rowb), slo = st.add(slots.data(), s * 4ull),
             qo = st.add(q, qb), po = st.add(pos, s * 4ull), bo = st.add(blocks, n_table * 4),
             tao = st.add(table_at, s * 4ull), oo = st.reserve(qb);
    StagedSegments ss;
    ss.add(st, sg);
    if (int rc = st.upload(dev)) return rc;
    time_start(dev);
    hipError_t e = hipSuccess;
    if (n_sync)
        e = qvkv::launch_append(g, pool->ptr, held, st.at<float>(dev, sko), st.at<float>(dev, svo),
                                st.at<uint32_t>(dev, sto), n_sync, dev->own->d_err, dev->stream);
    if (int rc = launched(dev, e, "append launch (sync rows)")) return rc;
    e = qvkv::launch_append(g, pool->ptr, held, st.at<float>(dev, kno), st.at<float>(dev, vno),
                            st.at<uint32_t>(dev, slo), s, dev->own->d_err, dev->stream);
    if (int rc = launched(dev, e, "append launch (new rows)")) return rc;
    auto attend = [&](bool f16_values) {
        return attend_tokens(dev, g, p, sg, ss, st, pool->ptr, held, st.at<float>(dev, qo),
                             st.at<uint32_t>(dev, bo), n_table, st.at<uint32_t>(dev, tao),
                             st.at<uint32_t>(dev, po), s, heads, max_pos, st.at<float>(dev, oo),
                             f16_values);
    };
    e = attend(true);
    if (int rc = launched(dev, e, "attention launch")) return rc;
    time_stop(dev);
    if (int rc = download(dev, out, st.at<void>(dev, oo), qb)) return rc;
    int rc = finish_timed(dev);
    if (rc == QVKV_E_UNSUPPORTED) {  // q8_0 values past the f16 prefill's range: f32 form
        time_start(dev);
        if (int rc2 = launched(dev, attend(false), "attention launch")) return rc2;
        time_stop(dev);
        if (int rc2 = download(dev, out, st.at<void>(dev, oo), qb)) return rc2;
        rc = finish_timed(dev);
    }
    return rc;
}

// ---------------------------------------------------------------------------------
// prelude
// ---------------------------------------------------------------------------------

static int prelude_shape(const Geometry &g, const qvkv_prelude_t *p) {
    if (!p) return fail(QVKV_E_SHAPE, "shape mismatch in prelude: null parameters");
    if (p->heads == 0 || p->heads % g.G != 0)
        return fail(QVKV_E_SHAPE, "shape mismatch in prelude: %u heads, %d KV heads", p->heads, g.G);
    if (g.D % 2 != 0) return fail(QVKV_E_SHAPE, "shape mismatch in prelude: odd head_dim");
    if ((uint64_t)p->heads * g.D > 16384)
        return fail(QVKV_E_SHAPE, "shape mismatch in prelude: heads*head_dim above 16384");
    if (p->norm > QVKV_NORM_PER_HEAD) return fail(QVKV_E_UNSUPPORTED, "hip backend has no such norm");
    if (!p->rope) return fail(QVKV_E_SHAPE, "shape mismatch in prelude: no rope rows");
    return QVKV_OK;
}

static qvkv::PreludeArgs prelude_args(const qvkv_prelude_t *p) {
    return qvkv::PreludeArgs{p->norm, p->has_clip, p->clip, p->eps, p->q_bias, p->k_bias,
                             p->v_bias, p->norm ? p->q_norm : nullptr,
                             p->norm ? p->k_norm : nullptr, p->rope};
}

int qvkv_prelude_async(qvkv_dev *dev, const qvkv_layout *layout, const qvkv_prelude_t *p,
                       float *q, float *k, float *v, uint32_t s, void *stream) {
    if (!dev) return fail(QVKV_E_SHAPE, "null device");
    SubmitTimer timer(dev);
    Geometry g;
    if (int rc = geometry(layout, &g)) return rc;
    if (int rc = prelude_shape(g, p)) return rc;
    if (s == 0) return QVKV_OK;
    if (!q || !k || !v) return fail(QVKV_E_SHAPE, "shape mismatch in prelude: null pointer");
    if (int rc = set_device(dev)) return rc;
    return launched(dev, qvkv::launch_prelude(q, k, v, s, p->heads, (uint32_t)g.G, (uint32_t)g.D,
                                              prelude_args(p), (hipStream_t)stream),
                    "prelude launch");
}

int qvkv_prelude_attention(qvkv_dev *dev, const qvkv_layout *layout, qvkv_buf *pool,
                           const qvkv_prelude_t *p, const float *q, const float *k,
                           const float *v, const uint32_t *pos, uint32_t s,
                           const uint32_t *blocks, uint64_t n_table, const uint32_t *table_at,
                           const float *sync, const uint32_t *sync_to, uint32_t n_sync,
                           float *out, float *k_new, float *v_new) {
    if (!dev) return fail(QVKV_E_SHAPE, "null device");
    SubmitTimer timer(dev);
    Geometry g;
    if (int rc = geometry(layout, &g)) return rc;
    if (int rc = prelude_shape(g, p)) return rc;
    uint64_t held;
    if (int rc = pool_of(dev, pool, g, &held)) return rc;
    const uint32_t heads = p->heads;
    qvkv::AttnPlan plan;
    const char *why = "";
    if (s && (!q || !k || !v || !pos || !blocks || !table_at || !out ||
              (n_sync && (!sync || !sync_to))))
        return fail(QVKV_E_SHAPE, "shape mismatch in routed moe attention: null pointer");
    uint32_t max_pos = 0;
    for (uint32_t t = 0; t < s; t++) max_pos = std::max(max_pos, pos[t]);
    if (int rc = qvkv::plan_attention(g, s, heads, max_pos, &plan, &why))
        return fail(rc, "shape mismatch in routed moe attention: %s", why);
    if (s == 0) return QVKV_OK;
    const Segments sg = segments_of(table_at, pos, s);
    if (int rc = qvkv::check_prefill(g, (uint32_t)sg.n_tok.size(), heads, sg.max_tok, &why))
        return fail(rc, "shape mismatch in routed moe attention: %s", why);
    for (uint64_t i = 0; i < n_table; i++)
        if (blocks[i] >= held)
            return fail(QVKV_E_SHAPE, "shape mismatch in routed moe attention: a block past the pool's %llu",
                        (unsigned long long)held);
    for (uint32_t i = 0; i < n_sync; i++)
        if (sync_to[i] / g.B >= held)
            return fail(QVKV_E_SHAPE, "shape mismatch in routed moe attention: a block past the pool's %llu",
                        (unsigned long long)held);
    std::vector<uint32_t> slots(s);
    for (uint32_t t = 0; t < s; t++) {
        if ((uint64_t)table_at[t] + pos[t] / g.B + 1 > n_table)
            return fail(QVKV_E_SHAPE, "shape mismatch in routed moe attention: token %u has no block for position %u",
                        t, pos[t]);
        slots[t] = blocks[table_at[t] + pos[t] / g.B] * g.B + pos[t] % g.B;
    }
    std::vector<float> sk((uint64_t)n_sync * g.kv_out), sv((uint64_t)n_sync * g.kv_out);
    for (uint32_t r = 0; r < n_sync; r++) {
        memcpy(&sk[(uint64_t)r * g.kv_out], sync + (uint64_t)r * 2 * g.kv_out, g.kv_out * 4);
        memcpy(&sv[(uint64_t)r * g.kv_out], sync + ((uint64_t)r * 2 + 1) * g.kv_out, g.kv_out * 4);
    }
    std::lock_guard<std::mutex> lk(dev->host_mu);
    if (int rc = set_device(dev)) return rc;
    if (int rc = ensure_attention(dev, dev->own, plan)) return rc;
    const uint64_t q_out = (uint64_t)heads * g.D, rowb = g.kv_out * 4, qb = s * q_out * 4;
    const uint64_t nq = p->norm == QVKV_NORM_PER_HEAD ? g.D : q_out;
    const uint64_t nk = p->norm == QVKV_NORM_PER_HEAD ? g.D : g.kv_out;
    Stager st;
    const uint64_t qo = st.add(q, qb), ko = st.add(k, s * rowb), vo = st.add(v, s * rowb),
                   ro = st.add(p->rope, (uint64_t)s * g.D * 4),
                   qbo = p->q_bias ? st.add(p->q_bias, q_out * 4) : 0,
                   kbo = p->k_bias ? st.add(p->k_bias, rowb) : 0,
                   vbo = p->v_bias ? st.add(p->v_bias, rowb) : 0,
                   qno = (p->norm && p->q_norm) ? st.add(p->q_norm, nq * 4) : 0,
                   kno = (p->norm && p->k_norm) ? st.add(p->k_norm, nk * 4) : 0,
                   sko = st.add(sk.data(), n_sync * rowb), svo = st.add(sv.data(), n_sync * rowb),
                   sto = st.add(sync_to, n_sync * 4ull), slo = st.add(slots.data(), s * 4ull),
                   po = st.add(pos, s * 4ull), bo = st.add(blocks, n_table * 4),
                   tao = st.add(table_at, s * 4ull), oo = st.reserve(qb);
    StagedSegments ss;
    ss.add(st, sg);
    if (int rc = st.upload(dev)) return rc;
    qvkv::PreludeArgs a = prelude_args(p);
    a.q_bias = p->q_bias ? st.at<float>(dev, qbo) : nullptr;
    a.k_bias = p->k_bias ? st.at<float>(dev, kbo) : nullptr;
    a.v_bias = p->v_bias ? st.at<float>(dev, vbo) : nullptr;
    a.q_norm = (p->norm && p->q_norm) ? st.at<float>(dev, qno) : nullptr;
    a.k_norm = (p->norm && p->k_norm) ? st.at<float>(dev, kno) : nullptr;
    a.rope = st.at<float>(dev, ro);
    float *dq = st.at<float>(dev, qo), *dk = st.at<float>(dev, ko), *dv = st.at<float>(dev, vo);
    time_start(dev);
    hipError_t e = qvkv::launch_prelude(dq, dk, dv, s, heads, (uint32_t)g.G, (uint32_t)g.D, a,
                                        dev->stream);
    if (int rc = launched(dev, e, "prelude launch")) return rc;
    if (n_sync) {
        e = qvkv::launch_append(g, pool->ptr, held, st.at<float>(dev, sko), st.at<float>(dev, svo),
                                st.at<uint32_t>(dev, sto), n_sync, dev->own->d_err, dev->stream);
        if (int rc = launched(dev, e, "append launch (sync rows)")) return rc;
    }
    e = qvkv::launch_append(g, pool->ptr, held, dk, dv, st.at<uint32_t>(dev, slo), s, dev->own->d_err,
                            dev->stream);
    if (int rc = launched(dev, e, "append launch (new rows)")) return rc;
    auto attend = [&](bool f16_values) {
        return attend_tokens(dev, g, plan, sg, ss, st, pool->ptr, held, dq,
                             st.at<uint32_t>(dev, bo), n_table, st.at<uint32_t>(dev, tao),
                             st.at<uint32_t>(dev, po), s, heads, max_pos, st.at<float>(dev, oo),
                             f16_values);
    };
    e = attend(true);
    if (int rc = launched(dev, e, "attention launch")) return rc;
    time_stop(dev);
    if (int rc = download(dev, out, st.at<void>(dev, oo), qb)) return rc;
    if (k_new)
        if (int rc = download(dev, k_new, dk, s * rowb)) return rc;
    if (v_new)
        if (int rc = download(dev, v_new, dv, s * rowb)) return rc;
    int rc = finish_timed(dev);
    if (rc == QVKV_E_UNSUPPORTED) {  // q8_0 values past the f16 prefill's range: f32 form
        time_start(dev);
        if (int rc2 = launched(dev, attend(false), "attention launch")) return rc2;
        time_stop(dev);
        if (int rc2 = download(dev, out, st.at<void>(dev, oo), qb)) return rc2;
        rc = finish_timed(dev);
    }
    return rc;
}

}  // extern "C"

// The host-memory block copy, optionally ordered after the work already queued on a
// caller's stream: an event recorded there makes the device's own stream wait before
// the copy kernel reads the source blocks (the pool manager's copy-on-write and
// compaction copies, whose source rows the caller may have appended asynchronously).
int qvkv::block_copy_after(qvkv_dev *dev, const qvkv_layout *layout, qvkv_buf *pool,
                           const uint32_t *src, const uint32_t *dst, uint32_t n, bool ordered,
                           void *after, void (*overlap)(void *), void *ctx) {
    if (!dev) return fail(QVKV_E_SHAPE, "null device");
    Geometry g;
    if (int rc = geometry(layout, &g)) return rc;
    uint64_t held;
    if (int rc = pool_of(dev, pool, g, &held)) return rc;
    if (n && (!src || !dst)) return fail(QVKV_E_SHAPE, "shape mismatch in block copy: null pointer");
    for (uint32_t i = 0; i < n; i++)
        if (src[i] >= held || dst[i] >= held)
            return fail(QVKV_E_SHAPE, "shape mismatch in block copy: a block past the pool's %llu",
                        (unsigned long long)held);
    if (n == 0) return QVKV_OK;
    std::lock_guard<std::mutex> lk(dev->host_mu);
    if (int rc = set_device(dev)) return rc;
    Stager st;
    uint64_t so = st.add(src, n * 4ull), dd = st.add(dst, n * 4ull);
    if (int rc = st.upload(dev)) return rc;
    if (ordered && (hipStream_t)after != dev->stream) {
        hipError_t e = hipEventRecord(dev->order_ev, (hipStream_t)after);
        if (e == hipSuccess) e = hipStreamWaitEvent(dev->stream, dev->order_ev, 0);
        if (e != hipSuccess) return hip_fail(e, "ordering after the caller's stream");
        dev->stream_waits.fetch_add(1);
    }
    time_start(dev);
    if (int rc = launched(dev, qvkv::launch_block_copy(g, pool->ptr, held, st.at<uint32_t>(dev, so),
                                                       st.at<uint32_t>(dev, dd), n, dev->own->d_err,
                                                       dev->stream),
                          "block copy launch"))
        return rc;
    time_stop(dev);
    if (overlap) overlap(ctx);
    return finish_timed(dev);
}
