// HIP runtime glue of libgen9blas: init, errors, memory resolution, work buffers, waiting, profiling.
//
// Replaces two layers of the reference: its OpenCL-subset device runtime that built i915 command buffers
// (reference: lib/kcl.c) and the glue above it (reference: lib/src/core.c). On MI355X the HIP runtime already does
// command submission, so what remains is the contract of the glue:
// - gen9blas_init runs once per process under pthread_once and a failure is final (reference: core.c:205-219);
// - operands are resolved per call (reference: get_obj, core.c:328-340): device memory is used in place; host memory
//   (pageable or pinned) is copied into growing device work buffers, with matrix rows re-pitched to 16 bytes so the
//   vectorized kernels always apply, and written results are copied back after the one wait of the call
//   (reference: to_host, core.c:363-367);
// - errors map to gen9blas_status codes (reference: internal.h:28-35).
#include "internal.h"
#include <pthread.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#include <unistd.h>
#include <condition_variable>
#include <functional>
#include <map>
#include <mutex>
#include <thread>

namespace g9 {

char errbuf[1200];
int gst;
int last_zc;
double last_ms;
hipStream_t stream;
int device = -1;
int profile;
int nowait;
int num_cus;

double now_s() {
    struct timespec t;
    clock_gettime(CLOCK_MONOTONIC, &t);
    return t.tv_sec + t.tv_nsec * 1e-9;
}

int fail(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(errbuf, sizeof errbuf, fmt, ap);
    va_end(ap);
    gst = code;
    return code;
}

int hip_fail(hipError_t e, const char *what, const char *file, int line) {
    const int code = e == hipErrorOutOfMemory ? GEN9BLAS_ERR_OUT_OF_MEMORY : GEN9BLAS_ERR;
    const char *base = strrchr(file, '/');
    return fail(code, "%s:%d: %s = %s", base ? base + 1 : file, line, what, hipGetErrorString(e));
}

// ---------------- init ----------------
static pthread_once_t init_once = PTHREAD_ONCE_INIT;
static int init_status = GEN9BLAS_ERR_NO_DEVICE;
static char init_err[sizeof errbuf];
static int arch;
static hipEvent_t ev_start, ev_stop;
static bool ev_used;
static unsigned *done_word;   // host-coherent completion word (wait_done), or null
static unsigned done_seq;

static int init_impl() {
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n <= 0) {
        (void)hipGetLastError();
        G9_FAIL(GEN9BLAS_ERR_NO_DEVICE, "no HIP device (%s)", e != hipSuccess ? hipGetErrorString(e) : "count 0");
    }
    int d = 0;
    const char *env = getenv("GEN9BLAS_DEVICE");
    if (env) d = atoi(env);
    else if (hipGetDevice(&d) != hipSuccess) d = 0;
    if (d < 0 || d >= n) G9_FAIL(GEN9BLAS_ERR_NO_DEVICE, "GEN9BLAS_DEVICE=%d: %d devices", d, n);
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, d) != hipSuccess) G9_FAIL(GEN9BLAS_ERR_NO_DEVICE, "hipGetDeviceProperties(%d) failed", d);
    if (strncmp(p.gcnArchName, "gfx950", 6) != 0)
        G9_FAIL(GEN9BLAS_ERR_NO_DEVICE, "device %d is %s; this build has gfx950 kernels only", d, p.gcnArchName);
    if (hipSetDevice(d) != hipSuccess) G9_FAIL(GEN9BLAS_ERR_NO_DEVICE, "hipSetDevice(%d) failed", d);
    device = d;
    noalloc_setup(d);
    arch = 950;
    num_cus = p.multiProcessorCount;
    // Default flags and default priority: the stream orders itself with the legacy null stream.
    if (hipStreamCreate(&stream) != hipSuccess) G9_FAIL(GEN9BLAS_ERR_NO_DEVICE, "hipStreamCreate failed");
    if (hipEventCreate(&ev_start) != hipSuccess || hipEventCreate(&ev_stop) != hipSuccess)
        G9_FAIL(GEN9BLAS_ERR_NO_DEVICE, "hipEventCreate failed");
    void *w = nullptr;
    if (hipHostMalloc(&w, 256, hipHostMallocCoherent) == hipSuccess) {
        done_word = (unsigned *)w;
        __atomic_store_n(done_word, 0u, __ATOMIC_RELEASE);
    } else {
        (void)hipGetLastError();   // wait_done falls back to hipStreamSynchronize
    }
    profile = getenv("GEN9BLAS_PROFILE") != nullptr;
    errbuf[0] = 0;
    return 0;
}

static void init_run() {
    init_status = init_impl();
    if (init_status) snprintf(init_err, sizeof init_err, "%s", errbuf[0] ? errbuf : "GPU initialization failed");
}

namespace stage {
static void bounce_reset();
}

int begin() {
    gst = 0;
    pthread_once(&init_once, init_run);
    if (init_status) {
        snprintf(errbuf, sizeof errbuf, "%s", init_err);
        gst = GEN9BLAS_ERR_NO_DEVICE;
        return gst;
    }
    int cur = -1;
    if (hipGetDevice(&cur) != hipSuccess || cur != device) G9_HIP(hipSetDevice(device));
    stage::bounce_reset();
    return 0;
}

// ---------------- work buffers ----------------
static void *sbuf[NSLOTS];
static size_t ssize[NSLOTS];

static void *fixed_base;
static size_t fixed_bytes;
static const char *fixed_who;

void set_fixed_workspace(void *base, size_t bytes, const char *who) {
    fixed_base = base;
    fixed_bytes = base ? bytes : 0;
    fixed_who = who;
}

int scratch(int slot, size_t bytes, void **p) {
    if (fixed_base) {
        if (slot != SLOT_P)
            G9_FAIL(GEN9BLAS_ERR_INVALID_ARG, "%s takes device operands only: an operand in host memory would need a "
                    "staging buffer", fixed_who);
        if (bytes > fixed_bytes)
            G9_FAIL(GEN9BLAS_ERR_INVALID_ARG, "%s: this product needs %zu bytes of work space (split-K slices, or a "
                    "skinny product's gathered operand and partial sums), more than its fixed maximum of %zu", fixed_who, bytes, fixed_bytes);
        *p = fixed_base;
        return 0;
    }
    if (bytes == 0) bytes = 256;
    if (ssize[slot] < bytes) {
        if (sbuf[slot]) {
            G9_HIP(hipStreamSynchronize(stream));
            G9_HIP(hipFree(sbuf[slot]));
            sbuf[slot] = nullptr;
            ssize[slot] = 0;
        }
        size_t nb = (bytes + (1u << 21) - 1) & ~(size_t)((1u << 21) - 1);
        hipError_t e = hipMalloc(&sbuf[slot], nb);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            sbuf[slot] = nullptr;
            G9_FAIL(GEN9BLAS_ERR_OUT_OF_MEMORY, "hipMalloc(%zu) for a work buffer: %s", nb, hipGetErrorString(e));
        }
        ssize[slot] = nb;
    }
    *p = sbuf[slot];
    return 0;
}

// ---------------- operand resolution ----------------
int mem_kind(const void *p, size_t bytes) {
    if (!p) return MEM_HOST;
    hipPointerAttribute_t a;
    if (hipPointerGetAttributes(&a, p) != hipSuccess) {
        (void)hipGetLastError();   // plain host memory: the query fails, clear the error
        return MEM_HOST;
    }
    if (a.type == hipMemoryTypeHost) return MEM_PINNED;   // hipHostMalloc'd or registered
    if (a.type != hipMemoryTypeDevice && a.type != hipMemoryTypeManaged && a.type != hipMemoryTypeUnified)
        return MEM_HOST;
    hipDeviceptr_t base = nullptr;
    size_t size = 0;
    if (hipMemGetAddressRange(&base, &size, (hipDeviceptr_t)p) != hipSuccess) {
        (void)hipGetLastError();
        return MEM_DEVICE;   // device memory whose extent the runtime does not report: trust the caller
    }
    return (uintptr_t)p + bytes <= (uintptr_t)base + size ? MEM_DEVICE : MEM_DEVICE_OVERRUN;
}

int is_device(const void *p, size_t bytes) { return mem_kind(p, bytes) == MEM_DEVICE; }

// ---------------- staged copies between pageable host memory and the device ----------------
// From pageable memory hipMemcpy reaches about 30 GB/s to the device and 18 GB/s back on an MI355X host, against
// 57 GB/s from pinned memory, while four or more host threads copy pageable → pinned at about 70 GB/s. Large transfers
// therefore go through a ring of pinned chunks: host threads fill chunk i while the DMA engine moves chunk i−1 (to the
// device), or copy chunk i out while chunks i+1.. are in flight (back to the host). A 2D transfer (re-pitched rows)
// is chunked by whole rows. GEN9BLAS_STAGE=0 leaves every transfer to hipMemcpy.
namespace stage {
// 4 chunks of 8 MiB and 6 threads: HGEMM n = 4096 on pageable buffers 2.30-2.33 ms per call (3 × 8 MiB, 4 threads:
// 2.48; 8 threads: 2.30-2.31, 12: 2.36-2.37; 2 MiB chunks: 2.74; unstaged: 4.2-6.6)
constexpr size_t CHUNK = 8u << 20, MIN_BYTES = 4u << 20;
constexpr int NBUF = 4, NTHREADS = 6;
static char *buf[NBUF];
static hipEvent_t done[NBUF];
static bool used[NBUF];
static int cursor;  // next chunk to fill: consecutive transfers go round the ring instead of waiting on chunk 0
static int state;   // 0: not set up, 1: on, -1: off

// A pool of NTHREADS - 1 copy threads; the caller runs part 0 of each job. Never destroyed: the threads wait on the
// condition variable until the process ends.
struct Pool {
    std::mutex mu;
    std::condition_variable cv, cv_done;
    std::function<void(int)> job;
    int parts = 0, next = 0, left = 0;
    unsigned gen = 0;
    void worker() {
        unsigned seen = 0;
        std::unique_lock<std::mutex> lk(mu);
        for (;;) {
            cv.wait(lk, [&] { return gen != seen; });
            seen = gen;
            while (next < parts) {
                const int i = next++;
                lk.unlock();
                job(i);
                lk.lock();
                if (--left == 0) cv_done.notify_one();
            }
        }
    }
    void run(int n, const std::function<void(int)> &f) {   // f(0 .. n-1), part 0 on the calling thread
        {
            std::lock_guard<std::mutex> lk(mu);
            job = f;
            parts = n;
            next = 1;
            left = n - 1;
            gen++;
        }
        cv.notify_all();
        f(0);
        std::unique_lock<std::mutex> lk(mu);
        cv_done.wait(lk, [&] { return left == 0; });
    }
};
static Pool *pool;
static pid_t pool_pid;   // a forked child has none of the parent's copy threads: it starts its own

static bool on() {
    if (state > 0 && pool_pid != getpid()) {
        pool = new Pool;
        pool_pid = getpid();
        for (int t = 1; t < NTHREADS; t++) std::thread([] { pool->worker(); }).detach();
    }
    if (state == 0) {
        const char *e = getenv("GEN9BLAS_STAGE");
        state = e && !strcmp(e, "0") ? -1 : 1;
        for (int b = 0; b < NBUF && state > 0; b++) {
            if (hipHostMalloc((void **)&buf[b], CHUNK, hipHostMallocDefault) != hipSuccess ||
                hipEventCreateWithFlags(&done[b], hipEventDisableTiming) != hipSuccess) {
                (void)hipGetLastError();
                state = -1;   // no pinned ring: plain copies
            }
        }
        if (state > 0) {
            pool = new Pool;
            pool_pid = getpid();
            for (int t = 1; t < NTHREADS; t++) std::thread([] { pool->worker(); }).detach();
        }
    }
    return state > 0;
}
// Copies `rows` rows of `width` bytes (row strides sp, dp) with the pool: split by rows, or by bytes for one row.
static void pcopy(char *dst, size_t dp, const char *src, size_t sp, size_t width, size_t rows) {
    if (rows == 1) {
        const size_t part = (width + NTHREADS - 1) / NTHREADS;
        pool->run(NTHREADS, [&](int i) {
            const size_t a = (size_t)i * part, b = a + part < width ? a + part : width;
            if (a < b) memcpy(dst + a, src + a, b - a);
        });
        return;
    }
    const size_t per = (rows + NTHREADS - 1) / NTHREADS;
    pool->run(NTHREADS, [&](int i) {
        const size_t a = (size_t)i * per, b = a + per < rows ? a + per : rows;
        for (size_t r = a; r < b; r++) memcpy(dst + r * dp, src + r * sp, width);
    });
}
// rows of `width` bytes per chunk: the whole transfer is one "row" when contiguous (pitches equal to width)
static void plan(size_t width, size_t rows, size_t pitch, size_t &unit, size_t &units, size_t &per_chunk) {
    if (rows == 1) {
        unit = 1;
        units = width;
        per_chunk = CHUNK;
    } else {
        unit = pitch;
        units = rows;
        per_chunk = CHUNK / pitch;
    }
}
// host (row stride hpitch) → device (row stride dpitch), rows of width bytes; enqueued on stream s
static char *bounce_take(size_t bytes);
static int h2d(char *dev, size_t dpitch, const char *host, size_t hpitch, size_t width, size_t rows, bool pinned,
               hipStream_t s) {
    const size_t total = rows == 1 ? width : rows * dpitch;
    if (pinned) {   // page-locked: one asynchronous DMA straight from the caller's memory
        if (rows == 1) G9_HIP(hipMemcpyAsync(dev, host, width, hipMemcpyHostToDevice, s));
        else G9_HIP(hipMemcpy2DAsync(dev, dpitch, host, hpitch, width, rows, hipMemcpyHostToDevice, s));
        return 0;
    }
    if (char *bb = bounce_take(rows == 1 ? width : rows * width)) {   // small: through the pinned bounce area
        if (rows == 1) {
            memcpy(bb, host, width);
            G9_HIP(hipMemcpyAsync(dev, bb, width, hipMemcpyHostToDevice, s));
        } else {
            for (size_t r = 0; r < rows; r++) memcpy(bb + r * width, host + r * hpitch, width);
            G9_HIP(hipMemcpy2DAsync(dev, dpitch, bb, width, width, rows, hipMemcpyHostToDevice, s));
        }
        return 0;
    }
    if (total < MIN_BYTES || !on() || (rows > 1 && dpitch > CHUNK)) {
        if (rows == 1) G9_HIP(hipMemcpyAsync(dev, host, width, hipMemcpyHostToDevice, s));
        else G9_HIP(hipMemcpy2DAsync(dev, dpitch, host, hpitch, width, rows, hipMemcpyHostToDevice, s));
        return 0;
    }
    size_t unit, units, per;
    plan(width, rows, dpitch, unit, units, per);
    int b = cursor;
    for (size_t u0 = 0; u0 < units; u0 += per) {
        const size_t n = units - u0 < per ? units - u0 : per;
        if (used[b]) G9_HIP(hipEventSynchronize(done[b]));   // the DMA that last read this chunk has finished
        if (rows == 1) pcopy(buf[b], 0, host + u0, 0, n, 1);
        else pcopy(buf[b], dpitch, host + u0 * hpitch, hpitch, width, n);
        G9_HIP(hipMemcpyAsync(dev + u0 * unit, buf[b], n * unit, hipMemcpyHostToDevice, s));
        G9_HIP(hipEventRecord(done[b], s));
        used[b] = true;
        b = b + 1 == NBUF ? 0 : b + 1;
    }
    cursor = b;
    return 0;
}
// device (row stride dpitch) → host (row stride hpitch); returns once the data is in host memory
static int d2h(char *host, size_t hpitch, const char *dev, size_t dpitch, size_t width, size_t rows) {
    size_t unit, units, per;
    plan(width, rows, dpitch, unit, units, per);
    const size_t nchunks = (units + per - 1) / per;
    auto issue = [&](size_t c) -> int {   // chunk c into buffer c % NBUF
        const int b = (int)(c % NBUF);
        const size_t u0 = c * per, n = units - u0 < per ? units - u0 : per;
        G9_HIP(hipMemcpyAsync(buf[b], dev + u0 * unit, n * unit, hipMemcpyDeviceToHost, stream));
        G9_HIP(hipEventRecord(done[b], stream));
        used[b] = true;
        return 0;
    };
    for (size_t c = 0; c < nchunks && c < (size_t)NBUF; c++) G9_TRY(issue(c));
    for (size_t c = 0; c < nchunks; c++) {
        const int b = (int)(c % NBUF);
        const size_t u0 = c * per, n = units - u0 < per ? units - u0 : per;
        G9_HIP(hipEventSynchronize(done[b]));
        if (rows == 1) pcopy(host + u0, 0, buf[b], 0, n, 1);
        else pcopy(host + u0 * hpitch, hpitch, buf[b], dpitch, width, n);
        if (c + NBUF < nchunks) G9_TRY(issue(c + NBUF));
    }
    return 0;
}
static bool d2h_staged(size_t width, size_t rows, size_t dpitch) {
    const size_t total = rows == 1 ? width : rows * dpitch;
    return total >= MIN_BYTES && on() && !(rows > 1 && dpitch > CHUNK);
}

// A second stream (default flags and priority) for copies that run beside the library stream's kernels: inputs
// through the ring above, and results, in pieces of at most one chunk, each into one of two pinned chunks of its own.
// The kernels wait for the inputs, and the results for the kernels, through events; the DMA engine then never waits
// for a kernel it does not depend on.
static hipStream_t ostream;
static char *obuf[2];
static hipEvent_t kdone[2], odone[2], iready;
static bool oused[2];
static int ostate;   // 0: not set up, 1: on, -1: off
static bool out_on() {
    if (ostate == 0) {
        ostate = on() && hipStreamCreate(&ostream) == hipSuccess &&
                 hipEventCreateWithFlags(&iready, hipEventDisableTiming) == hipSuccess ? 1 : -1;
        for (int q = 0; q < 2 && ostate > 0; q++)
            if (hipHostMalloc((void **)&obuf[q], CHUNK, hipHostMallocDefault) != hipSuccess ||
                hipEventCreateWithFlags(&kdone[q], hipEventDisableTiming) != hipSuccess ||
                hipEventCreateWithFlags(&odone[q], hipEventDisableTiming) != hipSuccess)
                ostate = -1;
        if (ostate < 0) (void)hipGetLastError();   // no second direction: results go back after the whole product
    }
    return ostate > 0;
}

// Small transfers (at most SMALL bytes) go through a pinned bounce area instead: the host copies into it (or out of
// it after the wait) and the DMA engine moves it asynchronously, where a copy from or to pageable memory makes the
// runtime stage and wait itself. MI355X, one copy and the wait: 16 KiB host → device 18.6 → 8.8 µs, device → host
// 25.1 → 9.6 µs; 64 KiB 17.0 → 13.7 and 18.7 → 14.5; 256 KiB 20.2 → 18.3 and 26.7 → 22.4; 1 MiB 42 → 55 (one host
// thread's memcpy loses there; so does a whole 256² FP32 product on host buffers, its three 256 KiB copies through the
// area taking 82.7 against 66.8 µs per call, while 64² goes from 33.0 to 21.0 µs). A call takes its pieces from the
// area in order; the next call starts over once this one has waited (begin()). Page-locked caller memory skips the
// area: the DMA engine reads or writes it directly.
constexpr size_t SMALL = 128u << 10, BOUNCE = 1u << 20;
static char *bounce;
static int bounce_state;     // 0: not set up, 1: on, -1: off
static size_t bounce_used;   // bytes taken by the current call
static bool bounce_busy;     // copies through the area may still be in flight (no completed wait since)
static char *bounce_take(size_t bytes) {
    if (bounce_state == 0) {
        const char *e = getenv("GEN9BLAS_STAGE");
        bounce_state = e && !strcmp(e, "0") ? -1 : 1;
        if (bounce_state > 0 && hipHostMalloc((void **)&bounce, BOUNCE, hipHostMallocDefault) != hipSuccess) {
            (void)hipGetLastError();
            bounce_state = -1;
        }
    }
    const size_t need = (bytes + 255) & ~(size_t)255;
    if (bounce_state < 0 || bytes > SMALL || bounce_used + need > BOUNCE) return nullptr;
    char *p = bounce + bounce_used;
    bounce_used += need;
    bounce_busy = true;
    return p;
}
// start of a call: the area is free again once the previous call's copies are known to be done
static void bounce_reset() {
    if (!bounce_used) return;
    if (bounce_busy) (void)hipStreamSynchronize(stream);
    bounce_used = 0;
    bounce_busy = false;
}
}  // namespace stage

int resolve(Operand &op, int slot, bool copy_in, bool written, bool repitch) {
    const size_t es = op.es;
    const size_t span = ((size_t)(op.rows - 1) * (size_t)op.caller_ld + (size_t)op.cols) * es;
    op.written = written;
    const int kind = mem_kind(op.host, span);
    if (kind == MEM_DEVICE_OVERRUN)
        G9_FAIL(GEN9BLAS_ERR_INVALID_ARG, "an operand of %zu bytes (with its leading dimension or increment) runs past "
                "the end of its device allocation", span);
    if (kind == MEM_DEVICE) {
        op.dev = const_cast<void *>(op.host);
        op.ld = op.caller_ld;
        op.zc = true;
        return 0;
    }
    op.zc = false;
    op.pinned = kind == MEM_PINNED;
    // Host memory moves in one 1D copy of the caller's span with the caller's leading dimension: from pageable
    // memory a 2D copy goes row by row (about 20 µs per row). Only a matrix whose row gaps make up more than half of
    // its span is packed by a 2D copy instead.
    const size_t dense = (size_t)op.rows * (size_t)op.cols * es;
    if (repitch && op.rows > 1 && span > 2 * dense) {
        const size_t pitch = ((size_t)op.cols * es + 15) / 16 * 16;
        op.ld = (long long)(pitch / es);
        G9_TRY(scratch(slot, pitch * (size_t)op.rows, &op.dev));
        if (copy_in)
            G9_TRY(stage::h2d((char *)op.dev, pitch, (const char *)op.host, (size_t)op.caller_ld * es, (size_t)op.cols * es,
                              (size_t)op.rows, op.pinned, stream));
        return 0;
    }
    op.ld = op.caller_ld;
    G9_TRY(scratch(slot, span, &op.dev));
    // the copy back rewrites the whole span: gap elements of a written operand must hold the caller's values
    if (written && span > dense) copy_in = true;
    if (copy_in) G9_TRY(stage::h2d((char *)op.dev, span, (const char *)op.host, span, span, 1, op.pinned, stream));
    return 0;
}

size_t out_chunk() { return stage::out_on() ? stage::CHUNK : 0; }

int out_mark(int q) {
    G9_HIP(hipEventRecord(stage::kdone[q], stream));
    return 0;
}

int out_start(int q, const void *dev, size_t bytes) {
    using namespace stage;
    if (oused[q]) G9_HIP(hipEventSynchronize(odone[q]));   // the piece last in this chunk has left it
    G9_HIP(hipStreamWaitEvent(ostream, kdone[q], 0));
    G9_HIP(hipMemcpyAsync(obuf[q], dev, bytes, hipMemcpyDeviceToHost, ostream));
    G9_HIP(hipEventRecord(odone[q], ostream));
    oused[q] = true;
    return 0;
}

int out_finish(int q, void *host, size_t bytes) {
    G9_HIP(hipEventSynchronize(stage::odone[q]));
    stage::pcopy((char *)host, 0, stage::obuf[q], 0, bytes, 1);
    return 0;
}

void out_drain() {
    if (stage::ostate > 0) (void)hipStreamSynchronize(stage::ostream);
}

int stage_in(void *dev, const void *host, size_t bytes) {
    return stage::h2d((char *)dev, bytes, (const char *)host, bytes, bytes, 1, false, stage::ostream);
}

int stage_in_ready() {
    G9_HIP(hipEventRecord(stage::iready, stage::ostream));
    G9_HIP(hipStreamWaitEvent(stream, stage::iready, 0));
    return 0;
}

int wait_stream() {
    G9_HIP(hipStreamSynchronize(stream));
    G9_HIP(hipGetLastError());
    stage::bounce_busy = false;
    return 0;
}

// One thread stores the sequence number with a system-scope release; the kernel starts only after everything queued
// before it on the stream has completed.
__global__ void done_signal(unsigned *word, unsigned seq) {
    if (threadIdx.x == 0) __hip_atomic_store(word, seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

// The 64 bytes after the completion word's cache line: a call's scalar result, written by its last kernel.
void *result_slot() { return done_word ? (void *)((char *)done_word + 128) : nullptr; }

// Waits for the stream by spinning on a host-coherent word that a one-thread kernel, queued behind the call's work,
// sets. MI355X, median of 2000 calls: a kernel and the signal 8.4 µs, a kernel and hipStreamSynchronize 11.0 µs.
// Only for calls whose device-to-host copies, if any, land in page-locked memory (the bounce area, or the caller's
// own): a copy into pageable memory may complete on the host after the GPU's part. After 2 ms (a long queue ahead,
// or a fault that keeps the signal from coming) it falls back to hipStreamSynchronize, which also reports kernel
// errors; so does a signal overtaken by another thread's (the word then holds a later number, which also means this
// call's work is done).
int wait_done() {
    if (!done_word) return wait_stream();
    const unsigned seq = __atomic_add_fetch(&done_seq, 1u, __ATOMIC_RELAXED);
    hipLaunchKernelGGL(done_signal, dim3(1), dim3(64), 0, stream, done_word, seq);
    G9_HIP(hipGetLastError());
    const double t0 = now_s();
    while ((int)(__atomic_load_n(done_word, __ATOMIC_ACQUIRE) - seq) < 0)
        if (now_s() - t0 > 2e-3) return wait_stream();
    stage::bounce_busy = false;
    return 0;
}

int finish(Operand *ops, int n, bool host_copy) {
    bool all_zc = true;
    for (int i = 0; i < n; i++) all_zc &= ops[i].zc || !ops[i].host;
    if (nowait && all_zc) {
        G9_HIP(hipGetLastError());   // launch errors are reported at once; kernel errors at gen9blas_flush
        return 0;
    }
    bool copied = host_copy;
    struct Out { char *host; size_t hpitch; const char *bb; size_t width, rows; };
    Out outs[4];
    int nout = 0;
    for (int i = 0; i < n; i++) {
        const Operand &o = ops[i];
        if (!o.written || o.zc || !o.host) continue;
        const size_t es = o.es;
        char *h = (char *)const_cast<void *>(o.host);
        const char *d = (const char *)o.dev;
        const bool pitched = o.ld != o.caller_ld && o.rows > 1;
        const size_t width = pitched ? (size_t)o.cols * es : ((size_t)(o.rows - 1) * (size_t)o.caller_ld + (size_t)o.cols) * es;
        const size_t rows = pitched ? (size_t)o.rows : 1, dpitch = pitched ? (size_t)o.ld * es : width;
        const size_t hpitch = pitched ? (size_t)o.caller_ld * es : width;
        if (o.pinned) {   // page-locked: the DMA writes the caller's memory; done once the stream is
            if (rows == 1) G9_HIP(hipMemcpyAsync(h, d, width, hipMemcpyDeviceToHost, stream));
            else G9_HIP(hipMemcpy2DAsync(h, hpitch, d, dpitch, width, rows, hipMemcpyDeviceToHost, stream));
            continue;
        }
        // small: into the pinned bounce area by DMA, copied out on the host after the wait
        char *bb = nout < 4 ? stage::bounce_take(rows * width) : nullptr;
        if (bb) {
            if (rows == 1) G9_HIP(hipMemcpyAsync(bb, d, width, hipMemcpyDeviceToHost, stream));
            else G9_HIP(hipMemcpy2DAsync(bb, width, d, dpitch, width, rows, hipMemcpyDeviceToHost, stream));
            outs[nout++] = Out{h, hpitch, bb, width, rows};
            continue;
        }
        copied = true;
        if (stage::d2h_staged(width, rows, dpitch)) {
            G9_TRY(stage::d2h(h, pitched ? (size_t)o.caller_ld * es : width, d, dpitch, width, rows));
        } else if (pitched) {
            G9_HIP(hipMemcpy2DAsync(h, (size_t)o.caller_ld * es, d, dpitch, width, rows, hipMemcpyDeviceToHost, stream));
        } else {
            G9_HIP(hipMemcpyAsync(h, d, width, hipMemcpyDeviceToHost, stream));
        }
    }
    G9_TRY(copied ? wait_stream() : wait_done());
    for (int i = 0; i < nout; i++) {
        const Out &u = outs[i];
        if (u.rows == 1) memcpy(u.host, u.bb, u.width);
        else for (size_t r = 0; r < u.rows; r++) memcpy(u.host + r * u.hpitch, u.bb + r * u.width, u.width);
    }
    return 0;
}

// ---------------- profiling ----------------
void prof_begin() {
    if (profile) {
        (void)hipEventRecord(ev_start, stream);
        ev_used = true;
    }
}
void prof_end() {
    if (profile && ev_used) (void)hipEventRecord(ev_stop, stream);
}
void prof_collect(double t_call_start) {
    last_ms = (now_s() - t_call_start) * 1e3;
    if (profile && ev_used && !nowait) {
        float ms = 0;
        if (hipEventSynchronize(ev_stop) == hipSuccess && hipEventElapsedTime(&ms, ev_start, ev_stop) == hipSuccess)
            last_ms = ms;
        else
            (void)hipGetLastError();
    }
    ev_used = false;
}

// ---------------- pinned host memory registry (gen9blas_alloc / gen9blas_is_usm) ----------------
static std::mutex alloc_mu;
static std::map<uintptr_t, size_t> &blocks() {
    static std::map<uintptr_t, size_t> m;
    return m;
}

}  // namespace g9

using namespace g9;

extern "C" {

int gen9blas_version(void) { return GEN9BLAS_VERSION; }

int gen9blas_init(void) { return begin(); }

int gen9blas_device_gen(void) { return begin() ? 0 : 9; }

int gen9blas_device_arch(void) { return begin() ? 0 : arch; }
int gen9blas_is_device(const void *p, size_t bytes) { return begin() ? 0 : is_device(p, bytes ? bytes : 1); }

int gen9blas_has(int f) {
    if (begin()) return 0;
    switch (f) {
    case GEN9BLAS_FEAT_FP16:
    case GEN9BLAS_FEAT_FP32:
    case GEN9BLAS_FEAT_FP64:
    case GEN9BLAS_FEAT_SKINNY_PB: return 1;
    default: return 0;   // the other ML features of the reference are not part of this library
    }
}

const char *gen9blas_error(void) { return errbuf; }
int gen9blas_last_status(void) { return gst; }
double gen9blas_last_time_ms(void) { return last_ms; }
int gen9blas_last_zero_copy(void) { return last_zc; }

void *gen9blas_alloc(size_t bytes) {
    if (begin()) return nullptr;
    void *p = nullptr;
    hipError_t e = hipHostMalloc(&p, bytes ? bytes : 1, hipHostMallocDefault);
    if (e != hipSuccess || !p) {
        (void)hipGetLastError();
        fail(GEN9BLAS_ERR_OUT_OF_MEMORY, "hipHostMalloc(%zu): %s", bytes, hipGetErrorString(e));
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(alloc_mu);
    blocks()[(uintptr_t)p] = bytes ? bytes : 1;
    return p;
}

void gen9blas_free(void *p) {
    if (!p) return;
    {
        std::lock_guard<std::mutex> lk(alloc_mu);
        auto it = blocks().find((uintptr_t)p);
        if (it == blocks().end()) return;
        blocks().erase(it);
    }
    if (stream) (void)hipStreamSynchronize(stream);
    (void)hipHostFree(p);
}

int gen9blas_is_usm(const void *p, size_t bytes) {
    if (!p) return 0;
    std::lock_guard<std::mutex> lk(alloc_mu);
    auto &m = blocks();
    auto it = m.upper_bound((uintptr_t)p);
    if (it == m.begin()) return 0;
    --it;
    return (uintptr_t)p + bytes <= it->first + it->second;
}

void *gen9blas_hip_stream(void) { return begin() ? nullptr : (void *)stream; }

void *gen9blas_device_alloc(size_t bytes) {
    if (begin()) return nullptr;
    void *p = nullptr;
    hipError_t e = hipMalloc(&p, bytes ? bytes : 1);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        fail(GEN9BLAS_ERR_OUT_OF_MEMORY, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
        return nullptr;
    }
    return p;
}

void gen9blas_device_free(void *p) {
    if (!p || begin()) return;
    (void)hipStreamSynchronize(stream);
    (void)hipFree(p);
}

int gen9blas_memcpy(void *dst, const void *src, size_t bytes) {
    G9_TRY(begin());
    if (!bytes) return 0;
    if (!dst || !src) G9_FAIL(GEN9BLAS_ERR_INVALID_ARG, "gen9blas_memcpy: NULL pointer");
    G9_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDefault, stream));
    return wait_stream();
}

void gen9blas_set_nowait(int on) { nowait = on != 0; }

int gen9blas_flush(void) {
    G9_TRY(begin());
    return wait_stream();
}

}  // extern "C"
