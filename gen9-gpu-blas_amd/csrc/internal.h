// Shared state and helpers of libgen9blas (not installed). Everything here has hidden visibility.
//
// Roles (reference: lib/src/internal.h, lib/src/core.c, lib/kcl.c):
// - error state: the text of the last error and the gen9blas_status of the current call;
// - one-time init: device selection, the HIP stream, profiling events;
// - operand resolution: device memory is used in place, host memory is staged through growing device work buffers;
// - synchronization: one wait per call (or none in no-wait mode), then copies of staged results back to the host.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>
#include "gen9blas.h"
#include "gen9blas_hip.h"

#define G9_HIDDEN __attribute__((visibility("hidden")))

namespace g9 {

// ---- error state (reference: lib/src/internal.h:28-35, lib/src/core.c:385-392) ----
G9_HIDDEN extern char errbuf[1200];
G9_HIDDEN extern int gst;            // status of the current call
G9_HIDDEN extern int last_zc;        // zero-copy bits of the last level 3 call
G9_HIDDEN extern double last_ms;     // gen9blas_last_time_ms
G9_HIDDEN int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
G9_HIDDEN int hip_fail(hipError_t e, const char *what, const char *file, int line);
#define G9_FAIL(code, ...) return ::g9::fail((code), __VA_ARGS__)
#define G9_HIP(x) do { hipError_t e_ = (x); if (e_ != hipSuccess) return ::g9::hip_fail(e_, #x, __FILE__, __LINE__); } while (0)
#define G9_TRY(x) do { int r_ = (x); if (r_) return r_; } while (0)

// ---- runtime ----
G9_HIDDEN extern hipStream_t stream;
G9_HIDDEN extern int device;
G9_HIDDEN extern int profile;        // GEN9BLAS_PROFILE set: time the main kernels with events
G9_HIDDEN extern int nowait;         // gen9blas_set_nowait
G9_HIDDEN extern int num_cus;
// Start of every entry point: reset the status, make sure the device is open and current. 0 or an error.
G9_HIDDEN int begin();
G9_HIDDEN double now_s();

// ---- operands ----
enum Slot { SLOT_A = 0, SLOT_B, SLOT_C, SLOT_P, SLOT_Q, SLOT_T, SLOT_X, SLOT_Y, SLOT_W, NSLOTS };
// Device scratch owned by the library, grown on demand and kept between calls (the reference's work buffers,
// reference: lib/src/core.c:272-277). Growing waits for queued work first.
G9_HIDDEN int scratch(int slot, size_t bytes, void **p);
// While a fixed work space is set (base != nullptr), scratch() allocates nothing: the split-K slices (SLOT_P) are
// placed at `base` if they fit in `bytes`, and every other request (staging of host operands, other work buffers)
// fails with INVALID_ARG. set_fixed_workspace(nullptr, 0) returns to the growing buffers.
G9_HIDDEN void set_fixed_workspace(void *base, size_t bytes, const char *who);
// Largest split-K partial tile, in bytes: the FP16 256×256 tile of FP32 sums and the FP64 256×128 tile of FP64 sums.
// A split of s > 1 slices is chosen only while tiles · s ≤ CUs, so the slices of one product never exceed
// CUs × this many bytes (the launch asserts every split tile against it).
constexpr size_t SPLITK_TILE_BYTES_MAX = 256 * 256 * 4;
// Set-up of the no-allocation entry point on `dev` (called by init with `dev` current): finds the device address of
// its static work space. A failure is kept and reported by that entry point only.
G9_HIDDEN void noalloc_setup(int dev);

// A vector or matrix operand. Matrices are described as rows × cols elements with row stride ld; vectors as
// rows = 1, cols = span (elements from the lowest address), ld = cols.
struct Operand {
    const void *host = nullptr;  // caller's pointer
    void *dev = nullptr;         // pointer the kernels use
    long long ld = 0;            // row stride (elements) the kernels must use; may differ from the caller's for staged matrices
    long long caller_ld = 0;
    long long rows = 0, cols = 0;
    int es = 0;
    bool zc = false;             // caller's memory used in place
    bool pinned = false;         // caller's host memory is page-locked: copied by DMA straight from or into it
    bool written = false;        // kernels write it: copy back after the wait when staged
};
// Resolves op (host, rows, cols, ld, es set by the caller) for the kernels. Device memory is used in place; host
// memory goes into the work buffer `slot` as one copy of the caller's span with the caller's row stride, or, when
// `repitch` and row gaps make up more than half of the span, packed with a row stride rounded up to 16 bytes
// (copy_in: with the data; otherwise the buffer contents are undefined, as for outputs not read, except the gaps of
// a written operand, which are copied in so the copy back preserves them).
G9_HIDDEN int resolve(Operand &op, int slot, bool copy_in, bool written, bool repitch);
// Where p .. p+bytes lies: host memory (pageable or pinned, or NULL), inside one device (or managed) allocation, or in
// device memory but running past the end of its allocation (an ld or increment too large for the buffer).
enum { MEM_HOST = 0, MEM_DEVICE = 1, MEM_DEVICE_OVERRUN = 2, MEM_PINNED = 3 };   // MEM_PINNED: page-locked host memory
G9_HIDDEN int mem_kind(const void *p, size_t bytes);
// 1 if p .. p+bytes lies in one device allocation.
G9_HIDDEN int is_device(const void *p, size_t bytes);
// End of a call: in no-wait mode with every operand in place, returns at once; otherwise waits for the stream and
// copies staged written operands back (through wait_done when nothing is copied back and the caller queued no
// device-to-host copy of its own: host_copy).
G9_HIDDEN int finish(Operand *ops, int n, bool host_copy = false);
// Waits for the stream (no copies). 0 or an error.
G9_HIDDEN int wait_stream();
// Copies beside the kernels, on a second stream (available when out_chunk() > 0). stage_in: pageable host bytes
// into device memory, through the pinned ring when large (returns once the host side is copied; the DMA is queued);
// stage_in_ready: work queued on the library stream from now on waits for the inputs queued so far. out_chunk() is
// the most one result piece may hold (0: not available); out_mark(q) marks the work queued so far on the library
// stream; out_start(q, dev, bytes) queues the piece, once that marked work is done, into pinned chunk q (0 or 1);
// out_finish(q, host, bytes) waits for it and copies it to the host. out_drain() waits for the second stream (after an error, before buffers it may still
// read are reused).
G9_HIDDEN int stage_in(void *dev, const void *host, size_t bytes);
G9_HIDDEN int stage_in_ready();
G9_HIDDEN size_t out_chunk();
G9_HIDDEN int out_mark(int q);
G9_HIDDEN int out_start(int q, const void *dev, size_t bytes);
G9_HIDDEN int out_finish(int q, void *host, size_t bytes);
G9_HIDDEN void out_drain();
// Waits for the stream through a completion word set by a kernel queued behind the call's work (falls back to
// wait_stream); for calls whose device-to-host copies, if any, go into page-locked memory.
G9_HIDDEN int wait_done();
// 64 bytes of pinned host-coherent memory that kernels may write a call's scalar result into (read after wait_done),
// or null when it could not be allocated.
G9_HIDDEN void *result_slot();

// Kernel timing for GEN9BLAS_PROFILE=1: events around the main kernels of a call.
G9_HIDDEN void prof_begin();
G9_HIDDEN void prof_end();
G9_HIDDEN void prof_collect(double t_call_start);

// Scalars for kernels: double for FP64, float otherwise (reference: lib/src/core.c:356-359).
inline int elem_size(int type) { return type == GEN9BLAS_S ? 4 : type == GEN9BLAS_D ? 8 : 2; }

}  // namespace g9

// ---- kernel launchers (one translation unit each) ----
namespace g9 {
struct GemmCall {
    int type;                      // GEN9BLAS_H / HS / S / D
    int tA, tB, M, N, K, count;
    double alpha, beta;
    const void *A; long long lda, sA;
    const void *B; long long ldb, sB;
    void *C; long long ldc, sC;
};
G9_HIDDEN int launch_gemm(const GemmCall &c);
// Lower (upper) triangle only of a square product, C = alpha·op(A)·op(B) + beta·C there (tA != tB, count 1).
G9_HIDDEN int launch_gemm_tri(const GemmCall &c, bool lower);
// NN product (or strided batch of them) whose tiles take only the k range where a triangular operand is non-zero:
// klim 1 op(A) lower, 2 op(A) upper, 3 op(B) lower, 4 op(B) upper.
G9_HIDDEN int launch_gemm_klim(const GemmCall &c, int klim);
// Inverses, computed in FP64 (level3.hip), of the `count` 128-row diagonal blocks of lower-triangular leaves of lb
// rows (lb a multiple of 128): leaf p's element (i, j) at L[p·bstride + i·ld + j]; the inverses go to leaf p at
// Inv + p·istride (row stride lb), with zeros right of each block's inverse to the end of its leaf; es 4 (float) or
// 8 (double). Each block's entries above its diagonal are read as zeros, and with `unit` its diagonal as ones.
G9_HIDDEN int launch_tri_inverse(int es, const void *L, long long ld, long long bstride, int count, void *Inv, int lb,
                                 long long istride, int unit);
// The whole gen9blas_gemm_batched call: checks, operand resolution, skinny / MFMA dispatch, wait (gemm.hip).
G9_HIDDEN int gemm_impl(int type, int tA, int tB, int M, int N, int K, double alpha, const void *A, int lda, long long sA,
                        const void *B, int ldb, long long sB, double beta, void *C, int ldc, long long sC, int count);
struct SkinnyCall {
    int type;                                // GEN9BLAS_H / HS / S
    int M, N, K;                             // C (M×N) = alpha·a·wᵀ + beta·C, a M×K, w N×K
    double alpha, beta;
    const void *a; long long sam, sak = 1;   // a[m][k] = a[m·sam + k·sak]
    const void *w; long long swn, swk = 1;   // w[n][k] = w[n·swn + k·swk]; swk = 1 (K-contiguous) or swn = 1
    void *C; long long scm, scn;             // C[m][n] = C[m·scm + n·scn]
};
G9_HIDDEN int launch_skinny(const SkinnyCall &c);
// Level 1/2: element i of a vector is at p[o + i·inc], o = (n-1)·(-inc) for inc < 0.
G9_HIDDEN int launch_axpy(int es, int n, double a, const void *x, long long ox, long long ix, void *y, long long oy, long long iy);
G9_HIDDEN int launch_scal(int es, int n, double a, void *x, long long ox, long long ix);
G9_HIDDEN int launch_copy(int es, int n, const void *x, long long ox, long long ix, void *y, long long oy, long long iy);
G9_HIDDEN int launch_rot(int es, int n, void *x, long long ox, long long ix, void *y, long long oy, long long iy,
                         double h11, double h12, double h21, double h22, int swap);
// mode 0: Σ x·y, 1: Σ|x|, 2: Σ x² (FP64). Result written to *result (a double in device memory or in the pinned
// result slot).
G9_HIDDEN int launch_reduce(int es, int mode, int n, const void *x, long long ox, long long ix, const void *y, long long oy,
                            long long iy, double *result);
G9_HIDDEN int launch_iamax(int es, int n, const void *x, long long ox, long long ix, long long *result);
G9_HIDDEN int launch_gemv(int es, int trans, int M, int N, double alpha, const void *A, long long lda, const void *x, long long ox,
                          long long ix, double beta, void *y, long long oy, long long iy);
G9_HIDDEN int launch_ger(int es, int M, int N, double alpha, const void *x, long long ox, long long ix, const void *y,
                         long long oy, long long iy, void *A, long long lda);
}  // namespace g9
