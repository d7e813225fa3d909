// gen9blas_gemm_noalloc: gen9blas_gemm for callers that cannot allocate device memory (tight serving loops, harnesses
// that forbid hipMalloc). It runs the same kernels with the same dispatch as gen9blas_gemm; the only work buffer a
// GEMM on device operands uses comes from a static device array instead of the library's growing buffers, so the
// call itself allocates nothing. That buffer holds the split-K partial slices of the tile kernels, or, for a skinny
// product (min(M, N) ≤ 16), a transposed small operand gathered K-contiguous (M·K elements) and the K-split partial
// sums of weights stored K×N (parts · M · N FP32 values, with parts · N ≤ 4 · 64 · CUs: 4 MiB at M = 16 on 256 CUs).
//
// Size of that array: without a split forced by GEN9BLAS_SPLITK, a product splits K into s > 1 slices only while
// tiles · s ≤ CUs, and the slices hold ns ≤ s partial copies of C, M · N ≤ tiles · BM · BN elements each. So one
// call needs at most CUs × (largest split tile: 256 × 256 FP32 sums = 256 × 128 FP64 sums = 256 KiB) bytes,
// 64 MiB on MI355X's 256 CUs: an FP16 product on the general kernel with 128 tiles of 256×256 split two ways
// (2048×4096×1000, say) uses all of it. A forced split can
// need more, as can a skinny product whose gathered operand alone passes about 60 MiB (M · K · element size); both
// are rejected with INVALID_ARG before anything is launched (as is every product on a device with more CUs than the
// bound assumes, should one need more).
#include "internal.h"
#include <stdio.h>

namespace {
constexpr int MAX_CUS = 256;   // MI355X
constexpr size_t NOALLOC_SCRATCH_BYTES = (size_t)MAX_CUS * g9::SPLITK_TILE_BYTES_MAX;
static_assert(NOALLOC_SCRATCH_BYTES == 64u << 20, "64 MiB per GPU");
constexpr int MAX_DEVICES = 64;
}  // namespace

// One copy per GPU, held until the process ends. In host code `scratch` is only a stand-in for the symbol: its device
// address comes from hipGetSymbolAddress (scratch_dev below), and only that address is passed to kernels.
static __device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];

namespace g9 {

static void *scratch_dev[MAX_DEVICES];
static char setup_error[256];

void noalloc_setup(int dev) {
    if (dev < 0 || dev >= MAX_DEVICES) {
        snprintf(setup_error, sizeof setup_error, "gen9blas_gemm_noalloc: device %d beyond the first %d", dev,
                 MAX_DEVICES);
        return;
    }
    void *ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(::scratch));
    if (e != hipSuccess || !ptr) {
        (void)hipGetLastError();
        snprintf(setup_error, sizeof setup_error, "gen9blas_gemm_noalloc: no device address for its work space (%s)",
                 hipGetErrorString(e));
        return;
    }
    scratch_dev[dev] = ptr;
}

// Span in bytes of a rows × cols row-major operand with row stride ld.
static size_t span(int rows, int cols, int ld, int es) { return ((size_t)(rows - 1) * ld + cols) * es; }

}  // namespace g9

using namespace g9;

extern "C" int gen9blas_gemm_noalloc(int type, int transA, int transB, int M, int N, int K, double alpha, const void *A,
                                     int lda, const void *B, int ldb, double beta, void *C, int ldc) {
    G9_TRY(begin());
    void *ws = device >= 0 && device < MAX_DEVICES ? scratch_dev[device] : nullptr;
    if (!ws) G9_FAIL(GEN9BLAS_ERR, "%s", setup_error[0] ? setup_error : "gen9blas_gemm_noalloc: not set up");
    // Operands must lie in device memory. Checked before any dispatch: host operands would reach the staging paths
    // (pinned rings, copy threads), which allocate on first use.
    if (type >= 0 && type <= 3 && M > 0 && N > 0 && K > 0 && A && B && C && lda >= (transA ? M : K) &&
        ldb >= (transB ? K : N) && ldc >= N) {
        const int es = elem_size(type);
        const bool ok = mem_kind(A, transA ? span(K, M, lda, es) : span(M, K, lda, es)) == MEM_DEVICE &&
                        mem_kind(B, transB ? span(N, K, ldb, es) : span(K, N, ldb, es)) == MEM_DEVICE &&
                        mem_kind(C, span(M, N, ldc, es)) == MEM_DEVICE;
        if (!ok)
            G9_FAIL(GEN9BLAS_ERR_INVALID_ARG, "gen9blas_gemm_noalloc takes device operands only: an operand in host "
                    "memory (or past the end of its device allocation) would need a staging buffer");
    }
    set_fixed_workspace(ws, NOALLOC_SCRATCH_BYTES, "gen9blas_gemm_noalloc");
    const int r = gemm_impl(type, transA, transB, M, N, K, alpha, A, lda, 0, B, ldb, 0, beta, C, ldc, 0, 1);
    set_fixed_workspace(nullptr, 0, nullptr);
    return r;
}
