// gen9blas_gemm_noalloc: gen9blas_gemm for callers that cannot allocate device memory (code under HIP graph capture,
// tight serving loops, harnesses that forbid hipMalloc). It runs the same kernels with the same dispatch as
// gen9blas_gemm; the only work buffer a GEMM on device operands uses, the split-K partial slices, comes from a static
// device array instead of the library's growing buffers, so the call itself allocates nothing.
//
// Size of that array: split-K runs only for products whose tiles times slices stay within half of the CUs (at most
// 128 tile-slices on MI355X), on the small tiles: 128×128 for FP16 (FP32 sums), 64×64 for FP32, 64×128 for FP64
// (FP64 sums). So a default dispatch needs at most 128 × 16384 × 4 = 128 × 8192 × 8 = 8 MiB. Only a split forced
// with GEN9BLAS_SPLITK can need more, and is then rejected with INVALID_ARG before anything is launched.
#include "internal.h"
#include <stdio.h>

namespace {
constexpr size_t NOALLOC_SCRATCH_BYTES = 8u << 20;
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

}  // namespace g9

using namespace g9;

extern "C" int gen9blas_gemm_noalloc(int type, int transA, int transB, int M, int N, int K, double alpha, const void *A,
                                     int lda, const void *B, int ldb, double beta, void *C, int ldc) {
    G9_TRY(begin());
    void *ws = device >= 0 && device < MAX_DEVICES ? scratch_dev[device] : nullptr;
    if (!ws) G9_FAIL(GEN9BLAS_ERR, "%s", setup_error[0] ? setup_error : "gen9blas_gemm_noalloc: not set up");
    set_fixed_workspace(ws, NOALLOC_SCRATCH_BYTES, "gen9blas_gemm_noalloc");
    const int r = gemm_impl(type, transA, transB, M, N, K, alpha, A, lda, 0, B, ldb, 0, beta, C, ldc, 0, 1);
    set_fixed_workspace(nullptr, 0, nullptr);
    return r;
}
