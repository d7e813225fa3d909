// Launcher of the skinny GEMM kernel (C = alpha·a·wᵀ + beta·C, a M×K with M ≤ 16, w N×K, both K-contiguous).
// Kernel selection replaces the reference's skinny_k1 / skinny_r4 / skinny_r8 choice (reference: lib/src/gemm.c:225-245)
// with one template over the M tile. Per M tile, the weight rows per workgroup (RW), the waves splitting K (KS) and
// the chunks prefetched per lane (NC) are the fastest of a sweep over 155 configurations on MI355X for
// C = A·Wᵀ with W 4096×4096 FP16 rotated over 32 copies (1 GiB, beyond the 256 MB MALL).
#include "skinny_kernel.h"

namespace g9 {

template <class T, int MT, int RW, int KS, int NC>
static int launch_cfg(const sk::Params &p, bool vec) {
    const dim3 grid((unsigned)((p.N + RW - 1) / RW), (unsigned)((p.M + MT - 1) / MT)), block(KS * 64);
    if (vec) hipLaunchKernelGGL((sk::skinny_kernel<T, MT, RW, KS, NC, true>), grid, block, 0, stream, p);
    else hipLaunchKernelGGL((sk::skinny_kernel<T, MT, RW, KS, NC, false>), grid, block, 0, stream, p);
    G9_HIP(hipGetLastError());
    return 0;
}

template <int MT, int KS, int NS>
static int launch_mfma(const sk::Params &p) {
    const dim3 grid((unsigned)((p.N + 15) / 16), (unsigned)((p.M + MT - 1) / MT)), block(KS * 64);
    hipLaunchKernelGGL((sk::skinny_mfma_kernel<MT, KS, NS>), grid, block, 0, stream, p);
    G9_HIP(hipGetLastError());
    return 0;
}

template <class T>
static int launch_typed(const sk::Params &p, bool vec) {
    //                                       MT  RW  KS  NC
    if (p.M <= 1) return launch_cfg<T, 1, 1, 4, 2>(p, vec);
    if (p.M <= 2) return launch_cfg<T, 2, 2, 4, 1>(p, vec);
    if (p.M <= 4) return launch_cfg<T, 4, 4, 8, 1>(p, vec);
    if (p.M <= 8) return launch_cfg<T, 8, 4, 4, 1>(p, vec);
    return launch_cfg<T, 16, 8, 4, 1>(p, vec);   // M > 16 (forced threshold): tiles of 16 rows, w re-read per tile
}

int launch_skinny(const SkinnyCall &c) {
    sk::Params p;
    p.a = c.a; p.w = c.w; p.C = c.C;
    p.sam = c.sam; p.swn = c.swn; p.scm = c.scm; p.scn = c.scn;
    p.M = c.M; p.N = c.N; p.K = c.K;
    p.alpha = (float)c.alpha;
    p.beta = (float)c.beta;
    const int es = c.type == GEN9BLAS_S ? 4 : 2;
    const bool vec = ((uintptr_t)c.a % 16 == 0) && ((uintptr_t)c.w % 16 == 0) && (c.sam * es) % 16 == 0 &&
                     (c.swn * es) % 16 == 0;
    if ((long long)c.N > 0x7fffffffLL || (c.M + 15) / 16 > 65535)
        G9_FAIL(GEN9BLAS_ERR_UNSUPPORTED, "skinny grid too large (M %d, N %d)", c.M, c.N);
    if (c.type == GEN9BLAS_S) return launch_typed<float>(p, vec);
    // FP16, M > 2: the matrix-core kernel when K is a multiple of its 256-k groups and the rows are 16-byte aligned
    // (MI355X, W 4096×4096 rotated over 32 copies, µs per call: M = 4 7.6 against 8.7-9.1 for the dot kernel; M = 8
    // 7.8-8.0, M = 16 8.3-8.5 against 11.1 and 16.0 for the dot kernel; 2 waves with 4 stages (M = 16: 3) against
    // 1 or 4 waves and 2-6 stages; M ≤ 2 stays on the dot kernel: 7.1-7.7 against 7.6-7.7)
    if (p.M > 2 && vec && p.K % 256 == 0 && (c.swn + c.sam) * 2 * 16 < (1LL << 32)) {   // 32-bit lane offsets
        if (p.M <= 4) return launch_mfma<4, 2, 4>(p);
        if (p.M <= 8) return launch_mfma<8, 2, 4>(p);
        return launch_mfma<16, 2, 3>(p);
    }
    return launch_typed<sk::f16>(p, vec);
}

}  // namespace g9
