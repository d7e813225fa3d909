// Launchers of the skinny GEMM kernels (C = alpha·a·wᵀ + beta·C, a M×K with M ≤ 16, w N×K), for every layout the
// reference's skinny path takes (reference: lib/src/gemm.c:197-263): w K-contiguous (its rows are the weight rows)
// or N-contiguous (row-major x·W, W stored K×N), and a K-contiguous or not (a transposed a is gathered first).
// Kernel selection replaces the reference's skinny_k1 / skinny_r4 / skinny_r8 choice (reference: lib/src/gemm.c:225-245)
// with one template over the M tile. Per M tile, the weight rows per workgroup (RW), the waves splitting K (KS) and
// the chunks prefetched per lane (NC) are the fastest of a sweep over 155 configurations on MI355X for
// C = A·Wᵀ with W 4096×4096 FP16 rotated over 32 copies (1 GiB, beyond the 256 MB MALL).
#include "skinny_kernel.h"
#include <algorithm>

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

// Weights contiguous along N (c.swn == 1, W element (k, n) at w[k·swk + n]), a K-contiguous.
template <int MT>
static int launch_n_mfma(sk::ParamsNP p, void *work) {
    constexpr int SWB = 128, SW = SWB / 2, KS = 2, NS = 4;
    const long long strips = (p.N + SW - 1) / SW;
    if (strips * p.parts > 0x7fffffffLL || (p.M + MT - 1) / MT > 65535)
        G9_FAIL(GEN9BLAS_ERR_UNSUPPORTED, "skinny grid too large (M %d, N %d)", p.M, p.N);
    p.P = reinterpret_cast<float *>(work);
    const dim3 grid((unsigned)(strips * p.parts), (unsigned)((p.M + MT - 1) / MT)), block(KS * 64);
    hipLaunchKernelGGL((sk::skinny_np_mfma_kernel<SWB, MT, KS, NS>), grid, block, 0, stream, p);
    G9_HIP(hipGetLastError());
    if (p.parts > 1) {
        const long long total = (long long)p.M * p.N;
        const unsigned blocks = (unsigned)std::min<long long>((total + 255) / 256, (long long)num_cus * 4);
        hipLaunchKernelGGL((sk::skinny_n_sum_kernel<sk::f16>), dim3(blocks), dim3(256), 0, stream, p.P, p.parts, p.M,
                           p.N, p.alpha, p.beta, reinterpret_cast<sk::f16 *>(p.C), p.scm, p.scn);
        G9_HIP(hipGetLastError());
    }
    return 0;
}

template <class T, int MT, int KS>
static int launch_n_valu(const sk::ParamsN &p, bool vec) {
    const dim3 grid((unsigned)(8 * p.per_xcd), (unsigned)((p.M + MT - 1) / MT)), block(KS * 64);
    if (vec) hipLaunchKernelGGL((sk::skinny_n_valu_kernel<T, MT, KS, true>), grid, block, 0, stream, p);
    else hipLaunchKernelGGL((sk::skinny_n_valu_kernel<T, MT, KS, false>), grid, block, 0, stream, p);
    G9_HIP(hipGetLastError());
    return 0;
}

template <class T>
static int launch_n_typed(const sk::ParamsN &p, bool vec) {
    if (p.M <= 1) return launch_n_valu<T, 1, 4>(p, vec);
    if (p.M <= 2) return launch_n_valu<T, 2, 4>(p, vec);
    if (p.M <= 4) return launch_n_valu<T, 4, 4>(p, vec);
    if (p.M <= 8) return launch_n_valu<T, 8, 4>(p, vec);
    return launch_n_valu<T, 16, 4>(p, vec);
}

// Parts of K for the matrix-core form (0: the form does not apply). FP16 with 16-byte aligned rows, N ≥ 64 and a
// multiple of 8, K a multiple of 64. Four parts where K allows (N = 4096: 64 strips × 4 = 256 workgroups); measured
// on MI355X, W 4096² rotated over 32 copies, µs per call at M = 1 / 4 / 16 including the sum: 2 parts 13.5 / 13.8 /
// 15.3, 4 parts 11.8 / 12.0 / 13.0, 8 parts 13.2 / 13.6 / 14.7; strips of 128 columns with 8 parts 12.2 / 12.6 /
// 14.1.
static int n_parts(const SkinnyCall &c) {
    if (c.type == GEN9BLAS_S) return 0;
    const bool aligned = (uintptr_t)c.w % 16 == 0 && (c.swk * 2) % 16 == 0 && (uintptr_t)c.a % 16 == 0 &&
                         (c.sam * 2) % 16 == 0;
    if (!aligned || c.N < 64 || c.N % 8 || c.K % 64 || 64 * c.swk * 2 >= (1LL << 32) || c.sam * 2 * 16 >= (1LL << 32))
        return 0;
    const int groups = c.K / 64;
    const long long strips = (c.N + 63) / 64;
    int parts = groups % 4 == 0 ? 4 : groups % 2 == 0 ? 2 : 1;
    while (parts > 1 && strips * parts > 4LL * num_cus) parts /= 2;   // enough workgroups without the split
    return parts;
}

static int launch_skinny_n(const SkinnyCall &c, void *work) {
    const int parts = n_parts(c);
    if (parts > 0) {
        sk::ParamsNP p;
        p.a = c.a; p.w = c.w; p.C = c.C; p.P = nullptr;
        p.sam = c.sam; p.swk = c.swk; p.scm = c.scm; p.scn = c.scn;
        p.M = c.M; p.N = c.N; p.K = c.K; p.parts = parts;
        p.alpha = (float)c.alpha;
        p.beta = (float)c.beta;
        if (p.M <= 4) return launch_n_mfma<4>(p, work);
        if (p.M <= 8) return launch_n_mfma<8>(p, work);
        return launch_n_mfma<16>(p, work);
    }
    sk::ParamsN p;
    p.a = c.a; p.w = c.w; p.C = c.C;
    p.sam = c.sam; p.swk = c.swk; p.scm = c.scm; p.scn = c.scn;
    p.M = c.M; p.N = c.N; p.K = c.K;
    p.alpha = (float)c.alpha;
    p.beta = (float)c.beta;
    p.strips = (c.N + 15) / 16;
    p.per_xcd = (p.strips + 7) / 8;
    if ((long long)p.per_xcd * 8 > 0x7fffffffLL || (c.M + 15) / 16 > 65535)
        G9_FAIL(GEN9BLAS_ERR_UNSUPPORTED, "skinny grid too large (M %d, N %d)", c.M, c.N);
    const int es = c.type == GEN9BLAS_S ? 4 : 2, V = 16 / es;
    const bool wvec = (uintptr_t)c.w % 16 == 0 && (c.swk * es) % 16 == 0 && c.N >= 16 && c.N % V == 0;
    if (c.type == GEN9BLAS_S) return launch_n_typed<float>(p, wvec);
    return launch_n_typed<sk::f16>(p, wvec);
}

int launch_skinny(const SkinnyCall &c0) {
    SkinnyCall c = c0;
    // One work buffer for the call: the gathered a (when a has a k stride) and the partial sums of the split
    // N-contiguous form. It is the split-K slot, which a skinny call never uses otherwise.
    const int es = c.type == GEN9BLAS_S ? 4 : 2;
    const long long ldo = (c.K + 7) / 8 * 8;
    const size_t gather = c.sak != 1 ? ((size_t)c.M * ldo * es + 255) / 256 * 256 : 0;
    SkinnyCall probe = c;
    if (c.sak != 1) { probe.sam = ldo; probe.sak = 1; probe.a = nullptr; }   // alignment as after the gather
    const int parts = c.swk != 1 ? n_parts(probe) : 0;
    const size_t partials = parts > 1 ? (size_t)parts * c.M * c.N * sizeof(float) : 0;
    void *work = nullptr;
    if (gather + partials) G9_TRY(scratch(SLOT_P, gather + partials, &work));
    if (c.sak != 1) {
        // a with a k stride (transposed a): gathered K-contiguous first (M·K elements, M ≤ 16 on the default
        // threshold)
        const long long total = (long long)c.M * c.K;
        const unsigned blocks = (unsigned)std::min<long long>((total + 255) / 256, (long long)num_cus * 4);
        if (es == 4)
            hipLaunchKernelGGL((sk::gather_a_kernel<float>), dim3(blocks), dim3(256), 0, stream,
                               (const float *)c.a, c.sam, c.sak, c.M, c.K, (float *)work, ldo);
        else
            hipLaunchKernelGGL((sk::gather_a_kernel<sk::f16>), dim3(blocks), dim3(256), 0, stream,
                               (const sk::f16 *)c.a, c.sam, c.sak, c.M, c.K, (sk::f16 *)work, ldo);
        G9_HIP(hipGetLastError());
        c.a = work;
        c.sam = ldo;
        c.sak = 1;
    }
    if (c.swk != 1) return launch_skinny_n(c, (char *)work + gather);
    sk::Params p;
    p.a = c.a; p.w = c.w; p.C = c.C;
    p.sam = c.sam; p.swn = c.swn; p.scm = c.scm; p.scn = c.scn;
    p.M = c.M; p.N = c.N; p.K = c.K;
    p.alpha = (float)c.alpha;
    p.beta = (float)c.beta;
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
