// Wave-level (64-lane) reductions shared by the skinny GEMM and GEMV kernels.
#pragma once
#include <hip/hip_runtime.h>

namespace g9 {

// Transposing butterfly: each of the 64 lanes holds NV partial sums v[0..NV-1] of the same NV outputs; afterwards
// lane l holds the complete sums of outputs base .. base + max(1, NV/64) - 1 in v[0..].
// At exchange distance d the lane keeps half of its values (the upper half when bit d of its index is set) and adds
// the partner's copy of that half, so NV sums cost NV/2 + NV/4 + ... exchanges instead of 6·NV. Once one value is
// left, the remaining distances are plain pairwise sums (the lanes that differ only in those bits end up with the
// same value). The recursion is over compile-time distances, so every index into v is a constant and v stays in
// registers.
template <int S, int NV, class R>
__device__ __forceinline__ void butterfly(R *v, int lane, int &base) {
    if constexpr (S < 6) {
        constexpr int d = 32 >> S, h = NV >> (S + 1);
        const bool up = (lane & d) != 0;
        if constexpr (h >= 1) {
#pragma unroll
            for (int i = 0; i < h; i++) {
                const R keep = up ? v[i + h] : v[i], send = up ? v[i] : v[i + h];
                v[i] = keep + __shfl_xor(send, d);
            }
            if (up) base += h;
        } else {
            v[0] += __shfl_xor(v[0], d);
        }
        butterfly<S + 1, NV, R>(v, lane, base);
    }
}

// Sums per lane after butterfly<0, NV>, and how many lanes hold each sum.
template <int NV> struct Butterfly {
    static constexpr int per_lane = NV >= 64 ? NV / 64 : 1;
    static constexpr int dup = NV >= 64 ? 1 : 64 / NV;
};

}  // namespace g9
