// Direct global→LDS copies (global_load_lds_dwordx4) and the waits that go with them, shared by the FP16 GEMM and
// the skinny kernels.
#pragma once
#include <hip/hip_runtime.h>

namespace g9 {

#define G9_LDS __attribute__((address_space(3)))

// One global→LDS copy of 16 bytes per lane: lane L writes LDS bytes lds + 16·L .. +15 with the 16 bytes at
// base + voff (global_load_lds_dwordx4, M0 = LDS address; one wait state between the M0 write and the load).
// Issued by inline assembly: the compiler does not track these writes, so it adds no wait for them before
// unrelated LDS reads. Callers wait for them themselves (wait_vm, and a barrier before other waves read the
// data). Nothing else in the kernels that use it touches M0.
__device__ __forceinline__ void lds_dma16(const void *base, unsigned voff, unsigned lds) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" : : "v"(voff), "s"(base), "s"(lds) : "memory");
}

// s_waitcnt fields (gfx9): vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8; a field at its maximum does not wait.
template <int N> __device__ __forceinline__ void wait_vm() {   // at most N vector-memory loads of this wave in flight
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4)); }
// At most s stages of LPS loads each still in flight, s in [0, MAXS].
template <int MAXS, int LPS> __device__ __forceinline__ void wait_vm_stages(int s) {
    if constexpr (MAXS > 0) {
        if (s >= MAXS) { wait_vm<MAXS * LPS>(); return; }
        wait_vm_stages<MAXS - 1, LPS>(s);
    } else {
        wait_vm<0>();
    }
}

}  // namespace g9
