// Calibration kernels for bench.py, built into libgen9blas_calib.so (not part of libgen9blas.so or its ABI). They
// measure, on the same box and in the same run, the ceilings the library's kernels are compared with:
// - g9cal_stream_read: a pure streaming read (the HBM read rate, and the floor of a one-pass 32 MiB call such as the
//   skinny product's weight stream). Each block reads 32 KiB contiguous per step with all 8 of a lane's 16-byte
//   nontemporal loads issued before they are consumed; one float per block is written so the loads stay.
// - g9cal_touch: the one-word kernel, back to back: the launch-to-launch floor of dependent kernels on one stream.
// - g9cal_mfma: sustained matrix-core loops on random FP16 operands, v_mfma_f32_32x32x16_f16 or
//   v_mfma_f32_16x16x32_f16 at the same flops per iteration. Operands rotate through 8 register fragments per lane, so
//   their bits toggle as in a GEMM; FP16 GEMMs on random data run at the board's power limit, and this loop is the
//   rate the matrix cores sustain there with no data movement at all.
#include <hip/hip_runtime.h>
#include <algorithm>
#include <chrono>
#include <vector>
#include <stddef.h>

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int RT = 256, RU = 8;                     // threads per block, loads in flight per lane
constexpr size_t STEP = (size_t)RT * RU * 16;       // bytes per block step

__global__ void __launch_bounds__(RT) stream_read(const u32x4 *p, size_t steps, float *sink) {
    unsigned a = 0;
    for (size_t s = blockIdx.x; s < steps; s += gridDim.x) {
        const u32x4 *q = p + s * (RT * RU) + threadIdx.x;
        u32x4 v[RU];
#pragma unroll
        for (int u = 0; u < RU; u++) v[u] = __builtin_nontemporal_load(q + u * RT);
#pragma unroll
        for (int u = 0; u < RU; u++) a ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
    }
    __shared__ unsigned red[RT / 64];
    for (int o = 32; o > 0; o >>= 1) a ^= __shfl_xor(a, o);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = a;
    __syncthreads();
    if (threadIdx.x == 0) sink[blockIdx.x] = (float)(red[0] ^ red[1] ^ red[2] ^ red[3]);
}

constexpr int NSRC = 1 << 20;                       // f16x8 fragments in the source buffer (16 MiB)

__global__ void __launch_bounds__(256) mfma32(const f16x8 *src, float *out, int iters) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    f16x8 a[8], b[8];
#pragma unroll
    for (int i = 0; i < 8; i++) { a[i] = src[(t * 16 + i) % NSRC]; b[i] = src[(t * 16 + 8 + i) % NSRC]; }
    f32x16 acc[4] = {};
    for (int it = 0; it < iters; it++)
#pragma unroll
        for (int i = 0; i < 8; i++)
#pragma unroll
            for (int j = 0; j < 4; j++)
                acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[(i + j) & 7], b[(i + 2 * j) & 7], acc[j], 0, 0, 0);
    float s = 0;
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
        for (int r = 0; r < 16; r++) s += acc[j][r];
    out[t] = s;
}

__global__ void __launch_bounds__(256) mfma16(const f16x8 *src, float *out, int iters) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    f16x8 a[8], b[8];
#pragma unroll
    for (int i = 0; i < 8; i++) { a[i] = src[(t * 16 + i) % NSRC]; b[i] = src[(t * 16 + 8 + i) % NSRC]; }
    f32x4 acc[16] = {};
    for (int it = 0; it < iters; it++)
#pragma unroll
        for (int i = 0; i < 8; i++)
#pragma unroll
            for (int j = 0; j < 8; j++)
                acc[(i & 1) * 8 + j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[(i + j) & 7], b[(i + 2 * j) & 7],
                                                                              acc[(i & 1) * 8 + j], 0, 0, 0);
    float s = 0;
#pragma unroll
    for (int j = 0; j < 16; j++)
#pragma unroll
        for (int r = 0; r < 4; r++) s += acc[j][r];
    out[t] = s;
}

// One word written by one lane: the smallest kernel, for the launch-and-wait round trip.
__global__ void touch(float *out) {
    if (blockIdx.x == 0 && threadIdx.x == 0) out[0] = 1.f;
}

}  // namespace

extern "C" {

// Reads `bytes` (a multiple of 32 KiB) from p with `blocks` blocks; sink receives `blocks` floats. 0 or a HIP error.
__attribute__((visibility("default"))) int g9cal_stream_read(const void *p, size_t bytes, float *sink, int blocks,
                                                             void *stream) {
    if (!p || !sink || blocks <= 0 || bytes % STEP) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(stream_read, dim3(blocks), dim3(RT), 0, (hipStream_t)stream, (const u32x4 *)p, bytes / STEP,
                       sink);
    return (int)hipGetLastError();
}

// shape 32: v_mfma_f32_32x32x16_f16, 16: v_mfma_f32_16x16x32_f16. src: at least 16 MiB of FP16 data; out: blocks·256
// floats. Each of the blocks·4 waves runs iters × 2^20 flops.
__attribute__((visibility("default"))) int g9cal_mfma(int shape, const void *src, size_t src_bytes, float *out,
                                                      int blocks, int iters, void *stream) {
    if (!src || !out || blocks <= 0 || iters <= 0 || src_bytes < (size_t)NSRC * 16 || (shape != 32 && shape != 16))
        return (int)hipErrorInvalidValue;
    if (shape == 32) hipLaunchKernelGGL(mfma32, dim3(blocks), dim3(256), 0, (hipStream_t)stream, (const f16x8 *)src, out, iters);
    else hipLaunchKernelGGL(mfma16, dim3(blocks), dim3(256), 0, (hipStream_t)stream, (const f16x8 *)src, out, iters);
    return (int)hipGetLastError();
}

// Median over `reps` of: launch the one-word kernel on `stream`, then hipStreamSynchronize (µs); < 0 on a HIP error.
__attribute__((visibility("default"))) double g9cal_round_trip_us(float *out, int reps, void *stream) {
    if (!out || reps <= 0 || reps > 100000) return -1.0;
    std::vector<double> t((size_t)reps);
    for (int i = 0; i < reps; i++) {
        const auto t0 = std::chrono::steady_clock::now();
        hipLaunchKernelGGL(touch, dim3(1), dim3(64), 0, (hipStream_t)stream, out);
        if (hipStreamSynchronize((hipStream_t)stream) != hipSuccess) return -1.0;
        t[(size_t)i] = std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0).count();
    }
    std::sort(t.begin(), t.end());
    return t[(size_t)reps / 2];
}

// The one-word kernel launched on `stream` without waiting: back to back, the launch-to-launch floor of dependent
// kernels on one stream. 0 or a HIP error.
__attribute__((visibility("default"))) int g9cal_touch(float *out, void *stream) {
    if (!out) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(touch, dim3(1), dim3(64), 0, (hipStream_t)stream, out);
    return (int)hipGetLastError();
}

}  // extern "C"
