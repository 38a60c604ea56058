// qt_device.h — device-side helpers shared by the gfx950 decode kernels.
//
// Weight storage on the device (set up once by qwen_tts_hip.c at init):
//   bf16  rows of 2*cols bytes, the reference's row-major bits unchanged;
//   int8  rows of cols bytes holding u = q ^ 0x80 (= q + 128), so one
//         v_cvt_f32_ubyteN converts a byte; the -128 offset is folded into a
//         per-lane sum of the activation slice.  Scale f32 per row.
//   q4_0  the reference's 18-byte blocks split into qs rows (cols/2 bytes) and a
//         [rows][cols/32] array of f16 scale bits, so qs rows are 16-byte aligned
//         and one 128-bit load covers exactly one block.
// Every matvec streams weights with 128-bit loads: one 16-byte "chunk" per lane per
// load, consecutive lanes on consecutive chunks of a row, so a wave reads 1 KiB of a
// row per load instruction.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define QT_WG 256          // threads per workgroup in every matvec/attention kernel
#define QT_WAVES 4

enum { QT_BF16 = 0, QT_INT8 = 1, QT_Q4 = 2 };
enum { QT_EPI_STORE = 0, QT_EPI_RESID = 1, QT_EPI_SWIGLU = 2, QT_EPI_BIAS = 3 };

struct QtMat {
    const uint8_t *w;      // chunk rows (see above)
    const float *scale;    // int8 per-row scale
    const uint16_t *s16;   // q4 per-block f16 scale bits [rows][cols/32]
    int rows, cols;
};

__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }
__device__ __forceinline__ float bf16f(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }
__device__ __forceinline__ uint16_t f2bf_trunc(float f) { return (uint16_t)(__float_as_uint(f) >> 16); }

// binary16 -> f32 exactly as the reference's portable branch (qwen_tts_kernels.h:162-179),
// including its subnormal mapping (exponent field 112 - shift).
__device__ __forceinline__ float ref_f16_to_f32(uint32_t h) {
    uint32_t sign = (h & 0x8000u) << 16;
    uint32_t em = h & 0x7FFFu, bits;
    if (em >= 0x7C00u) bits = sign | 0x7F800000u | ((em & 0x3FFu) << 13);
    else if (em >= 0x0400u) bits = sign | ((em + (112u << 10)) << 13);
    else if (em == 0) bits = sign;
    else {
        uint32_t sh = __clz(em) - 21;          // shifts until bit 10 is set
        uint32_t m = em << sh;
        bits = sign | ((112u - sh) << 23) | ((m & 0x3FFu) << 13);
    }
    return __uint_as_float(bits);
}

template <int W>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int o = W / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
template <int W>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
    for (int o = W / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// Block-wide sum over QT_WG threads; every thread gets the result.  `red` >= QT_WAVES floats.
__device__ __forceinline__ float block_sum(float v, float *red) {
    v = group_sum<64>(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < QT_WAVES; i++) t += red[i];
    return t;
}

// Agent-scope relaxed accesses: compiled to global_load/store with the sc1 bit, so they
// go to the device coherence point instead of a (per-XCD, non-coherent) L2 line.  Used
// for the few values one workgroup publishes to workgroups on other XCDs inside one
// kernel; ordering is by s_waitcnt + a device-scope atomic, no L2 write-back/invalidate.
__device__ __forceinline__ void st_agent(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_agent(const float *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint4 ld_chunk(const uint8_t *p) {
    return *reinterpret_cast<const uint4 *>(p);
}
