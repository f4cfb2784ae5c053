// dev_common.h -- small device helpers shared by the gfx950 kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define DRACO_WAVE 64

// Exact IEEE half -> float (hardware v_cvt_f32_f16 handles subnormals exactly).
__device__ __forceinline__ float h2f(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}

__device__ __forceinline__ float ubyte_f(uint32_t w, int k) {
    return (float)((w >> (8 * k)) & 0xFFu);  // lowers to v_cvt_f32_ubyteK
}

__device__ __forceinline__ float sbyte_f(uint32_t w, int k) {
    return (float)(int)(int8_t)(w >> (8 * k));  // v_bfe_i32 + v_cvt_f32_i32
}

// Full-wave (64 lane) sum, butterfly; every lane receives the total.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, DRACO_WAVE);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, DRACO_WAVE));
    return v;
}

__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, DRACO_WAVE);
    return v;
}

// Workgroup barrier that orders LDS only.  __syncthreads() carries a
// workgroup fence over all address spaces, which on gfx9 waits for every
// outstanding global load (vmcnt(0)); this one waits for LDS operations only,
// so weight loads issued before it stay in flight.  Use it only where the
// barrier protects LDS data.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }

__device__ __forceinline__ uint4 ldu4(const uint8_t* p) { return *reinterpret_cast<const uint4*>(p); }
