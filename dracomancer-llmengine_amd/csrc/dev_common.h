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

// ---- cross-lane exchange inside the VALU --------------------------------------
// A DPP row move (rows are 16 lanes) or a gfx950 permlane swap moves a value
// between lanes without the LDS round trip that ds_bpermute (__shfl_xor) costs
// per step.  A reduction step pairs lanes by an involution: xor 1, xor 2,
// mirror within 8 lanes, mirror within 16 lanes, xor 16, xor 32.  After the
// steps before it each half of a mirror is uniform, so the mirror stands in for
// xor 4 / xor 8.  Both lanes of a pair apply the same commutative operation to
// the same two values, so every lane of a group ends with bit-identical
// results.  Every lane of the groups involved must be active.
enum : int { DPP_XOR1 = 0xB1, DPP_XOR2 = 0x4E, DPP_MIRROR8 = 0x141, DPP_MIRROR16 = 0x140 };

template <int CTRL, class T>
__device__ __forceinline__ T dpp(T v) {
    static_assert(sizeof(T) == 4, "32-bit lane values");
    return __builtin_bit_cast(T, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Own value and the partner's (lane i ^ 16, resp. i ^ 32), in an order that
// depends on the lane; .x + .y (or any commutative op) is the pair's result.
template <class T>
struct LanePair {
    T x, y;
};
template <class T>
__device__ __forceinline__ LanePair<T> swap16(T v) {
    const int b = __builtin_bit_cast(int, v);
    const auto p = __builtin_amdgcn_permlane16_swap(b, b, false, false);
    return {__builtin_bit_cast(T, (int)p[0]), __builtin_bit_cast(T, (int)p[1])};
}
template <class T>
__device__ __forceinline__ LanePair<T> swap32(T v) {
    const int b = __builtin_bit_cast(int, v);
    const auto p = __builtin_amdgcn_permlane32_swap(b, b, false, false);
    return {__builtin_bit_cast(T, (int)p[0]), __builtin_bit_cast(T, (int)p[1])};
}

// The value lane i ^ 16 (resp. i ^ 32) holds.  permlane16_swap leaves the
// first result's even rows and the second's odd rows in place, so a lane reads
// its partner from the other one.
template <class T>
__device__ __forceinline__ T lane_xor16(T v) {
    const LanePair<T> p = swap16(v);
    return (__lane_id() & 16) ? p.x : p.y;
}
template <class T>
__device__ __forceinline__ T lane_xor32(T v) {
    const LanePair<T> p = swap32(v);
    return (__lane_id() & 32) ? p.x : p.y;
}

// A lane pairing that flips bit log2(m) of the lane index (m = 1, 2, ..., 32):
// xor m for m = 1, 2, 16, 32, the mirror within 2m lanes for m = 4, 8.  The
// two lanes of a pair always differ in that bit, so (lane & m) still tells
// them apart, which is all a reduce-scatter step needs.  m must be a
// compile-time constant after unrolling.
template <class T>
__device__ __forceinline__ T lane_flip(T v, int m) {
    switch (m) {
    case 32: return lane_xor32(v);
    case 16: return lane_xor16(v);
    case 8: return dpp<DPP_MIRROR16>(v);
    case 4: return dpp<DPP_MIRROR8>(v);
    case 2: return dpp<DPP_XOR2>(v);
    default: return dpp<DPP_XOR1>(v);
    }
}

// Reduction over each aligned group of G lanes (G = 1, 2, 4, ..., 64) with a
// commutative op; every lane of the group receives the result.
template <int G, class T, class Op>
__device__ __forceinline__ T group_reduce(T v, Op op) {
    static_assert(G >= 1 && G <= 64 && (G & (G - 1)) == 0, "power-of-two group");
    if constexpr (G >= 2) v = op(v, dpp<DPP_XOR1>(v));
    if constexpr (G >= 4) v = op(v, dpp<DPP_XOR2>(v));
    if constexpr (G >= 8) v = op(v, dpp<DPP_MIRROR8>(v));
    if constexpr (G >= 16) v = op(v, dpp<DPP_MIRROR16>(v));
    if constexpr (G >= 32) {
        const LanePair<T> p = swap16(v);
        v = op(p.x, p.y);
    }
    if constexpr (G >= 64) {
        const LanePair<T> p = swap32(v);
        v = op(p.x, p.y);
    }
    return v;
}

// Reduction over the four rows: lanes i, i^16, i^32, i^48.
template <class T, class Op>
__device__ __forceinline__ T rows_reduce(T v, Op op) {
    const LanePair<T> p = swap16(v);
    v = op(p.x, p.y);
    const LanePair<T> q = swap32(v);
    return op(q.x, q.y);
}

struct OpAdd {
    template <class T>
    __device__ __forceinline__ T operator()(T a, T b) const { return a + b; }
};
struct OpMax {
    __device__ __forceinline__ float operator()(float a, float b) const { return fmaxf(a, b); }
};

template <int G = 64>
__device__ __forceinline__ float group_sum(float v) { return group_reduce<G>(v, OpAdd{}); }
template <int G = 64>
__device__ __forceinline__ float group_max(float v) { return group_reduce<G>(v, OpMax{}); }

// Full-wave (64 lane) reductions; every lane receives the result.
__device__ __forceinline__ float wave_sum(float v) { return group_reduce<64>(v, OpAdd{}); }
__device__ __forceinline__ float wave_max(float v) { return group_reduce<64>(v, OpMax{}); }
__device__ __forceinline__ int wave_sum_i(int v) { return group_reduce<64>(v, OpAdd{}); }
__device__ __forceinline__ float rows_sum(float v) { return rows_reduce(v, OpAdd{}); }
__device__ __forceinline__ int rows_sum_i(int v) { return rows_reduce(v, OpAdd{}); }

// (value, index) maximum over each aligned group of G lanes, ties to the lower
// index (the first maximum in index order, whatever order the pairs meet in).
// NaN ranks above every number, as in np.argmax (src/smol_engine.py:212):
// any NaN makes the result the first NaN's index.
__device__ __forceinline__ void am_merge(float& v, int& i, float v2, int i2) {
    const bool n1 = v != v, n2 = v2 != v2;
    const bool take = n2 ? (!n1 || i2 < i) : (!n1 && (v2 > v || (v2 == v && i2 < i)));
    if (take) {
        v = v2;
        i = i2;
    }
}
template <int G>
__device__ __forceinline__ void group_argmax(float& v, int& i) {
    static_assert(G >= 1 && G <= 64 && (G & (G - 1)) == 0, "power-of-two group");
    if constexpr (G >= 2) am_merge(v, i, dpp<DPP_XOR1>(v), dpp<DPP_XOR1>(i));
    if constexpr (G >= 4) am_merge(v, i, dpp<DPP_XOR2>(v), dpp<DPP_XOR2>(i));
    if constexpr (G >= 8) am_merge(v, i, dpp<DPP_MIRROR8>(v), dpp<DPP_MIRROR8>(i));
    if constexpr (G >= 16) am_merge(v, i, dpp<DPP_MIRROR16>(v), dpp<DPP_MIRROR16>(i));
    if constexpr (G >= 32) am_merge(v, i, lane_xor16(v), lane_xor16(i));
    if constexpr (G >= 64) am_merge(v, i, lane_xor32(v), lane_xor32(i));
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

// The pending accumulator's flag (a uniform int64) through a vector load at
// an opaque per-lane offset of 0: a plain uniform load becomes a scalar load
// that the compiler schedules after the vector loads and then waits for.
__device__ __forceinline__ long long load_flag(const long long* p) {
    int z;
    asm volatile("v_mov_b32 %0, 0" : "=v"(z));
    return p[z];
}

// x + acc * 2^-32 for a pending residual held as int64 fixed point (acc of
// four inputs in a, b), or NaN in every lane when the accumulator's flag is
// set.  Branch-free: under an if / else the compiler moves the x and acc
// loads into the branch, behind the flag's load, which costs a memory round
// trip.
__device__ __forceinline__ float4 fx_pending(float4 v, longlong2 a, longlong2 b, bool bad) {
    constexpr float S = 2.3283064365386963e-10f;  // 2^-32
    const float n = __builtin_nanf("");
    const float x = v.x + (float)a.x * S, y = v.y + (float)a.y * S;
    const float z = v.z + (float)b.x * S, w = v.w + (float)b.y * S;
    return make_float4(bad ? n : x, bad ? n : y, bad ? n : z, bad ? n : w);
}


// Streaming load of data read once per launch (quantized weights): the
// non-temporal hint marks the lines for early eviction, so a weight stream
// does not push activations, KV rows and other reused data out of L2.
// Measured on the decode chain: 1919 -> 1943 tok/s.
typedef unsigned int v4u32 __attribute__((ext_vector_type(4)));
// Weight streams live in global memory.  A pointer read from memory (an
// expert table) is generic to the compiler, and a generic (flat) load also
// counts against the LDS wait counter, so every LDS barrier behind it would
// wait for the weights; the cast makes it a global load.
template <class T>
__device__ __forceinline__ const __attribute__((address_space(1))) T* gptr(const void* p) {
    return (const __attribute__((address_space(1))) T*)p;
}
// 16 weight bytes through the global address space (the grouped expert GEMMs' items)
__device__ __forceinline__ uint4 ldu4(const uint8_t* p) {
    const v4u32 v = *gptr<v4u32>(p);
    return make_uint4(v.x, v.y, v.z, v.w);
}
// Lane s's pointer (s wave-uniform) read into SGPRs: a table of up to 64
// pointers held one per lane is indexed without writing a VGPR (a VGPR
// temporary can land on the destination of a load still in flight, and the
// compiler then waits for every load before writing it).
__device__ __forceinline__ const uint8_t* lane_ptr(const uint8_t* p, int s) {
    const unsigned long long v = reinterpret_cast<unsigned long long>(p);
    const unsigned lo = __builtin_amdgcn_readlane((unsigned)v, s);
    const unsigned hi = __builtin_amdgcn_readlane((unsigned)(v >> 32), s);
    return reinterpret_cast<const uint8_t*>(((unsigned long long)hi << 32) | lo);
}

__device__ __forceinline__ uint4 ldnt4(const uint8_t* p) {
    const v4u32 v = __builtin_nontemporal_load(gptr<v4u32>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}
