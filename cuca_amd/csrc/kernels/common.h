// common.h -- shared device helpers of the gfx950 per-layer kernels.
//
// Every kernel is wave64 and bandwidth-bound: activations move in 16-byte
// chunks (4 f32 or 8 f16 per lane, one global_load/store_dwordx4), all
// arithmetic is f32, and f16 results are rounded once (v_cvt_f16_f32,
// round-to-nearest-even).  The whole code object is built with
// -ffp-contract=off, so a*c - b*s is two rounded products and a rounded
// difference, as in the reference's scalar f32 code; fmaf() is written out
// where a fused multiply-add is wanted.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../kernel_args.h"

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

#define CUCA_WAVE 64
#define CUCA_BLOCK 256

// A 16-byte chunk of activations of type T, widened to f32 in registers.
// v, materialised as an f32 value: an operation written before it cannot be
// merged with one written after it (a multiply with the next multiply's
// rounding, or with a conversion to f16 into one v_fma_mix*_f16).
__device__ static inline float pin_f32(float v) {
    asm volatile("" : "+v"(v));
    return v;
}

template <typename T> struct Chunk;

template <> struct Chunk<float> {
    static constexpr int N = 4;
    __device__ static inline void load(const void *base, int64_t chunk, float (&v)[4]) {
        f32x4 t = reinterpret_cast<const f32x4 *>(base)[chunk];
        v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
    }
    // Streaming load (nontemporal hint): for inputs read once that are larger
    // than the last-level cache, so they do not evict data that is reused.
    __device__ static inline void load_nt(const void *base, int64_t chunk, float (&v)[4]) {
        f32x4 t = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(base) + chunk);
        v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
    }
    __device__ static inline void store(void *base, int64_t chunk, const float (&v)[4]) {
        f32x4 t = {v[0], v[1], v[2], v[3]};
        reinterpret_cast<f32x4 *>(base)[chunk] = t;
    }
    // Streaming store (nontemporal hint): the vector kernels write every
    // output this way.  Their outputs are read by a different kernel (a
    // GEMM, the next layer), not by the next instructions; kept in the
    // caches they would be written back to HBM during that next kernel and
    // slow it.  Measured on MI355X over the five-op prefill step of the
    // Llama-3-8B shapes: 154 -> 147 us at 4096 tokens, 550 -> 513 us at
    // 16384; decode-graph latency unchanged.
    __device__ static inline void store_nt(void *base, int64_t chunk, const float (&v)[4]) {
        f32x4 t = {v[0], v[1], v[2], v[3]};
        __builtin_nontemporal_store(t, reinterpret_cast<f32x4 *>(base) + chunk);
    }
    // The value the activation type holds for v (identity for f32).
    __device__ static inline float as_stored(float v) { return v; }
    // The chunk's raw 16 bytes, and their values.
    __device__ static inline u32x4 load_raw(const void *base, int64_t chunk) {
        return reinterpret_cast<const u32x4 *>(base)[chunk];
    }
    // (The whole vector is cast: __builtin_bit_cast(float, r.y) of one
    // element compiled to a read of element 0.)
    __device__ static inline void widen(u32x4 r, float (&v)[4]) {
        const f32x4 t = __builtin_bit_cast(f32x4, r);
        v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
    }
};

template <> struct Chunk<_Float16> {
    static constexpr int N = 8;
    __device__ static inline void load(const void *base, int64_t chunk, float (&v)[8]) {
        f16x8 t = reinterpret_cast<const f16x8 *>(base)[chunk];
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = (float)t[i];
    }
    __device__ static inline void load_nt(const void *base, int64_t chunk, float (&v)[8]) {
        f16x8 t = __builtin_nontemporal_load(reinterpret_cast<const f16x8 *>(base) + chunk);
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = (float)t[i];
    }
    // (each f32 value is pinned before its conversion, so the f16 output is
    // the f32 result rounded once more, never a single fused rounding)
    __device__ static inline void store(void *base, int64_t chunk, const float (&v)[8]) {
        f16x8 t;
#pragma unroll
        for (int i = 0; i < 8; i++) t[i] = (_Float16)pin_f32(v[i]);
        reinterpret_cast<f16x8 *>(base)[chunk] = t;
    }
    __device__ static inline void store_nt(void *base, int64_t chunk, const float (&v)[8]) {
        f16x8 t;
#pragma unroll
        for (int i = 0; i < 8; i++) t[i] = (_Float16)pin_f32(v[i]);
        __builtin_nontemporal_store(t, reinterpret_cast<f16x8 *>(base) + chunk);
    }
    // (the f32 value is pinned first: otherwise the compiler may fold the
    // operation that produced it and this rounding into one v_fma_mix*_f16,
    // which rounds once to f16 where the f32 result rounded to f16 is asked)
    __device__ static inline float as_stored(float v) {
        asm volatile("" : "+v"(v));
        return (float)(_Float16)v;
    }
    __device__ static inline u32x4 load_raw(const void *base, int64_t chunk) {
        return reinterpret_cast<const u32x4 *>(base)[chunk];
    }
    __device__ static inline void widen(u32x4 r, float (&v)[8]) {
        const f16x8 t = __builtin_bit_cast(f16x8, r);
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = (float)t[i];
    }
};

// Load chunk `c` of `base`, streaming (NT) or cached.
template <typename T, bool NT, int N>
__device__ static inline void load_chunk(const void *base, int64_t c, float (&v)[N]) {
    if (NT) Chunk<T>::load_nt(base, c, v);
    else Chunk<T>::load(base, c, v);
}

// Scalar element access for the shape-generic fallback kernels.
template <typename T> __device__ static inline float load1(const void *p, int64_t i) {
    return (float)reinterpret_cast<const T *>(p)[i];
}
// The value stored as T: an f16 store rounds the pinned f32 value.
template <typename T> __device__ static inline T to_stored(float v) {
    if constexpr (sizeof(T) == 2) return (T)pin_f32(v);
    else return (T)v;
}
template <typename T> __device__ static inline void store1(void *p, int64_t i, float v) {
    reinterpret_cast<T *>(p)[i] = to_stored<T>(v);
}

// Sum over aligned groups of G lanes (G a power of two <= 64).  A butterfly:
// at every step lane i adds lane i^off, and float addition is commutative,
// so every lane of a group ends with the same bits; the order is fixed by
// the lane layout alone, so a row's result never depends on its neighbours.
//
// Each step takes lane i ^ off's value without a trip through LDS memory
// (__shfl_xor compiles to ds_bpermute, an LDS-pipe round trip per step):
//   off 32, 16: v_permlane32_swap / v_permlane16_swap (gfx950) of v with
//               itself give each lane its own value and its partner's, in
//               one order or the other (a + b == b + a in IEEE arithmetic);
//   off 8:      DPP row_ror:8 (rotating a 16-lane row by 8 is xor 8);
//   off 4:      ds_swizzle in bit mode (xor 4 within 32 lanes);
//   off 2, 1:   DPP quad_perm [2,3,0,1] / [1,0,3,2].
// The partner and the order are the butterfly's, so the bits are those of
// the __shfl_xor form.  Every lane of the group must be active.
template <int OFF> __device__ static inline float xor_add(float v) {
    const int b = __builtin_bit_cast(int, v);
    if constexpr (OFF == 32) {
        const auto r = __builtin_amdgcn_permlane32_swap(b, b, false, false);
        return __builtin_bit_cast(float, (int)r[0]) + __builtin_bit_cast(float, (int)r[1]);
    } else if constexpr (OFF == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(b, b, false, false);
        return __builtin_bit_cast(float, (int)r[0]) + __builtin_bit_cast(float, (int)r[1]);
    } else if constexpr (OFF == 8) {
        return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, b, 0x128, 0xF, 0xF, false));
    } else if constexpr (OFF == 4) {
        return v + __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(b, 0x1F | (4 << 10)));
    } else if constexpr (OFF == 2) {
        return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, b, 0x4E, 0xF, 0xF, false));
    } else {
        static_assert(OFF == 1, "xor offsets 1 to 32");
        return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, b, 0xB1, 0xF, 0xF, false));
    }
}

// The bits of lane i ^ off's value, for off a power of two up to 32 known
// at compile time (after unrolling), every lane of the wave active: DPP
// quad_perm (1, 2) and row_ror:8 (8), ds_swizzle in bit mode (4, 16), and
// v_permlane32_swap plus a select (32), in place of __shfl_xor's
// ds_bpermute.  The caller combines the partner with its own value in the
// order it always did, so results keep their bits whatever the operation.
__device__ static inline uint32_t xor_partner_bits(uint32_t b, int off) {
    const int x = (int)b;
    switch (off) {
    case 1: return (uint32_t)__builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, false);
    case 2: return (uint32_t)__builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, false);
    case 4: return (uint32_t)__builtin_amdgcn_ds_swizzle(x, 0x1F | (4 << 10));
    case 8: return (uint32_t)__builtin_amdgcn_update_dpp(0, x, 0x128, 0xF, 0xF, false);
    case 16: return (uint32_t)__builtin_amdgcn_ds_swizzle(x, 0x1F | (16 << 10));
    default: {
        const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
        return (uint32_t)(__lane_id() < 32 ? r[1] : r[0]);
    }
    }
}

__device__ static inline float xor_partner(float v, int off) {
    return __builtin_bit_cast(float, xor_partner_bits(__builtin_bit_cast(uint32_t, v), off));
}

template <int G> __device__ static inline float group_sum(float v) {
    if constexpr (G >= 64) v = xor_add<32>(v);
    if constexpr (G >= 32) v = xor_add<16>(v);
    if constexpr (G >= 16) v = xor_add<8>(v);
    if constexpr (G >= 8) v = xor_add<4>(v);
    if constexpr (G >= 4) v = xor_add<2>(v);
    if constexpr (G >= 2) v = xor_add<1>(v);
    return v;
}

// g a power of two up to 64, uniform over the wave
__device__ static inline float group_sum_rt(float v, int g) {
    switch (g) {
    case 64: return group_sum<64>(v);
    case 32: return group_sum<32>(v);
    case 16: return group_sum<16>(v);
    case 8: return group_sum<8>(v);
    case 4: return group_sum<4>(v);
    case 2: return group_sum<2>(v);
    default: return v;
    }
}

// The reference form of group_sum (kept for the test kernel that checks
// the two give the same bits).
template <int G> __device__ static inline float group_sum_shfl(float v) {
#pragma unroll
    for (int off = G / 2; off >= 1; off >>= 1) v += __shfl_xor(v, off, CUCA_WAVE);
    return v;
}

// Sum over the whole block (blockDim.x a multiple of 64, <= 1024); every
// thread receives the same value.  `red` holds 16 floats of LDS.
__device__ static inline float block_sum(float v, float *red) {
    v = group_sum<CUCA_WAVE>(v);
    const int wave = threadIdx.x / CUCA_WAVE, nw = blockDim.x / CUCA_WAVE;
    __syncthreads(); // `red` may still be read by a previous call
    if ((threadIdx.x & (CUCA_WAVE - 1)) == 0) red[wave] = v;
    __syncthreads();
    float s = 0.0f;
    for (int i = 0; i < nw; i++) s += red[i];
    return s;
}

// Record (row, value) of a bad input in a status word, keeping the
// smallest row (global atomic, vector memory path).
__device__ static inline void record_bad(unsigned long long *word, uint32_t row, uint32_t value) {
    atomicMin(word, ((unsigned long long)row << 32) | value);
}
