// glu.hip -- gated activation act(gate) * up on gfx950 (SwiGLU, GeGLU-tanh).
//
// Replaces Glu::apply / activate (cpu.rs:342-371, 3644-3649) and the GPU
// activate / gelu chain (gpu.rs:5899-5913); the ragged entry serves the MoE
// rows grouped by expert (moe.rs:39-94, cpu.rs:3599-3642), whose
// activation the reference fuses into up_kernel (moe_kernel.rs:1265-1288).
//
// Elementwise and HBM-bound: each lane reads one 16-byte chunk of gate and
// of up and writes one chunk of out, so each tensor crosses HBM once.  One
// workgroup covers BT chunks of one row (row = blockIdx / blocks per row), so
// strided rows -- the fused [gate | up] projection -- need no copy.  The
// streaming kernels run one wave per workgroup (BT = 64): at 16384 x 14336
// f16 that is 208 us against 218 us with four waves, the same bits -- a
// one-wave group retires as soon as its own loads land, so the CU takes new
// work without waiting for a group's slowest wave.
//
// The activation is evaluated with the hardware transcendental unit,
// keeping the ALU work well under the memory time:
//   SiLU      g * rcp(1 + 2^(-g log2 e))                   = g / (1 + e^-g)
//   GELU-tanh g * rcp(1 + 2^(-2 k log2 e * g (1 + 0.044715 g^2)))
//             = 0.5 g (1 + tanh(k g (1 + 0.044715 g^2))),  k = sqrt(2 / pi)
// (the identity 1 + tanh(z) = 2 / (1 + e^-2z) removes the cancellation of
// 1 + tanh(z) for z << 0).  v_exp_f32 and v_rcp_f32 are accurate to 1 ulp;
// the relative error stays below 1e-5 for |g| < 88 (the argument's own
// rounding, |arg| * 2^-24, dominates for large |g|); below that the result
// underflows through the denormals to -0, as the reference's does.

#include "common.h"

#define CUCA_LOG2E 1.4426950408889634f

// g * rcp(t) for t >= 1.  v_rcp_f32 flushes a denormal result to zero, so
// for t >= 2^64 (g < -44 in SiLU) the reciprocal is taken of t * 2^-64 and
// the product rescaled: near the f32 maximum (g < -87) the result then
// underflows gradually, as g / t does in the reference (candle's
// v / (1 + exp(-v))).  Scaling by a power of two does not change the
// reciprocal's significand.
__device__ static inline float mul_rcp(float g, float t) {
    return t < 0x1p64f ? g * __builtin_amdgcn_rcpf(t)
                       : (g * __builtin_amdgcn_rcpf(t * 0x1p-64f)) * 0x1p-64f;
}

__device__ static inline float act_silu(float g) {
    const float e = __builtin_amdgcn_exp2f(g * -CUCA_LOG2E);
    return mul_rcp(g, 1.0f + e);
}

__device__ static inline float act_gelu_tanh(float g) {
    // -2 * sqrt(2/pi) * log2(e)
    const float k2 = -2.0f * 0.7978845608028654f * CUCA_LOG2E;
    const float p = fmaf(0.044715f, g * g, 1.0f);
    const float e = __builtin_amdgcn_exp2f((k2 * g) * p);
    return mul_rcp(g, 1.0f + e);
}

template <int ACT> __device__ static inline float act_fn(float g) {
    return ACT == 0 ? act_silu(g) : act_gelu_tanh(g);
}

template <typename T, int ACT, bool RAGGED, bool NTL, int BT = CUCA_BLOCK>
__device__ static inline void glu_body(const GluArgs &a) {
    constexpr int N = Chunk<T>::N;
    const uint32_t bpr = (uint32_t)a.blocks_per_row;
    const uint32_t row = blockIdx.x / bpr;
    const uint32_t cblk = blockIdx.x - row * bpr;
    int64_t nrows = a.rows;
    if (RAGGED) {
        const int64_t total = a.offsets[a.n_experts];
        nrows = total < 0 ? 0 : (total < a.rows ? total : a.rows);
    }
    if ((int64_t)row >= nrows) return;
    const int cpr = a.ff / N;
    const int c = (int)cblk * BT + (int)threadIdx.x;
    if (c >= cpr) return;
    float g[N], u[N], o[N];
    load_chunk<T, NTL>(reinterpret_cast<const T *>(a.gate) + (int64_t)row * a.gate_ld, c, g);
    load_chunk<T, NTL>(reinterpret_cast<const T *>(a.up) + (int64_t)row * a.up_ld, c, u);
    if (a.clamp > 0.0f) { // Glu::apply's clamp (cpu.rs:364-368)
#pragma unroll
        for (int i = 0; i < N; i++) {
            g[i] = fminf(g[i], a.clamp);
            u[i] = fminf(fmaxf(u[i], -a.clamp), a.clamp);
        }
    }
#pragma unroll
    for (int i = 0; i < N; i++) o[i] = act_fn<ACT>(g[i]) * u[i];
    Chunk<T>::store_nt(reinterpret_cast<T *>(a.out) + (int64_t)row * a.out_ld, c, o);
}

// Any shape or alignment: one element per thread.
template <typename T, int ACT, bool RAGGED>
__device__ static inline void glu_generic_body(const GluArgs &a) {
    const uint32_t bpr = (uint32_t)a.blocks_per_row;
    const uint32_t row = blockIdx.x / bpr;
    const int j = (int)(blockIdx.x - row * bpr) * CUCA_BLOCK + (int)threadIdx.x;
    int64_t nrows = a.rows;
    if (RAGGED) {
        const int64_t total = a.offsets[a.n_experts];
        nrows = total < 0 ? 0 : (total < a.rows ? total : a.rows);
    }
    if ((int64_t)row >= nrows || j >= a.ff) return;
    float g = load1<T>(a.gate, (int64_t)row * a.gate_ld + j);
    float u = load1<T>(a.up, (int64_t)row * a.up_ld + j);
    if (a.clamp > 0.0f) {
        g = fminf(g, a.clamp);
        u = fminf(fmaxf(u, -a.clamp), a.clamp);
    }
    store1<T>(a.out, (int64_t)row * a.out_ld + j, act_fn<ACT>(g) * u);
}

#define CUCA_GLU(NAME, BODY, ...)                                                          \
    extern "C" __global__ __launch_bounds__(CUCA_BLOCK) void NAME(GluArgs a) {             \
        BODY<__VA_ARGS__>(a);                                                              \
    }
#define CUCA_GLU_W(NAME, BODY, ...)                                                        \
    extern "C" __global__ __launch_bounds__(CUCA_GLU_NT_BLOCK) void NAME(GluArgs a) {      \
        BODY<__VA_ARGS__, CUCA_GLU_NT_BLOCK>(a);                                           \
    }
// "nt" variants stream gate and up (inputs larger than the last-level cache).
#define CUCA_GLU_SET(TN, T)                                                                \
    CUCA_GLU(cuca_glu_##TN##_silu, glu_body, T, 0, false, false)                           \
    CUCA_GLU(cuca_glu_##TN##_gelu, glu_body, T, 1, false, false)                           \
    CUCA_GLU_W(cuca_glu_##TN##_silu_nt, glu_body, T, 0, false, true)                       \
    CUCA_GLU_W(cuca_glu_##TN##_gelu_nt, glu_body, T, 1, false, true)                       \
    CUCA_GLU(cuca_glu_##TN##_silu_ragged, glu_body, T, 0, true, false)                     \
    CUCA_GLU(cuca_glu_##TN##_gelu_ragged, glu_body, T, 1, true, false)                     \
    CUCA_GLU(cuca_glu_##TN##_silu_generic, glu_generic_body, T, 0, false)                  \
    CUCA_GLU(cuca_glu_##TN##_gelu_generic, glu_generic_body, T, 1, false)                  \
    CUCA_GLU(cuca_glu_##TN##_silu_ragged_generic, glu_generic_body, T, 0, true)            \
    CUCA_GLU(cuca_glu_##TN##_gelu_ragged_generic, glu_generic_body, T, 1, true)

CUCA_GLU_SET(f32, float)
CUCA_GLU_SET(f16, _Float16)
