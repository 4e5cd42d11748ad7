// norm.hip -- fused residual add + RMSNorm on gfx950.
//
// Replaces the add / rms pairs of Transformer::block (cpu.rs:2650-2711) and
// the GPU attn_tail / ffn_half / ffn_tail (gpu.rs:5420-5483), whose rms is
// a chain of burn ops (gpu.rs:5883-5896).  One pass over HBM: read x and the
// branch, write x' = x + rs * [rms(branch, w_post)] and h = rms(x', w).
//
// Vector kernel: LPR lanes per row (64 = one wave64 per row for hidden >=
// 64 chunks; fewer lanes, several rows per wave, for short rows).  The row
// lives in registers (NCH 16-byte chunks per lane), so x' is never re-read;
// the sum of squares is a per-lane sum in index order followed by a
// butterfly over the row's lanes.  m = sqrt(sum / H + eps) and
// y = v / m * w use IEEE division and square root, the reference's formula;
// only the summation order differs from candle's sequential sum.
//
// Generic kernel (any hidden, any alignment): one workgroup per row, scalar
// loads, block reduction through LDS, x' re-read from x_out (or recomputed).

#include "common.h"

template <int N>
__device__ static inline void load_w(const float *w, int64_t c, float (&v)[N]) {
    const f32x4 *p = reinterpret_cast<const f32x4 *>(w) + c * (N / 4);
#pragma unroll
    for (int j = 0; j < N / 4; j++) {
        f32x4 t = p[j];
        v[4 * j] = t.x; v[4 * j + 1] = t.y; v[4 * j + 2] = t.z; v[4 * j + 3] = t.w;
    }
}

template <typename T, int LPR, int NCH>
__device__ static inline void norm_body(const NormArgs &a) {
    constexpr int N = Chunk<T>::N;
    constexpr int RPW = CUCA_WAVE / LPR;
    const int lane = threadIdx.x & (CUCA_WAVE - 1);
    const int wave = threadIdx.x / CUCA_WAVE;
    const int li = lane & (LPR - 1);
    const int64_t row = ((int64_t)blockIdx.x * (CUCA_BLOCK / CUCA_WAVE) + wave) * RPW + lane / LPR;
    const bool live = row < a.rows;
    const int H = a.hidden;
    const int nch = H / N;
    const int64_t cb = live ? row * nch : 0; // first chunk of the row

    float v[NCH][N];
#pragma unroll
    for (int k = 0; k < NCH; k++) {
        const int c = li + k * LPR;
        if (live && c < nch) {
            Chunk<T>::load(a.x, cb + c, v[k]);
        } else {
#pragma unroll
            for (int i = 0; i < N; i++) v[k][i] = 0.0f;
        }
    }
    if (a.branch) {
        float b[NCH][N];
#pragma unroll
        for (int k = 0; k < NCH; k++) {
            const int c = li + k * LPR;
            if (live && c < nch) {
                Chunk<T>::load(a.branch, cb + c, b[k]);
            } else {
#pragma unroll
                for (int i = 0; i < N; i++) b[k][i] = 0.0f;
            }
        }
        if (a.w_post) { // Gemma sandwich: rms(branch, w_post, post_eps)
            float ss = 0.0f;
#pragma unroll
            for (int k = 0; k < NCH; k++)
#pragma unroll
                for (int i = 0; i < N; i++) ss += b[k][i] * b[k][i];
            ss = group_sum<LPR>(ss);
            const float m = sqrtf(ss / (float)H + a.post_eps);
#pragma unroll
            for (int k = 0; k < NCH; k++) {
                const int c = li + k * LPR;
                if (c < nch) {
                    float w[N];
                    load_w<N>(a.w_post, c, w);
#pragma unroll
                    for (int i = 0; i < N; i++) b[k][i] = b[k][i] / m * w[i];
                }
            }
        }
        if (a.rs != 1.0f) { // `scaled`: branch.affine(rs, 0)
#pragma unroll
            for (int k = 0; k < NCH; k++)
#pragma unroll
                for (int i = 0; i < N; i++) b[k][i] = b[k][i] * a.rs + 0.0f;
        }
#pragma unroll
        for (int k = 0; k < NCH; k++)
#pragma unroll
            for (int i = 0; i < N; i++) v[k][i] = Chunk<T>::as_stored(v[k][i] + b[k][i]);
        if (a.x_out && live) {
#pragma unroll
            for (int k = 0; k < NCH; k++) {
                const int c = li + k * LPR;
                if (c < nch) Chunk<T>::store(a.x_out, cb + c, v[k]);
            }
        }
    } else if (a.x_out && live) {
#pragma unroll
        for (int k = 0; k < NCH; k++) {
            const int c = li + k * LPR;
            if (c < nch) Chunk<T>::store(a.x_out, cb + c, v[k]);
        }
    }
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < NCH; k++)
#pragma unroll
        for (int i = 0; i < N; i++) ss += v[k][i] * v[k][i];
    ss = group_sum<LPR>(ss);
    const float m = sqrtf(ss / (float)H + a.eps);
    if (!live) return;
#pragma unroll
    for (int k = 0; k < NCH; k++) {
        const int c = li + k * LPR;
        if (c < nch) {
            float h[N];
            if (a.w) {
                float w[N];
                load_w<N>(a.w, c, w);
#pragma unroll
                for (int i = 0; i < N; i++) h[i] = v[k][i] / m * w[i];
            } else {
#pragma unroll
                for (int i = 0; i < N; i++) h[i] = v[k][i] / m;
            }
            Chunk<T>::store(a.h_out, cb + c, h);
        }
    }
}

template <typename T>
__device__ static inline void norm_generic_body(const NormArgs &a) {
    __shared__ float red[16];
    const int64_t row = blockIdx.x;
    const int H = a.hidden;
    const int64_t base = row * H;
    float mb = 1.0f;
    if (a.branch && a.w_post) {
        float ss = 0.0f;
        for (int i = threadIdx.x; i < H; i += blockDim.x) {
            const float b = load1<T>(a.branch, base + i);
            ss += b * b;
        }
        ss = block_sum(ss, red);
        mb = sqrtf(ss / (float)H + a.post_eps);
    }
    float ss = 0.0f;
    for (int i = threadIdx.x; i < H; i += blockDim.x) {
        float v = load1<T>(a.x, base + i);
        if (a.branch) {
            float b = load1<T>(a.branch, base + i);
            if (a.w_post) b = b / mb * a.w_post[i];
            if (a.rs != 1.0f) b = b * a.rs + 0.0f;
            v = Chunk<T>::as_stored(v + b);
        }
        if (a.x_out) store1<T>(a.x_out, base + i, v);
        ss += v * v;
    }
    ss = block_sum(ss, red);
    const float m = sqrtf(ss / (float)H + a.eps);
    for (int i = threadIdx.x; i < H; i += blockDim.x) {
        float v;
        if (a.x_out) { // this thread wrote element i above
            v = load1<T>(a.x_out, base + i);
        } else {
            v = load1<T>(a.x, base + i);
            if (a.branch) {
                float b = load1<T>(a.branch, base + i);
                if (a.w_post) b = b / mb * a.w_post[i];
                if (a.rs != 1.0f) b = b * a.rs + 0.0f;
                v = Chunk<T>::as_stored(v + b);
            }
        }
        const float h = a.w ? v / m * a.w[i] : v / m;
        store1<T>(a.h_out, base + i, h);
    }
}

#define CUCA_NORM(NAME, T, LPR, NCH)                                                       \
    extern "C" __global__ __launch_bounds__(CUCA_BLOCK) void NAME(NormArgs a) {            \
        norm_body<T, LPR, NCH>(a);                                                         \
    }
#define CUCA_NORM_SET(TN, T)                                                               \
    CUCA_NORM(cuca_norm_##TN##_l64_c1, T, 64, 1)                                           \
    CUCA_NORM(cuca_norm_##TN##_l64_c2, T, 64, 2)                                           \
    CUCA_NORM(cuca_norm_##TN##_l64_c4, T, 64, 4)                                           \
    CUCA_NORM(cuca_norm_##TN##_l64_c8, T, 64, 8)                                           \
    CUCA_NORM(cuca_norm_##TN##_l64_c16, T, 64, 16)                                         \
    CUCA_NORM(cuca_norm_##TN##_l32_c1, T, 32, 1)                                           \
    CUCA_NORM(cuca_norm_##TN##_l16_c1, T, 16, 1)                                           \
    CUCA_NORM(cuca_norm_##TN##_l8_c1, T, 8, 1)                                             \
    CUCA_NORM(cuca_norm_##TN##_l4_c1, T, 4, 1)                                             \
    CUCA_NORM(cuca_norm_##TN##_l2_c1, T, 2, 1)                                             \
    CUCA_NORM(cuca_norm_##TN##_l1_c1, T, 1, 1)                                             \
    extern "C" __global__ __launch_bounds__(CUCA_BLOCK) void cuca_norm_##TN##_generic(     \
        NormArgs a) {                                                                      \
        norm_generic_body<T>(a);                                                           \
    }

CUCA_NORM_SET(f32, float)
CUCA_NORM_SET(f16, _Float16)
// 8192-wide f32 rows (32 chunks per lane) still fit in registers; f16 rows
// of 32 chunks would spill and take the generic kernel instead.
CUCA_NORM(cuca_norm_f32_l64_c32, float, 64, 32)
