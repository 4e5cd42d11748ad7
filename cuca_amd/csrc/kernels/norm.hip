// norm.hip -- fused residual add + RMSNorm on gfx950.
//
// Replaces the add / rms pairs of Transformer::block (cpu.rs:2650-2711) and
// the GPU attn_tail / ffn_half / ffn_tail (gpu.rs:5420-5483), whose rms is
// a chain of burn ops (gpu.rs:5883-5896).  One pass over HBM: read x and the
// branch, write x' = x + rs * [rms(branch, w_post)] and h = rms(x', w).
//
// Vector kernel: TPR threads per row, NCH 16-byte chunks per thread; the
// row lives in registers, so x' is never re-read.  Short rows share a wave
// (TPR < 64); long rows spread over up to 16 waves (TPR up to 1024, one row
// per workgroup) so a few rows at decode still issue many loads at once and
// a prefill wave holds only a few chunks.  The sum of squares is a
// per-thread sum in index order, a butterfly inside the wave and, across
// waves, an LDS sum in wave order: a fixed order, independent of the other
// rows.  y = x * (1 / sqrt(sum / H + eps)) * w, the reciprocal form of the
// reference's GPU rms (gpu.rs:5883-5896), with IEEE sqrt and reciprocal;
// against candle's x / m it differs by the rounding of one product.
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

// TPR threads per row (a power of two up to 1024), NCH chunks per thread.
// TPR <= 64: a block of 256 threads holds 256 / TPR rows.  TPR > 64: a block
// is one row of TPR threads.
// Rows wider than a wave reduce through LDS (one slot per wave), in a fixed
// order, so every thread of the row gets the same bits.
// RPB rows of TPR > 64 threads share a block, each with its own W slots.
template <int TPR, int RPB = 1>
__device__ static inline float row_sum(float v, float *red) {
    if (TPR <= CUCA_WAVE) return group_sum<TPR>(v);
    constexpr int W = TPR / CUCA_WAVE; // waves per row
    v = group_sum<CUCA_WAVE>(v);
    const int wave = threadIdx.x / CUCA_WAVE; // = row in block * W + the row's wave
    if ((threadIdx.x & (CUCA_WAVE - 1)) == 0) red[wave] = v;
    __syncthreads();
    const float *rr = red + (RPB > 1 ? (int)(threadIdx.x / TPR) * W : 0);
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < W; i++) s += rr[i];
    return s;
}

template <typename T, int TPR, int NCH, bool NTL, int RPB = 1>
__device__ static inline void norm_body(const NormArgs &a) {
    constexpr int N = Chunk<T>::N;
    constexpr int B = TPR > CUCA_WAVE ? TPR * RPB : CUCA_BLOCK;
    __shared__ float red_post[TPR > CUCA_WAVE ? RPB * TPR / CUCA_WAVE : 1];
    __shared__ float red_main[TPR > CUCA_WAVE ? RPB * TPR / CUCA_WAVE : 1];
    const int li = threadIdx.x & (TPR - 1);
    const int64_t row = (int64_t)blockIdx.x * (B / TPR) + threadIdx.x / TPR;
    // TPR > 64: the block is RPB whole rows, so `live` is uniform over a
    // row, and no thread returns before the barriers of row_sum
    const bool live = row < a.rows;
    const int H = a.hidden;
    const int nch = H / N;
    const int64_t cb = live ? row * nch : 0; // first chunk of the row

    float v[NCH][N];
#pragma unroll
    for (int k = 0; k < NCH; k++) {
        const int c = li + k * TPR;
        if (live && c < nch) {
            load_chunk<T, NTL>(a.x, cb + c, v[k]);
        } else {
#pragma unroll
            for (int i = 0; i < N; i++) v[k][i] = 0.0f;
        }
    }
    if (a.branch) {
        float b[NCH][N];
#pragma unroll
        for (int k = 0; k < NCH; k++) {
            const int c = li + k * TPR;
            if (live && c < nch) {
                load_chunk<T, NTL>(a.branch, cb + c, b[k]);
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
            ss = row_sum<TPR, RPB>(ss, red_post);
            const float inv = 1.0f / sqrtf(ss / (float)H + a.post_eps);
#pragma unroll
            for (int k = 0; k < NCH; k++) {
                const int c = li + k * TPR;
                if (c < nch) {
                    float w[N];
                    load_w<N>(a.w_post, c, w);
#pragma unroll
                    for (int i = 0; i < N; i++) b[k][i] = b[k][i] * inv * w[i];
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
    }
    if (a.x_out && live) {
#pragma unroll
        for (int k = 0; k < NCH; k++) {
            const int c = li + k * TPR;
            if (c < nch) Chunk<T>::store_nt(a.x_out, cb + c, v[k]);
        }
    }
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < NCH; k++)
#pragma unroll
        for (int i = 0; i < N; i++) ss += v[k][i] * v[k][i];
    ss = row_sum<TPR, RPB>(ss, red_main);
    // y = x * (1 / sqrt(mean + eps)) * w, the GPU mirror's form (gpu.rs:5883-5896)
    const float inv = 1.0f / sqrtf(ss / (float)H + a.eps);
    if (!live) return;
#pragma unroll
    for (int k = 0; k < NCH; k++) {
        const int c = li + k * TPR;
        if (c < nch) {
            float h[N];
            // each product rounded to f32 before the store rounds to the
            // activation type (pinned: the compiler may otherwise fold the
            // last multiply and the f16 conversion into one v_fma_mixlo_f16,
            // which rounds once)
            if (a.w) {
                float w[N];
                load_w<N>(a.w, c, w);
#pragma unroll
                for (int i = 0; i < N; i++) h[i] = pin_f32(pin_f32(v[k][i] * inv) * w[i]);
            } else {
#pragma unroll
                for (int i = 0; i < N; i++) h[i] = pin_f32(v[k][i] * inv);
            }
            Chunk<T>::store_nt(a.h_out, cb + c, h);
        }
    }
}

// The prefill form of the plain residual step -- a branch, no sandwich,
// rs = 1, weights, x' written, one chunk a thread covering the row -- with
// nothing else in it: streaming loads of x and the branch issued
// unconditionally (a row past the call reads row 0 and stores nothing),
// the weights read after the sum.  The same arithmetic and order as
// norm_body, so the same bits.  Measured on MI355X in the prefill steps
// (median of three windows): config C at 4096 rows 0.703-0.704 -> 0.72-0.74
// of the HBM peak, config E at 8192 rows 0.71-0.72 -> 0.725-0.73.
template <typename T, int TPR, int RPB = 1>
__device__ static inline void norm_plain_body(const NormArgs &a) {
    constexpr int N = Chunk<T>::N;
    constexpr int B = TPR > CUCA_WAVE ? TPR * RPB : CUCA_BLOCK;
    __shared__ float red_main[TPR > CUCA_WAVE ? RPB * TPR / CUCA_WAVE : 1];
    const int li = threadIdx.x & (TPR - 1);
    const int64_t row = (int64_t)blockIdx.x * (B / TPR) + threadIdx.x / TPR;
    const bool live = row < a.rows;
    const int H = a.hidden; // = TPR * N (the host's choice)
    const int64_t c = (live ? row * TPR : 0) + li;
    float v[N], b[N];
    load_chunk<T, true>(a.x, c, v);
    load_chunk<T, true>(a.branch, c, b);
#pragma unroll
    for (int i = 0; i < N; i++) v[i] = Chunk<T>::as_stored(v[i] + b[i]);
    if (live) Chunk<T>::store_nt(a.x_out, c, v);
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < N; i++) ss += v[i] * v[i];
    ss = row_sum<TPR, RPB>(ss, red_main);
    const float inv = 1.0f / sqrtf(ss / (float)H + a.eps);
    if (!live) return;
    float w[N], h[N];
    load_w<N>(a.w, li, w);
#pragma unroll
    for (int i = 0; i < N; i++) h[i] = pin_f32(pin_f32(v[i] * inv) * w[i]);
    Chunk<T>::store_nt(a.h_out, c, h);
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
        mb = 1.0f / sqrtf(ss / (float)H + a.post_eps);
    }
    float ss = 0.0f;
    for (int i = threadIdx.x; i < H; i += blockDim.x) {
        float v = load1<T>(a.x, base + i);
        if (a.branch) {
            float b = load1<T>(a.branch, base + i);
            if (a.w_post) b = b * mb * a.w_post[i];
            if (a.rs != 1.0f) b = b * a.rs + 0.0f;
            v = Chunk<T>::as_stored(v + b);
        }
        if (a.x_out) store1<T>(a.x_out, base + i, v);
        ss += v * v;
    }
    ss = block_sum(ss, red);
    const float inv = 1.0f / sqrtf(ss / (float)H + a.eps);
    for (int i = threadIdx.x; i < H; i += blockDim.x) {
        float v;
        if (a.x_out) { // this thread wrote element i above
            v = load1<T>(a.x_out, base + i);
        } else {
            v = load1<T>(a.x, base + i);
            if (a.branch) {
                float b = load1<T>(a.branch, base + i);
                if (a.w_post) b = b * mb * a.w_post[i];
                if (a.rs != 1.0f) b = b * a.rs + 0.0f;
                v = Chunk<T>::as_stored(v + b);
            }
        }
        const float h = a.w ? v * inv * a.w[i] : v * inv;
        store1<T>(a.h_out, base + i, h);
    }
}

#define CUCA_NORM(NAME, T, TPR, NCH, NTL)                                                  \
    extern "C" __global__ __launch_bounds__(TPR > CUCA_WAVE ? TPR : CUCA_BLOCK) void NAME(    \
        NormArgs a) {                                                                      \
        norm_body<T, TPR, NCH, NTL>(a);                                                    \
    }
// Rows of 256 threads go two to a block of 512.  Measured on MI355X in config
// E's prefill step (8192 f16 rows of 2048): the norms unchanged (0.70-0.71),
// the step 140.8-143.8 -> 139.2-141.9 us, the kernels after the norms running
// faster (SwiGLU 0.77-0.79 -> 0.81-0.82 of the HBM peak).  The bits are the same.
#define CUCA_NORM_R2(NAME, T, TPR, NCH, NTL)                                               \
    extern "C" __global__ __launch_bounds__(2 * TPR) void NAME(NormArgs a) {               \
        norm_body<T, TPR, NCH, NTL, 2>(a);                                                 \
    }
// Shapes: TPR = 2^k threads per row with one chunk each up to 1024 (every
// hidden size up to 1024 chunks: 4096 f32, 8192 f16), then 1024 threads with
// 2 or 4 chunks (8 for f32); "nt" variants stream x and the branch.
#define CUCA_NORM_SET(TN, T)                                                               \
    CUCA_NORM(cuca_norm_##TN##_t1, T, 1, 1, false)                                         \
    CUCA_NORM(cuca_norm_##TN##_t2, T, 2, 1, false)                                         \
    CUCA_NORM(cuca_norm_##TN##_t4, T, 4, 1, false)                                         \
    CUCA_NORM(cuca_norm_##TN##_t8, T, 8, 1, false)                                         \
    CUCA_NORM(cuca_norm_##TN##_t16, T, 16, 1, false)                                       \
    CUCA_NORM(cuca_norm_##TN##_t32, T, 32, 1, false)                                       \
    CUCA_NORM(cuca_norm_##TN##_t64, T, 64, 1, false)                                       \
    CUCA_NORM(cuca_norm_##TN##_t128, T, 128, 1, false)                                     \
    CUCA_NORM_R2(cuca_norm_##TN##_t256, T, 256, 1, false)                                     \
    CUCA_NORM(cuca_norm_##TN##_t512, T, 512, 1, false)                                     \
    CUCA_NORM(cuca_norm_##TN##_t1024, T, 1024, 1, false)                                   \
    CUCA_NORM(cuca_norm_##TN##_t1024_c2, T, 1024, 2, false)                                \
    CUCA_NORM(cuca_norm_##TN##_t1024_c4, T, 1024, 4, false)                                \
    CUCA_NORM(cuca_norm_##TN##_t128_nt, T, 128, 1, true)                                   \
    CUCA_NORM_R2(cuca_norm_##TN##_t256_nt, T, 256, 1, true)                                   \
    CUCA_NORM(cuca_norm_##TN##_t512_nt, T, 512, 1, true)                                   \
    CUCA_NORM(cuca_norm_##TN##_t1024_nt, T, 1024, 1, true)                                 \
    CUCA_NORM(cuca_norm_##TN##_t1024_c2_nt, T, 1024, 2, true)                              \
    extern "C" __global__ __launch_bounds__(CUCA_BLOCK) void cuca_norm_##TN##_generic(     \
        NormArgs a) {                                                                      \
        norm_generic_body<T>(a);                                                           \
    }

CUCA_NORM_SET(f32, float)
CUCA_NORM_SET(f16, _Float16)
#define CUCA_NORM_PLAIN(NAME, T, TPR, RPB)                                                 \
    extern "C" __global__ __launch_bounds__(TPR * RPB) void NAME(NormArgs a) {             \
        norm_plain_body<T, TPR, RPB>(a);                                                   \
    }
CUCA_NORM_PLAIN(cuca_norm_f32_t256_nts, float, 256, 2)
CUCA_NORM_PLAIN(cuca_norm_f32_t512_nts, float, 512, 1)
CUCA_NORM_PLAIN(cuca_norm_f32_t1024_nts, float, 1024, 1)
CUCA_NORM_PLAIN(cuca_norm_f16_t256_nts, _Float16, 256, 2)
CUCA_NORM_PLAIN(cuca_norm_f16_t512_nts, _Float16, 512, 1)
CUCA_NORM_PLAIN(cuca_norm_f16_t1024_nts, _Float16, 1024, 1)
// 8 chunks per thread: f32 rows of up to 32768 values fit in registers; f16
// rows that wide would spill and take the generic kernel.
CUCA_NORM(cuca_norm_f32_t1024_c8, float, 1024, 8, false)

// Self-test of group_sum: every group size, the library's reduction and the
// __shfl_xor butterfly side by side (the two must give the same bits).
extern "C" __global__ __launch_bounds__(CUCA_BLOCK) void cuca_selftest_group_sum(SelftestArgs a) {
    const int64_t i = (int64_t)blockIdx.x * CUCA_BLOCK + threadIdx.x; // n is a multiple of 256
    const float v = a.in[i];
    float *o = a.out;
    o[0 * a.n + i] = group_sum<2>(v);
    o[1 * a.n + i] = group_sum_shfl<2>(v);
    o[2 * a.n + i] = group_sum<4>(v);
    o[3 * a.n + i] = group_sum_shfl<4>(v);
    o[4 * a.n + i] = group_sum<8>(v);
    o[5 * a.n + i] = group_sum_shfl<8>(v);
    o[6 * a.n + i] = group_sum<16>(v);
    o[7 * a.n + i] = group_sum_shfl<16>(v);
    o[8 * a.n + i] = group_sum<32>(v);
    o[9 * a.n + i] = group_sum_shfl<32>(v);
    o[10 * a.n + i] = group_sum<64>(v);
    o[11 * a.n + i] = group_sum_shfl<64>(v);
}
