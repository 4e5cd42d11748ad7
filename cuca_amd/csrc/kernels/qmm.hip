// qmm.hip -- the CPU engine's quantized matmul (QmmWeight, qmm.rs) on gfx950,
// bit-exact, for Q4_0 and Q8_0 weights, with the gated activation fused in
// for the gate/up pair.
//
// Arithmetic (qmm.rs:14-45, restated by qmm/tests.rs:151-191): the
// activations are quantised to Q8_0 per 32 values (Acts::new,
// qmm.rs:1217-1343); out[j][r] is sixteen f32 lanes, lane l adding block by
// block, in row order,
//     (float)(w[l] q[l] + w[l+16] q[l+16]) * (dw * dx)
// with the product and the sum rounded separately, and the lanes reduced by
// the fixed tree of hsum (qmm.rs:1345-1353).  The kernel keeps every one of
// these roundings, so a row's bits equal the reference CPU engine's, and do
// not depend on the other rows of the call.
//
// Mapping.  A thread owns one (weight row, lane) pair: its lane accumulator
// is a sequential chain over the blocks, exactly the definition's order.  A
// workgroup is 16 weight rows x 16 lanes (256 threads) and a tile of MT
// activation rows; the 16 lanes of a row are 16 consecutive threads, and
// the final tree is a butterfly over them (xor 8, 4, 1, 2: h[i] = a[i] +
// a[i+8], then (h0+h4), (h1+h5), ..., then the pairs, then the halves).
//
// Integer part.  v_dot2_f32_f16 of two f16 pairs of small integers is exact
// (every product and partial sum is an integer below 2^24).  A weight pair
// is built as f16 values 1024 + u (bit pattern 0x6400 | u): Q4_0 u = the
// nibble (element l low, l+16 high), Q8_0 u = q + 128.  The activation pair
// is (f16 q[l], f16 q[l+16]) and the accumulator input of the dot is
// C = -(1024 + bias) (q[l] + q[l+16]), bias 8 for Q4_0 and 128 for Q8_0, so
// the dot returns the exact pair sum w[l] q[l] + w[l+16] q[l+16].
//
// Weight layout (QmmPack, built once by cuca_qpack_* from the GGUF rows):
// per row, groups of G blocks of GB bytes -- the scales first (G f16), then
// sixteen 16-byte lane chunks, so a thread reads G blocks of its lane with
// one dwordx4 load:
//   Q4_0: G = 16, GB = 288: lane chunk l, byte i = nibble byte l of block i;
//   Q8_0: G =  8, GB = 272: lane chunk l, bytes 2i, 2i+1 = quants l, l+16 of
//         block i.
// Blocks past the row's end (a partial last group) are zero.
//
// Chunks.  The blocks are processed in chunks of CB = 64.  Per chunk the
// workgroup quantises its activation tile into LDS (four threads per 32
// values), stages the 16 rows' weight scales as f32, and every thread then
// runs its chains over the chunk; the next chunk's weight loads are issued
// before the current chunk is computed.  Grid: the workgroups of one XCD
// take consecutive row blocks with all their activation tiles, so the
// weight rows a tile re-reads stay in that XCD's L2.
#include "common.h"

#define QMM_CB 64          // blocks per chunk
#define QMM_RPW 16         // weight rows per workgroup
#define QMM_XS (QMM_CB + 2) // lane stride of the staged activations (uint2 units)
#define QMM_WSS (QMM_CB + 4) // row stride of the staged weight scales (floats)

typedef _Float16 qmm_h2 __attribute__((ext_vector_type(2)));
typedef uint32_t qmm_u2 __attribute__((ext_vector_type(2)));

template <int FMT> struct QFmt;
template <> struct QFmt<0> { // Q4_0
    static constexpr int G = 16, GB = 288, SCB = 32, BB = 18;
    static constexpr float BIAS = 1032.0f; // 1024 + 8
    // the f16 pair (1024 + low nibble, 1024 + high nibble) of block i of a
    // lane chunk (byte i)
    __device__ static inline uint32_t pair(const u32x4 &v, int i) {
        const uint32_t d = v[i >> 2];
        const uint32_t sel = 0x0c000c00u | ((uint32_t)(4 + (i & 3)) << 16) | (uint32_t)(i & 3);
        return (__builtin_amdgcn_perm(d >> 4, d, sel) & 0x000f000fu) | 0x64006400u;
    }
};
template <> struct QFmt<1> { // Q8_0
    static constexpr int G = 8, GB = 272, SCB = 16, BB = 34;
    static constexpr float BIAS = 1152.0f; // 1024 + 128
    // (1024 + q[l] + 128, 1024 + q[l+16] + 128) of block i (bytes 2i, 2i+1)
    __device__ static inline uint32_t pair(const u32x4 &v, int i) {
        const uint32_t d = v[i >> 1];
        const uint32_t sel = 0x0c000c00u | ((uint32_t)(2 * (i & 1) + 1) << 16) | (uint32_t)(2 * (i & 1));
        return (__builtin_amdgcn_perm(d, d, sel) ^ 0x00800080u) + 0x64006400u;
    }
};

__device__ static inline float qmm_dot(uint32_t w, uint32_t x, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(qmm_h2, w), __builtin_bit_cast(qmm_h2, x), c,
                                  false);
}

// round_away (qmm.rs:1194-1201) then Rust's saturating `as i8` (NaN -> 0),
// as an exact integer-valued float.
__device__ static inline float qmm_quant(float t) {
    float r = roundf(t);
    r = fminf(fmaxf(r, -128.0f), 127.0f);
    return r == r ? r : 0.0f;
}

template <typename T> __device__ static inline void qmm_load8(const T *p, float (&v)[8]);
template <> __device__ inline void qmm_load8<float>(const float *p, float (&v)[8]) {
    const f32x4 a = reinterpret_cast<const f32x4 *>(p)[0];
    const f32x4 b = reinterpret_cast<const f32x4 *>(p)[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}
template <> __device__ inline void qmm_load8<_Float16>(const _Float16 *p, float (&v)[8]) {
    const f16x8 a = reinterpret_cast<const f16x8 *>(p)[0];
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = (float)a[i];
}

// LDS of one chunk.
template <int MT, bool GLU> struct QmmLds {
    qmm_u2 xe[MT][16][QMM_XS];     // per act row, lane, block: (f16 pair, C)
    float xs[MT][QMM_CB];          // act block scales
    float ws[QMM_RPW][QMM_WSS];    // gate (or plain) weight scales
    float wu[GLU ? QMM_RPW : 1][QMM_WSS]; // up weight scales
};

// Quantise the activation tile's blocks of chunk c into LDS: four threads
// per (act row, block), eight values each (Acts::new, qmm.rs:1217-1240).
template <typename T, int FMT, int MT, bool GLU>
__device__ static inline void qmm_stage_acts(const QmmArgs &a, QmmLds<MT, GLU> &L, int j0, int c) {
    const int tid = threadIdx.x;
    const int b = tid >> 2, sub = tid & 3;
    const int gb = c * QMM_CB + b;
#pragma unroll
    for (int j = 0; j < MT; j++) {
        const int ja = j0 + j;
        const bool valid = ja < a.m && gb < a.nb;
        float v[8];
        if (valid) {
            qmm_load8<T>(reinterpret_cast<const T *>(a.x) + (int64_t)ja * a.ldx + (int64_t)gb * 32 +
                             sub * 8, v);
        } else {
#pragma unroll
            for (int e = 0; e < 8; e++) v[e] = 0.0f;
        }
        float amax = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; e++) amax = fmaxf(amax, fabsf(v[e]));
        amax = fmaxf(amax, __shfl_xor(amax, 1, CUCA_WAVE));
        amax = fmaxf(amax, __shfl_xor(amax, 2, CUCA_WAVE));
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        // own quants as f16 pairs of consecutive elements (exact integers)
        uint32_t own[4], other[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            own[i] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(
                                                      qmm_quant(v[2 * i] * id), qmm_quant(v[2 * i + 1] * id)));
            other[i] = (uint32_t)__shfl_xor((int)own[i], 2, CUCA_WAVE);
        }
        // threads 0/1 own elements 0-7 / 8-15, threads 2/3 own 16-23 / 24-31;
        // sub < 2 writes lanes 8s..8s+3, sub >= 2 lanes 8s+4..8s+7 (s = sub & 1)
        const bool low = sub < 2;
        const int base = 8 * (sub & 1) + (low ? 0 : 4);
        const qmm_h2 negb = {(_Float16)(-QFmt<FMT>::BIAS), (_Float16)(-QFmt<FMT>::BIAS)};
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const uint32_t lo = low ? own[q >> 1] : other[2 + (q >> 1)];
            const uint32_t hi = low ? other[q >> 1] : own[2 + (q >> 1)];
            const uint32_t xp = __builtin_amdgcn_perm(hi, lo, (q & 1) ? 0x07060302u : 0x05040100u);
            const float cc = __builtin_amdgcn_fdot2(__builtin_bit_cast(qmm_h2, xp), negb, 0.0f, false);
            L.xe[j][base + q][b] = qmm_u2{xp, __builtin_bit_cast(uint32_t, cc)};
        }
        if (sub == 0) L.xs[j][b] = valid ? (float)(_Float16)d : 0.0f;
    }
}

// Stage the chunk's weight scales of the 16 rows as f32: threads 0..127 the
// gate (or plain) weight, 128..255 the up weight; eight blocks per thread.
template <int FMT, int MT, bool GLU>
__device__ static inline void qmm_stage_wscales(const QmmArgs &a, QmmLds<MT, GLU> &L, int row0, int c) {
    using F = QFmt<FMT>;
    const int tid = threadIdx.x;
    const int which = tid >> 7;
    if (which == 1 && !GLU) return;
    const int t = tid & 127;
    const int r = t >> 3, piece = t & 7;            // eight blocks of the chunk
    const int blk0 = c * QMM_CB + piece * 8;         // first block of the piece
    const int g = blk0 / F::G;
    const int row = row0 + r;
    float s[8];
    if (row < a.rows && g < a.ng) {
        const uint8_t *w = which ? a.w_up : a.w;
        const u32x4 raw = *reinterpret_cast<const u32x4 *>(w + (int64_t)row * a.row_bytes +
                                                           (int64_t)g * F::GB + (blk0 % F::G) * 2);
        const f16x8 h = __builtin_bit_cast(f16x8, raw);
#pragma unroll
        for (int i = 0; i < 8; i++) s[i] = (float)h[i];
    } else {
#pragma unroll
        for (int i = 0; i < 8; i++) s[i] = 0.0f;
    }
    float *dst = which ? &L.wu[GLU ? r : 0][piece * 8] : &L.ws[r][piece * 8];
    reinterpret_cast<f32x4 *>(dst)[0] = f32x4{s[0], s[1], s[2], s[3]};
    reinterpret_cast<f32x4 *>(dst)[1] = f32x4{s[4], s[5], s[6], s[7]};
}

template <int FMT>
__device__ static inline void qmm_load_w(const uint8_t *w, const QmmArgs &a, int row, int lane, int c,
                                         u32x4 (&v)[QMM_CB / QFmt<FMT>::G]) {
    using F = QFmt<FMT>;
    constexpr int NG = QMM_CB / F::G;
#pragma unroll
    for (int gg = 0; gg < NG; gg++) {
        const int g = c * NG + gg;
        if (row < a.rows && g < a.ng)
            v[gg] = *reinterpret_cast<const u32x4 *>(w + (int64_t)row * a.row_bytes + (int64_t)g * F::GB +
                                                     F::SCB + 16 * lane);
        else
            v[gg] = u32x4{0u, 0u, 0u, 0u};
    }
}

// One chunk of the chains of a thread: acc[j] += (float)p * (dw * dx).
template <int FMT, int MT, bool GLU>
__device__ static inline void qmm_chunk(const QmmLds<MT, GLU> &L, int rloc, int lane,
                                        const u32x4 (&wg)[QMM_CB / QFmt<FMT>::G],
                                        const u32x4 (&wu)[QMM_CB / QFmt<FMT>::G], float (&acc)[MT],
                                        float (&accu)[MT]) {
    using F = QFmt<FMT>;
    constexpr int NG = QMM_CB / F::G;
#pragma unroll
    for (int gg = 0; gg < NG; gg++) {
#pragma unroll
        for (int i0 = 0; i0 < F::G; i0 += 4) {
            const int b0 = gg * F::G + i0;
            const f32x4 dw = *reinterpret_cast<const f32x4 *>(&L.ws[rloc][b0]);
            f32x4 du = {0.0f, 0.0f, 0.0f, 0.0f};
            if (GLU) du = *reinterpret_cast<const f32x4 *>(&L.wu[GLU ? rloc : 0][b0]);
#pragma unroll
            for (int j = 0; j < MT; j++) {
                const f32x4 dx = *reinterpret_cast<const f32x4 *>(&L.xs[j][b0]);
                const u32x4 x01 = *reinterpret_cast<const u32x4 *>(&L.xe[j][lane][b0]);
                const u32x4 x23 = *reinterpret_cast<const u32x4 *>(&L.xe[j][lane][b0 + 2]);
                const uint32_t xp[4] = {x01.x, x01.z, x23.x, x23.z};
                const uint32_t xc[4] = {x01.y, x01.w, x23.y, x23.w};
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float c = __builtin_bit_cast(float, xc[i]);
                    const float p = qmm_dot(F::pair(wg[gg], i0 + i), xp[i], c);
                    const float s = dw[i] * dx[i];
                    acc[j] = acc[j] + p * s;
                    if (GLU) {
                        const float pu = qmm_dot(F::pair(wu[gg], i0 + i), xp[i], c);
                        const float su = du[i] * dx[i];
                        accu[j] = accu[j] + pu * su;
                    }
                }
            }
        }
    }
}

// hsum (qmm.rs:1345-1353) over the 16 lanes of a row: xor 8, 4, 1, 2.
__device__ static inline float qmm_hsum(float v) {
    v = v + __shfl_xor(v, 8, CUCA_WAVE);
    v = v + __shfl_xor(v, 4, CUCA_WAVE);
    v = v + __shfl_xor(v, 1, CUCA_WAVE);
    v = v + __shfl_xor(v, 2, CUCA_WAVE);
    return v;
}

template <typename T, int FMT, int MT, bool GLU, int ACT>
__device__ static inline void qmm_body(const QmmArgs &a) {
    using F = QFmt<FMT>;
    constexpr int NG = QMM_CB / F::G;
    __shared__ QmmLds<MT, GLU> L;
    // XCD-aware tile order: the workgroups of one XCD (id % 8) take row
    // blocks x, x + 8, ... each with all of its activation tiles in a row.
    const int id = blockIdx.x;
    const int xcd = id & 7, k = id >> 3;
    const int rb = (k / a.ntile) * 8 + xcd;
    const int tile = k % a.ntile;
    if (rb >= a.nrb) return;
    const int tid = threadIdx.x;
    const int rloc = tid >> 4, lane = tid & 15;
    const int row0 = rb * QMM_RPW, row = row0 + rloc;
    const int j0 = tile * MT;
    const int nch = (a.ng * F::G + QMM_CB - 1) / QMM_CB;

    float acc[MT], accu[MT];
#pragma unroll
    for (int j = 0; j < MT; j++) { acc[j] = 0.0f; accu[j] = 0.0f; }
    u32x4 wg[NG], wu[NG], ng_[NG], nu[NG];
    qmm_load_w<FMT>(a.w, a, row, lane, 0, wg);
    if (GLU) qmm_load_w<FMT>(a.w_up, a, row, lane, 0, wu);
    for (int c = 0; c < nch; c++) {
        qmm_stage_acts<T, FMT, MT, GLU>(a, L, j0, c);
        qmm_stage_wscales<FMT, MT, GLU>(a, L, row0, c);
        __syncthreads();
        if (c + 1 < nch) {
            qmm_load_w<FMT>(a.w, a, row, lane, c + 1, ng_);
            if (GLU) qmm_load_w<FMT>(a.w_up, a, row, lane, c + 1, nu);
        }
        qmm_chunk<FMT, MT, GLU>(L, rloc, lane, wg, wu, acc, accu);
        __syncthreads();
#pragma unroll
        for (int gg = 0; gg < NG; gg++) { wg[gg] = ng_[gg]; if (GLU) wu[gg] = nu[gg]; }
    }
#pragma unroll
    for (int j = 0; j < MT; j++) {
        float g = qmm_hsum(acc[j]);
        float o = g;
        if (GLU) {
            float u = qmm_hsum(accu[j]);
            if (a.clamp > 0.0f) { // Glu::apply's clamp (cpu.rs:364-368)
                g = fminf(g, a.clamp);
                u = fminf(fmaxf(u, -a.clamp), a.clamp);
            }
            o = (ACT == 0 ? act_silu(g) : act_gelu_tanh(g)) * u;
        }
        if (lane == 0 && row < a.rows && j0 + j < a.m)
            reinterpret_cast<T *>(a.out)[(int64_t)(j0 + j) * a.out_ld + row] = (T)o;
    }
}

// Repack GGUF Q4_0 / Q8_0 rows (src, [n][nb blocks of BB bytes]) into the
// layout above (dst, [n][ng][GB]); one thread per 16-byte piece.
template <int FMT> __device__ static inline void qpack_body(const QPackArgs &a) {
    using F = QFmt<FMT>;
    constexpr int PPG = F::GB / 16, SP = F::SCB / 16; // pieces per group, scale pieces
    const int64_t t = (int64_t)blockIdx.x * CUCA_BLOCK + threadIdx.x;
    const int64_t per_row = (int64_t)a.ng * PPG;
    if (t >= (int64_t)a.n * per_row) return;
    const int64_t row = t / per_row;
    const int rem = (int)(t - row * per_row);
    const int g = rem / PPG, piece = rem - g * PPG;
    const uint8_t *src = a.src + row * (int64_t)a.nb * F::BB;
    uint8_t out[16];
    if (piece < SP) {
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int blk = g * F::G + piece * 8 + i;
            out[2 * i] = blk < a.nb ? src[(int64_t)blk * F::BB] : 0;
            out[2 * i + 1] = blk < a.nb ? src[(int64_t)blk * F::BB + 1] : 0;
        }
    } else {
        const int l = piece - SP;
        if (FMT == 0) {
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int blk = g * 16 + i;
                out[i] = blk < a.nb ? src[(int64_t)blk * F::BB + 2 + l] : 0;
            }
        } else {
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int blk = g * 8 + i;
                out[2 * i] = blk < a.nb ? src[(int64_t)blk * F::BB + 2 + l] : 0;
                out[2 * i + 1] = blk < a.nb ? src[(int64_t)blk * F::BB + 2 + 16 + l] : 0;
            }
        }
    }
    u32x4 v;
#pragma unroll
    for (int i = 0; i < 4; i++)
        v[i] = (uint32_t)out[4 * i] | ((uint32_t)out[4 * i + 1] << 8) | ((uint32_t)out[4 * i + 2] << 16) |
               ((uint32_t)out[4 * i + 3] << 24);
    reinterpret_cast<u32x4 *>(a.dst)[t] = v;
}

extern "C" __global__ __launch_bounds__(CUCA_BLOCK) void cuca_qpack_q4_0(QPackArgs a) { qpack_body<0>(a); }
extern "C" __global__ __launch_bounds__(CUCA_BLOCK) void cuca_qpack_q8_0(QPackArgs a) { qpack_body<1>(a); }

#define CUCA_QMM(NAME, ...)                                                                \
    extern "C" __global__ __launch_bounds__(CUCA_BLOCK) void NAME(QmmArgs a) {             \
        qmm_body<__VA_ARGS__>(a);                                                          \
    }
// [act dtype][format][act rows per tile]: plain, SwiGLU, GeGLU-tanh
#define CUCA_QMM_MT(TN, T, FN, FMT, MT)                                                    \
    CUCA_QMM(cuca_qmm_##TN##_##FN##_m##MT, T, FMT, MT, false, 0)                           \
    CUCA_QMM(cuca_qmm_glu_##TN##_##FN##_silu_m##MT, T, FMT, MT, true, 0)                   \
    CUCA_QMM(cuca_qmm_glu_##TN##_##FN##_gelu_m##MT, T, FMT, MT, true, 1)
#define CUCA_QMM_SET(TN, T, FN, FMT)                                                       \
    CUCA_QMM_MT(TN, T, FN, FMT, 1)                                                         \
    CUCA_QMM_MT(TN, T, FN, FMT, 2)                                                         \
    CUCA_QMM_MT(TN, T, FN, FMT, 4)

CUCA_QMM_SET(f32, float, q4_0, 0)
CUCA_QMM_SET(f32, float, q8_0, 1)
CUCA_QMM_SET(f16, _Float16, q4_0, 0)
CUCA_QMM_SET(f16, _Float16, q8_0, 1)
