// attn_rows.hip -- paged attention of many query rows of one sequence
// (a prefill chunk, verification rows) on gfx950, on the matrix cores.
//
// Replaces attend_paged_rows / attend_latent_rows (cpu/paged_attn.rs:
// 177-309) and the GPU engine's gather-then-matmul prefill attention
// (paged_kernel.rs:6-8): row r of q attends to the positions ranges[r] =
// [lo, hi) of one block table, query head h reading KV head h / G (G =
// n_head / n_kv), the scores scaled by `scale`, an online softmax over the
// keys, the values a pool of their own.  The pools are [n_blocks, n_kv, 16,
// d], read in place through the table (no gather copy).
//
// Matrix-core kernel: a workgroup per (16 query rows, KV head), one wave per
// query head of the GQA group (G waves).  Per 16-position block of the
// table (the paged block), the workgroup stages the block's K rows and V
// rows in LDS, and every wave computes the block's scores transposed, S^T =
// K Q^T (16 keys x 16 rows, MFMA), so that a lane holds four keys of ONE
// query row: the row's softmax statistics are per lane, reduced over four
// lanes, and S^T is already the P^T operand of O^T = V^T P^T (d x 16 rows,
// MFMA), whose lane holds four consecutive output columns of its row.
// - f16 pools: v_mfma_f32_16x16x16f16; the score products are exact, their
//   sums f32.  The probabilities enter the value product as two f16 parts,
//   p = hi + lo / 2048 (hi = f16(p), lo = f16((p - hi) 2048)), into two
//   accumulators: 22 bits of p, where one f16 part would round p to 11 bits
//   (5e-4 relative, far outside the 1e-5 bar).
// - f32 pools: v_mfma_f32_16x16x4f32, every operand f32.
// Scores, exponentials and sums are f32; the order of the sums differs from
// the reference's sequential one, which the bar absorbs (1e-5 relative plus
// 1e-5 of the range's largest value).  A row's keys, block order and masking
// depend only on its own range (positions outside it get probability 0 and
// leave the maximum alone), so a row's result does not depend on the other
// rows of its tile or call.
// A row with an empty range, or one past the table, gives zeros and is
// recorded (CUCA_STATUS_KV_RANGE, value all ones); a block of a row's range
// outside the pool too (value: the block's first position in the range),
// as the decode kernel records them.
//
// Generic kernel (any head_dim and group, and the latent form): a wave per
// (row, query head), the reference's own loop -- block by block, scores,
// block maximum, rescale, weighted values -- with the dot products a lane
// per column and a butterfly.

#include "common.h"

#pragma clang fp contract(off)

typedef _Float16 attn_h4 __attribute__((ext_vector_type(4)));

// The block's status for a row: its range [lo, hi) meets positions
// [16 b, 16 b + 16).
__device__ static inline bool rows_meets(int lo, int hi, int b) { return lo < 16 * b + 16 && hi > 16 * b; }

template <typename T, int D, int G>
__device__ static inline void attn_rows_body(const AttnRowsArgs &a) {
    constexpr bool F16 = sizeof(T) == 2;
    constexpr int NT = 64 * G;                 // threads
    constexpr int NS = D / 16;                 // output column slices
    constexpr int KST = F16 ? D + 16 : D + 4;  // K row stride in LDS (elements)
    constexpr int VST = F16 ? 16 : D + 4;      // f16: V^T [D][16]; f32: V [16][D + 4]
    __shared__ __align__(16) T ks[16 * KST];
    __shared__ __align__(16) T vs[F16 ? D * 16 : 16 * (D + 4)];
    const int wave = threadIdx.x / 64, lane = threadIdx.x & 63;
    const int r = lane & 15, grp = lane >> 4;
    const int tile = blockIdx.x / a.n_kv, kvh = blockIdx.x - tile * a.n_kv;
    const int row = tile * 16 + r;
    const int head = kvh * G + wave;
    const bool in_call = row < a.rows;
    int lo = 0, hi = 0;
    if (in_call) {
        lo = a.ranges[2 * row];
        hi = a.ranges[2 * row + 1];
    }
    const bool valid = in_call && lo >= 0 && hi > lo && (int64_t)hi <= (int64_t)a.max_blocks * 16;
    if (in_call && !valid && kvh == 0 && wave == 0 && grp == 0)
        record_bad(a.status + CUCA_STATUS_KV_RANGE, (uint32_t)row, 0xffffffffu);
    // the tile's blocks: the union of its valid rows' ranges (the same in
    // every wave)
    int tlo = valid ? lo : 0x7fffffff, thi = valid ? hi : 0;
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) {
        tlo = min(tlo, __shfl_xor(tlo, off));
        thi = max(thi, __shfl_xor(thi, off));
    }
    T *orow = reinterpret_cast<T *>(a.out) + (int64_t)(in_call ? row : 0) * a.out_ld + (int64_t)head * D;
    // the query: lane (r, grp) holds row r's dims 16 j + 4 grp .. + 3 (f16)
    // or 4 j + grp (f32), j over the k-steps
    constexpr int QN = F16 ? NS : D / 4;
    attn_h4 qh[F16 ? NS : 1];
    float qf[F16 ? 1 : D / 4];
    {
        const T *qrow = reinterpret_cast<const T *>(a.q) + (int64_t)(in_call ? row : 0) * a.q_ld + (int64_t)head * D;
#pragma unroll
        for (int j = 0; j < QN; j++) {
            if constexpr (F16) qh[j] = *reinterpret_cast<const attn_h4 *>(qrow + 16 * j + 4 * grp);
            else qf[j] = (float)qrow[4 * j + grp];
        }
    }
    f32x4 acc[NS], acl[F16 ? NS : 1];
#pragma unroll
    for (int s = 0; s < NS; s++) {
        acc[s] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        if constexpr (F16) acl[s] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    float m = -__builtin_huge_valf(), l = 0.0f;
    bool bad = false;
    const T *pv = reinterpret_cast<const T *>(a.pool_v ? a.pool_v : a.pool_k);
    if (thi > 0) {
        const int b0 = tlo >> 4, b1 = (thi - 1) >> 4;
        for (int b = b0; b <= b1; b++) {
            const uint32_t blk = a.table[b];
            const bool ok = (int64_t)blk < a.n_blocks;
            if (!ok && valid && rows_meets(lo, hi, b)) {
                bad = true;
                if (kvh == 0 && wave == 0 && grp == 0)
                    record_bad(a.status + CUCA_STATUS_KV_RANGE, (uint32_t)row, (uint32_t)max(16 * b, lo));
            }
            const int64_t base = ((int64_t)(ok ? blk : 0u) * a.n_kv + kvh) * 16 * D; // the block's 16 rows
            // stage K and V of the block (16 x D each) in LDS
            constexpr int CH = 16 * D * (int)sizeof(T) / 16; // 16-byte chunks per block
            constexpr int CPR = D * (int)sizeof(T) / 16;     // chunks per row
#pragma unroll
            for (int c0 = 0; c0 < CH; c0 += NT) {
                const int c = c0 + (int)threadIdx.x;
                if (CH % NT == 0 || c < CH) {
                    const int key = c / CPR, col = (c - key * CPR) * (16 / (int)sizeof(T));
                    const u32x4 kc = *reinterpret_cast<const u32x4 *>(reinterpret_cast<const T *>(a.pool_k) + base +
                                                                      key * D + col);
                    const u32x4 vc = *reinterpret_cast<const u32x4 *>(pv + base + key * D + col);
                    *reinterpret_cast<u32x4 *>(ks + key * KST + col) = kc;
                    if constexpr (F16) {
                        const f16x8 v8 = __builtin_bit_cast(f16x8, vc);
#pragma unroll
                        for (int i = 0; i < 8; i++) vs[(col + i) * 16 + key] = v8[i];
                    } else {
                        *reinterpret_cast<u32x4 *>(vs + key * VST + col) = vc;
                    }
                }
            }
            __syncthreads();
            // S^T: lane (r, grp) gets the scores of keys 4 grp + i with row r
            f32x4 st = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            if constexpr (F16) {
#pragma unroll
                for (int j = 0; j < NS; j++) {
                    const attn_h4 kk = *reinterpret_cast<const attn_h4 *>(ks + r * KST + 16 * j + 4 * grp);
                    st = __builtin_amdgcn_mfma_f32_16x16x16f16(kk, qh[j], st, 0, 0, 0);
                }
            } else {
#pragma unroll
                for (int j = 0; j < D / 4; j++)
                    st = __builtin_amdgcn_mfma_f32_16x16x4f32((float)ks[r * KST + 4 * j + grp], qf[j], st, 0, 0, 0);
            }
            float x[4];
            bool in[4];
            float bmax = -__builtin_huge_valf();
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int p = 16 * b + 4 * grp + i;
                in[i] = valid && p >= lo && p < hi;
                x[i] = st[i] * a.scale;
                if (in[i]) bmax = fmaxf(bmax, x[i]);
            }
            bmax = fmaxf(bmax, __shfl_xor(bmax, 16));
            bmax = fmaxf(bmax, __shfl_xor(bmax, 32));
            if (bmax > m) { // rescale what was accumulated under the old maximum
                const float corr = expf(m - bmax);
                l *= corr;
#pragma unroll
                for (int s = 0; s < NS; s++) {
                    acc[s] *= corr;
                    if constexpr (F16) acl[s] *= corr;
                }
                m = bmax;
            }
            float e[4], es = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                e[i] = in[i] ? expf(x[i] - m) : 0.0f;
                es += e[i];
            }
            es += __shfl_xor(es, 16);
            es += __shfl_xor(es, 32);
            l += es;
            // O^T += V^T P^T
            if constexpr (F16) {
                attn_h4 ph, pl;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    ph[i] = (_Float16)e[i];
                    pl[i] = (_Float16)((e[i] - (float)ph[i]) * 2048.0f);
                }
#pragma unroll
                for (int s = 0; s < NS; s++) {
                    const attn_h4 vv = *reinterpret_cast<const attn_h4 *>(vs + (16 * s + r) * 16 + 4 * grp);
                    acc[s] = __builtin_amdgcn_mfma_f32_16x16x16f16(vv, ph, acc[s], 0, 0, 0);
                    acl[s] = __builtin_amdgcn_mfma_f32_16x16x16f16(vv, pl, acl[s], 0, 0, 0);
                }
            } else {
#pragma unroll
                for (int s = 0; s < NS; s++)
#pragma unroll
                    for (int j = 0; j < 4; j++)
                        acc[s] = __builtin_amdgcn_mfma_f32_16x16x4f32((float)vs[(4 * grp + j) * VST + 16 * s + r], e[j],
                                                                      acc[s], 0, 0, 0);
            }
            __syncthreads(); // before the next block overwrites the tiles
        }
    }
    if (!in_call) return;
    // lane (r, grp) holds O^T[16 s + 4 grp + i][row r]
    const bool zero = !valid || bad;
#pragma unroll
    for (int s = 0; s < NS; s++) {
        float o[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float v = F16 ? acc[s][i] + acl[s][i] * (1.0f / 2048.0f) : acc[s][i];
            o[i] = zero ? 0.0f : v / l;
        }
        T *dst = orow + 16 * s + 4 * grp;
        if constexpr (F16) {
            attn_h4 h;
#pragma unroll
            for (int i = 0; i < 4; i++) h[i] = (_Float16)pin_f32(o[i]);
            *reinterpret_cast<attn_h4 *>(dst) = h;
        } else {
            *reinterpret_cast<f32x4 *>(dst) = f32x4{o[0], o[1], o[2], o[3]};
        }
    }
}

// The generic kernel: a wave per (row, query head), the reference's loop.
// Values: pool_v rows, or the first v_width columns of the key rows.
template <typename T>
__device__ static inline void attn_rows_generic_body(const AttnRowsArgs &a) {
    const int lane = threadIdx.x & 63;
    const int64_t job = (int64_t)blockIdx.x * 4 + threadIdx.x / 64;
    if (job >= (int64_t)a.rows * a.n_head) return; // whole wave
    const int row = (int)(job / a.n_head), head = (int)(job - (int64_t)row * a.n_head);
    const int G = a.n_head / a.n_kv, kvh = head / G;
    const int D = a.head_dim, VW = a.v_width;
    const int lo = a.ranges[2 * row], hi = a.ranges[2 * row + 1];
    T *orow = reinterpret_cast<T *>(a.out) + (int64_t)row * a.out_ld + (int64_t)head * VW;
    const bool valid = lo >= 0 && hi > lo && (int64_t)hi <= (int64_t)a.max_blocks * 16;
    bool bad = !valid;
    if (!valid && head == 0 && lane == 0) record_bad(a.status + CUCA_STATUS_KV_RANGE, (uint32_t)row, 0xffffffffu);
    const T *q = reinterpret_cast<const T *>(a.q) + (int64_t)row * a.q_ld + (int64_t)head * D;
    const T *pk = reinterpret_cast<const T *>(a.pool_k);
    const T *pv = reinterpret_cast<const T *>(a.pool_v ? a.pool_v : a.pool_k);
    constexpr int MAXC = 8;            // value columns a lane, v_width <= 512
    float acc[MAXC];
#pragma unroll
    for (int c = 0; c < MAXC; c++) acc[c] = 0.0f;
    float m = -__builtin_huge_valf(), sum = 0.0f;
    for (int b = valid ? lo >> 4 : 1, be = valid ? (hi - 1) >> 4 : 0; b <= be && !bad; b++) {
        const uint32_t blk = a.table[b];
        if ((int64_t)blk >= a.n_blocks) {
            bad = true;
            if (head == 0 && lane == 0)
                record_bad(a.status + CUCA_STATUS_KV_RANGE, (uint32_t)row, (uint32_t)max(16 * b, lo));
            break;
        }
        const int p0 = max(lo, 16 * b), p1 = min(hi, 16 * b + 16);
        const int64_t base = ((int64_t)blk * a.n_kv + kvh) * 16;
        float sc[16];
        float bmax = -__builtin_huge_valf();
        for (int p = p0; p < p1; p++) {
            const T *kr = pk + (base + (p & 15)) * D;
            float d = 0.0f;
            for (int c = lane; c < D; c += 64) d += (float)q[c] * (float)kr[c];
            d = group_sum<64>(d);
            const float s = d * a.scale;
            sc[p - p0] = s;
            bmax = fmaxf(bmax, s);
        }
        if (bmax > m) {
            const float corr = expf(m - bmax);
            sum *= corr;
#pragma unroll
            for (int c = 0; c < MAXC; c++) acc[c] *= corr;
            m = bmax;
        }
        for (int p = p0; p < p1; p++) {
            const float e = expf(sc[p - p0] - m);
            sum += e;
            const T *vr = pv + (base + (p & 15)) * D; // a value row sits where its key row does
#pragma unroll
            for (int c = 0; c < MAXC; c++) {
                const int col = lane + 64 * c;
                if (col < VW) acc[c] += e * (float)vr[col];
            }
        }
    }
#pragma unroll
    for (int c = 0; c < MAXC; c++) {
        const int col = lane + 64 * c;
        if (col < VW) orow[col] = to_stored<T>(bad ? 0.0f : acc[c] / sum);
    }
}

#define CUCA_ATTN_ROWS(NAME, T, D, G)                                                      \
    extern "C" __global__ __launch_bounds__(64 * G) void NAME(AttnRowsArgs a) {            \
        attn_rows_body<T, D, G>(a);                                                        \
    }
#define CUCA_ATTN_ROWS_SET(TN, T)                                                          \
    CUCA_ATTN_ROWS(cuca_attn_rows_##TN##_d64_g1, T, 64, 1)                                 \
    CUCA_ATTN_ROWS(cuca_attn_rows_##TN##_d64_g2, T, 64, 2)                                 \
    CUCA_ATTN_ROWS(cuca_attn_rows_##TN##_d64_g4, T, 64, 4)                                 \
    CUCA_ATTN_ROWS(cuca_attn_rows_##TN##_d64_g8, T, 64, 8)                                 \
    CUCA_ATTN_ROWS(cuca_attn_rows_##TN##_d128_g1, T, 128, 1)                               \
    CUCA_ATTN_ROWS(cuca_attn_rows_##TN##_d128_g2, T, 128, 2)                               \
    CUCA_ATTN_ROWS(cuca_attn_rows_##TN##_d128_g4, T, 128, 4)                               \
    CUCA_ATTN_ROWS(cuca_attn_rows_##TN##_d128_g8, T, 128, 8)                               \
    CUCA_ATTN_ROWS(cuca_attn_rows_##TN##_d256_g1, T, 256, 1)                               \
    CUCA_ATTN_ROWS(cuca_attn_rows_##TN##_d256_g2, T, 256, 2)                               \
    CUCA_ATTN_ROWS(cuca_attn_rows_##TN##_d256_g4, T, 256, 4)                               \
    CUCA_ATTN_ROWS(cuca_attn_rows_##TN##_d256_g8, T, 256, 8)                               \
    extern "C" __global__ __launch_bounds__(CUCA_BLOCK) void cuca_attn_rows_##TN##_generic( \
        AttnRowsArgs a) {                                                                  \
        attn_rows_generic_body<T>(a);                                                      \
    }
CUCA_ATTN_ROWS_SET(f32, float)
CUCA_ATTN_ROWS_SET(f16, _Float16)
