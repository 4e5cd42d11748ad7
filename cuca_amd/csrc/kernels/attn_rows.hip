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
// Matrix-core kernel: a workgroup per (RT tiles of 16 query rows, KV head),
// one wave per (query head of the GQA group, row tile): G RT waves, with RT
// = 4 for groups of 1 and 2 and 8 / G above (8 waves a workgroup from
// groups of 2 on).  Per 16-position block of the table (the paged block),
// the workgroup stages the block's K rows and V rows in LDS once for all
// its waves -- double-buffered: the next block's loads are in flight while
// the current one computes -- and every wave computes the block's scores
// transposed, S^T = K Q^T (16 keys x 16 rows, MFMA), so that a lane holds
// four keys of ONE query row: the row's softmax statistics are per lane,
// reduced over four lanes, and S^T is already the P^T operand of O^T =
// V^T P^T (d x 16 rows, MFMA), whose lane holds four consecutive output
// columns of its row.  The exponentials are base 2, the scale folded with
// log2(e) into the scores.
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

template <typename T, int D, int G, int RT, int SBO = 0>
__device__ static inline void attn_rows_body(const AttnRowsArgs &a) {
    constexpr bool F16 = sizeof(T) == 2;
    constexpr int W = G * RT;                  // waves: (query head, row tile)
    constexpr int NT = 64 * W;                 // threads
    constexpr int NS = D / 16;                 // output column slices
    // K row stride in LDS (elements): rows 8 bytes (f16) or 16 bytes (f32)
    // past a multiple of 128, so the 16 rows of a score fragment, read 8
    // bytes a lane, start on 16 different bank pairs.  (At D + 16 the f16
    // rows started 8 banks apart and four rows shared each bank pair: 53 % of
    // the kernel's LDS cycles were bank conflicts, SQ_LDS_BANK_CONFLICT /
    // SQ_LDS_IDX_ACTIVE.)  Staged with 8-byte writes (f16 rows are 8-byte
    // aligned).
    constexpr int KST = D + 4;
    constexpr int VT = 20;                     // f16: V^T [D][16 keys + 4 padding]
    constexpr int VST = D + 4;                 // f32: V [16][D + 4]
    constexpr int KSZ = 16 * KST, VSZ = F16 ? D * VT : 16 * VST;
    // blocks of 16 positions per iteration: one.  Measured on MI355X,
    // config C's causal attention of 4096 f16 rows at the 128-register cap:
    // 1 block 702 us, 2 blocks 675 us but 13 registers spilled to scratch,
    // 4 blocks (57 spilled) 974 us; without the cap 2 blocks 850 us.
    constexpr int SB = SBO ? SBO : 1;
    constexpr int CH = 16 * D * (int)sizeof(T) / 16; // 16-byte chunks of a block's K (and of its V)
    constexpr int CPR = D * (int)sizeof(T) / 16;     // chunks per row
    constexpr int LPT = (2 * CH + NT - 1) / NT;      // chunks a thread loads per block
    __shared__ __align__(16) T ks[2][SB][KSZ];
    __shared__ __align__(16) T vs[2][SB][VSZ];
    __shared__ int span[2][RT];
    // The f16 kernels under the 128-register cap keep each wave's query rows
    // in LDS (read back per block, rows padded as K's), which frees the
    // registers of the loads two blocks ahead.
    constexpr bool QL = F16 && D <= 128 && G >= 2;
    constexpr int QST = D + 4;
    __shared__ __align__(16) T qs[QL ? W : 1][QL ? 16 * QST : 1];
    // a launch of another shape would leave row tiles' spans unwritten (they
    // bound the block loop and index the table): do nothing
    if (blockDim.x != NT) return;
    const int wave = threadIdx.x / 64, lane = threadIdx.x & 63;
    const int g = wave % G, rt = wave / G;
    const int r = lane & 15, grp = lane >> 4;
    const int wg_tile = blockIdx.x / a.n_kv, kvh = blockIdx.x - wg_tile * a.n_kv;
    const int row = (wg_tile * RT + rt) * 16 + r;
    const int head = kvh * G + g;
    const bool in_call = row < a.rows;
    int lo = 0, hi = 0;
    if (in_call) {
        lo = a.ranges[2 * row];
        hi = a.ranges[2 * row + 1];
    }
    const bool valid = in_call && lo >= 0 && hi > lo && (int64_t)hi <= (int64_t)a.max_blocks * 16;
    if (in_call && !valid && kvh == 0 && g == 0 && grp == 0)
        record_bad(a.status + CUCA_STATUS_KV_RANGE, (uint32_t)row, 0xffffffffu);
    // the workgroup's blocks: the union of its valid rows' ranges
    int tlo = valid ? lo : 0x7fffffff, thi = valid ? hi : 0;
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) {
        tlo = min(tlo, __shfl_xor(tlo, off));
        thi = max(thi, __shfl_xor(thi, off));
    }
    if (g == 0 && lane == 0) {
        span[0][rt] = tlo;
        span[1][rt] = thi;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < RT; i++) {
        tlo = min(tlo, span[0][i]);
        thi = max(thi, span[1][i]);
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
        if constexpr (QL) { // (read after the barrier that follows the first blocks' staging)
#pragma unroll
            for (int j = 0; j < QN; j++) *reinterpret_cast<attn_h4 *>(&qs[wave][r * QST + 16 * j + 4 * grp]) = qh[j];
        }
    }
    f32x4 acc[NS], acl[F16 ? NS : 1];
#pragma unroll
    for (int s = 0; s < NS; s++) {
        acc[s] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        if constexpr (F16) acl[s] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    // scores in the base-2 domain: x = q.k * scale * log2(e), weights
    // 2^(x - max) (v_exp_f32); the exponent's extra rounding is a relative
    // error of about |x| 2^-24 in a weight, far inside the bar
    const float scale2 = a.scale * 1.4426950408889634f;
    float m = -__builtin_huge_valf(), l = 0.0f;
    bool bad = false;
    const T *pk = reinterpret_cast<const T *>(a.pool_k);
    const T *pv = reinterpret_cast<const T *>(a.pool_v ? a.pool_v : a.pool_k);
    if (thi > 0) { // uniform over the workgroup
        const int b0 = tlo >> 4, b1 = (thi - 1) >> 4;
        // the table entries of the blocks, 64 at a time: lane i holds block
        // b0 + 64 c + i (entries past b1 repeat b1's: their keys are masked)
        uint32_t tabv = 0;
        auto load_tab = [&](int c) {
            const int bi = b0 + 64 * c + lane;
            tabv = a.table[bi <= b1 ? bi : b1];
        };
        auto blk_of = [&](int b) -> uint32_t { return (uint32_t)__builtin_amdgcn_readlane((int)tabv, (b - b0) & 63); };
        // a thread's chunks of a block: c < CH of K (16 bytes along a row),
        // the rest of V: f16, 4 keys x 2 columns (four dwords down the rows,
        // written to the transposed tile as two 8-byte pieces); f32, 16
        // bytes of a row, keys fastest.  Two register slots: the blocks are
        // loaded two iterations before they are computed (one before they
        // are staged into LDS).  With the loads one iteration ahead, every
        // iteration waited for a block's memory latency: config C's causal
        // attention of 4096 f16 rows spent about 5000 cycles an iteration,
        // its matrix cores and LDS each busy under a fifth of the time.
        // okb: the slot's blocks exist in the pool (taken when the block is
        // loaded, while the table window holds its entry).
        u32x4 pre[2][SB][LPT];
        bool okb[2][SB];
        auto fetch = [&](int bs, int slot) {
#pragma unroll
            for (int i = 0; i < SB; i++) {
                const uint32_t blk = blk_of(bs + i);
                okb[slot][i] = (int64_t)blk < a.n_blocks;
                const int64_t base = ((int64_t)((int64_t)blk < a.n_blocks ? blk : 0u) * a.n_kv + kvh) * 16 * D;
#pragma unroll
                for (int t = 0; t < LPT; t++) {
                    const int c = (int)threadIdx.x + t * NT;
                    if (2 * CH % NT == 0 || c < 2 * CH) {
                        if (c < CH) {
                            const int key = c / CPR, col = (c - key * CPR) * (16 / (int)sizeof(T));
                            pre[slot][i][t] = *reinterpret_cast<const u32x4 *>(pk + base + key * D + col);
                        } else if constexpr (F16) {
                            // 4 keys x 2 columns: the dwords of columns 2 dp, 2 dp + 1 of rows 4 kq .. + 3
                            const int u = c - CH, kq = u & 3, dp = u >> 2;
                            const uint32_t *vr = reinterpret_cast<const uint32_t *>(pv + base + 4 * kq * D + 2 * dp);
                            pre[slot][i][t] = u32x4{vr[0], vr[D / 2], vr[D], vr[3 * D / 2]};
                        } else {
                            const int key = (c - CH) & 15, col = ((c - CH) >> 4) * 4;
                            pre[slot][i][t] = *reinterpret_cast<const u32x4 *>(pv + base + key * D + col);
                        }
                    }
                }
            }
        };
        auto stage = [&](int buf, int slot) {
#pragma unroll
            for (int i = 0; i < SB; i++) {
#pragma unroll
                for (int t = 0; t < LPT; t++) {
                    const int c = (int)threadIdx.x + t * NT;
                    if (2 * CH % NT == 0 || c < 2 * CH) {
                        if (c < CH) {
                            const int key = c / CPR, col = (c - key * CPR) * (16 / (int)sizeof(T));
                            if constexpr (F16) {
                                uint2 *kd = reinterpret_cast<uint2 *>(&ks[buf][i][key * KST + col]);
                                kd[0] = uint2{pre[slot][i][t].x, pre[slot][i][t].y};
                                kd[1] = uint2{pre[slot][i][t].z, pre[slot][i][t].w};
                            } else {
                                *reinterpret_cast<u32x4 *>(&ks[buf][i][key * KST + col]) = pre[slot][i][t];
                            }
                        } else if constexpr (F16) {
                            // the low halves are column 2 dp of the 4 keys, the high halves 2 dp + 1
                            const int u = c - CH, kq = u & 3, dp = u >> 2;
                            const u32x4 w = pre[slot][i][t];
                            const uint2 lo2 = {(w.x & 0xffffu) | (w.y << 16), (w.z & 0xffffu) | (w.w << 16)};
                            const uint2 hi2 = {(w.x >> 16) | (w.y & 0xffff0000u), (w.z >> 16) | (w.w & 0xffff0000u)};
                            *reinterpret_cast<uint2 *>(&vs[buf][i][(2 * dp) * VT + 4 * kq]) = lo2;
                            *reinterpret_cast<uint2 *>(&vs[buf][i][(2 * dp + 1) * VT + 4 * kq]) = hi2;
                        } else {
                            const int key = (c - CH) & 15, col = ((c - CH) >> 4) * 4;
                            *reinterpret_cast<u32x4 *>(&vs[buf][i][key * VST + col]) = pre[slot][i][t];
                        }
                    }
                }
            }
        };
        // one iteration: blocks bs (register slot `slot`, LDS buffer `buf`)
        // computed, bs + SB staged from the other slot into the other
        // buffer, bs + 2 SB loaded into this slot (block k in slot k % 2,
        // buffer k % 2; the slot is free once its blocks are staged)
        auto iter = [&](int bs, int slot, int buf) {
            const bool more = bs + SB <= b1, more2 = bs + 2 * SB <= b1;
            bool okc[SB];
#pragma unroll
            for (int i = 0; i < SB; i++) okc[i] = okb[slot][i];
            if (more2 && ((bs + 2 * SB - b0) & 63) == 0) load_tab((bs + 2 * SB - b0) >> 6);
            if (more2) fetch(bs + 2 * SB, slot); // in flight during this and the next iteration
            // scores: lane (r, grp) gets keys 4 grp + i of each block with row r
            float x[SB][4];
            bool in[SB][4];
            float bmax = -__builtin_huge_valf();
#pragma unroll
            for (int sb = 0; sb < SB; sb++) {
                const int b = bs + sb;
                if (b <= b1 && !okc[sb] && valid && rows_meets(lo, hi, b)) {
                    bad = true;
                    if (kvh == 0 && g == 0 && grp == 0)
                        record_bad(a.status + CUCA_STATUS_KV_RANGE, (uint32_t)row, (uint32_t)max(16 * b, lo));
                }
                const T *kt = ks[buf][sb];
                f32x4 st = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                if constexpr (F16) {
#pragma unroll
                    for (int j = 0; j < NS; j++) {
                        const attn_h4 kk = *reinterpret_cast<const attn_h4 *>(kt + r * KST + 16 * j + 4 * grp);
                        const attn_h4 qq =
                            QL ? *reinterpret_cast<const attn_h4 *>(&qs[wave][r * QST + 16 * j + 4 * grp]) : qh[j];
                        st = __builtin_amdgcn_mfma_f32_16x16x16f16(kk, qq, st, 0, 0, 0);
                    }
                } else {
#pragma unroll
                    for (int j = 0; j < D / 4; j++)
                        st = __builtin_amdgcn_mfma_f32_16x16x4f32((float)kt[r * KST + 4 * j + grp], qf[j], st, 0, 0,
                                                                  0);
                }
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int p = 16 * b + 4 * grp + i;
                    in[sb][i] = valid && p >= lo && p < hi;
                    x[sb][i] = st[i] * scale2;
                    if (in[sb][i]) bmax = fmaxf(bmax, x[sb][i]);
                }
            }
            bmax = fmaxf(bmax, __shfl_xor(bmax, 16));
            bmax = fmaxf(bmax, __shfl_xor(bmax, 32));
            // Rescale what was accumulated under the old maximum only when the
            // block's maximum exceeds it by more than 8 (base 2): the weights
            // are then at most 2^8, which f16 holds with room (the hi part up
            // to 256, the lo part (p - hi) 2048 up to 256), and the f32 sums
            // too.  Rescaling at every new maximum ran most blocks' 64
            // accumulator multiplies; config C's causal attention of 4096
            // f16 rows 605 -> 551 us.
            if (bmax > m + 8.0f) {
                const float corr = __builtin_amdgcn_exp2f(m - bmax);
                l *= corr;
#pragma unroll
                for (int s = 0; s < NS; s++) {
                    acc[s] *= corr;
                    if constexpr (F16) acl[s] *= corr;
                }
                m = bmax;
            }
            float es = 0.0f;
#pragma unroll
            for (int sb = 0; sb < SB; sb++) {
                float e[4];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    e[i] = in[sb][i] ? __builtin_amdgcn_exp2f(x[sb][i] - m) : 0.0f;
                    es += e[i];
                }
                // O^T += V^T P^T
                const T *vt = vs[buf][sb];
                if constexpr (F16) {
                    attn_h4 ph, pl;
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        ph[i] = (_Float16)e[i];
                        pl[i] = (_Float16)((e[i] - (float)ph[i]) * 2048.0f);
                    }
#pragma unroll
                    for (int s = 0; s < NS; s++) {
                        const attn_h4 vv = *reinterpret_cast<const attn_h4 *>(vt + (16 * s + r) * VT + 4 * grp);
                        acc[s] = __builtin_amdgcn_mfma_f32_16x16x16f16(vv, ph, acc[s], 0, 0, 0);
                        acl[s] = __builtin_amdgcn_mfma_f32_16x16x16f16(vv, pl, acl[s], 0, 0, 0);
                    }
                } else {
#pragma unroll
                    for (int s = 0; s < NS; s++)
#pragma unroll
                        for (int j = 0; j < 4; j++)
                            acc[s] = __builtin_amdgcn_mfma_f32_16x16x4f32((float)vt[(4 * grp + j) * VST + 16 * s + r],
                                                                          e[j], acc[s], 0, 0, 0);
                }
            }
            es += __shfl_xor(es, 16);
            es += __shfl_xor(es, 32);
            l += es;
            if (more) stage(buf ^ 1, slot ^ 1);
            // the next blocks' tiles are in place, and every wave is done
            // with these before the blocks after overwrite them
            __syncthreads();
        };
        load_tab(0);
        fetch(b0, 0);
        if (b0 + SB <= b1) fetch(b0 + SB, 1); // (within the first table window: SB < 64)
        stage(0, 0);
        __syncthreads();
        for (int bs = b0; bs <= b1; bs += 2 * SB) {
            iter(bs, 0, 0);
            if (bs + SB <= b1) iter(bs + SB, 1, 1);
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

// Row tiles of 16 a workgroup: 4 at groups 1 and 2, 2 at 4, 1 at 8 (4 to 8
// waves, every wave a query head and a row tile, all sharing the block's
// K and V in LDS).
// f16 up to head_dim 128: at most 128 registers (four waves per SIMD, two
// workgroups of 8 waves per CU), which they fit without spilling.
#define CUCA_ATTN_ROWS(NAME, T, D, G)                                                      \
    extern "C" __global__ __launch_bounds__(64 * G * (G <= 2 ? 4 : 8 / G),                 \
                                            sizeof(T) == 2 && D <= 128 && G >= 2 ? 4 : 1)  \
        void NAME(AttnRowsArgs a) {                                                        \
        attn_rows_body<T, D, G, (G <= 2 ? 4 : 8 / G)>(a);                                  \
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
