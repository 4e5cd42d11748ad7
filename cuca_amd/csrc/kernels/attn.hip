// attn.hip -- paged decode attention on gfx950: one query row per sequence
// over its keys in the paged K/V pools, read in place.
//
// Replaces the GPU engine's decode kernel (paged_kernel.rs:92-282:
// paged_decode_kernel + paged_merge_kernel) and, for one query row, the
// CPU's attend_paged_rows (cpu/paged_attn.rs:105-290).  The pools are
// [n_blocks, n_kv, 16, d] (the layout cuca_hip_rope_store_kv writes); row
// r's key positions lo..hi (ranges[r]) map to block tables[r][p / 16], row
// p % 16.  Query head h reads KV head h / (n_head / n_kv).
//
// Split pass: a workgroup of 4 waves per (row, KV head, part of 4 CP key
// positions); wave w takes the part's CP positions w*CP.. (CP = 64 / LPP,
// LPP lanes per position: a K row slice of at most 256 bytes per lane, 128
// for a group of 8).  f16 groups of 4 at head_dim 64 / 128 take 8 waves of
// twice the lanes per position: the same part length.  Chunks start at the range's first block (positions
// before lo are masked), so a wave's positions are CP / 16 whole blocks and
// every value row is one of CP / 16 scalar block bases plus a constant
// offset.  The group's query heads (the GQA group) are staged once in LDS
// (f16 pairs, or f32).  Every lane issues all of its loads at once -- its
// slice of its position's K row and its d/64 value columns of all CP
// positions (about 64 VGPRs each) -- so a wave's 16-32 KiB are in flight
// together.  Scores: f16 dot2 (exact products) or f32 fma over the lane's
// columns, then across its LPP lanes, times `scale`; the wave's maximum and
// sum are wave reductions; the weights exp(s - max) go through LDS to every
// lane, which accumulates its value columns in position order (fma).  The 4
// waves' partials are combined in LDS, in wave order, into the part's
// (values, max, sum).  Part sizes depend on the dtype, head_dim and group
// only, so a row's result depends on its own range, never on the batch it
// is computed in.
//
// Measured on MI355X (f16, 32/8 heads of 128, 8192 keys per row): 60 % of
// 8 TB/s at 32-64 rows, against 72 % for a kernel that only issues the
// same loads (the block-scattered 4 KiB K/V pieces cap it below a
// streaming copy's 80 %).  16-byte value loads (4 rows per instruction)
// measured slower (53 % loads-only).
//
// When no row can have more than one part (max_parts == 1, short
// contexts), the split writes each head's output itself and there is no
// merge launch: the merge of one part multiplies by e^0 = 1 and divides by
// the part's own sum, so the bits are the same.
//
// Merge pass: one wave per (row, query head) combines the row's parts in
// part order -- the global maximum M, then sum_p acc_p e^(m_p - M) /
// sum_p sum_p e^(m_p - M), the reference's merge (paged_kernel.rs:
// 185-215) -- with the per-part weights computed lane-parallel and 16
// parts' loads in flight.
//
// HBM-bound: a row reads 2 (hi - lo) n_kv d s bytes of K and V; the
// arithmetic (2 G d flops per key byte pair) is VALU work far below it.

#include "common.h"

#pragma clang fp contract(off)

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// An f16 pair from a dword taken by value (a bit_cast straight from an
// ext-vector element compiled to a read of element 0).
__device__ static inline f16x2 as_h2(uint32_t u) { return __builtin_bit_cast(f16x2, u); }

__device__ static inline float wave_max(float v) {
#pragma unroll
    for (int off = CUCA_WAVE / 2; off >= 1; off >>= 1) v = fmaxf(v, xor_partner(v, off));
    return v;
}

// A bad row: an empty or inverted range, or one past the table.
__device__ static inline bool attn_range_ok(const AttnArgs &a, int lo, int hi) {
    return lo >= 0 && hi > lo && (int64_t)hi <= (int64_t)a.max_blocks * 16;
}

// Pool row index of position p of `row` (block table lookup), and whether
// the block exists.
__device__ static inline int64_t attn_pool_row(const AttnArgs &a, int row, int kvh, int p, bool &ok) {
    const uint32_t blk = a.tables[(int64_t)row * a.max_blocks + (p >> 4)];
    ok = (int64_t)blk < a.n_blocks;
    return ((int64_t)(ok ? blk : 0) * a.n_kv + kvh) * 16 + (p & 15);
}

// Lanes per key position for a d-wide row of T and a group of G query
// heads: a lane's K slice is at most 256 bytes (64 VGPRs), and at most 128
// for G = 8 (whose scores and weights need the registers).
template <typename T, int D, int G, int LPPO = 0> struct AttnShape {
    static constexpr int ROWB = D * (int)sizeof(T);
    static constexpr int LPP0 = ROWB > 256 ? ROWB / 256 : 1;
    static constexpr int LPP = LPPO ? LPPO : G >= 8 && LPP0 < 2 ? 2 : LPP0;
    static constexpr int CP = CUCA_WAVE / LPP; // positions per wave
    static constexpr int CPL = D / CUCA_WAVE;  // value columns per lane
};

__device__ static inline void pin_u(uint32_t &x) { asm volatile("" : "+v"(x)); }

template <typename T, int D, int G, int WPB = 4, int LPPO = 0>
__device__ static inline void attn_split_body(const AttnArgs &a) {
    using S = AttnShape<T, D, G, LPPO>;
    constexpr int BT = WPB * CUCA_WAVE;
    constexpr int VP = Chunk<T>::N;        // values per 16-byte chunk
    constexpr int LPP = S::LPP, CP = S::CP, CPL = S::CPL;
    constexpr int KCH = D / VP / LPP;      // 16-byte K chunks per lane
    constexpr int VW = CPL * (int)sizeof(T) <= 4 ? 1 : CPL * (int)sizeof(T) / 4; // dwords per value load
    // the group's query heads: f16 pairs (f16) or f32, as the pools, one
    // slice of SL dwords per (head, lane of a position).  With several lanes
    // per position the slices are padded by 16 bytes, so that the lanes of a
    // position read from different banks (unpadded, a 256-byte slice put
    // them on the same banks: 28 % of the f32 kernel's LDS cycles were bank
    // conflicts, SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE)
    constexpr int SL = D / LPP / (sizeof(T) == 2 ? 2 : 1);
    constexpr int SLP = LPP > 1 ? SL + 4 : SL;
    __shared__ __align__(16) uint32_t qs[G * LPP * SLP];
    __shared__ __align__(16) float wsh[WPB][CP][G];      // each wave's weights
    __shared__ __align__(16) float red[WPB][G][D + 2];   // each wave's partial
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / CUCA_WAVE);
    const int lane = threadIdx.x & (CUCA_WAVE - 1);
    const int rk = blockIdx.x / a.max_parts;
    const int part = blockIdx.x - rk * a.max_parts;
    const int row = rk / a.n_kv, kvh = rk - row * a.n_kv;
    // The query dwords are loaded into registers first and written to LDS
    // only after the K/V loads are issued: waiting for them before the
    // range, block-table and K/V loads put one more memory latency in front
    // of the part's bulk reads.
    constexpr int NW = G * D / (sizeof(T) == 2 ? 2 : 1);
    constexpr int NQ = (NW + BT - 1) / BT;
    uint32_t qv[NQ];
    {
        const uint32_t *qg = reinterpret_cast<const uint32_t *>(
            reinterpret_cast<const T *>(a.q) + (int64_t)row * a.q_ld + (int64_t)kvh * G * D);
#pragma unroll
        for (int k = 0; k < NQ; k++) {
            const int i = (int)threadIdx.x + k * BT;
            qv[k] = i < NW ? qg[i] : 0u;
        }
    }
    constexpr int NB = CP / 16;
    const uint32_t *tab = a.tables + (int64_t)row * a.max_blocks;
    // The table entries of the wave's blocks for a range that starts in the
    // first block (lo < 16, every decode row without a window), loaded
    // beside the range so that the K/V loads wait for one load, not two.
    const int s0 = (part * WPB + wave) * (CP / 16);
    uint32_t sblk[NB];
#pragma unroll
    for (int k = 0; k < NB; k++) sblk[k] = tab[min(s0 + k, a.max_blocks - 1)];
    const int lo = a.ranges[2 * row], hi = a.ranges[2 * row + 1];
    const bool valid = attn_range_ok(a, lo, hi);
    if (!valid && kvh == 0 && part == 0 && threadIdx.x == 0)
        record_bad(a.status + CUCA_STATUS_KV_RANGE, row, 0xffffffffu);
    // Chunks start at lo rounded down to a block, so a wave's CP positions
    // are CP / 16 whole blocks; positions before lo or from hi on are masked.
    const int lo_al = lo & ~15;
    if (valid && part * WPB * CP >= hi - lo_al) return; // a part past this row's range (whole workgroup)
    const int p0 = lo_al + (part * WPB + wave) * CP;   // wave-uniform, a block boundary
    const bool wave_live = valid && p0 < hi;
    const int pi = lane / LPP, sub = lane - pi * LPP;
    const int p = p0 + pi;
    const bool live = wave_live && p >= lo && p < hi;
    // the pool row of each block's first position (a missing block in the
    // range reads block 0 and is recorded; blocks past the range, whose
    // positions are all masked, read any existing block)
    const int last_b = (hi - 1) >> 4;
    int64_t brow[NB];
#pragma unroll
    for (int k = 0; k < NB; k++) {
        const int bk = (p0 >> 4) + k;
        const bool in = wave_live && bk <= last_b;
        const uint32_t blk = lo_al == 0 || !in ? sblk[k] : tab[bk]; // (bk == s0 + k when lo_al is 0)
        const bool ok = (int64_t)blk < a.n_blocks;
        if (!ok && in && lane == 0)
            record_bad(a.status + CUCA_STATUS_KV_RANGE, row, (uint32_t)max(bk * 16, lo));
        brow[k] = ((int64_t)(ok ? blk : 0) * a.n_kv + kvh) * 16;
    }

    // all loads: this lane's K slice, and its value columns of the CP positions
    int64_t kb = brow[0];
#pragma unroll
    for (int k = 1; k < NB; k++) kb = (pi >> 4) == k ? brow[k] : kb;
    u32x4 kraw[KCH];
    const T *krow = reinterpret_cast<const T *>(a.pool_k) + (kb + (pi & 15)) * D + sub * (D / LPP);
#pragma unroll
    for (int j = 0; j < KCH; j++) kraw[j] = Chunk<T>::load_raw(krow, j);
    uint32_t vraw[CP][VW];
#pragma unroll
    for (int j = 0; j < CP; j++) {
        // a block's scalar base plus a constant row offset
        const char *src = reinterpret_cast<const char *>(a.pool_v) +
                          ((brow[j >> 4] + (j & 15)) * D + lane * CPL) * (int64_t)sizeof(T);
        if constexpr (VW == 1 && CPL * sizeof(T) == 2) {
            vraw[j][0] = *reinterpret_cast<const uint16_t *>(src);
        } else if constexpr (VW == 1) {
            vraw[j][0] = *reinterpret_cast<const uint32_t *>(src);
        } else if constexpr (VW == 2) {
            const uint2 t = *reinterpret_cast<const uint2 *>(src);
            vraw[j][0] = t.x; vraw[j][1] = t.y;
        } else {
            const u32x4 t = *reinterpret_cast<const u32x4 *>(src);
            vraw[j][0] = t.x; vraw[j][1] = t.y; vraw[j][2] = t.z; vraw[j][3] = t.w;
        }
    }
    __builtin_amdgcn_sched_barrier(0); // every load above is issued first
#pragma unroll
    for (int k = 0; k < NQ; k++) {
        const int i = (int)threadIdx.x + k * BT;
        if (i < NW) qs[(i / SL) * SLP + i % SL] = qv[k];
    }
    __syncthreads();                   // qs is staged
#pragma unroll
    for (int j = 0; j < KCH; j++) pin(kraw[j]);

    // scores: this lane's columns in order (f16: dot2 of f16 pairs, exact
    // products; f32: fma), then across the LPP lanes
    // (head by head, with a scheduling barrier between heads: hoisting every
    // head's query reads at once would take more registers than the loads)
    float s[G];
#pragma unroll
    for (int g = 0; g < G; g++) {
        s[g] = 0.0f;
#pragma unroll
        for (int j = 0; j < KCH; j++) {
            if constexpr (sizeof(T) == 2) {
                const u32x4 qq = *reinterpret_cast<const u32x4 *>(qs + (g * LPP + sub) * SLP + j * (VP / 2));
                s[g] = __builtin_amdgcn_fdot2(as_h2(kraw[j].x),
                                              as_h2(qq.x), s[g], false);
                s[g] = __builtin_amdgcn_fdot2(as_h2(kraw[j].y),
                                              as_h2(qq.y), s[g], false);
                s[g] = __builtin_amdgcn_fdot2(as_h2(kraw[j].z),
                                              as_h2(qq.z), s[g], false);
                s[g] = __builtin_amdgcn_fdot2(as_h2(kraw[j].w),
                                              as_h2(qq.w), s[g], false);
            } else {
                const f32x4 qq = *reinterpret_cast<const f32x4 *>(
                    reinterpret_cast<const float *>(qs) + (g * LPP + sub) * SLP + j * VP);
                const f32x4 kk = __builtin_bit_cast(f32x4, kraw[j]);
                s[g] = fmaf(qq.x, kk.x, s[g]);
                s[g] = fmaf(qq.y, kk.y, s[g]);
                s[g] = fmaf(qq.z, kk.z, s[g]);
                s[g] = fmaf(qq.w, kk.w, s[g]);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int off = 1; off < LPP; off <<= 1) s[g] += xor_partner(s[g], off);

    // the wave's softmax pieces; the weights go to LDS for every lane
    float m[G], sum[G];
#pragma unroll
    for (int g = 0; g < G; g++) {
        const float sc = live ? s[g] * a.scale : -INFINITY;
        m[g] = wave_max(sc);
        const float w = live ? expf(sc - m[g]) : 0.0f;
        sum[g] = group_sum<CUCA_WAVE>(sub == 0 ? w : 0.0f);
        if (sub == 0) wsh[wave][pi][g] = w;
    }
    __syncthreads();
    // values: lane owns columns lane*CPL .. +CPL, positions in order
    float acc[G][CPL];
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int c = 0; c < CPL; c++) acc[g][c] = 0.0f;
#pragma unroll
    for (int j = 0; j < CP; j++) {
        // (8 positions at a time: hoisting every position's weight reads
        // would take more registers than the loads)
        if (j % 8 == 0) __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int c = 0; c < VW; c++) pin_u(vraw[j][c]);
        if (wave_live && p0 + j >= lo && p0 + j < hi) { // wave-uniform
            float v[CPL];
            if constexpr (sizeof(T) == 2) {
                if constexpr (CPL == 1) {
                    v[0] = (float)__builtin_bit_cast(_Float16, (uint16_t)vraw[j][0]);
                } else {
#pragma unroll
                    for (int c = 0; c < CPL / 2; c++) {
                        const f16x2 h = as_h2(vraw[j][c]);
                        v[2 * c] = (float)h.x; v[2 * c + 1] = (float)h.y;
                    }
                }
            } else {
#pragma unroll
                for (int c = 0; c < CPL; c++) v[c] = __builtin_bit_cast(float, vraw[j][c]);
            }
#pragma unroll
            for (int g = 0; g < G; g++) {
                const float wj = wsh[wave][j][g];
#pragma unroll
                for (int c = 0; c < CPL; c++) acc[g][c] = fmaf(wj, v[c], acc[g][c]);
            }
        }
    }
    // combine the WPB waves in LDS, in wave order
#pragma unroll
    for (int g = 0; g < G; g++) {
#pragma unroll
        for (int c = 0; c < CPL; c++) red[wave][g][lane * CPL + c] = acc[g][c];
        if (lane == 0) {
            red[wave][g][D] = wave_live ? m[g] : -INFINITY;
            red[wave][g][D + 1] = wave_live ? sum[g] : 0.0f;
        }
    }
    __syncthreads();
    if (!valid) {
        if (a.direct) { // the merge's zero rows for a bad range
            T *o = reinterpret_cast<T *>(a.out) + ((int64_t)row * a.n_head + kvh * G) * D;
            for (int e = threadIdx.x; e < G * D; e += BT) store1<T>(o, e, 0.0f);
        }
        return;
    }
    // wave w combines query heads w, w + WPB, ...
    for (int g = wave; g < G; g += WPB) {
        float top = red[0][g][D];
        for (int w2 = 1; w2 < WPB; w2++) top = fmaxf(top, red[w2][g][D]);
        float tot = 0.0f, f[WPB];
        for (int w2 = 0; w2 < WPB; w2++) {
            f[w2] = red[w2][g][D + 1] > 0.0f ? expf(red[w2][g][D] - top) : 0.0f;
            tot += red[w2][g][D + 1] * f[w2];
        }
        const int head = kvh * G + g;
        float *pp = a.part + (((int64_t)row * a.n_head + head) * a.max_parts + part) * (D + 2);
        T *o = reinterpret_cast<T *>(a.out) + ((int64_t)row * a.n_head + head) * D;
        for (int e = lane; e < D; e += CUCA_WAVE) {
            float v = 0.0f;
            for (int w2 = 0; w2 < WPB; w2++) v += red[w2][g][e] * f[w2];
            // one part: what the merge computes from it, acc e^0 / (sum e^0)
            if (a.direct) store1<T>(o, e, v / tot);
            else pp[e] = v;
        }
        if (lane == 0 && !a.direct) {
            pp[D] = top;
            pp[D + 1] = tot;
        }
    }
}

// Any head_dim and group size: one wave per (row, query head, chunk); lane
// = position, one wave reduction per value column.
template <typename T>
__device__ static inline void attn_split_generic_body(const AttnArgs &a) {
    const int wave = threadIdx.x / CUCA_WAVE, lane = threadIdx.x & (CUCA_WAVE - 1);
    const int64_t item = (int64_t)blockIdx.x * (CUCA_BLOCK / CUCA_WAVE) + wave;
    const int64_t per_row = (int64_t)a.n_head * a.max_parts;
    if (item >= (int64_t)a.rows * per_row) return;
    const int row = (int)(item / per_row);
    const int head = (int)((item - row * per_row) / a.max_parts);
    const int chunk = (int)(item - row * per_row - (int64_t)head * a.max_parts);
    const int G = a.n_head / a.n_kv, kvh = head / G, D = a.head_dim;
    const int lo = a.ranges[2 * row], hi = a.ranges[2 * row + 1];
    if (!attn_range_ok(a, lo, hi)) {
        if (head == 0 && chunk == 0 && lane == 0) record_bad(a.status + CUCA_STATUS_KV_RANGE, row, 0xffffffffu);
        return;
    }
    const int p0 = (lo & ~15) + chunk * CUCA_WAVE; // part_positions = 64, from lo's block
    if (p0 >= hi) return;
    const bool live = p0 + lane >= lo && p0 + lane < hi;
    const int p = live ? p0 + lane : max(p0, lo);
    bool ok;
    const int64_t prow = attn_pool_row(a, row, kvh, p, ok);
    if (!ok && live) record_bad(a.status + CUCA_STATUS_KV_RANGE, row, (uint32_t)p);
    const T *qh = reinterpret_cast<const T *>(a.q) + (int64_t)row * a.q_ld + (int64_t)head * D;
    float s = 0.0f;
    for (int e = 0; e < D; e++) s += (float)qh[e] * load1<T>(a.pool_k, prow * D + e);
    const float sc = live ? s * a.scale : -INFINITY;
    const float m = wave_max(sc);
    const float w = live ? expf(sc - m) : 0.0f;
    const float sum = group_sum<CUCA_WAVE>(w);
    float *pp = a.part + (((int64_t)row * a.n_head + head) * a.max_parts + chunk) * (D + 2);
    for (int e = 0; e < D; e++) {
        const float acc = group_sum<CUCA_WAVE>(live ? w * load1<T>(a.pool_v, prow * D + e) : 0.0f);
        if (lane == 0) pp[e] = acc;
    }
    if (lane == 0) {
        pp[D] = m;
        pp[D + 1] = sum;
    }
}

// Parts a merge holds in registers per lane (up to 256 parts per row: 32768
// f16 or 16384 f32 keys at head_dim 128); longer rows walk them in turn.
#define MERGE_PL 4

// Merge of one (row, query head) = job by one wave; lane owns columns lane,
// lane + 64, ... -- or, for two columns a lane (an even head_dim of
// 66..128), the adjacent columns 2 lane and 2 lane + 1, read with one
// 8-byte load: the
// preload of 32 parts is then 32 loads, not 64, and with the (max, sum)
// loads stays under the 63 loads a wave can have in flight (past that the
// wave waits for its first loads before it issues the rest: two memory
// round trips instead of one).  Each column still sums the parts in order.
template <int MAXC> __device__ static inline int merge_col(int lane, int k) {
    return MAXC == 2 ? 2 * lane + k : lane + k * CUCA_WAVE;
}
template <int MAXC>
__device__ static inline void merge_load(const float *pc, int D, int lane, float (&v)[MAXC]) {
    if constexpr (MAXC == 2) { // an even head_dim (the host's choice): 8-byte aligned part rows
        const int e = 2 * lane;
        const float2 t = e < D ? *reinterpret_cast<const float2 *>(pc + e) : make_float2(0.0f, 0.0f);
        v[0] = t.x;
        v[1] = t.y;
    } else {
#pragma unroll
        for (int k = 0; k < MAXC; k++) {
            const int e = lane + k * CUCA_WAVE;
            v[k] = e < D ? pc[e] : 0.0f;
        }
    }
}

// This lane's (max, sum) of parts lane, lane + 64, ... below lim and the
// values of parts 0 .. R-1 (the last part below lim repeated past it).
template <int MAXC, int R>
__device__ static inline void attn_merge_preload(const float *pp, int64_t stride, int D, int lim, int lane,
                                                 float (&mv)[MERGE_PL], float (&sv)[MERGE_PL],
                                                 float (&v0)[R > 0 ? R : 1][MAXC]) {
#pragma unroll
    for (int q = 0; q < MERGE_PL; q++) {
        const int c = lane + q * CUCA_WAVE;
        mv[q] = c < lim ? pp[(int64_t)c * stride + D] : -INFINITY;
        sv[q] = c < lim ? pp[(int64_t)c * stride + D + 1] : 0.0f;
    }
#pragma unroll
    for (int jj = 0; jj < R; jj++) merge_load<MAXC>(pp + (int64_t)min(jj, lim - 1) * stride, D, lane, v0[jj]);
}

template <typename T, int MAXC>
__device__ static inline void attn_merge_job(const AttnArgs &a, int64_t job, int lane) {
    const int row = (int)(job / a.n_head);
    const int D = a.head_dim;
    const int64_t stride = D + 2;
    const float *pp = a.part + job * a.max_parts * stride;
    // Every load of the short path is issued at once: this lane's (max, sum)
    // of parts lane, lane + 64, ... and the values of the first R parts, so
    // the merge waits for one round of loads (walking the parts' maxima, sums
    // and values in turn made four).  When a row can have no more parts than
    // that path takes (max_parts <= MERGE_PL * 64), they are loaded before the
    // row's range, up to max_parts: the range and the parts then arrive in
    // the same round.  Those loads stay inside the workspace, which holds
    // max_parts parts per (row, head), and a part past the row's count is
    // loaded but never used.  The arithmetic and its order are those of the
    // loop below.
    constexpr int R = MAXC <= 2 ? 32 : MAXC == 4 ? 16 : 0; // whole blocks of 16 parts
    float mv[MERGE_PL], sv[MERGE_PL];
    float v0[R > 0 ? R : 1][MAXC];
    const bool early = a.max_parts <= MERGE_PL * CUCA_WAVE; // uniform
    if (early) attn_merge_preload<MAXC, R>(pp, stride, D, a.max_parts, lane, mv, sv, v0);
    const int lo = a.ranges[2 * row], hi = a.ranges[2 * row + 1];
    T *o = reinterpret_cast<T *>(a.out) + job * D;
    if (!attn_range_ok(a, lo, hi)) {
        for (int e = lane; e < D; e += CUCA_WAVE) store1<T>(o, e, 0.0f);
        return;
    }
    const int np = (hi - (lo & ~15) + a.part_positions - 1) / a.part_positions;
    float acc[MAXC]; // columns per lane: head_dim <= 64 MAXC
#pragma unroll
    for (int k = 0; k < MAXC; k++) acc[k] = 0.0f;
    float total;
    if (np <= MERGE_PL * CUCA_WAVE) {
        if (!early) attn_merge_preload<MAXC, R>(pp, stride, D, np, lane, mv, sv, v0);
        float mx = -INFINITY;
#pragma unroll
        for (int q = 0; q < MERGE_PL; q++)
            if (lane + q * CUCA_WAVE < np) mx = fmaxf(mx, mv[q]);
        const float top = wave_max(mx);
        float t = 0.0f;
#pragma unroll
        for (int q = 0; q < MERGE_PL; q++)
            if (lane + q * CUCA_WAVE < np) t += sv[q] * expf(mv[q] - top);
        total = group_sum<CUCA_WAVE>(t);
#pragma unroll
        for (int q = 0; q < MERGE_PL; q++) {
            const int c0 = q * CUCA_WAVE;
            if (c0 >= np) break;
            const float wl = c0 + lane < np ? expf(mv[q] - top) : 0.0f;
            const int nc = min(CUCA_WAVE, np - c0);
#pragma unroll
            for (int j0 = 0; j0 < CUCA_WAVE; j0 += 16) {
                if (j0 >= nc) break;
                float v[16][MAXC];
#pragma unroll
                for (int jj = 0; jj < 16; jj++) {
                    if (q == 0 && j0 + 16 <= R) {
#pragma unroll
                        for (int k = 0; k < MAXC; k++) v[jj][k] = v0[R > 0 ? (j0 + jj) % R : 0][k];
                    } else {
                        merge_load<MAXC>(pp + (int64_t)(c0 + min(j0 + jj, nc - 1)) * stride, D, lane, v[jj]);
                    }
                }
#pragma unroll
                for (int jj = 0; jj < 16; jj++) {
                    if (j0 + jj < nc) {
                        const float wj = __builtin_bit_cast(
                            float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wl), j0 + jj));
#pragma unroll
                        for (int k = 0; k < MAXC; k++) acc[k] += v[jj][k] * wj;
                    }
                }
            }
        }
    } else {
        // the global maximum, then each lane's parts' weighted sums (in order)
        float mx = -INFINITY;
        for (int c = lane; c < np; c += CUCA_WAVE) mx = fmaxf(mx, pp[c * stride + D]);
        const float top = wave_max(mx);
        float t = 0.0f;
        for (int c = lane; c < np; c += CUCA_WAVE) t += pp[c * stride + D + 1] * expf(pp[c * stride + D] - top);
        total = group_sum<CUCA_WAVE>(t);
        for (int c0 = 0; c0 < np; c0 += CUCA_WAVE) {
            // lane l holds the weight of part c0 + l
            const int cl = c0 + lane;
            const float wl = cl < np ? expf(pp[cl * stride + D] - top) : 0.0f;
            const int nc = min(CUCA_WAVE, np - c0);
            for (int j0 = 0; j0 < nc; j0 += 16) {
                float v[16][MAXC];
#pragma unroll
                for (int jj = 0; jj < 16; jj++)
                    merge_load<MAXC>(pp + (int64_t)(c0 + min(j0 + jj, nc - 1)) * stride, D, lane, v[jj]);
#pragma unroll
                for (int jj = 0; jj < 16; jj++) {
                    if (j0 + jj < nc) {
                        const float wj = __builtin_bit_cast(
                            float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wl), j0 + jj));
#pragma unroll
                        for (int k = 0; k < MAXC; k++) acc[k] += v[jj][k] * wj;
                    }
                }
            }
        }
    }
#pragma unroll
    for (int k = 0; k < MAXC; k++) {
        const int e = merge_col<MAXC>(lane, k);
        if (e < D) store1<T>(o, e, acc[k] / total);
    }
}

// Merge pass: one wave per (row, query head).
template <typename T, int MAXC>
__device__ static inline void attn_merge_body(const AttnArgs &a) {
    const int wave = threadIdx.x / CUCA_WAVE, lane = threadIdx.x & (CUCA_WAVE - 1);
    const int64_t job = (int64_t)blockIdx.x * (CUCA_BLOCK / CUCA_WAVE) + wave;
    if (job >= (int64_t)a.rows * a.n_head) return;
    attn_merge_job<T, MAXC>(a, job, lane);
}

#define CUCA_ATTN(NAME, BODY, ...)                                                         \
    extern "C" __global__ __launch_bounds__(CUCA_BLOCK) void NAME(AttnArgs a) {            \
        BODY<__VA_ARGS__>(a);                                                              \
    }
// f16 group-4 splits at head_dim 64 and 128 run as 8 waves of half the
// positions each (twice the lanes per position), so a part covers the same
// positions as the 4-wave form and a SIMD holds two waves.  Measured on
// MI355X (32/8 heads of 128): 1 row x 8192 f16 keys 19.4 -> 16.5 us; 32-64
// rows x 8192 f16 keys 1.5-2.5 % slower.  For f32 pools the 8-wave form was
// faster at one row (4096 keys 16.4 -> 15.0 us) but slower in the 8B decode
// step at 32 rows x 1024 keys (attention 58.3 -> 62.2 us per layer), so f32
// keeps 4 waves.  The form depends on (dtype, head_dim, group) only, never
// on the batch, so a row's bits do not either.
#define CUCA_ATTN_W8(NAME, ...)                                                            \
    extern "C" __global__ __launch_bounds__(8 * CUCA_WAVE) void NAME(AttnArgs a) {         \
        attn_split_body<__VA_ARGS__>(a);                                                   \
    }
#define CUCA_ATTN_D(TN, T, D)                                                              \
    CUCA_ATTN(cuca_attn_split_##TN##_d##D##_g1, attn_split_body, T, D, 1)                  \
    CUCA_ATTN(cuca_attn_split_##TN##_d##D##_g2, attn_split_body, T, D, 2)
#define CUCA_ATTN_G4_f32                                                                   \
    CUCA_ATTN(cuca_attn_split_f32_d64_g4, attn_split_body, float, 64, 4)                   \
    CUCA_ATTN(cuca_attn_split_f32_d128_g4, attn_split_body, float, 128, 4)
#define CUCA_ATTN_G4_f16                                                                   \
    CUCA_ATTN_W8(cuca_attn_split_f16_d64_g4, _Float16, 64, 4, 8, 2 * AttnShape<_Float16, 64, 4>::LPP) \
    CUCA_ATTN_W8(cuca_attn_split_f16_d128_g4, _Float16, 128, 4, 8, 2 * AttnShape<_Float16, 128, 4>::LPP)
#define CUCA_ATTN_SET(TN, T)                                                               \
    CUCA_ATTN_D(TN, T, 64)                                                                 \
    CUCA_ATTN_D(TN, T, 128)                                                                \
    CUCA_ATTN_D(TN, T, 256)                                                                \
    CUCA_ATTN_G4_##TN                                                                      \
    CUCA_ATTN(cuca_attn_split_##TN##_d256_g4, attn_split_body, T, 256, 4)                  \
    CUCA_ATTN(cuca_attn_split_##TN##_d64_g8, attn_split_body, T, 64, 8)                    \
    CUCA_ATTN(cuca_attn_split_##TN##_d128_g8, attn_split_body, T, 128, 8)                  \
    CUCA_ATTN(cuca_attn_split_##TN##_generic, attn_split_generic_body, T)                  \
    CUCA_ATTN(cuca_attn_merge_##TN##_c1, attn_merge_body, T, 1)                           \
    CUCA_ATTN(cuca_attn_merge_##TN##_c2, attn_merge_body, T, 2)                           \
    CUCA_ATTN(cuca_attn_merge_##TN##_c4, attn_merge_body, T, 4)                           \
    CUCA_ATTN(cuca_attn_merge_##TN##_c8, attn_merge_body, T, 8)

CUCA_ATTN_SET(f32, float)
CUCA_ATTN_SET(f16, _Float16)
