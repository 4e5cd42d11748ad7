// pick.hip -- the end of a decode step on gfx950: greedy argmax and top-k
// selection over logits rows, so that a step reads back one id, or k
// (logit, id) candidates, per row instead of the whole vocabulary.
//
// Replaces the host-side scans of the reference's sampler (sampler.rs):
//   greedy       (sampler.rs:44-56): the first maximum (strict >, so a NaN
//                never wins and all -inf / NaN rows give 0);
//   select_top_k (sampler.rs:254-286): after logit / temperature, the k best
//                finite logits in (logit desc by total order, id asc) order --
//                exactly those of a full sort (the reference's own test,
//                sampler.rs:578-596).  The host then runs the rest of
//                warp_candidates / sample on those k candidates.
//
// A decode step has one row per sequence, often a single one, so a row is
// split into slices that separate workgroups take (the host picks the
// slice count from the rows and the CU count), and a second launch combines
// the slices' results; a row taken whole by one workgroup (many rows) needs
// no second launch.
//
// argmax: a workgroup scans its slice, each thread a strided subsequence in
// increasing index order with the strict comparison (its first maximum);
// results combine as (larger value, or the smaller id on equal values), so
// any split gives the first maximum of the row.
//
// top-k: a finite logit l becomes the 64-bit composite (key << 32) | ~id,
// where the 32-bit key's unsigned order is f32::total_cmp's (sign bit set:
// ~bits, else bits | 2^31).  Composites are distinct, and the k largest are
// exactly the k best of (logit desc, id asc).  A workgroup holds up to
// PICK_CAP composites in LDS; a radix select, 8 bits a pass from the top,
// finds the k-th largest (stopping as soon as one bucket holds exactly the
// entries still needed) and keeps the composites at or above it.  A slice
// longer than the LDS is taken in rounds (the k kept ones plus the next
// values).  The slices' candidates are a superset of the row's k best; the
// combining workgroup selects among them the same way and writes the k in
// order, each thread placing one candidate at its rank.
#include "common.h"

#define PICK_THREADS 1024
#define PICK_CAP CUCA_PICK_CAP
#define PICK_PER ((PICK_CAP + PICK_THREADS - 1) / PICK_THREADS)
#define PICK_MAX_SLICES CUCA_PICK_MAX_SLICES
#define ARGMAX_UNROLL 8

typedef unsigned long long u64;

template <typename T> __device__ static inline float pick_load(const void *p, int64_t i) {
    return (float)reinterpret_cast<const T *>(p)[i];
}

// (value, id) pairs: the larger value wins, the smaller id on equal values;
// id 0xffffffff is "none" (every value NaN or -inf so far).
__device__ static inline void argmax_merge(float &best, uint32_t &bi, float ov, uint32_t oi) {
    if (ov > best || (ov == best && oi < bi)) { best = ov; bi = oi; }
}
__device__ static inline u64 argmax_pack(float v, uint32_t id) {
    return ((u64)__builtin_bit_cast(uint32_t, v) << 32) | id;
}

__device__ static inline void argmax_wave(float &best, uint32_t &bi) {
#pragma unroll
    for (int off = CUCA_WAVE / 2; off >= 1; off >>= 1) {
        const float ov = xor_partner(best, off);
        const uint32_t oi = xor_partner_bits(bi, off);
        argmax_merge(best, bi, ov, oi);
    }
}

// mode 0: the workgroup takes the whole row and writes the id; mode 1: it
// takes slice blockIdx % slices and writes its (value, id) to cand.
template <typename T> __device__ static inline void argmax_body(const PickArgs &a) {
    const int row = blockIdx.x / a.slices, s = blockIdx.x - row * a.slices;
    if (row >= a.rows) return;
    const void *lg = reinterpret_cast<const T *>(a.logits) + (int64_t)row * a.ld;
    const int lo = s * a.slice_len, hi = min(a.vocab, lo + a.slice_len);
    float best = -__builtin_inff();
    uint32_t bi = 0xffffffffu;
    for (int i0 = lo + (int)threadIdx.x; i0 < hi; i0 += ARGMAX_UNROLL * CUCA_BLOCK) {
        float v[ARGMAX_UNROLL];
#pragma unroll
        for (int u = 0; u < ARGMAX_UNROLL; u++) {
            const int i = i0 + u * CUCA_BLOCK;
            v[u] = i < hi ? pick_load<T>(lg, i) : -__builtin_inff();
        }
#pragma unroll
        for (int u = 0; u < ARGMAX_UNROLL; u++)
            if (v[u] > best) { best = v[u]; bi = (uint32_t)(i0 + u * CUCA_BLOCK); }
    }
    argmax_wave(best, bi);
    __shared__ float sv[CUCA_BLOCK / CUCA_WAVE];
    __shared__ uint32_t si[CUCA_BLOCK / CUCA_WAVE];
    const int wave = threadIdx.x / CUCA_WAVE;
    if ((threadIdx.x & (CUCA_WAVE - 1)) == 0) { sv[wave] = best; si[wave] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < CUCA_BLOCK / CUCA_WAVE; w++) argmax_merge(best, bi, sv[w], si[w]);
        if (a.mode == 0) a.out_ids[row] = bi == 0xffffffffu ? 0u : bi;
        else a.cand[(int64_t)row * a.slices + s] = argmax_pack(best, bi);
    }
}

// One wave per row over the row's slices, in any order (the merge is
// order-free), CUCA_BLOCK / 64 rows per workgroup.
__device__ static inline void argmax_merge_body(const PickArgs &a) {
    const int row = blockIdx.x * (CUCA_BLOCK / CUCA_WAVE) + (int)threadIdx.x / CUCA_WAVE;
    const int lane = threadIdx.x & (CUCA_WAVE - 1);
    if (row >= a.rows) return;
    float best = -__builtin_inff();
    uint32_t bi = 0xffffffffu;
    for (int s = lane; s < a.slices; s += CUCA_WAVE) {
        const u64 p = a.cand[(int64_t)row * a.slices + s];
        argmax_merge(best, bi, __builtin_bit_cast(float, (uint32_t)(p >> 32)), (uint32_t)p);
    }
    argmax_wave(best, bi);
    if (lane == 0) a.out_ids[row] = bi == 0xffffffffu ? 0u : bi;
}

// f32::total_cmp order as an unsigned key.
__device__ static inline uint32_t pick_key(float v) {
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ static inline float pick_unkey(uint32_t k) {
    return __builtin_bit_cast(float, (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

struct PickLds {
    u64 c[PICK_CAP];
    int hist[256];
    int wsum[4];
    int cnt[PICK_MAX_SLICES];
    int count;
    u64 prefix;
    int need, exact;
};

// Number of nonzero entries of c[0, n) (block-uniform result).
__device__ static inline int pick_nonzero(PickLds &L, const u64 (&e)[PICK_PER]) {
    if (threadIdx.x == 0) L.count = 0;
    __syncthreads();
    int n = 0;
#pragma unroll
    for (int i = 0; i < PICK_PER; i++) n += e[i] != 0ull;
#pragma unroll
    for (int off = CUCA_WAVE / 2; off >= 1; off >>= 1) n += (int)xor_partner_bits((uint32_t)n, off);
    if ((threadIdx.x & (CUCA_WAVE - 1)) == 0 && n) atomicAdd(&L.count, n);
    __syncthreads();
    const int r = L.count;
    __syncthreads();
    return r;
}

// Keep the kk = min(k, nonzero) largest composites of c[0, n), moved to
// c[0, kk) in any order; returns kk.
__device__ static inline int pick_select(PickLds &L, int n, int k) {
    const int tid = threadIdx.x;
    u64 e[PICK_PER];
#pragma unroll
    for (int i = 0; i < PICK_PER; i++) {
        const int j = tid + i * PICK_THREADS;
        e[i] = j < n ? L.c[j] : 0ull;
    }
    const int nnz = pick_nonzero(L, e);
    const int kk = nnz < k ? nnz : k;
    u64 thr = 1ull; // keep e >= thr (and nonzero)
    if (nnz > k) {
        u64 prefix = 0ull;
        int need = kk;
        for (int shift = 56; shift >= 0; shift -= 8) {
            if (tid < 256) L.hist[tid] = 0;
            __syncthreads();
#pragma unroll
            for (int i = 0; i < PICK_PER; i++) {
                const bool match = e[i] != 0ull && (shift == 56 || (e[i] >> (shift + 8)) == (prefix >> (shift + 8)));
                if (match) atomicAdd(&L.hist[(int)((e[i] >> shift) & 255ull)], 1);
            }
            __syncthreads();
            // buckets from the top (thread t holds bucket 255 - t): the one
            // where the running count reaches `need`
            const int lane = tid & (CUCA_WAVE - 1), w = tid / CUCA_WAVE;
            int v = 0, incl = 0;
            if (tid < 256) {
                v = L.hist[255 - tid];
                incl = v;
#pragma unroll
                for (int off = 1; off < CUCA_WAVE; off <<= 1) {
                    const int o = __shfl_up(incl, off, CUCA_WAVE);
                    if (lane >= off) incl += o;
                }
                if (lane == CUCA_WAVE - 1) L.wsum[w] = incl;
            }
            __syncthreads();
            if (tid < 256) {
                for (int q = 0; q < w; q++) incl += L.wsum[q];
                const int excl = incl - v;
                if (excl < need && need <= incl) {
                    L.prefix = prefix | ((u64)(255 - tid) << shift);
                    L.need = need - excl;
                    L.exact = v == need - excl;
                }
            }
            __syncthreads();
            // L.prefix / need / exact are written again only after the next
            // pass's barriers, and hist was last read above
            prefix = L.prefix;
            need = L.need;
            if (L.exact) break;
        }
        thr = prefix;
    }
    // compaction (order-free: composites are distinct)
    if (tid == 0) L.count = 0;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < PICK_PER; i++)
        if (e[i] != 0ull && e[i] >= thr) L.c[atomicAdd(&L.count, 1)] = e[i];
    __syncthreads();
    return kk;
}

// The composite of element i of a logits row.
template <typename T>
__device__ static inline u64 pick_composite(const void *lg, int i, float temperature) {
    const float l = pick_load<T>(lg, i) / temperature;
    if (!__builtin_isfinite(l)) return 0ull;
    return ((u64)pick_key(l) << 32) | (uint32_t)~(uint32_t)i;
}

// Final: c[0, kk) sorted best first into the row's outputs.
__device__ static inline void pick_write(PickLds &L, const PickArgs &a, int row, int kk) {
    for (int t = threadIdx.x; t < kk; t += PICK_THREADS) {
        const u64 mine = L.c[t];
        int rank = 0;
        for (int j = 0; j < kk; j++) rank += L.c[j] > mine;
        a.out_logits[(int64_t)row * a.k + rank] = pick_unkey((uint32_t)(mine >> 32));
        a.out_ids[(int64_t)row * a.k + rank] = ~(uint32_t)mine;
    }
    if (threadIdx.x == 0) a.out_count[row] = kk;
}

// SRC 0: the logits (mode 0 the whole row, final; mode 1 slice
// blockIdx % slices, candidates to cand / cand_count); SRC 1: the row's
// slices' candidates (final).
template <typename T, int SRC> __device__ static inline void topk_body(const PickArgs &a) {
    __shared__ PickLds L;
    const int S = SRC == 1 ? 1 : a.slices;
    const int row = blockIdx.x / S, s = blockIdx.x - row * S;
    if (row >= a.rows) return;
    const int tid = threadIdx.x;
    const void *lg = reinterpret_cast<const T *>(a.logits) + (int64_t)row * a.ld;
    int lo = 0, total = 0;
    const u64 *cand = nullptr;
    if (SRC == 0) {
        lo = s * a.slice_len;
        total = max(0, min(a.vocab, lo + a.slice_len) - lo);
    } else {
        for (int j = tid; j < a.slices; j += PICK_THREADS) L.cnt[j] = a.cand_count[(int64_t)row * a.slices + j];
        cand = a.cand + (int64_t)row * a.slices * a.k;
        total = a.slices * a.k; // slot (slice j, i) holds a candidate when i < cnt[j]
        __syncthreads();
    }
    int held = 0, pos = 0;
    for (;;) {
        const int take = min(PICK_CAP - held, total - pos);
        for (int j = tid; j < take; j += PICK_THREADS) {
            const int q = pos + j;
            u64 c;
            if (SRC == 0) {
                c = pick_composite<T>(lg, lo + q, a.temperature);
            } else {
                const int sl = q / a.k;
                c = q - sl * a.k < L.cnt[sl] ? cand[q] : 0ull;
            }
            L.c[held + j] = c;
        }
        pos += take;
        __syncthreads();
        held = pick_select(L, held + take, a.k);
        if (pos >= total) break;
    }
    if (SRC == 0 && a.mode == 1) {
        u64 *dst = a.cand + ((int64_t)row * a.slices + s) * a.k;
        for (int j = tid; j < held; j += PICK_THREADS) dst[j] = L.c[j];
        if (tid == 0) a.cand_count[(int64_t)row * a.slices + s] = held;
    } else {
        pick_write(L, a, row, held);
    }
}

extern "C" __global__ __launch_bounds__(CUCA_BLOCK) void cuca_argmax_f32(PickArgs a) { argmax_body<float>(a); }
extern "C" __global__ __launch_bounds__(CUCA_BLOCK) void cuca_argmax_f16(PickArgs a) { argmax_body<_Float16>(a); }
extern "C" __global__ __launch_bounds__(CUCA_BLOCK) void cuca_argmax_merge(PickArgs a) { argmax_merge_body(a); }
extern "C" __global__ __launch_bounds__(PICK_THREADS) void cuca_topk_f32(PickArgs a) { topk_body<float, 0>(a); }
extern "C" __global__ __launch_bounds__(PICK_THREADS) void cuca_topk_f16(PickArgs a) { topk_body<_Float16, 0>(a); }
extern "C" __global__ __launch_bounds__(PICK_THREADS) void cuca_topk_merge(PickArgs a) { topk_body<float, 1>(a); }

// The indexed LM head's weight rows (head_indexed, cpu.rs:2603-2606;
// QMatMul::forward_indexed, qmm.rs:1818-1843): workgroup j copies packed
// row ids[j] of the head into row j of a contiguous matrix, which the
// quantized matmul then runs as a row prefix -- the same kernel per row,
// so the same bits as the full head's column ids[j].  An id past the head
// is recorded and gives a zero row.
extern "C" __global__ __launch_bounds__(CUCA_BLOCK) void cuca_gather_rows(RowGatherArgs a) {
    const int j = blockIdx.x;
    const uint32_t id = a.ids[j];
    const bool ok = (int64_t)id < a.n_src;
    if (!ok && threadIdx.x == 0) record_bad(a.status + CUCA_STATUS_HEAD_ROW, (uint32_t)j, id);
    const u32x4 *src = reinterpret_cast<const u32x4 *>(a.src + (int64_t)(ok ? id : 0u) * a.row_bytes);
    u32x4 *dst = reinterpret_cast<u32x4 *>(a.dst + (int64_t)j * a.row_bytes);
    for (int64_t c = threadIdx.x; c < a.row_bytes / 16; c += CUCA_BLOCK)
        dst[c] = ok ? src[c] : u32x4{0u, 0u, 0u, 0u};
}
