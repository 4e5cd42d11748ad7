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
// argmax: one workgroup per row; each thread scans a strided subsequence
// with the strict comparison (its first maximum), and the workgroup keeps the
// larger value, the smaller id on ties.
//
// top-k: one workgroup of 1024 threads per row.  A finite logit l becomes
// the 32-bit key whose unsigned order is f32::total_cmp's (sign bit set:
// ~bits, else bits | 2^31).  Four 8-bit radix passes (LDS histograms) find
// the k-th largest key K; every key > K is kept, and the lowest ids with key
// == K fill the rest (thread t scans a contiguous range, so a block scan of
// the per-thread counts keeps id order).  The k candidates are sorted in
// LDS by a bitonic sort of (key, ~id) and written best first.
#include "common.h"

#define PICK_THREADS 1024
#define PICK_MAX_K 1024

template <typename T> __device__ static inline float pick_load(const void *p, int64_t i) {
    return (float)reinterpret_cast<const T *>(p)[i];
}

template <typename T> __device__ static inline void argmax_body(const PickArgs &a) {
    const int row = blockIdx.x;
    if (row >= a.rows) return;
    const void *lg = reinterpret_cast<const T *>(a.logits) + (int64_t)row * a.ld;
    float best = -__builtin_inff();
    uint32_t bi = 0xffffffffu;
    for (int i = threadIdx.x; i < a.vocab; i += CUCA_BLOCK) {
        const float v = pick_load<T>(lg, i);
        if (v > best) { best = v; bi = (uint32_t)i; }
    }
    // larger value; equal values: the smaller id (the earlier first maximum)
#pragma unroll
    for (int off = CUCA_WAVE / 2; off >= 1; off >>= 1) {
        const float ov = __shfl_xor(best, off, CUCA_WAVE);
        const uint32_t oi = (uint32_t)__shfl_xor((int)bi, off, CUCA_WAVE);
        if (ov > best || (ov == best && oi < bi)) { best = ov; bi = oi; }
    }
    __shared__ float sv[CUCA_BLOCK / CUCA_WAVE];
    __shared__ uint32_t si[CUCA_BLOCK / CUCA_WAVE];
    const int wave = threadIdx.x / CUCA_WAVE;
    if ((threadIdx.x & (CUCA_WAVE - 1)) == 0) { sv[wave] = best; si[wave] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < CUCA_BLOCK / CUCA_WAVE; w++)
            if (sv[w] > best || (sv[w] == best && si[w] < bi)) { best = sv[w]; bi = si[w]; }
        a.out_ids[row] = bi == 0xffffffffu ? 0u : bi;
    }
}

// f32::total_cmp order as an unsigned key.
__device__ static inline uint32_t pick_key(float v) {
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ static inline float pick_unkey(uint32_t k) {
    return __builtin_bit_cast(float, (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// Exclusive block-wide prefix sum of v (PICK_THREADS threads); *total gets
// the sum.  `red` holds PICK_THREADS / 64 ints.
__device__ static inline int pick_scan(int v, int *red, int *total) {
    const int lane = threadIdx.x & (CUCA_WAVE - 1), wave = threadIdx.x / CUCA_WAVE;
    int incl = v;
#pragma unroll
    for (int off = 1; off < CUCA_WAVE; off <<= 1) {
        const int o = __shfl_up(incl, off, CUCA_WAVE);
        if (lane >= off) incl += o;
    }
    __syncthreads();
    if (lane == CUCA_WAVE - 1) red[wave] = incl;
    __syncthreads();
    int before = 0, all = 0;
    for (int w = 0; w < PICK_THREADS / CUCA_WAVE; w++) {
        if (w < wave) before += red[w];
        all += red[w];
    }
    *total = all;
    return before + incl - v;
}

template <typename T> __device__ static inline void topk_body(const PickArgs &a) {
    const int row = blockIdx.x;
    if (row >= a.rows) return;
    const void *lg = reinterpret_cast<const T *>(a.logits) + (int64_t)row * a.ld;
    const int tid = threadIdx.x;
    __shared__ int hist[256];
    __shared__ int red[PICK_THREADS / CUCA_WAVE];
    __shared__ uint32_t sh_prefix;
    __shared__ int sh_need;
    __shared__ unsigned long long cand[PICK_MAX_K];
    // contiguous range of this thread (id order for the compaction)
    const int per = (a.vocab + PICK_THREADS - 1) / PICK_THREADS;
    const int lo = tid * per, hi = min(a.vocab, lo + per);
    // the logit of element i as sample() sees it: l / temperature, finite only
    auto key_at = [&](int i, bool *ok) -> uint32_t {
        const float l = pick_load<T>(lg, i) / a.temperature;
        *ok = __builtin_isfinite(l);
        return pick_key(l);
    };
    // 1. radix select the k-th largest finite key, 8 bits at a time
    uint32_t prefix = 0, mask = 0;
    int need = a.k; // rank of the wanted key among those matching the prefix
    int n_finite_total = 0;
    for (int pass = 0; pass < 4; pass++) {
        const int shift = 24 - 8 * pass;
        for (int b = tid; b < 256; b += PICK_THREADS) hist[b] = 0;
        __syncthreads();
        int n_finite = 0;
        for (int i = lo; i < hi; i++) {
            bool ok;
            const uint32_t key = key_at(i, &ok);
            if (!ok) continue;
            n_finite++;
            if ((key & mask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1);
        }
        if (pass == 0) {
            int tot;
            (void)pick_scan(n_finite, red, &tot);
            n_finite_total = tot;
        }
        __syncthreads();
        if (tid == 0) {
            int kk = need < n_finite_total ? need : n_finite_total;
            if (kk <= 0) kk = 1;
            int d = 255, acc = 0;
            for (; d > 0; d--) {
                if (acc + hist[d] >= kk) break;
                acc += hist[d];
            }
            sh_prefix = prefix | ((uint32_t)d << shift);
            sh_need = kk - acc;
        }
        __syncthreads();
        prefix = sh_prefix;
        need = sh_need;
        mask |= 255u << shift;
    }
    const int kk = a.k < n_finite_total ? a.k : n_finite_total;
    if (kk <= 0) {
        if (tid == 0) a.out_count[row] = 0;
        return;
    }
    // prefix is the k-th largest key K; `need` keys equal to K are kept
    // 2. compaction: keys > K anywhere, then the first `need` keys == K in id order
    int n_gt = 0, n_eq = 0;
    for (int i = lo; i < hi; i++) {
        bool ok;
        const uint32_t key = key_at(i, &ok);
        if (!ok) continue;
        n_gt += key > prefix;
        n_eq += key == prefix;
    }
    int tot_gt, tot_eq;
    const int at_gt = pick_scan(n_gt, red, &tot_gt);
    const int at_eq = pick_scan(n_eq, red, &tot_eq);
    int wgt = at_gt, weq = tot_gt + at_eq;
    for (int i = lo; i < hi; i++) {
        bool ok;
        const uint32_t key = key_at(i, &ok);
        if (!ok) continue;
        const unsigned long long c = ((unsigned long long)key << 32) | (0xffffffffu - (uint32_t)i);
        if (key > prefix) {
            if (wgt < PICK_MAX_K) cand[wgt] = c;
            wgt++;
        } else if (key == prefix) {
            if (weq < tot_gt + need && weq < PICK_MAX_K) cand[weq] = c;
            weq++;
        }
    }
    // pad to a power of two for the bitonic sort
    int n = 1;
    while (n < kk) n <<= 1;
    for (int i = kk + tid; i < n; i += PICK_THREADS) cand[i] = 0ull;
    __syncthreads();
    // 3. bitonic sort, descending
    for (int size = 2; size <= n; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = tid; i < n; i += PICK_THREADS) {
                const int j = i ^ stride;
                if (j > i) {
                    const bool desc = (i & size) == 0;
                    const unsigned long long x = cand[i], y = cand[j];
                    if ((x < y) == desc) { cand[i] = y; cand[j] = x; }
                }
            }
            __syncthreads();
        }
    }
    for (int i = tid; i < kk; i += PICK_THREADS) {
        const unsigned long long c = cand[i];
        a.out_logits[(int64_t)row * a.k + i] = pick_unkey((uint32_t)(c >> 32));
        a.out_ids[(int64_t)row * a.k + i] = 0xffffffffu - (uint32_t)c;
    }
    if (tid == 0) a.out_count[row] = kk;
}

extern "C" __global__ __launch_bounds__(CUCA_BLOCK) void cuca_argmax_f32(PickArgs a) { argmax_body<float>(a); }
extern "C" __global__ __launch_bounds__(CUCA_BLOCK) void cuca_argmax_f16(PickArgs a) { argmax_body<_Float16>(a); }
extern "C" __global__ __launch_bounds__(PICK_THREADS) void cuca_topk_f32(PickArgs a) { topk_body<float>(a); }
extern "C" __global__ __launch_bounds__(PICK_THREADS) void cuca_topk_f16(PickArgs a) { topk_body<_Float16>(a); }
