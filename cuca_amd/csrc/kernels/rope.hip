// rope.hip -- rotary embedding on Q and K in place, with the optional fused
// per-head QK-norm, on gfx950; and the same fused with the paged K/V store.
//
// Replaces apply_rope / rotate_calls (cpu.rs:2996-3026, 3672-3688; candle's
// rope and rope_i) and the GPU rope (gpu.rs:5922-5964: narrow / cat / mul,
// several launches and copies), plus the QK-norm in front of it
// (cpu.rs:2840-2864, 3040-3055).  One launch covers the Q and the K heads
// of every row, in the projection's own [rows, heads, head_dim] layout
// (row stride q_ld / k_ld, so Q and K may sit inside a fused QKV buffer).
//
// Vector kernel: a head is handled by TPH lanes, each owning whole 16-byte
// chunks (VP = 4 f32 or 8 f16 values; the layouts are described at
// rope_body).  The cos/sin row of the position (n_dims / 2 f32) is shared by
// all heads of the row and stays in cache.  The QK-norm sum is a butterfly
// over the head's TPH lanes.
//
// a' = a*c - b*s, b' = a*s + b*c with separately rounded products
// (-ffp-contract=off, and the pragma below): without the norm the result is
// bit-identical to the reference's f32 rotation, in f16 too (exact widening,
// one rounding).
//
// The _kv kernels replace store_kv (cpu.rs:3028-3097) and KvPool::write
// (gpu.rs:1786-1806): K is normalised, rotated and written straight into
// the layer's paged pool, V (optionally RMS-normalised without a weight,
// gpu.rs:5277) copied into its pool, so K makes one trip through HBM
// instead of two.  The pools are [n_blocks, n_kv_head, 16, head_dim]
// (paged_attn.rs:1-38); row r goes to pool row slots[r] = block * 16 +
// position % 16, which the host derives from the sequence's block table.
//
// Generic kernel (any head_dim / n_dims / alignment): one wave per head.

#include "common.h"

#pragma clang fp contract(off)

// `n` consecutive f32 of a table (n = 2, 4 or 8; 8-byte aligned for 2,
// 16-byte aligned otherwise).
// Empty asm on loaded registers: the loads must complete before this point
// and cannot be sunk past it (emits no instruction, only a wait).
template <int n>
__device__ static inline void pin(float (&v)[n]) {
#pragma unroll
    for (int i = 0; i < n; i++) asm volatile("" : "+v"(v[i]));
}

__device__ static inline void pin(u32x4 &r) { asm volatile("" : "+v"(r)); }

// Head-chunk load policies of rope_body.
//   LP_DEV:    device-scope buffer loads (`buffer_load_dwordx4 ... sc1`);
//   LP_NT:     nontemporal global loads;
//   LP_CACHED: plain global loads (rows whose offsets do not fit 32 bits).
// RoPE rewrites its rows in place.  A plain or nontemporal load leaves the
// line in this XCD's L2, the store then hits it and leaves it dirty there,
// to be written back later (by an eviction or the end-of-kernel release)
// instead of streaming out.  A device-scope load does not leave it there.
// Measured on MI355X, in-place 1:1 streams with streaming stores, cold:
//   40 MiB  15.0 us (plain 17.2, nontemporal 20.6);
//   160 MiB 49.8 us (plain 59.7, nontemporal 72.2);
// and in the config C prefill step (4096 tokens) RoPE 15.8 -> 14.9 us,
// the fused K/V-store RoPE 19.4 -> 17.9 us.
#define LP_CACHED 0
#define LP_NT 1
#define LP_DEV 2

// A buffer resource of 2^32 bytes at `base` (wave-uniform), raw dwords.
__device__ static inline __amdgpu_buffer_rsrc_t rsrc_4g(const void *base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, -1, 0x00020000);
}

// The 16-byte chunk at byte offset `off` of `r`, loaded at device scope
// (aux 16 = sc1).
__device__ static inline u32x4 load_dev16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 16);
}

template <int n>
__device__ static inline void load_tab(const float *t, int64_t first, float (&v)[n]) {
    if constexpr (n == 2) {
        const float2 x = *reinterpret_cast<const float2 *>(t + first);
        v[0] = x.x; v[1] = x.y;
    } else {
        const f32x4 *p = reinterpret_cast<const f32x4 *>(t + first);
#pragma unroll
        for (int j = 0; j < n / 4; j++) {
            f32x4 x = p[j];
            v[4 * j] = x.x; v[4 * j + 1] = x.y; v[4 * j + 2] = x.z; v[4 * j + 3] = x.w;
        }
    }
}

// Lane layout (TPH lanes per head, VP values per 16-byte chunk):
//   NEOX: TPH = head_dim / (2 VP); lane u owns chunk u of the first half and
//         its partner chunk u + n/(2 VP) (values i and i + n/2), or two
//         pass-through chunks past n_dims -- both of a wave's load
//         instructions cover contiguous bytes;
//   NORM: TPH = head_dim / VP; lane u owns chunk u, i.e. VP/2 whole (2i,
//         2i+1) pairs (or a pass-through chunk) -- one contiguous chunk per
//         lane.  (Two adjacent chunks per lane measured 74 % of peak at 16384
//         f16 rows against 80 % for this layout: each load instruction then
//         touched every other chunk.)
// A row's heads, in launch order: nq Q heads, nk K heads, then (STORE) nk
// V heads.  Without STORE every head is rotated in place.  With STORE the K
// heads are rotated and the V heads (optionally RMS-normalised without a
// weight) copied into the paged pools, at pool row slots[row] of their KV
// head; Q stays in place.
// LP: the load policy of the head chunks (LP_DEV, LP_NT, LP_CACHED above).
// LP_DEV addresses a row's chunks by 32-bit byte offsets from q, k and v:
// the host checks that rows * row stride fits.
// WHOLE (the _h2w kernels; the host launches them for in-place RoPE whose
// rotated dims cover the head, with QK-norm only when both projections have
// norm weights, at a power-of-two head_dim, two heads a lane): every lane
// rotates and every head is normalised with weights, so the per-value
// selects of pass-through lanes and weightless heads drop out; the mean is
// the sum times 1 / head_dim (exact for a power of two: the same bits as
// the division); and the two heads' norm factors are computed once per lane
// pair (below).  (In config E's prefill step, 8192 tokens of QK-norm NEOX
// f16, the waves wait on memory 42 % of their resident time against 67 %
// for config C's RoPE: instruction issue holds them.  The whole-head form
// takes about 10 % of the per-lane instructions off and ran 2 % faster.)
template <typename T, int KIND, bool NORM, bool STORE, int LP, int HPL = 1, bool WHOLE = false>
__device__ static inline void rope_body(const RopeArgs &a) {
    static_assert(!WHOLE || (HPL == 2 && !STORE), "whole-head kernels: two heads a lane, in place");
    constexpr int VP = Chunk<T>::N;
    constexpr int NC = KIND == 2 ? 2 : 1;       // chunks per lane
    constexpr int NT = KIND == 2 ? VP : VP / 2; // cos/sin entries per lane
    const int tl = a.tph_log2;
    const int tph = 1 << tl;
    const uint32_t gh = blockIdx.x * (uint32_t)(CUCA_BLOCK >> tl) + (threadIdx.x >> tl);
    const int u = threadIdx.x & (tph - 1);
    const int nqk = a.nq + a.nk;
    // a lane takes HPL consecutive heads of one projection (the host checks
    // that HPL divides nq and nk): gh counts groups of them
    const uint32_t heads = (uint32_t)(nqk + (STORE ? a.nv : 0));
    const uint32_t groups = heads / HPL;
    const bool live = gh < (uint32_t)a.rows * groups;
    const uint32_t row = live ? gh / groups : 0;
    const int h = live ? (int)(gh - row * groups) * HPL : 0;
    const int hk = h < a.nq ? 0 : (h < nqk ? 1 : 2); // Q, K or V head
    const int D = a.head_dim;
    const T *src = hk == 0 ? reinterpret_cast<const T *>(a.q) + (int64_t)row * a.q_ld + (int64_t)h * D
                 : hk == 1 ? reinterpret_cast<const T *>(a.k) + (int64_t)row * a.k_ld + (int64_t)(h - a.nq) * D
                           : reinterpret_cast<const T *>(a.v) + (int64_t)row * a.v_ld + (int64_t)(h - nqk) * D;
    const float *nw = hk == 0 ? a.q_norm_w : (hk == 1 ? a.k_norm_w : nullptr);
    const bool scale_h = hk == 2 ? a.v_norm != 0 : nw != nullptr; // this head is normalised
    const int half = a.n_dims >> 1;

    // This lane's chunks: element offsets e[0] (and e[1] for NEOX).
    int e[NC];
    bool rot;
    if (KIND == 2) {
        const int nr = half / VP;
        if (u < nr) {
            e[0] = u * VP; e[NC - 1] = e[0] + half; rot = true;
        } else {
            e[0] = a.n_dims + (u - nr) * 2 * VP; e[NC - 1] = e[0] + VP; rot = false;
        }
    } else {
        e[0] = u * VP; rot = e[0] < a.n_dims;
    }
    rot = WHOLE || (rot && hk != 2);
    // Every load is issued up front and unconditionally, from addresses that
    // are always valid (a lane past the last head reads row 0, a position
    // outside the table or a pass-through lane reads table entry 0, a head
    // without norm weights reads the other projection's), and pinned there
    // by an empty asm on the loaded registers: the position (and slot), the
    // head's chunks, the cos/sin entries and the norm weights are all in
    // flight together.  Left to itself the compiler sinks the table loads
    // into the predicated store's branch, behind a wait for the chunks
    // (56-63 us against 53.5 us per 16384 f16 rows of 40 heads).
    const int32_t pos = a.pos[row];
    const int32_t slot = STORE ? a.slots[row] : 0;
    u32x4 raw[HPL][NC];
    if constexpr (LP == LP_DEV) {
        // the byte offset of the head in its projection; one load per
        // projection, so each resource stays wave-uniform
        const uint32_t ho = (uint32_t)(hk == 0 ? (int64_t)row * a.q_ld + (int64_t)h * D
                                      : hk == 1 ? (int64_t)row * a.k_ld + (int64_t)(h - a.nq) * D
                                                : (int64_t)row * a.v_ld + (int64_t)(h - nqk) * D) *
                            (uint32_t)sizeof(T);
#pragma unroll
        for (int j = 0; j < HPL; j++)
#pragma unroll
            for (int k = 0; k < NC; k++) {
                const uint32_t off = ho + (uint32_t)((j * D + e[k]) * (int)sizeof(T));
                if (hk == 0) raw[j][k] = load_dev16(rsrc_4g(a.q), off);
                else if (hk == 1) raw[j][k] = load_dev16(rsrc_4g(a.k), off);
                else raw[j][k] = load_dev16(rsrc_4g(a.v), off);
            }
    } else {
#pragma unroll
        for (int j = 0; j < HPL; j++)
#pragma unroll
            for (int k = 0; k < NC; k++)
                raw[j][k] = LP == LP_NT
                                ? __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(src + j * D) + e[k] / VP)
                                : Chunk<T>::load_raw(src + j * D, e[k] / VP);
    }
    const bool pos_ok = pos >= 0 && (int64_t)pos < a.table_rows;
    const bool slot_ok = !STORE || (slot >= 0 && (int64_t)slot < a.n_slots);
    const int64_t t0 = (rot && pos_ok) ? (int64_t)pos * half + (KIND == 2 ? e[0] : (e[0] >> 1)) : 0;
    float c[NT], s[NT];
    load_tab<NT>(a.cos_t, t0, c);
    load_tab<NT>(a.sin_t, t0, s);
    float w[NC][VP];
    // a uniform condition: are there norm weights at all?
    const float *any_w = a.q_norm_w ? a.q_norm_w : a.k_norm_w;
    if (NORM && any_w) {
        const float *wp = nw ? nw : any_w;
#pragma unroll
        for (int k = 0; k < NC; k++) load_tab<VP>(wp, e[k], w[k]);
    }
    __builtin_amdgcn_sched_barrier(0); // every load above is issued first
    pin(c);
    pin(s);
#pragma unroll
    for (int j = 0; j < HPL; j++)
#pragma unroll
        for (int k = 0; k < NC; k++) pin(raw[j][k]);
    // WHOLE with QK-norm: both heads' sums of squares first.  The butterfly's
    // first step (xor tph/2) is taken transposed -- the lower half of a
    // head's lanes keeps head 0's partial sums and the upper half head 1's,
    // each lane adding its partner's partial of the head it keeps -- and the
    // rest of the butterfly runs within each half, so every lane ends with
    // exactly the sum the per-head butterfly gives (the same additions in
    // the same order), of one head; each lane computes that head's factor,
    // and takes the other head's from its partner.  (tph >= 2: a head_dim of
    // at least 32 f16 or 16 f32 values; the host launches WHOLE only then.)
    float winv[WHOLE && NORM ? HPL : 1];
    if constexpr (WHOLE && NORM) {
        float ssh[HPL];
#pragma unroll
        for (int j = 0; j < HPL; j++) {
            float v[NC][VP];
#pragma unroll
            for (int k = 0; k < NC; k++) Chunk<T>::widen(raw[j][k], v[k]);
            float ss = 0.0f;
#pragma unroll
            for (int k = 0; k < NC; k++)
#pragma unroll
                for (int i = 0; i < VP; i++) ss += v[k][i] * v[k][i];
            ssh[j] = ss;
        }
        const int hb = tph >> 1;
        const bool upper = (u & hb) != 0;
        float t = (upper ? ssh[1] : ssh[0]) + xor_partner(upper ? ssh[0] : ssh[1], hb);
        t = group_sum_rt(t, hb);
        // (a power-of-two head_dim: the mean times 2^-log2(D) is the division's value)
        const float rd = __builtin_amdgcn_ldexpf(1.0f, -(tl + (KIND == 2 ? 1 : 0) + (VP == 8 ? 3 : 2)));
        const float mine = 1.0f / sqrtf(t * rd + a.eps);
        const float other = xor_partner(mine, hb);
        winv[0] = upper ? other : mine;
        winv[1] = upper ? mine : other;
        // widened again below, head by head: keeping both heads' widened
        // values from the sums took 83 registers (5 waves per SIMD)
#pragma unroll
        for (int j = 0; j < HPL; j++)
#pragma unroll
            for (int k = 0; k < NC; k++) pin(raw[j][k]);
    }
#pragma unroll
    for (int j = 0; j < HPL; j++) {
    float v[NC][VP];
#pragma unroll
    for (int k = 0; k < NC; k++) Chunk<T>::widen(raw[j][k], v[k]);
    if (NORM) {
        if (any_w && j == 0) {
#pragma unroll
            for (int k = 0; k < NC; k++) pin(w[k]);
        }
        float inv;
        if constexpr (WHOLE) {
            inv = winv[j];
        } else {
            float ss = 0.0f;
#pragma unroll
            for (int k = 0; k < NC; k++)
#pragma unroll
                for (int i = 0; i < VP; i++) ss += v[k][i] * v[k][i];
            ss = group_sum_rt(ss, tph);
            // the norm kernel's reciprocal form, x * (1 / sqrt(mean + eps)) * w;
            // a weightless norm multiplies by 1 (exact)
            inv = 1.0f / sqrtf(ss / (float)D + a.eps);
        }
#pragma unroll
        for (int k = 0; k < NC; k++)
#pragma unroll
            for (int i = 0; i < VP; i++) {
                if constexpr (WHOLE) {
                    v[k][i] = v[k][i] * inv * w[k][i];
                } else {
                    const float wi = nw ? w[k][i] : 1.0f;
                    v[k][i] = scale_h ? v[k][i] * inv * wi : v[k][i];
                }
            }
    }
    // The rotation is computed on every lane and selected.
    if (KIND == 2) {
#pragma unroll
        for (int i = 0; i < VP; i++) {
            const float x0 = v[0][i], x1 = v[NC - 1][i];
            const float r0 = x0 * c[i] - x1 * s[i];
            const float r1 = x0 * s[i] + x1 * c[i];
            v[0][i] = WHOLE || rot ? r0 : x0;
            v[NC - 1][i] = WHOLE || rot ? r1 : x1;
        }
    } else {
#pragma unroll
        for (int j = 0; j < VP / 2; j++) {
            const float x0 = v[0][2 * j], x1 = v[0][2 * j + 1];
            const float r0 = x0 * c[j] - x1 * s[j];
            const float r1 = x0 * s[j] + x1 * c[j];
            v[0][2 * j] = WHOLE || rot ? r0 : x0;
            v[0][2 * j + 1] = WHOLE || rot ? r1 : x1;
        }
    }
    T *dst;
    if (STORE && hk != 0) {
        // pool [n_blocks, nk, 16, d]: block slot / 16, KV head, row slot % 16
        const int kvh = (hk == 1 ? h - a.nq : h - nqk) + j;
        const int64_t prow = ((int64_t)(slot >> 4) * a.nk + kvh) * 16 + (slot & 15);
        dst = reinterpret_cast<T *>(hk == 1 ? a.pool_k : a.pool_v) + prow * D;
    } else {
        dst = const_cast<T *>(src) + j * D;
    }
    if (live && pos_ok && slot_ok && (rot || scale_h || (STORE && hk != 0))) {
#pragma unroll
        for (int k = 0; k < NC; k++) Chunk<T>::store_nt(dst, e[k] / VP, v[k]);
    }
    }
    if (live && u == 0 && h == 0) {
        if (!pos_ok) record_bad(a.status + CUCA_STATUS_ROPE_POS, row, (uint32_t)pos);
        if (!slot_ok) record_bad(a.status + CUCA_STATUS_KV_SLOT, row, (uint32_t)slot);
    }
}

// Full-width QK-norm (the qk_norm_full archs, OLMo 2: cpu.rs:2838-2843 for
// Q, 3042-3045 for K; GPU gpu.rs:5233-5236): the norm runs over a row's
// whole Q (and K) projection, weights [nq * head_dim] / [nk * head_dim],
// before the heads are split and rotated.  One workgroup per row, its
// threads taking the row's (head, lane) slots of the layout above, thread t
// the slots t, t + blockDim, ... (RF_SLOTS at most).  blockDim is a power of
// two of at least 64, so a head's TPH slots sit on consecutive lanes of one
// wave (V's per-head norm stays a butterfly), and the Q and K sums are one
// block reduction each, in a fixed order.  The chunks stay in registers
// between the two passes; the tables and weights are read in the second.
#define RF_SLOTS 4
template <typename T, int KIND, bool STORE>
__device__ static inline void rope_full_body(const RopeArgs &a) {
    constexpr int VP = Chunk<T>::N;
    constexpr int NC = KIND == 2 ? 2 : 1;       // chunks per lane
    constexpr int NT = KIND == 2 ? VP : VP / 2; // cos/sin entries per lane
    __shared__ float red[2][CUCA_WAVE];
    const int tl = a.tph_log2;
    const int tph = 1 << tl;
    const uint32_t row = blockIdx.x;
    const int nqk = a.nq + a.nk;
    const int total = (nqk + (STORE ? a.nv : 0)) << tl;
    const int D = a.head_dim, half = a.n_dims >> 1;
    const int32_t pos = a.pos[row];
    const int32_t slot = STORE ? a.slots[row] : 0;
    const bool pos_ok = pos >= 0 && (int64_t)pos < a.table_rows;
    const bool slot_ok = !STORE || (slot >= 0 && (int64_t)slot < a.n_slots);
    if (!pos_ok || !slot_ok) { // uniform: the row is left untouched
        if (threadIdx.x == 0) {
            if (!pos_ok) record_bad(a.status + CUCA_STATUS_ROPE_POS, row, (uint32_t)pos);
            if (!slot_ok) record_bad(a.status + CUCA_STATUS_KV_SLOT, row, (uint32_t)slot);
        }
        return;
    }
    // this thread's slots: head h, lane u, kind hk (0 Q, 1 K, 2 V), chunks e
    auto head_src = [&](int h, int hk) -> const T * {
        return hk == 0 ? reinterpret_cast<const T *>(a.q) + (int64_t)row * a.q_ld + (int64_t)h * D
             : hk == 1 ? reinterpret_cast<const T *>(a.k) + (int64_t)row * a.k_ld + (int64_t)(h - a.nq) * D
                       : reinterpret_cast<const T *>(a.v) + (int64_t)row * a.v_ld + (int64_t)(h - nqk) * D;
    };
    auto lane_chunks = [&](int u, int (&e)[NC]) -> bool { // returns: rotated
        if (KIND == 2) {
            const int nr = half / VP;
            if (u < nr) { e[0] = u * VP; e[NC - 1] = e[0] + half; return true; }
            e[0] = a.n_dims + (u - nr) * 2 * VP; e[NC - 1] = e[0] + VP; return false;
        }
        e[0] = u * VP;
        return e[0] < a.n_dims;
    };
    u32x4 raw[RF_SLOTS][NC];
    float vss[RF_SLOTS]; // V: the head's sum of squares
    float ssq = 0.0f, ssk = 0.0f;
#pragma unroll
    for (int j = 0; j < RF_SLOTS; j++) {
        const int sl = (int)threadIdx.x + j * (int)blockDim.x;
        const bool live = sl < total;
        const int h = live ? sl >> tl : 0, u = sl & (tph - 1);
        const int hk = h < a.nq ? 0 : (h < nqk ? 1 : 2);
        int e[NC];
        (void)lane_chunks(u, e);
        const T *src = head_src(h, hk);
#pragma unroll
        for (int k = 0; k < NC; k++) raw[j][k] = Chunk<T>::load_raw(src, e[k] / VP);
        float part = 0.0f;
#pragma unroll
        for (int k = 0; k < NC; k++) {
            float v[VP];
            Chunk<T>::widen(raw[j][k], v);
#pragma unroll
            for (int i = 0; i < VP; i++) part += v[i] * v[i];
        }
        if (live && hk == 0) ssq += part;
        if (live && hk == 1) ssk += part;
        vss[j] = group_sum_rt(live && hk == 2 ? part : 0.0f, tph);
    }
    // the Q and K sums: a wave butterfly, then the waves in order
    ssq = group_sum<CUCA_WAVE>(ssq);
    ssk = group_sum<CUCA_WAVE>(ssk);
    const int wave = threadIdx.x / CUCA_WAVE, nw = blockDim.x / CUCA_WAVE;
    if ((threadIdx.x & (CUCA_WAVE - 1)) == 0) {
        red[0][wave] = ssq;
        red[1][wave] = ssk;
    }
    __syncthreads();
    float sq = 0.0f, sk = 0.0f;
    for (int i = 0; i < nw; i++) {
        sq += red[0][i];
        sk += red[1][i];
    }
    // the norm kernel's reciprocal form, x * (1 / sqrt(mean + eps)) * w
    const float invq = 1.0f / sqrtf(sq / (float)(a.nq * D) + a.eps);
    const float invk = 1.0f / sqrtf(sk / (float)(a.nk > 0 ? a.nk * D : 1) + a.eps);
#pragma unroll
    for (int j = 0; j < RF_SLOTS; j++) {
        const int sl = (int)threadIdx.x + j * (int)blockDim.x;
        if (sl >= total) continue;
        const int h = sl >> tl, u = sl & (tph - 1);
        const int hk = h < a.nq ? 0 : (h < nqk ? 1 : 2);
        int e[NC];
        const bool rot = lane_chunks(u, e) && hk != 2;
        const float *nw = hk == 0 ? a.q_norm_w : (hk == 1 ? a.k_norm_w : nullptr);
        const int64_t wbase = hk == 0 ? (int64_t)h * D : (int64_t)(h - a.nq) * D;
        const bool scale_h = hk == 2 ? a.v_norm != 0 : nw != nullptr;
        const float inv = hk == 0 ? invq : hk == 1 ? invk : 1.0f / sqrtf(vss[j] / (float)D + a.eps);
        float v[NC][VP];
#pragma unroll
        for (int k = 0; k < NC; k++) {
            Chunk<T>::widen(raw[j][k], v[k]);
            float w[VP];
            if (nw) load_tab<VP>(nw, wbase + e[k], w);
#pragma unroll
            for (int i = 0; i < VP; i++) v[k][i] = scale_h ? v[k][i] * inv * (nw ? w[i] : 1.0f) : v[k][i];
        }
        if (rot) {
            float c[NT], s[NT];
            const int64_t t0 = (int64_t)pos * half + (KIND == 2 ? e[0] : (e[0] >> 1));
            load_tab<NT>(a.cos_t, t0, c);
            load_tab<NT>(a.sin_t, t0, s);
            if (KIND == 2) {
#pragma unroll
                for (int i = 0; i < VP; i++) {
                    const float x0 = v[0][i], x1 = v[NC - 1][i];
                    v[0][i] = x0 * c[i] - x1 * s[i];
                    v[NC - 1][i] = x0 * s[i] + x1 * c[i];
                }
            } else {
#pragma unroll
                for (int i = 0; i < VP / 2; i++) {
                    const float x0 = v[0][2 * i], x1 = v[0][2 * i + 1];
                    v[0][2 * i] = x0 * c[i] - x1 * s[i];
                    v[0][2 * i + 1] = x0 * s[i] + x1 * c[i];
                }
            }
        }
        T *dst;
        if (STORE && hk != 0) {
            const int kvh = hk == 1 ? h - a.nq : h - nqk;
            const int64_t prow = ((int64_t)(slot >> 4) * a.nk + kvh) * 16 + (slot & 15);
            dst = reinterpret_cast<T *>(hk == 1 ? a.pool_k : a.pool_v) + prow * D;
        } else {
            dst = const_cast<T *>(head_src(h, hk));
        }
        if (rot || scale_h || (STORE && hk != 0)) {
#pragma unroll
            for (int k = 0; k < NC; k++) Chunk<T>::store_nt(dst, e[k] / VP, v[k]);
        }
    }
}

template <typename T>
__device__ static inline void rope_generic_body(const RopeArgs &a) {
    const int lane = threadIdx.x & (CUCA_WAVE - 1);
    const uint32_t gh = blockIdx.x * (uint32_t)(CUCA_BLOCK / CUCA_WAVE) + threadIdx.x / CUCA_WAVE;
    const int nqk = a.nq + a.nk;
    const uint32_t heads = (uint32_t)(nqk + a.nv);
    if (gh >= (uint32_t)a.rows * heads) return; // whole wave
    const uint32_t row = gh / heads;
    const int h = (int)(gh - row * heads);
    const int32_t pos = a.pos[row];
    const int32_t slot = a.slots ? a.slots[row] : 0;
    const bool pos_ok = pos >= 0 && (int64_t)pos < a.table_rows;
    const bool slot_ok = !a.slots || (slot >= 0 && (int64_t)slot < a.n_slots);
    if (!pos_ok || !slot_ok) {
        if (lane == 0 && h == 0) {
            if (!pos_ok) record_bad(a.status + CUCA_STATUS_ROPE_POS, row, (uint32_t)pos);
            if (!slot_ok) record_bad(a.status + CUCA_STATUS_KV_SLOT, row, (uint32_t)slot);
        }
        return;
    }
    const int hk = h < a.nq ? 0 : (h < nqk ? 1 : 2); // Q, K or V head
    const int D = a.head_dim;
    const T *src = hk == 0 ? reinterpret_cast<const T *>(a.q) + (int64_t)row * a.q_ld + (int64_t)h * D
                 : hk == 1 ? reinterpret_cast<const T *>(a.k) + (int64_t)row * a.k_ld + (int64_t)(h - a.nq) * D
                           : reinterpret_cast<const T *>(a.v) + (int64_t)row * a.v_ld + (int64_t)(h - nqk) * D;
    T *dst = const_cast<T *>(src);
    if (a.slots && hk != 0) {
        const int kvh = hk == 1 ? h - a.nq : h - nqk;
        const int64_t prow = ((int64_t)(slot >> 4) * a.nk + kvh) * 16 + (slot & 15);
        dst = reinterpret_cast<T *>(hk == 1 ? a.pool_k : a.pool_v) + prow * D;
    }
    const float *nw = hk == 0 ? a.q_norm_w : (hk == 1 ? a.k_norm_w : nullptr);
    const bool scale_h = hk == 2 ? a.v_norm != 0 : nw != nullptr;
    float inv = 1.0f;
    if (scale_h) {
        float ss = 0.0f;
        for (int e = lane; e < D; e += CUCA_WAVE) {
            const float v = load1<T>(src, e);
            ss += v * v;
        }
        ss = group_sum<CUCA_WAVE>(ss);
        inv = 1.0f / sqrtf(ss / (float)D + a.eps);
    }
    auto scaled = [&](int e) {
        const float x = load1<T>(src, e);
        return scale_h ? x * inv * (nw ? nw[e] : 1.0f) : x;
    };
    const int half = a.n_dims >> 1;
    const int rot_end = hk == 2 ? 0 : half; // V heads are not rotated
    const float *cs = a.cos_t + (int64_t)pos * half;
    const float *sn = a.sin_t + (int64_t)pos * half;
    // every lane reads its elements before any lane of the wave writes
    // (the norm pass above read all of them); pairs are disjoint per lane
    for (int i = lane; i < rot_end; i += CUCA_WAVE) {
        const int ea = a.kind == 2 ? i : 2 * i;
        const int eb = a.kind == 2 ? i + half : 2 * i + 1;
        const float x0 = scaled(ea), x1 = scaled(eb);
        store1<T>(dst, ea, x0 * cs[i] - x1 * sn[i]);
        store1<T>(dst, eb, x0 * sn[i] + x1 * cs[i]);
    }
    // pass-through values (past n_dims; a V head's whole row)
    if (scale_h || dst != src) {
        for (int e = (hk == 2 ? 0 : a.n_dims) + lane; e < D; e += CUCA_WAVE) store1<T>(dst, e, scaled(e));
    }
}

#define CUCA_ROPE(NAME, T, KIND, NORM, STORE)                                              \
    extern "C" __global__ __launch_bounds__(CUCA_BLOCK) void NAME(RopeArgs a) {            \
        rope_body<T, KIND, NORM, STORE, LP_DEV>(a);                                        \
    }                                                                                      \
    extern "C" __global__ __launch_bounds__(CUCA_BLOCK) void NAME##_h2(RopeArgs a) {       \
        rope_body<T, KIND, NORM, STORE, LP_DEV, 2>(a);                                     \
    }                                                                                      \
    extern "C" __global__ __launch_bounds__(CUCA_BLOCK) void NAME##_g(RopeArgs a) {        \
        rope_body<T, KIND, NORM, STORE, LP_CACHED>(a);                                     \
    }
// in-place RoPE of whole heads, two a lane (rope_body's WHOLE)
#define CUCA_ROPE_W(NAME, T, KIND, NORM, LP)                                               \
    extern "C" __global__ __launch_bounds__(CUCA_BLOCK) void NAME##_h2w(RopeArgs a) {      \
        rope_body<T, KIND, NORM, false, LP, 2, true>(a);                                   \
    }
// full-width QK-norm: a workgroup of up to 1024 threads per row
#define CUCA_ROPE_FULL(NAME, T, KIND, STORE)                                               \
    extern "C" __global__ __launch_bounds__(1024) void NAME(RopeArgs a) {                  \
        rope_full_body<T, KIND, STORE>(a);                                                 \
    }
// streaming variants of the QK-norm kernels (see the runtime's rope launch)
#define CUCA_ROPE_NT(NAME, T, KIND, STORE)                                                 \
    extern "C" __global__ __launch_bounds__(CUCA_BLOCK) void NAME(RopeArgs a) {            \
        rope_body<T, KIND, true, STORE, LP_NT>(a);                                         \
    }                                                                                      \
    extern "C" __global__ __launch_bounds__(CUCA_BLOCK) void NAME##_h2(RopeArgs a) {       \
        rope_body<T, KIND, true, STORE, LP_NT, 2>(a);                                      \
    }
#define CUCA_ROPE_SET(TN, T)                                                               \
    CUCA_ROPE(cuca_rope_##TN##_norm, T, 0, false, false)                                   \
    CUCA_ROPE(cuca_rope_##TN##_neox, T, 2, false, false)                                   \
    CUCA_ROPE(cuca_rope_##TN##_norm_qkn, T, 0, true, false)                                \
    CUCA_ROPE(cuca_rope_##TN##_neox_qkn, T, 2, true, false)                                \
    CUCA_ROPE(cuca_rope_##TN##_norm_kv, T, 0, false, true)                                 \
    CUCA_ROPE(cuca_rope_##TN##_neox_kv, T, 2, false, true)                                 \
    CUCA_ROPE(cuca_rope_##TN##_norm_qkn_kv, T, 0, true, true)                              \
    CUCA_ROPE(cuca_rope_##TN##_neox_qkn_kv, T, 2, true, true)                              \
    CUCA_ROPE_NT(cuca_rope_##TN##_norm_qkn_nt, T, 0, false)                                \
    CUCA_ROPE_NT(cuca_rope_##TN##_neox_qkn_nt, T, 2, false)                                \
    CUCA_ROPE_NT(cuca_rope_##TN##_norm_qkn_kv_nt, T, 0, true)                              \
    CUCA_ROPE_NT(cuca_rope_##TN##_neox_qkn_kv_nt, T, 2, true)                              \
    CUCA_ROPE_W(cuca_rope_##TN##_norm, T, 0, false, LP_DEV)                                \
    CUCA_ROPE_W(cuca_rope_##TN##_neox, T, 2, false, LP_DEV)                                \
    CUCA_ROPE_W(cuca_rope_##TN##_norm_qkn, T, 0, true, LP_DEV)                             \
    CUCA_ROPE_W(cuca_rope_##TN##_neox_qkn, T, 2, true, LP_DEV)                             \
    CUCA_ROPE_W(cuca_rope_##TN##_norm_qkn_nt, T, 0, true, LP_NT)                           \
    CUCA_ROPE_W(cuca_rope_##TN##_neox_qkn_nt, T, 2, true, LP_NT)                           \
    extern "C" __global__ __launch_bounds__(CUCA_BLOCK) void cuca_rope_##TN##_generic(     \
        RopeArgs a) {                                                                      \
        rope_generic_body<T>(a);                                                           \
    }                                                                                      \
    CUCA_ROPE_FULL(cuca_rope_##TN##_norm_full, T, 0, false)                                \
    CUCA_ROPE_FULL(cuca_rope_##TN##_neox_full, T, 2, false)                                \
    CUCA_ROPE_FULL(cuca_rope_##TN##_norm_full_kv, T, 0, true)                              \
    CUCA_ROPE_FULL(cuca_rope_##TN##_neox_full_kv, T, 2, true)

CUCA_ROPE_SET(f32, float)
CUCA_ROPE_SET(f16, _Float16)
