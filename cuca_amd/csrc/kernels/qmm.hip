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
// is two f16 values M + u (M a bit pattern with the quant's bits clear):
//   Q8_0: u = q + 128, stored biased; v_perm_b32 places the two bytes under
//         a 0x64 exponent byte: 1024 + u = 1152 + q;
//   Q4_0: the lanes' nibbles of four blocks share a dword (low nibbles in
//         bits 4i, high nibbles in bits 16 + 4i); one v_bfi_b32 inserts a
//         pair into M0 = 0x6480 (blocks 0, 2 of the dword: 1152 + n) or into
//         M1 = 0x6408 at bits 4-7 (blocks 1, 3: 1032 + 16 n).
// The activation pair is (f16 q[l], f16 q[l+16]) and the accumulator input
// of the dot is C = -K (q[l] + q[l+16]) with K = 1152 (Q8_0) or 1160 (Q4_0),
// so the dot returns the exact pair sum P = w[l] q[l] + w[l+16] q[l+16], or
// 16 P for the Q4_0 blocks in the odd position, whose f32 weight scale is
// staged as dw / 16: (16 P) * (dw / 16 * dx) is the same real number as
// P * (dw * dx) (f16 scales keep dw / 16 and its products normal), so every
// rounding is the definition's.
//
// Weight layout (QmmPack, built once by cuca_qpack_* from the GGUF rows):
// per row, groups of G blocks of GB bytes -- the scales first (G f16), then
// sixteen 16-byte lane chunks, so a thread reads G blocks of its lane with
// one dwordx4 load:
//   Q4_0: G = 16, GB = 288: lane chunk l, dword k = blocks 4k..4k+3: bits
//         4i..4i+3 the nibble of element l of block 4k+i, bits 16+4i..
//         16+4i+3 that of element l+16;
//   Q8_0: G =  8, GB = 272: lane chunk l, dword k = blocks 2k, 2k+1: bytes
//         q[l]+128 of 2k, of 2k+1, q[l+16]+128 of 2k, of 2k+1.
// Blocks past the row's end (a partial last group) are zero bytes with a
// zero scale, which add exact zeros.
//
// Chunks.  The blocks are processed in chunks of CB (64; 32 for four
// activation rows).  Per chunk the workgroup quantises its activation tile
// into LDS (four threads per 32 values), stages the 16 rows' weight scales as
// f32 and, for tiles of one or two rows, the products dw * dx per (row,
// block), which every lane of the row uses.  The loads of chunk c + 1 (its
// weights, activations and weight scales) are issued before chunk c is
// computed, and its staging is written into the other half of a double
// buffer.  Grid: the workgroups of one XCD take consecutive row blocks with
// all their activation tiles, so the weight rows a tile re-reads stay in
// that XCD's L2.
#include "common.h"

#define QMM_RPW 16 // weight rows per workgroup

typedef _Float16 qmm_h2 __attribute__((ext_vector_type(2)));
typedef uint32_t qmm_u2 __attribute__((ext_vector_type(2)));

// (d & mask) | (m & ~mask) as one v_bfi_b32 (the compiler splits the
// expression into an and and an or).
__device__ static inline uint32_t qmm_bfi(uint32_t mask, uint32_t d, uint32_t m) {
    uint32_t r;
    asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "v"(mask), "v"(d), "v"(m));
    return r;
}

template <int FMT> struct QFmt;
template <> struct QFmt<0> { // Q4_0
    static constexpr int G = 16, GB = 288, SCB = 32, BB = 18;
    static constexpr float K = 1160.0f;
    // the weight pair of block i of a lane chunk (see the layout above)
    __device__ static inline uint32_t pair(const u32x4 &v, int i) {
        const uint32_t d = v[i >> 2] >> ((i & 2) ? 8 : 0);
        return (i & 1) ? qmm_bfi(0x00f000f0u, d, 0x64086408u) : qmm_bfi(0x000f000fu, d, 0x64806480u);
    }
    // staged weight scale: the odd blocks' pairs carry a factor 16
    __device__ static inline float scale(float dw, int b) { return (b & 1) ? dw * 0.0625f : dw; }
};
template <> struct QFmt<1> { // Q8_0
    static constexpr int G = 8, GB = 272, SCB = 16, BB = 34;
    static constexpr float K = 1152.0f;
    __device__ static inline uint32_t pair(const u32x4 &v, int i) {
        return __builtin_amdgcn_perm(0x64646464u, v[i >> 1], (i & 1) ? 0x04030401u : 0x04020400u);
    }
    __device__ static inline float scale(float dw, int) { return dw; }
};

template <int MT> struct QShape {
    static constexpr int CB = MT == 4 ? 32 : 64; // blocks per chunk
    static constexpr bool PRE_S = MT <= 2;       // stage dw * dx per (row, block)
    static constexpr int XS = CB + 2;            // lane stride of xe (uint2 units)
    static constexpr int WSS = CB + 4;           // row stride of the f32 scale rows
    static constexpr int ITEMS = MT * CB / 64;   // (act row, block) items per thread
};

__device__ static inline float qmm_dot(uint32_t w, uint32_t x, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(qmm_h2, w), __builtin_bit_cast(qmm_h2, x), c,
                                  false);
}

// round_away (qmm.rs:1194-1201) then Rust's saturating `as i8` (NaN -> 0),
// as an exact integer-valued float.  Rounding half away from zero is
// trunc(t + copysign(0.5 - 2^-25, t)): the same bits as roundf for every
// finite f32 (checked exhaustively on the host, all 2^32 patterns), in two
// instructions fewer.  NaN is tested on t itself: the clamp's min / max
// return their other operand for a NaN, so a test after it never fires (it
// did not: a NaN activation quantised to -128).
__device__ static inline float qmm_quant(float t) {
    const float r = __builtin_truncf(t + __builtin_copysignf(0.49999997f, t));
    const float c = fminf(fmaxf(r, -128.0f), 127.0f);
    return t == t ? c : 0.0f;
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

// 16-byte aligned, so that every 16-byte operand read is one ds_read_b128:
// with the 8-byte alignment of its members the compiler split them into
// ds_read2_b64 pairs, which lost 35-40 % of the LDS cycles to bank
// conflicts (SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE) at this lane stride;
// ds_read_b128 reads it conflict-free.  Measured on MI355X: down 4096 x
// 14336 Q4_0 at one row 17.7 -> 14.9 us, gate+up 23.0 -> 20.0 us.
template <int MT, bool GLU> struct alignas(16) QmmLds {
    using S = QShape<MT>;
    static constexpr int SB = S::PRE_S ? 2 : 1;   // buffers of s
    static constexpr int WB = S::PRE_S ? 1 : 2;   // buffers of xs, ws
    qmm_u2 xe[2][MT][16][S::XS];                  // (f16 act pair, C) per act row, lane, block
    float s[SB][S::PRE_S ? MT : 1][QMM_RPW][S::WSS];             // dw * dx (gate or plain)
    float su[(S::PRE_S && GLU) ? 2 : 1][(S::PRE_S && GLU) ? MT : 1][(S::PRE_S && GLU) ? QMM_RPW : 1][S::WSS];
    float xs[WB][MT][S::CB];                      // act block scales
    float ws[WB][QMM_RPW][S::WSS];                // f32 weight scales (gate or plain)
    float wu[GLU ? WB : 1][GLU ? QMM_RPW : 1][S::WSS];
};

// The registers a chunk's staging starts from, loaded one chunk ahead.
template <int MT> struct QPre {
    float x[QShape<MT>::ITEMS][8];
    u32x4 wsc; // eight f16 weight scales
};

// The activation rows of a workgroup's tile and where its results go.
template <int MT> struct QTile {
    int64_t xrow[MT];     // element offset of act row j in x, or -1 (no row)
    int64_t orow[MT];     // element offset of output row j
    float weight[MT];     // MoE down: the pair's routing weight
    const uint8_t *w, *w_up;
};

// Element j_base (or j_base + 1 when `hi`) of a per-row array, with
// compile-time indices only.
template <typename V, int MT>
__device__ static inline V qmm_pick(const V (&arr)[MT], int jb, bool hi) {
    return (jb + 1 < MT && hi) ? arr[jb + 1 < MT ? jb + 1 : jb] : arr[jb];
}

// The tile's act row of an item of the staging (item = it * 64 + tid / 4):
// j = item / CB, a compile-time index when CB = 64, one of two otherwise.
template <int MT>
__device__ static inline int64_t qmm_item_row(const QTile<MT> &tl, int it, int tid) {
    using S = QShape<MT>;
    if constexpr (S::CB == 64) return tl.xrow[it];
    else return qmm_pick<int64_t, MT>(tl.xrow, 2 * it, (tid >> 2) >= 32);
}

template <typename T, int FMT, int MT>
__device__ static inline void qmm_prefetch(const QmmArgs &a, const QTile<MT> &tl, QPre<MT> &p, int row0,
                                           int c) {
    using S = QShape<MT>;
    using F = QFmt<FMT>;
    const int tid = threadIdx.x;
#pragma unroll
    for (int it = 0; it < S::ITEMS; it++) {
        const int item = it * 64 + (tid >> 2);
        const int b = item % S::CB, gb = c * S::CB + b;
        const int64_t xr = qmm_item_row<MT>(tl, it, tid);
        if (xr >= 0 && gb < a.nb) {
            qmm_load8<T>(reinterpret_cast<const T *>(a.x) + xr + (int64_t)gb * 32 + (tid & 3) * 8, p.x[it]);
        } else {
#pragma unroll
            for (int e = 0; e < 8; e++) p.x[it][e] = 0.0f;
        }
    }
    // weight scales: P = 2 CB pieces of eight per matrix (16 rows x CB / 8)
    constexpr int P = 2 * S::CB;
    const int which = tid / P, t = tid % P;
    const int r = t / (S::CB / 8), piece = t % (S::CB / 8);
    const int blk0 = c * S::CB + piece * 8, g = blk0 / F::G, row = row0 + r;
    p.wsc = u32x4{0u, 0u, 0u, 0u};
    if (which < (tl.w_up ? 2 : 1) && row < a.rows && g < a.ng) {
        const uint8_t *w = which ? tl.w_up : tl.w;
        p.wsc = *reinterpret_cast<const u32x4 *>(w + (int64_t)row * a.row_bytes + (int64_t)g * F::GB +
                                               (blk0 % F::G) * 2);
    }
}

// Stage A of chunk c from the prefetched registers: quantise the act tile
// (Acts::new, qmm.rs:1217-1240; four threads per (act row, block), eight
// values each) into xe[xb] and xs[wb]; the weight scales into ws[wb] / wu[wb].
template <int FMT, int MT, bool GLU>
__device__ static inline void qmm_stage_a(const QmmArgs &a, QmmLds<MT, GLU> &L, const QTile<MT> &tl,
                                          const QPre<MT> &p, int c, int xb, int wb) {
    using S = QShape<MT>;
    using F = QFmt<FMT>;
    const int tid = threadIdx.x, sub = tid & 3;
#pragma unroll
    for (int it = 0; it < S::ITEMS; it++) {
        const int item = it * 64 + (tid >> 2);
        const int j = item / S::CB, b = item % S::CB;
        float amax = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; e++) amax = fmaxf(amax, fabsf(p.x[it][e]));
        amax = fmaxf(amax, xor_partner(amax, 1));
        amax = fmaxf(amax, xor_partner(amax, 2));
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        // own quants as f16 pairs of consecutive elements (exact integers)
        uint32_t own[4], other[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            own[i] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(qmm_quant(p.x[it][2 * i] * id),
                                                                             qmm_quant(p.x[it][2 * i + 1] * id)));
            other[i] = xor_partner_bits(own[i], 2);
        }
        // threads 0/1 own elements 0-7 / 8-15, threads 2/3 own 16-23 / 24-31;
        // sub < 2 writes lanes 8s..8s+3, sub >= 2 lanes 8s+4..8s+7 (s = sub & 1)
        const bool low = sub < 2;
        const int base = 8 * (sub & 1) + (low ? 0 : 4);
        const qmm_h2 negk = {(_Float16)(-F::K), (_Float16)(-F::K)};
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const uint32_t lo = low ? own[q >> 1] : other[2 + (q >> 1)];
            const uint32_t hi = low ? other[q >> 1] : own[2 + (q >> 1)];
            const uint32_t xp = __builtin_amdgcn_perm(hi, lo, (q & 1) ? 0x07060302u : 0x05040100u);
            const float cc = __builtin_amdgcn_fdot2(__builtin_bit_cast(qmm_h2, xp), negk, 0.0f, false);
            L.xe[xb][j][base + q][b] = qmm_u2{xp, __builtin_bit_cast(uint32_t, cc)};
        }
        const bool valid = qmm_item_row<MT>(tl, it, tid) >= 0 && c * S::CB + b < a.nb;
        if (sub == 0) L.xs[wb][j][b] = valid ? (float)(_Float16)d : 0.0f;
    }
    constexpr int P = 2 * S::CB;
    const int which = tid / P, t = tid % P;
    if (which < (GLU ? 2 : 1)) {
        const int r = t / (S::CB / 8), piece = t % (S::CB / 8);
        const u32x4 raw = p.wsc;
        const f16x8 h = __builtin_bit_cast(f16x8, raw);
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = F::scale((float)h[i], i);
        float *dst = which ? &L.wu[GLU ? wb : 0][GLU ? r : 0][piece * 8] : &L.ws[wb][r][piece * 8];
        reinterpret_cast<f32x4 *>(dst)[0] = f32x4{v[0], v[1], v[2], v[3]};
        reinterpret_cast<f32x4 *>(dst)[1] = f32x4{v[4], v[5], v[6], v[7]};
    }
}

// Stage B (tiles of one or two rows): s[sb][j][r][b] = ws[r][b] * xs[j][b].
template <int MT, bool GLU>
__device__ static inline void qmm_stage_b(QmmLds<MT, GLU> &L, int sb) {
    using S = QShape<MT>;
    if constexpr (S::PRE_S) {
        const int tid = threadIdx.x;
        const int r = tid >> 4, b4 = (tid & 15) * 4; // CB = 64: 16 float4 per row
        const f32x4 w = *reinterpret_cast<const f32x4 *>(&L.ws[0][r][b4]);
        f32x4 u = {0.0f, 0.0f, 0.0f, 0.0f};
        if (GLU) u = *reinterpret_cast<const f32x4 *>(&L.wu[0][GLU ? r : 0][b4]);
#pragma unroll
        for (int j = 0; j < MT; j++) {
            const f32x4 x = *reinterpret_cast<const f32x4 *>(&L.xs[0][j][b4]);
            *reinterpret_cast<f32x4 *>(&L.s[sb][j][r][b4]) = w * x;
            if (GLU) *reinterpret_cast<f32x4 *>(&L.su[GLU ? sb : 0][GLU ? j : 0][GLU ? r : 0][b4]) = u * x;
        }
    }
}

template <int FMT, int MT>
__device__ static inline void qmm_load_w(const uint8_t *w, const QmmArgs &a, int row, int lane, int c,
                                         u32x4 (&v)[QShape<MT>::CB / QFmt<FMT>::G]) {
    using F = QFmt<FMT>;
    constexpr int NG = QShape<MT>::CB / F::G;
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

// The LDS operands of four blocks of one activation row.
struct QStep {
    f32x4 sg, su;     // dw * dx (gate / up), or the two scales' sources
    u32x4 x01, x23;   // (act pair, C) of the four blocks
};

template <int MT, bool GLU>
__device__ static inline void qmm_step_load(const QmmLds<MT, GLU> &L, int buf, int rloc, int lane, int b0,
                                            QStep (&st)[MT]) {
    using S = QShape<MT>;
    f32x4 dw = {0.0f, 0.0f, 0.0f, 0.0f}, du = {0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (!S::PRE_S) {
        dw = *reinterpret_cast<const f32x4 *>(&L.ws[buf][rloc][b0]);
        if (GLU) du = *reinterpret_cast<const f32x4 *>(&L.wu[GLU ? buf : 0][GLU ? rloc : 0][b0]);
    }
#pragma unroll
    for (int j = 0; j < MT; j++) {
        if constexpr (S::PRE_S) {
            st[j].sg = *reinterpret_cast<const f32x4 *>(&L.s[buf][j][rloc][b0]);
            if (GLU) st[j].su = *reinterpret_cast<const f32x4 *>(&L.su[GLU ? buf : 0][GLU ? j : 0][GLU ? rloc : 0][b0]);
        } else {
            const f32x4 dx = *reinterpret_cast<const f32x4 *>(&L.xs[buf][j][b0]);
            st[j].sg = dw * dx;
            if (GLU) st[j].su = du * dx;
        }
        st[j].x01 = *reinterpret_cast<const u32x4 *>(&L.xe[buf][j][lane][b0]);
        st[j].x23 = *reinterpret_cast<const u32x4 *>(&L.xe[buf][j][lane][b0 + 2]);
    }
}

// One chunk of a thread's chains: acc[j] += (float)P * (dw * dx), in steps of
// four blocks; the next step's LDS operands are read one step ahead, and a
// scheduling barrier after each step keeps the compiler from hoisting a
// whole chunk's reads into registers (measured: 256 VGPRs and spills
// without it).
template <int FMT, int MT, bool GLU>
__device__ static inline void qmm_chunk(const QmmLds<MT, GLU> &L, int buf, int rloc, int lane,
                                        const u32x4 (&wg)[QShape<MT>::CB / QFmt<FMT>::G],
                                        const u32x4 (&wu)[QShape<MT>::CB / QFmt<FMT>::G],
                                        float (&acc)[MT], float (&accu)[MT]) {
    using F = QFmt<FMT>;
    using S = QShape<MT>;
    constexpr int NSTEP = S::CB / 4;
    QStep cur[MT], nxt[MT];
    qmm_step_load<MT, GLU>(L, buf, rloc, lane, 0, cur);
#pragma unroll
    for (int step = 0; step < NSTEP; step++) {
        if (step + 1 < NSTEP) qmm_step_load<MT, GLU>(L, buf, rloc, lane, 4 * (step + 1), nxt);
        const int gg = (4 * step) / F::G, i0 = (4 * step) % F::G;
        uint32_t pg[4], pu[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            pg[i] = F::pair(wg[gg], i0 + i);
            pu[i] = GLU ? F::pair(wu[gg], i0 + i) : 0u;
        }
#pragma unroll
        for (int j = 0; j < MT; j++) {
            const uint32_t xp[4] = {cur[j].x01.x, cur[j].x01.z, cur[j].x23.x, cur[j].x23.z};
            const uint32_t xc[4] = {cur[j].x01.y, cur[j].x01.w, cur[j].x23.y, cur[j].x23.w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float cc = __builtin_bit_cast(float, xc[i]);
                acc[j] = acc[j] + qmm_dot(pg[i], xp[i], cc) * cur[j].sg[i];
                if (GLU) accu[j] = accu[j] + qmm_dot(pu[i], xp[i], cc) * cur[j].su[i];
            }
        }
        // pin this step's arithmetic here (the chains are only read at the
        // end, so the compiler would otherwise sink it past the barrier)
#pragma unroll
        for (int j = 0; j < MT; j++) {
            asm volatile("" : "+v"(acc[j]));
            if (GLU) asm volatile("" : "+v"(accu[j]));
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < MT; j++) cur[j] = nxt[j];
    }
}

// hsum (qmm.rs:1345-1353) over the 16 lanes of a row: xor 8, 4, 1, 2.
__device__ static inline float qmm_hsum(float v) {
    v = v + xor_partner(v, 8);
    v = v + xor_partner(v, 4);
    v = v + xor_partner(v, 1);
    v = v + xor_partner(v, 2);
    return v;
}

// MoE: the expert and pair range of activation tile `tile`.  Expert e has
// ceil(n_e / MT) tiles, in expert order; a workgroup (CUCA_BLOCK threads)
// finds its expert by a prefix sum over the offsets.  Returns false (for the
// whole workgroup) past the last tile.
template <int MT>
__device__ static inline bool moe_tile_lookup(const int32_t *offsets, int n_experts, int max_pairs, int tile,
                                              int *expert, int *p0, int *p1) {
    __shared__ int sh[CUCA_BLOCK / CUCA_WAVE + 2];
    const int tid = threadIdx.x, wave = tid / CUCA_WAVE, lane = tid % CUCA_WAVE;
    if (tid == 0) { sh[CUCA_BLOCK / CUCA_WAVE] = -1; sh[CUCA_BLOCK / CUCA_WAVE + 1] = 0; }
    int base = 0;
    for (int e0 = 0; e0 < n_experts; e0 += CUCA_BLOCK) {
        const int e = e0 + tid;
        int cnt = 0;
        if (e < n_experts) {
            const int lo = offsets[e], hi = offsets[e + 1];
            cnt = hi > lo ? (hi - lo + MT - 1) / MT : 0;
        }
        // inclusive scan: within the wave, then over the waves
        int incl = cnt;
#pragma unroll
        for (int off = 1; off < CUCA_WAVE; off <<= 1) {
            const int v = __shfl_up(incl, off, CUCA_WAVE);
            if (lane >= off) incl += v;
        }
        __syncthreads(); // sh[] of the previous round has been read
        if (lane == CUCA_WAVE - 1) sh[wave] = incl;
        __syncthreads();
        int before = base;
        for (int w = 0; w < wave; w++) before += sh[w];
        int total = 0;
        for (int w = 0; w < CUCA_BLOCK / CUCA_WAVE; w++) total += sh[w];
        const int excl = before + incl - cnt;
        if (cnt > 0 && tile >= excl && tile < excl + cnt) {
            sh[CUCA_BLOCK / CUCA_WAVE] = e;
            sh[CUCA_BLOCK / CUCA_WAVE + 1] = tile - excl;
        }
        base += total;
    }
    __syncthreads();
    const int e = sh[CUCA_BLOCK / CUCA_WAVE];
    if (e < 0) return false;
    const int local = sh[CUCA_BLOCK / CUCA_WAVE + 1];
    int lo = offsets[e] + local * MT;
    int hi = lo + MT < offsets[e + 1] ? lo + MT : offsets[e + 1];
    if (hi > max_pairs) hi = max_pairs;
    if (lo < 0) lo = 0;
    *expert = e;
    *p0 = lo;
    *p1 = hi;
    return true;
}

template <int MT>
__device__ static inline bool qmm_moe_tile(const QmmArgs &a, int tile, int *expert, int *p0, int *p1) {
    return moe_tile_lookup<MT>(a.offsets, a.n_experts, a.max_pairs, tile, expert, p0, p1);
}

// The Q|K|V epilogue (MODE 3): the output o of weight row `row` for
// activation row j, as the plain kernel would store it, then what
// rope_store_kv (rope.hip; store_kv, cpu.rs:3028-3097) does to it: Q and K
// rotated in NORM pairs (2i, 2i+1) -- rows row and row ^ 1, held by the
// lanes 16 apart in this wave -- as a' = a c - b s, b' = a s + b c with
// each product rounded on its own; Q stored in place of the plain output,
// K and V written to their pools at pool row slots[j].  The same bits as
// cuca_hip_qmm followed by cuca_hip_rope_store_kv.  A row whose position
// or slot is bad keeps Q unrotated and stores no K/V (as rope_store_kv
// leaves it), and is reported.
template <typename T>
__device__ static inline void qmm_rope_kv_store(const QmmArgs &a, int jg, bool valid, int64_t orow, int row,
                                                int lane, float o) {
    // the value the plain kernel stores, widened back (exact)
    const float v = (float)to_stored<T>(o);
    const float pv = xor_partner(v, 16); // row ^ 1: the pair partner
    if (lane != 0 || row >= a.rows || !valid) return;
    const int D = a.head_dim, half = a.n_dims >> 1;
    const int h = row / D, e = row - h * D;
    const int hk = h < a.nq ? 0 : (h < a.nq + a.nk ? 1 : 2); // Q, K or V head
    const int32_t pos = a.pos[jg], slot = a.slots[jg];
    const bool ok = pos >= 0 && (int64_t)pos < a.table_rows && slot >= 0 && (int64_t)slot < a.n_slots;
    if (!ok) {
        if (row == 0) {
            if (!(pos >= 0 && (int64_t)pos < a.table_rows))
                record_bad(a.status + CUCA_STATUS_ROPE_POS, (uint32_t)jg, (uint32_t)pos);
            else
                record_bad(a.status + CUCA_STATUS_KV_SLOT, (uint32_t)jg, (uint32_t)slot);
        }
        if (hk == 0) reinterpret_cast<T *>(a.out)[orow + row] = to_stored<T>(v);
        return;
    }
    float r = v;
    if (hk != 2 && e < a.n_dims) {
        const int64_t t = (int64_t)pos * half + (e >> 1);
        const float c = a.cos_t[t], s = a.sin_t[t];
        // a' = a c - b s (even element), b' = a s + b c (odd element)
        r = (e & 1) ? pv * s + v * c : v * c - pv * s;
    }
    if (hk == 0) {
        reinterpret_cast<T *>(a.out)[orow + row] = to_stored<T>(r);
    } else {
        const int kvh = h - a.nq - (hk == 2 ? a.nk : 0);
        const int64_t prow = ((int64_t)(slot >> 4) * a.nk + kvh) * 16 + (slot & 15);
        reinterpret_cast<T *>(hk == 1 ? a.pool_k : a.pool_v)[prow * D + e] = to_stored<T>(r);
    }
}

// MODE 0: dense (x rows j0.., out rows j0..); 1: MoE up (act row of pair p =
// x row pair_token[p], output row p); 2: MoE down (act row p of x, output
// row p of an f32 scratch, times pair_weight[p]); 3: dense Q|K|V with RoPE
// (NORM pairs) and the paged K/V store in the epilogue.
template <typename T, int FMT, int MT, bool GLU, int ACT, int MODE>
__device__ static inline void qmm_body(const QmmArgs &a) {
    using F = QFmt<FMT>;
    using S = QShape<MT>;
    constexpr int NG = S::CB / F::G;
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
    const int nch = (a.ng * F::G + S::CB - 1) / S::CB;

    QTile<MT> tl;
    if constexpr (MODE == 0 || MODE == 3) {
        const int j0 = tile * MT;
#pragma unroll
        for (int j = 0; j < MT; j++) {
            tl.xrow[j] = j0 + j < a.m ? (int64_t)(j0 + j) * a.ldx : -1;
            tl.orow[j] = (int64_t)(j0 + j) * a.out_ld;
            tl.weight[j] = 1.0f;
        }
        tl.w = a.w;
        tl.w_up = a.w_up;
    } else {
        int e, p0, p1;
        if (!qmm_moe_tile<MT>(a, tile, &e, &p0, &p1)) return;
#pragma unroll
        for (int j = 0; j < MT; j++) {
            const int p = p0 + j;
            int64_t xr = -1;
            float wt = 0.0f;
            if (p < p1) {
                if (MODE == 1) {
                    const int t = a.pair_token[p];
                    if (t >= 0 && t < a.n_tokens) xr = (int64_t)t * a.ldx;
                    else if (tid == 0) record_bad(a.status + CUCA_STATUS_MOE_PAIR, (uint32_t)p, (uint32_t)t);
                } else {
                    xr = (int64_t)p * a.ldx;
                    wt = a.pair_weight[p];
                }
            }
            tl.xrow[j] = xr;
            tl.orow[j] = (int64_t)p * a.out_ld;
            tl.weight[j] = wt;
        }
        tl.w = a.w + (int64_t)e * a.w_estride;
        tl.w_up = GLU ? a.w_up + (int64_t)e * a.w_estride : nullptr;
    }

    float acc[MT], accu[MT];
#pragma unroll
    for (int j = 0; j < MT; j++) { acc[j] = 0.0f; accu[j] = 0.0f; }
    u32x4 wg[NG], wu[NG], ng_[NG], nu[NG];
    QPre<MT> pre;
    // chunk 0
    qmm_load_w<FMT, MT>(tl.w, a, row, lane, 0, wg);
    if (GLU) qmm_load_w<FMT, MT>(tl.w_up, a, row, lane, 0, wu);
    qmm_prefetch<T, FMT, MT>(a, tl, pre, row0, 0);
    qmm_stage_a<FMT, MT, GLU>(a, L, tl, pre, 0, 0, 0);
    __syncthreads();
    if constexpr (S::PRE_S) {
        qmm_stage_b<MT, GLU>(L, 0);
        __syncthreads();
    }
    for (int c = 0; c < nch; c++) {
        const int buf = c & 1;
        const bool next = c + 1 < nch;
        if (next) {
            qmm_load_w<FMT, MT>(tl.w, a, row, lane, c + 1, ng_);
            if (GLU) qmm_load_w<FMT, MT>(tl.w_up, a, row, lane, c + 1, nu);
            qmm_prefetch<T, FMT, MT>(a, tl, pre, row0, c + 1);
        }
        qmm_chunk<FMT, MT, GLU>(L, buf, rloc, lane, wg, wu, acc, accu);
        if (next) qmm_stage_a<FMT, MT, GLU>(a, L, tl, pre, c + 1, buf ^ 1, S::PRE_S ? 0 : buf ^ 1);
        __syncthreads();
        if constexpr (S::PRE_S) {
            if (next) qmm_stage_b<MT, GLU>(L, buf ^ 1);
            __syncthreads();
        }
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
        if (MODE == 0 && !GLU && a.cap_flags) { // cap_logits (cpu.rs:2603-2617)
            if (a.cap_flags & 1) o = o * a.mul1 + 0.0f;
            if (a.cap_flags & 2) o = o * a.mul2 + 0.0f;
            if (a.cap_flags & 4) o = tanhf(o * a.softcap_inv + 0.0f) * a.softcap + 0.0f;
        }
        if constexpr (MODE == 3) {
            qmm_rope_kv_store<T>(a, tile * MT + j, tl.xrow[j] >= 0, tl.orow[j], row, lane, o);
            continue;
        }
        if (lane == 0 && row < a.rows && tl.xrow[j] >= 0) {
            if (MODE == 2) // CpuExpert::add_picks: y * weight (cpu.rs:400-417)
                reinterpret_cast<float *>(a.out)[tl.orow[j] + row] = o * tl.weight[j];
            else
                reinterpret_cast<T *>(a.out)[tl.orow[j] + row] = to_stored<T>(o);
        }
    }
}

// MoE expert sum (expert_sum's accumulation, cpu.rs:3599-3642, and the
// reference GPU engine's moe_sum, moe_kernel.rs:1370-1385): out[t] = sum
// over the token's pairs, in ascending expert order, of scratch[pair],
// f32 from 0.  Four elements per thread.
template <typename T> __device__ static inline void moe_sum_body(const MoeSumArgs &a) {
    const int nq = (a.n_embd + 3) / 4;
    const int64_t g = (int64_t)blockIdx.x * CUCA_BLOCK + threadIdx.x;
    if (g >= (int64_t)a.n_tokens * nq) return;
    const int t = (int)(g / nq), q = (int)(g - (int64_t)t * nq);
    const int h0 = 4 * q;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    // eight pairs at a time: their ids, then their rows, are all loaded
    // before the sums (in the pairs' order) use them
    for (int i0 = 0; i0 < a.n_used; i0 += 8) {
        int p[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            p[j] = i0 + j < a.n_used ? a.pairs[(int64_t)t * a.n_used + i0 + j] : -1;
            if (p[j] >= a.max_pairs) p[j] = -1;
        }
        float v[8][4];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float *src = a.scratch + (int64_t)(p[j] < 0 ? 0 : p[j]) * a.scratch_ld + h0;
#pragma unroll
            for (int e = 0; e < 4; e++) v[j][e] = (p[j] >= 0 && h0 + e < a.n_embd) ? src[e] : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < 8; j++)
            if (p[j] >= 0) {
#pragma unroll
                for (int e = 0; e < 4; e++) acc[e] = acc[e] + v[j][e];
            }
    }
    T *dst = reinterpret_cast<T *>(a.out) + (int64_t)t * a.out_ld + h0;
#pragma unroll
    for (int e = 0; e < 4; e++)
        if (h0 + e < a.n_embd) dst[e] = to_stored<T>(acc[e]);
}

extern "C" __global__ __launch_bounds__(CUCA_BLOCK) void cuca_moe_sum_f32(MoeSumArgs a) { moe_sum_body<float>(a); }
extern "C" __global__ __launch_bounds__(CUCA_BLOCK) void cuca_moe_sum_f16(MoeSumArgs a) { moe_sum_body<_Float16>(a); }

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
            // dword k: blocks 4k..4k+3; nibble i of the low half = element l
            // of block 4k+i, nibble i of the high half = element l+16
#pragma unroll
            for (int k = 0; k < 4; k++) {
                uint32_t lo = 0, hi = 0;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int blk = g * 16 + 4 * k + i;
                    const uint32_t byte = blk < a.nb ? src[(int64_t)blk * F::BB + 2 + l] : 0u;
                    lo |= (byte & 15u) << (4 * i);
                    hi |= (byte >> 4) << (4 * i);
                }
                const uint32_t word = lo | (hi << 16);
                out[4 * k] = word & 255u;
                out[4 * k + 1] = (word >> 8) & 255u;
                out[4 * k + 2] = (word >> 16) & 255u;
                out[4 * k + 3] = word >> 24;
            }
        } else {
            // dword k: q[l] + 128 of blocks 2k, 2k+1, then q[l+16] + 128 of both
#pragma unroll
            for (int k = 0; k < 4; k++) {
#pragma unroll
                for (int i = 0; i < 2; i++) {
                    const int blk = g * 8 + 2 * k + i;
                    out[4 * k + i] = blk < a.nb ? (uint8_t)(src[(int64_t)blk * F::BB + 2 + l] ^ 0x80u) : 0;
                    out[4 * k + 2 + i] = blk < a.nb ? (uint8_t)(src[(int64_t)blk * F::BB + 2 + 16 + l] ^ 0x80u) : 0;
                }
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
// [act dtype][format][act rows per tile]: plain, SwiGLU, GeGLU-tanh; MoE
// up (SwiGLU, GeGLU-tanh) and down
#define CUCA_QMM_MT(TN, T, FN, FMT, MT)                                                    \
    CUCA_QMM(cuca_qmm_##TN##_##FN##_m##MT, T, FMT, MT, false, 0, 0)                        \
    CUCA_QMM(cuca_qmm_glu_##TN##_##FN##_silu_m##MT, T, FMT, MT, true, 0, 0)                \
    CUCA_QMM(cuca_qmm_glu_##TN##_##FN##_gelu_m##MT, T, FMT, MT, true, 1, 0)                \
    CUCA_QMM(cuca_moe_up_##TN##_##FN##_silu_m##MT, T, FMT, MT, true, 0, 1)                 \
    CUCA_QMM(cuca_moe_up_##TN##_##FN##_gelu_m##MT, T, FMT, MT, true, 1, 1)                 \
    CUCA_QMM(cuca_moe_down_##TN##_##FN##_m##MT, T, FMT, MT, false, 0, 2)                  \
    CUCA_QMM(cuca_qmm_rope_kv_##TN##_##FN##_m##MT, T, FMT, MT, false, 0, 3)
#define CUCA_QMM_SET(TN, T, FN, FMT)                                                       \
    CUCA_QMM_MT(TN, T, FN, FMT, 1)                                                         \
    CUCA_QMM_MT(TN, T, FN, FMT, 2)                                                         \
    CUCA_QMM_MT(TN, T, FN, FMT, 4)

CUCA_QMM_SET(f32, float, q4_0, 0)
CUCA_QMM_SET(f32, float, q8_0, 1)
CUCA_QMM_SET(f16, _Float16, q4_0, 0)
CUCA_QMM_SET(f16, _Float16, q8_0, 1)
