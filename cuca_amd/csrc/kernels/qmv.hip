// qmv.hip -- the decode GEMV of the CPU engine's quantized matmul (qmm.rs)
// on gfx950: the same bits as qmm.hip, for one to four activation rows,
// shaped for the latency of a decode step, and the routed experts (MoE) at
// decode on the same kernel.
//
// A workgroup holds its activation rows for the whole row length in LDS,
// expanded once to what the integer dot reads: the f16 pair and C of
// qmm.hip per (row, lane, block), and the block scales.  The rows come
//   mode 0: quantised already (cuca_q8_acts_*: Acts::new, qmm.rs:1217-1343,
//           one thread per 32 values), shared by every workgroup;
//   mode 3: as f32 / f16 values, quantised by the workgroup (Acts::new,
//           the same bits), so a call is one launch;
//   mode 1 (MoE up) / 2 (MoE down): the rows of one tile of an expert's
//           pairs (up: the pairs' token rows of x; down: the pairs' hidden
//           rows), quantised by the workgroup.
// Its four waves then run independently.  A wave's task is four weight rows
// x sixteen lanes, each thread one chain over all blocks; a wave takes a
// sequence of tasks and streams their groups of G blocks back to back
// through a ring of QMV_D groups in flight, so the next task's weights load
// while the current one finishes.  Per group a wave stages dw * dx of its
// four rows in its own LDS area (no workgroup barrier).
// Modes 0 / 3: workgroups are persistent, a wave's tasks are strided over
// the grid.  Modes 1 / 2: workgroup (tile, split) takes tile `tile` of the
// expert order (moe_tile_lookup) and a contiguous range of the expert's row
// tasks; the outputs are those of the one-pass MoE kernels (hidden rows in
// pair order; f32 rows y * routing weight for moe_sum).
#include "common.h"

#define QMV_WAVES 4
#define QMV_D 8   // weight groups in flight per wave
#define QMV_NT 32 // tasks a wave streams before it writes their outputs

__device__ static inline float qmv_h2f(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// Acts::new for MIN_NONE of one 32-value block: v -> q (integers as f32)
// and the f16-rounded scale.
__device__ static inline float qmv_quant_block(float (&v)[32]) {
    float amax = 0.0f;
#pragma unroll
    for (int e = 0; e < 32; e++) amax = fmaxf(amax, fabsf(v[e]));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
#pragma unroll
    for (int e = 0; e < 32; e++) v[e] = qmm_quant(v[e] * id);
    return (float)(_Float16)d;
}

template <typename T> __device__ static inline void qmv_load32(const T *src, float (&v)[32]) {
#pragma unroll
    for (int q = 0; q < 4; q++) {
        float e[8];
        qmm_load8<T>(src + 8 * q, e);
#pragma unroll
        for (int i = 0; i < 8; i++) v[8 * q + i] = e[i];
    }
}

// One thread per (row, block).
template <typename T> __device__ static inline void q8_acts_body(const Q8ActsArgs &a) {
    const int64_t t = (int64_t)blockIdx.x * CUCA_BLOCK + threadIdx.x;
    if (t >= (int64_t)a.m * a.nb) return;
    const int j = (int)(t / a.nb), b = (int)(t - (int64_t)j * a.nb);
    float v[32];
    qmv_load32<T>(reinterpret_cast<const T *>(a.x) + (int64_t)j * a.ldx + (int64_t)b * 32, v);
    const float d = qmv_quant_block(v);
    u32x4 w0, w1;
#pragma unroll
    for (int q = 0; q < 8; q++) {
        uint32_t word = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) word |= ((uint32_t)(int32_t)v[4 * q + i] & 255u) << (8 * i);
        if (q < 4) w0[q] = word;
        else w1[q - 4] = word;
    }
    u32x4 *dst = reinterpret_cast<u32x4 *>(a.quants + (int64_t)j * a.q_ld + (int64_t)b * 32);
    dst[0] = w0;
    dst[1] = w1;
    a.scales[(int64_t)j * a.nb + b] = d;
}

extern "C" __global__ __launch_bounds__(CUCA_BLOCK) void cuca_q8_acts_f32(Q8ActsArgs a) { q8_acts_body<float>(a); }
extern "C" __global__ __launch_bounds__(CUCA_BLOCK) void cuca_q8_acts_f16(Q8ActsArgs a) { q8_acts_body<_Float16>(a); }

// Bytes of LDS a qmv workgroup needs for nbp (padded) blocks and MT rows:
// the expanded rows, their scales, per wave dw * dx of a group and the sums
// of QMV_NT tasks.
#define QMV_LDS_BYTES(MT, NBP, G)                                                          \
    ((MT) * 16 * ((NBP) + 2) * 8 + (MT) * (NBP) * 4 + QMV_WAVES * (MT) * 2 * 4 * (G) * 4 +  \
     QMV_WAVES * QMV_NT * (MT) * 2 * 4 * 4)

// The (f16 pair, C) entries of lane l of a block whose quants are q.
template <int FMT>
__device__ static inline void qmv_expand(qmm_u2 *xe, int xstr, int j, int b, const float (&q)[32]) {
    using F = QFmt<FMT>;
    const qmm_h2 negk = {(_Float16)(-F::K), (_Float16)(-F::K)};
#pragma unroll
    for (int l = 0; l < 16; l++) {
        const uint32_t xp = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(q[l], q[l + 16]));
        const float cc = __builtin_amdgcn_fdot2(__builtin_bit_cast(qmm_h2, xp), negk, 0.0f, false);
        xe[(j * 16 + l) * xstr + b] = qmm_u2{xp, __builtin_bit_cast(uint32_t, cc)};
    }
}

// One ring slot: the lane's 16-byte chunk of group g and the aligned pair
// of f16 scales that holds block l's (lanes l >= G read block l % G's;
// unused), picked by qmv_scale.  Loads are unconditional (a row or task
// past the end reads a valid row, whose results are never used), so the
// compiler's wait counts see every load; a whole dword keeps the register
// free of the zero-extension a 16-bit load would carry through the ring.
template <int FMT>
__device__ static inline void qmv_load(const uint8_t *w, int g, int l, u32x4 &chunk, uint32_t &sc) {
    using F = QFmt<FMT>;
    const uint8_t *grp = w + (int64_t)g * F::GB;
    chunk = *reinterpret_cast<const u32x4 *>(grp + F::SCB + 16 * l);
    sc = *reinterpret_cast<const uint32_t *>(grp + 4 * ((l % F::G) >> 1));
}
__device__ static inline float qmv_scale(uint32_t pair, int l) { return qmv_h2f(pair >> (16 * (l & 1))); }

// MODE 0: quantised rows (a.quants / a.scales), dense; 3: dense rows of
// a.x; 1: MoE up; 2: MoE down.  TX: the activation type (modes 1-3); TO:
// the output type.
template <int FMT, int MT, bool GLU, int ACT, typename TX, typename TO, int MODE>
__device__ static inline void qmv_body(const QmvArgs &a) {
    using F = QFmt<FMT>;
    constexpr int G = F::G;
    constexpr bool MOE = MODE == 1 || MODE == 2;
    extern __shared__ __attribute__((aligned(16))) unsigned char qmv_lds[];
    const int xstr = a.nbp + 2;
    qmm_u2 *xe = reinterpret_cast<qmm_u2 *>(qmv_lds);
    float *xsc = reinterpret_cast<float *>(xe + MT * 16 * xstr);
    float *sall = xsc + MT * a.nbp;
    // wave-uniform values are made scalar (readfirstlane), so that the
    // stream's loops are scalar loops and its wait counts exact
    const int tid = threadIdx.x, lt = tid % CUCA_WAVE;
    const int wave = __builtin_amdgcn_readfirstlane(tid / CUCA_WAVE);

    // the tile's rows and weights; the wave's tasks first, first + step, ... < tend
    const uint8_t *wm = a.w, *um = a.w_up;
    int p0 = 0, np = a.m, first, step, tend;
    if constexpr (MOE) {
        const int tile = blockIdx.x / a.splits, split = blockIdx.x - tile * a.splits;
        int e, q0, q1;
        if (!moe_tile_lookup<MT>(a.offsets, a.n_experts, a.max_pairs, tile, &e, &q0, &q1)) return;
        e = __builtin_amdgcn_readfirstlane(e);
        p0 = __builtin_amdgcn_readfirstlane(q0);
        np = __builtin_amdgcn_readfirstlane(q1) - p0;
        wm = a.w + (int64_t)e * a.w_estride;
        um = GLU ? a.w_up + (int64_t)e * a.w_estride : nullptr;
        const int t0 = split * a.tps;
        first = t0 + wave;
        step = QMV_WAVES;
        tend = min(a.ntask, t0 + a.tps);
    } else {
        first = blockIdx.x * QMV_WAVES + wave;
        step = gridDim.x * QMV_WAVES;
        tend = a.ntask;
    }

    // expand the tile's rows: (f16 pair, C) per (row, lane, block), scales
    if constexpr (MODE == 0) {
        const qmm_h2 negk = {(_Float16)(-F::K), (_Float16)(-F::K)};
        for (int e = tid; e < MT * a.nbp * 16; e += QMV_WAVES * CUCA_WAVE) {
            const int j = e / (a.nbp * 16), rem = e - j * (a.nbp * 16), b = rem >> 4, l = rem & 15;
            uint32_t xp = 0u;
            float cc = 0.0f;
            if (j < a.m && b < a.nb) {
                const int8_t *q = a.quants + (int64_t)j * a.q_ld + (int64_t)b * 32;
                xp = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz((float)q[l], (float)q[l + 16]));
                cc = __builtin_amdgcn_fdot2(__builtin_bit_cast(qmm_h2, xp), negk, 0.0f, false);
            }
            xe[(j * 16 + l) * xstr + b] = qmm_u2{xp, __builtin_bit_cast(uint32_t, cc)};
        }
        for (int e = tid; e < MT * a.nbp; e += QMV_WAVES * CUCA_WAVE) {
            const int j = e / a.nbp, b = e - j * a.nbp;
            xsc[e] = (j < a.m && b < a.nb) ? a.scales[(int64_t)j * a.nb + b] : 0.0f;
        }
    } else {
        for (int e = tid; e < MT * a.nbp; e += QMV_WAVES * CUCA_WAVE) {
            const int j = e / a.nbp, b = e - j * a.nbp;
            int64_t xr = -1;
            if (j < np && b < a.nb) {
                if (MODE == 1) {
                    const int t = a.pair_token[p0 + j];
                    if (t >= 0 && t < a.n_tokens) xr = (int64_t)t * a.ldx;
                    else if (b == 0) record_bad(a.status + CUCA_STATUS_MOE_PAIR, (uint32_t)(p0 + j), (uint32_t)t);
                } else {
                    xr = (int64_t)(p0 + j) * a.ldx;
                }
            }
            float v[32];
            float d = 0.0f;
            if (xr >= 0) {
                qmv_load32<TX>(reinterpret_cast<const TX *>(a.x) + xr + (int64_t)b * 32, v);
                d = qmv_quant_block(v);
            } else {
#pragma unroll
                for (int i = 0; i < 32; i++) v[i] = 0.0f;
            }
            qmv_expand<FMT>(xe, xstr, j, b, v);
            xsc[e] = d;
        }
    }
    __syncthreads();

    // which of the tile's rows have outputs (MoE up: a valid token)
    uint32_t jmask = 0;
#pragma unroll
    for (int j = 0; j < MT; j++) {
        bool v = j < np;
        if (MODE == 1 && v) {
            const int t = a.pair_token[p0 + j];
            v = t >= 0 && t < a.n_tokens;
        }
        jmask |= v ? 1u << j : 0u;
    }

    const int nt = first < tend ? (tend - first + step - 1) / step : 0;
    if (nt == 0) return;
    const int r = lt >> 4, l = lt & 15;
    float *S = sall + wave * (MT * 2 * 4 * G);                     // [MT][gate, up][4 rows][G]
    float *res = sall + QMV_WAVES * (MT * 2 * 4 * G) + wave * (QMV_NT * MT * 2 * 4); // [task][MT][g, u][4]
    // a task's weight rows (a row past the matrix reads row 0)
    auto row_off = [&](int ti) -> int64_t {
        const int row = (first + (ti < nt ? ti : nt - 1) * step) * 4 + r;
        return (int64_t)(row < a.rows ? row : 0) * a.row_bytes;
    };

    // chunks of QMV_NT tasks: the groups of a chunk's tasks stream through
    // the ring back to back; a task's sums go to LDS, and the chunk's
    // outputs are written after its stream (no stores inside the stream, so
    // the compiler's wait counts stay exact: one per slot)
    for (int c0 = 0; c0 < nt; c0 += QMV_NT) {
        // nothing outstanding when the ring starts (the last chunk's
        // stores included), so both paths into the stream's loop hold the
        // ring's loads only and each slot waits for exactly its own
        __builtin_amdgcn_s_waitcnt(0);
        const int cn = min(QMV_NT, nt - c0);
        const int total = cn * a.ng;
        u32x4 rg[QMV_D], ru[QMV_D];
        uint32_t sg[QMV_D], su[QMV_D];
        // load cursor (task lti, group lg) and its row offset
        int lti = c0, lg = 0;
        int64_t loff = row_off(lti);
#pragma unroll
        for (int i = 0; i < QMV_D; i++) {
            qmv_load<FMT>(wm + loff, lg, l, rg[i], sg[i]);
            if (GLU) qmv_load<FMT>(um + loff, lg, l, ru[i], su[i]);
            else { ru[i] = rg[i]; su[i] = 0u; }
            if (++lg == a.ng) { lg = 0; lti++; loff = row_off(lti); }
        }
        // consumption cursor (task cti of the chunk, group cg)
        int cti = 0, cg = 0;
        float acc[MT], accu[MT];
#pragma unroll
        for (int j = 0; j < MT; j++) { acc[j] = 0.0f; accu[j] = 0.0f; }
        for (int s0 = 0; s0 < total; s0 += QMV_D) {
#pragma unroll
            for (int i = 0; i < QMV_D; i++) {
                // whole rounds only (one path through the loop body, so the
                // wait counts are exact): past the stream's end a slot is
                // consumed with a scale product of exactly 0, which adds +-0
                // to every chain and leaves its bits as they are
                const bool live = s0 + i < total;
                // this wave's dw * dx for group cg (the odd Q4_0 blocks' dw / 16)
                if (l < G) {
#pragma unroll
                    for (int j = 0; j < MT; j++) {
                        const float dx = xsc[j * a.nbp + cg * G + l];
                        const float pg_ = F::scale(qmv_scale(sg[i], l), l) * dx;
                        S[((j * 2) * 4 + r) * G + l] = live ? pg_ : 0.0f;
                        if (GLU) {
                            const float pu_ = F::scale(qmv_scale(su[i], l), l) * dx;
                            S[((j * 2 + 1) * 4 + r) * G + l] = live ? pu_ : 0.0f;
                        }
                    }
                }
                __builtin_amdgcn_wave_barrier();
#pragma unroll
                for (int s1 = 0; s1 < G; s1 += 4) {
                    const int b0 = cg * G + s1;
                    uint32_t pg[4], pu[4];
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        pg[q] = F::pair(rg[i], s1 + q);
                        pu[q] = GLU ? F::pair(ru[i], s1 + q) : 0u;
                    }
#pragma unroll
                    for (int j = 0; j < MT; j++) {
                        const f32x4 s4 = *reinterpret_cast<const f32x4 *>(&S[((j * 2) * 4 + r) * G + s1]);
                        f32x4 u4 = s4;
                        if (GLU) u4 = *reinterpret_cast<const f32x4 *>(&S[((j * 2 + 1) * 4 + r) * G + s1]);
                        const u32x4 x01 = *reinterpret_cast<const u32x4 *>(&xe[(j * 16 + l) * xstr + b0]);
                        const u32x4 x23 = *reinterpret_cast<const u32x4 *>(&xe[(j * 16 + l) * xstr + b0 + 2]);
                        const uint32_t xp[4] = {x01.x, x01.z, x23.x, x23.z};
                        const uint32_t xc[4] = {x01.y, x01.w, x23.y, x23.w};
#pragma unroll
                        for (int q = 0; q < 4; q++) {
                            const float cc = __builtin_bit_cast(float, xc[q]);
                            acc[j] = acc[j] + qmm_dot(pg[q], xp[q], cc) * s4[q];
                            if (GLU) accu[j] = accu[j] + qmm_dot(pu[q], xp[q], cc) * u4[q];
                        }
                    }
#pragma unroll
                    for (int j = 0; j < MT; j++) {
                        asm volatile("" : "+v"(acc[j]));
                        if (GLU) asm volatile("" : "+v"(accu[j]));
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
                __builtin_amdgcn_wave_barrier();
                // refill this slot from the load cursor
                qmv_load<FMT>(wm + loff, lg, l, rg[i], sg[i]);
                if (GLU) qmv_load<FMT>(um + loff, lg, l, ru[i], su[i]);
                if (++lg == a.ng) { lg = 0; lti++; loff = row_off(lti); }
                // the task's last group: its sums to LDS
                if (live && ++cg == a.ng) {
#pragma unroll
                    for (int j = 0; j < MT; j++) {
                        const float o = qmm_hsum(acc[j]);
                        const float u = GLU ? qmm_hsum(accu[j]) : 0.0f;
                        if (l == 0) {
                            res[((cti * MT + j) * 2) * 4 + r] = o;
                            if (GLU) res[((cti * MT + j) * 2 + 1) * 4 + r] = u;
                        }
                        acc[j] = 0.0f;
                        accu[j] = 0.0f;
                    }
                    cg = 0;
                    cti++;
                }
            }
        }
        __builtin_amdgcn_wave_barrier();
        // the chunk's outputs: lane e takes (task, act row, weight row)
        for (int e = lt; e < cn * MT * 4; e += CUCA_WAVE) {
            const int ti = e / (MT * 4), j = (e / 4) % MT, rr = e % 4;
            const int row = (first + (c0 + ti) * step) * 4 + rr;
            if (row >= a.rows || !((jmask >> j) & 1u)) continue;
            float o = res[((ti * MT + j) * 2) * 4 + rr];
            if (GLU) {
                float gg = o, u = res[((ti * MT + j) * 2 + 1) * 4 + rr];
                if (a.clamp > 0.0f) { // Glu::apply's clamp (cpu.rs:364-368)
                    gg = fminf(gg, a.clamp);
                    u = fminf(fmaxf(u, -a.clamp), a.clamp);
                }
                o = (ACT == 0 ? act_silu(gg) : act_gelu_tanh(gg)) * u;
            } else if (!MOE && a.cap_flags) { // cap_logits (cpu.rs:2603-2617)
                if (a.cap_flags & 1) o = o * a.mul1 + 0.0f;
                if (a.cap_flags & 2) o = o * a.mul2 + 0.0f;
                if (a.cap_flags & 4) o = tanhf(o * a.softcap_inv + 0.0f) * a.softcap + 0.0f;
            }
            if (MODE == 2) // CpuExpert::add_picks: y * weight (cpu.rs:400-417)
                reinterpret_cast<float *>(a.out)[(int64_t)(p0 + j) * a.out_ld + row] = o * a.pair_weight[p0 + j];
            else
                reinterpret_cast<TO *>(a.out)[(int64_t)(p0 + j) * a.out_ld + row] = to_stored<TO>(o);
        }
        __builtin_amdgcn_wave_barrier();
    }
}

#define CUCA_QMV(NAME, ...)                                                                \
    extern "C" __global__ __launch_bounds__(QMV_WAVES * CUCA_WAVE) void NAME(QmvArgs a) {  \
        qmv_body<__VA_ARGS__>(a);                                                          \
    }
// mode 0 (quantised rows) and mode 3 (rows of x, type TN) for 1 or 2 rows
#define CUCA_QMV_SET(FN, FMT, MT, TN, T)                                                   \
    CUCA_QMV(cuca_qmv_##FN##_m##MT##_##TN, FMT, MT, false, 0, T, T, 0)                     \
    CUCA_QMV(cuca_qmv_glu_##FN##_silu_m##MT##_##TN, FMT, MT, true, 0, T, T, 0)             \
    CUCA_QMV(cuca_qmv_glu_##FN##_gelu_m##MT##_##TN, FMT, MT, true, 1, T, T, 0)             \
    CUCA_QMV(cuca_qmvx_##FN##_m##MT##_##TN, FMT, MT, false, 0, T, T, 3)                    \
    CUCA_QMV(cuca_qmvx_glu_##FN##_silu_m##MT##_##TN, FMT, MT, true, 0, T, T, 3)            \
    CUCA_QMV(cuca_qmvx_glu_##FN##_gelu_m##MT##_##TN, FMT, MT, true, 1, T, T, 3)
CUCA_QMV_SET(q4_0, 0, 1, f32, float)
CUCA_QMV_SET(q4_0, 0, 2, f32, float)
CUCA_QMV_SET(q8_0, 1, 1, f32, float)
CUCA_QMV_SET(q8_0, 1, 2, f32, float)
CUCA_QMV_SET(q4_0, 0, 1, f16, _Float16)
CUCA_QMV_SET(q4_0, 0, 2, f16, _Float16)
CUCA_QMV_SET(q8_0, 1, 1, f16, _Float16)
CUCA_QMV_SET(q8_0, 1, 2, f16, _Float16)
// MoE at decode: tiles of 1, 2 or 4 pairs
#define CUCA_QMV_MOE_SET(FN, FMT, MT, TN, T)                                               \
    CUCA_QMV(cuca_qmv_moe_up_##FN##_silu_m##MT##_##TN, FMT, MT, true, 0, T, T, 1)          \
    CUCA_QMV(cuca_qmv_moe_up_##FN##_gelu_m##MT##_##TN, FMT, MT, true, 1, T, T, 1)          \
    CUCA_QMV(cuca_qmv_moe_down_##FN##_m##MT##_##TN, FMT, MT, false, 0, T, float, 2)
CUCA_QMV_MOE_SET(q4_0, 0, 1, f32, float)
CUCA_QMV_MOE_SET(q4_0, 0, 2, f32, float)
CUCA_QMV_MOE_SET(q4_0, 0, 4, f32, float)
CUCA_QMV_MOE_SET(q8_0, 1, 1, f32, float)
CUCA_QMV_MOE_SET(q8_0, 1, 2, f32, float)
CUCA_QMV_MOE_SET(q8_0, 1, 4, f32, float)
CUCA_QMV_MOE_SET(q4_0, 0, 1, f16, _Float16)
CUCA_QMV_MOE_SET(q4_0, 0, 2, f16, _Float16)
CUCA_QMV_MOE_SET(q4_0, 0, 4, f16, _Float16)
CUCA_QMV_MOE_SET(q8_0, 1, 1, f16, _Float16)
CUCA_QMV_MOE_SET(q8_0, 1, 2, f16, _Float16)
CUCA_QMV_MOE_SET(q8_0, 1, 4, f16, _Float16)
