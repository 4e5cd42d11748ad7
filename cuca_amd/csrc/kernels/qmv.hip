// qmv.hip -- the decode GEMV of the CPU engine's quantized matmul (qmm.rs)
// on gfx950: the same bits as qmm.hip, for one or two activation rows,
// shaped for the latency of a decode step.
//
// The activations are quantised once per call (cuca_q8_acts_*: Acts::new,
// qmm.rs:1217-1343, one thread per 32 values) rather than by every
// workgroup.  A workgroup expands its tile's quants for the whole row length
// into LDS once (the f16 pair and C of qmm.hip per (row, lane, block), and
// the block scales), then its four waves run independently: a wave's task is
// four weight rows x sixteen lanes, each thread one chain over all blocks.
// Per group of G blocks a wave stages dw * dx of its four rows in its own
// LDS area (no workgroup barrier) and runs the chains; eight groups of
// weights per wave are kept in flight in a register ring.  Workgroups are
// persistent (a grid-stride loop over the tasks), so a large matrix (the LM
// head) pays the expansion once per workgroup.
#include "common.h"

#define QMV_WAVES 4
#define QMV_D 8 // weight groups in flight per wave

__device__ static inline float qmv_h2f(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// Acts::new for MIN_NONE: one thread per (row, block).
template <typename T> __device__ static inline void q8_acts_body(const Q8ActsArgs &a) {
    const int64_t t = (int64_t)blockIdx.x * CUCA_BLOCK + threadIdx.x;
    if (t >= (int64_t)a.m * a.nb) return;
    const int j = (int)(t / a.nb), b = (int)(t - (int64_t)j * a.nb);
    const T *src = reinterpret_cast<const T *>(a.x) + (int64_t)j * a.ldx + (int64_t)b * 32;
    float v[32];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        float e[8];
        qmm_load8<T>(src + 8 * q, e);
#pragma unroll
        for (int i = 0; i < 8; i++) v[8 * q + i] = e[i];
    }
    float amax = 0.0f;
#pragma unroll
    for (int e = 0; e < 32; e++) amax = fmaxf(amax, fabsf(v[e]));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    u32x4 w0, w1;
#pragma unroll
    for (int q = 0; q < 8; q++) {
        uint32_t word = 0;
#pragma unroll
        for (int i = 0; i < 4; i++)
            word |= ((uint32_t)(int32_t)qmm_quant(v[4 * q + i] * id) & 255u) << (8 * i);
        if (q < 4) w0[q] = word;
        else w1[q - 4] = word;
    }
    u32x4 *dst = reinterpret_cast<u32x4 *>(a.quants + (int64_t)j * a.q_ld + (int64_t)b * 32);
    dst[0] = w0;
    dst[1] = w1;
    a.scales[(int64_t)j * a.nb + b] = (float)(_Float16)d;
}

extern "C" __global__ __launch_bounds__(CUCA_BLOCK) void cuca_q8_acts_f32(Q8ActsArgs a) { q8_acts_body<float>(a); }
extern "C" __global__ __launch_bounds__(CUCA_BLOCK) void cuca_q8_acts_f16(Q8ActsArgs a) { q8_acts_body<_Float16>(a); }

// Bytes of LDS a qmv workgroup needs for nbp (padded) blocks and MT rows.
#define QMV_LDS_BYTES(MT, NBP, G) \
    ((MT) * 16 * ((NBP) + 2) * 8 + (MT) * (NBP) * 4 + QMV_WAVES * (MT) * 2 * 4 * (G) * 4)

// One ring slot: the lane's 16-byte chunk of group g and the scale of
// block l of the group (lanes l >= G read block l % G's; unused).  The
// loads are unconditional -- a row past the matrix reads row 0, whose
// results are never written -- so the loop body has no branches and the
// compiler's wait counts see every load of the ring.
template <int FMT>
__device__ static inline void qmv_load(const uint8_t *w, int g, int l, u32x4 &chunk, uint32_t &sc) {
    using F = QFmt<FMT>;
    const uint8_t *grp = w + (int64_t)g * F::GB;
    chunk = *reinterpret_cast<const u32x4 *>(grp + F::SCB + 16 * l);
    sc = *reinterpret_cast<const uint16_t *>(grp + 2 * (l % F::G));
}

template <int FMT, int MT, bool GLU, int ACT, typename TO>
__device__ static inline void qmv_body(const QmvArgs &a) {
    using F = QFmt<FMT>;
    constexpr int G = F::G;
    extern __shared__ __attribute__((aligned(16))) unsigned char qmv_lds[];
    const int xstr = a.nbp + 2;
    qmm_u2 *xe = reinterpret_cast<qmm_u2 *>(qmv_lds);
    float *xsc = reinterpret_cast<float *>(xe + MT * 16 * xstr);
    float *sall = xsc + MT * a.nbp;
    const int tid = threadIdx.x, wave = tid / CUCA_WAVE, lt = tid % CUCA_WAVE;

    // expand the tile's quants: (f16 pair, C) per (row, lane, block)
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
    __syncthreads();

    const int r = lt >> 4, l = lt & 15;
    float *S = sall + wave * (MT * 2 * 4 * G); // [MT][gate, up][4 rows][G]
    for (int t = blockIdx.x * QMV_WAVES + wave; t < a.ntask; t += gridDim.x * QMV_WAVES) {
        const int row = t * 4 + r;
        const bool rv = row < a.rows;
        const uint8_t *wr = a.w + (int64_t)(rv ? row : 0) * a.row_bytes;
        const uint8_t *ur = GLU ? a.w_up + (int64_t)(rv ? row : 0) * a.row_bytes : nullptr;
        u32x4 rg[QMV_D], ru[QMV_D];
        uint32_t sg[QMV_D], su[QMV_D];
#pragma unroll
        for (int i = 0; i < QMV_D; i++) {
            rg[i] = u32x4{0u, 0u, 0u, 0u};
            ru[i] = rg[i];
            sg[i] = 0u;
            su[i] = 0u;
        }
        // groups past the row's end (the last round of the ring) load and
        // read the last group again and use a scale product of exactly 0: a
        // finite integer dot times 0 adds +-0, which leaves every chain's
        // bits as they are.
#pragma unroll
        for (int i = 0; i < QMV_D; i++) {
            const int gi = i < a.ng ? i : a.ng - 1;
            qmv_load<FMT>(wr, gi, l, rg[i], sg[i]);
            if (GLU) qmv_load<FMT>(ur, gi, l, ru[i], su[i]);
        }
        float acc[MT], accu[MT];
#pragma unroll
        for (int j = 0; j < MT; j++) { acc[j] = 0.0f; accu[j] = 0.0f; }
        for (int g0 = 0; g0 < a.ng; g0 += QMV_D) {
#pragma unroll
            for (int i = 0; i < QMV_D; i++) {
                const int g = g0 + i;
                const bool live = g < a.ng;
                const int ge = live ? g : a.ng - 1;
                // this wave's dw * dx for group g (the odd Q4_0 blocks' dw / 16)
                if (l < G) {
#pragma unroll
                    for (int j = 0; j < MT; j++) {
                        const float dx = xsc[j * a.nbp + ge * G + l];
                        const float pg_ = F::scale(qmv_h2f(sg[i]), l) * dx;
                        S[((j * 2) * 4 + r) * G + l] = live ? pg_ : 0.0f;
                        if (GLU) {
                            const float pu_ = F::scale(qmv_h2f(su[i]), l) * dx;
                            S[((j * 2 + 1) * 4 + r) * G + l] = live ? pu_ : 0.0f;
                        }
                    }
                }
                __builtin_amdgcn_wave_barrier();
#pragma unroll
                for (int s0 = 0; s0 < G; s0 += 4) {
                    const int b0 = ge * G + s0;
                    uint32_t pg[4], pu[4];
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        pg[q] = F::pair(rg[i], s0 + q);
                        pu[q] = GLU ? F::pair(ru[i], s0 + q) : 0u;
                    }
#pragma unroll
                    for (int j = 0; j < MT; j++) {
                        const f32x4 s4 = *reinterpret_cast<const f32x4 *>(&S[((j * 2) * 4 + r) * G + s0]);
                        f32x4 u4 = s4;
                        if (GLU) u4 = *reinterpret_cast<const f32x4 *>(&S[((j * 2 + 1) * 4 + r) * G + s0]);
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
                // refill this slot with group g + D (or the last group again)
                const int gn = g + QMV_D < a.ng ? g + QMV_D : a.ng - 1;
                qmv_load<FMT>(wr, gn, l, rg[i], sg[i]);
                if (GLU) qmv_load<FMT>(ur, gn, l, ru[i], su[i]);
            }
        }
#pragma unroll
        for (int j = 0; j < MT; j++) {
            float o = qmm_hsum(acc[j]);
            if (GLU) {
                float gg = o, u = qmm_hsum(accu[j]);
                if (a.clamp > 0.0f) { // Glu::apply's clamp (cpu.rs:364-368)
                    gg = fminf(gg, a.clamp);
                    u = fminf(fmaxf(u, -a.clamp), a.clamp);
                }
                o = (ACT == 0 ? act_silu(gg) : act_gelu_tanh(gg)) * u;
            } else if (a.cap_flags) { // cap_logits (cpu.rs:2603-2617)
                if (a.cap_flags & 1) o = o * a.mul1 + 0.0f;
                if (a.cap_flags & 2) o = o * a.mul2 + 0.0f;
                if (a.cap_flags & 4) o = tanhf(o * a.softcap_inv + 0.0f) * a.softcap + 0.0f;
            }
            if (l == 0 && rv && j < a.m) reinterpret_cast<TO *>(a.out)[(int64_t)j * a.out_ld + row] = (TO)o;
        }
    }
}

#define CUCA_QMV(NAME, ...)                                                                \
    extern "C" __global__ __launch_bounds__(QMV_WAVES * CUCA_WAVE) void NAME(QmvArgs a) {  \
        qmv_body<__VA_ARGS__>(a);                                                          \
    }
#define CUCA_QMV_SET(FN, FMT, MT, TN, TO)                                                  \
    CUCA_QMV(cuca_qmv_##FN##_m##MT##_##TN, FMT, MT, false, 0, TO)                          \
    CUCA_QMV(cuca_qmv_glu_##FN##_silu_m##MT##_##TN, FMT, MT, true, 0, TO)                  \
    CUCA_QMV(cuca_qmv_glu_##FN##_gelu_m##MT##_##TN, FMT, MT, true, 1, TO)
CUCA_QMV_SET(q4_0, 0, 1, f32, float)
CUCA_QMV_SET(q4_0, 0, 2, f32, float)
CUCA_QMV_SET(q8_0, 1, 1, f32, float)
CUCA_QMV_SET(q8_0, 1, 2, f32, float)
CUCA_QMV_SET(q4_0, 0, 1, f16, _Float16)
CUCA_QMV_SET(q4_0, 0, 2, f16, _Float16)
CUCA_QMV_SET(q8_0, 1, 1, f16, _Float16)
CUCA_QMV_SET(q8_0, 1, 2, f16, _Float16)
