// qmd.hip -- the decode matmul of one activation row: the CPU engine's
// quantized matmul (QmmWeight, qmm.rs) bit for bit, as qmm.hip computes it,
// shaped for m = 1 at the layer shapes of a decode step.
//
// The arithmetic is qmm.hip's: sixteen lane chains per weight row, lane l
// adding block by block, in row order, (float)P * (dw * dx) with the
// product and the sum rounded separately, P the exact integer pair sum of
// v_dot2_f32_f16 over magic-number pairs; the fixed hsum tree at the end.
// Only the data movement differs:
//
//  * One wave is four weight rows x 16 lanes, each thread one chain over
//    the whole row; a workgroup is four waves and the grid holds every row
//    (no persistent loop): at one activation row the chains are the only
//    parallelism, so the chip needs all of them resident.
//  * Weight groups (G blocks: the lane's 16-byte chunk and the dword with
//    its block's f16 scale) stream through a ring of D slots in registers.
//    The first D loads are issued before anything else, so the workgroup's
//    quantisation of the activation row runs under their latency; after
//    that every consumed slot is refilled with the group D ahead.  D
//    divides the group count and the last round is peeled off, so every
//    load is used and the loop body has one path (exact wait counts).
//  * The activation row is quantised once per workgroup into LDS, as
//    qmv.hip does (Acts::new, qmm.rs:1217-1343): per (lane, block) the f16
//    pair and the dot's constant C, and the block scales.
//  * dw * dx: lane l of each row computes the product of block l of the
//    group, and the chain of block b reads it from lane b of its row by a
//    DPP row broadcast folded into the multiply (v_mul_f32_dpp
//    row_newbcast:b), so the per-block scale costs no LDS traffic and no
//    instruction of its own.  Per block and chain that leaves the pair
//    (one v_bfi_b32; Q4_0 adds a shift per four blocks), the dot, the
//    multiply and the add, and one 8-byte LDS read shared by the chains a
//    thread runs (gate and up for the GLU).
#include "common.h"

template <int V> struct QmdInt { static constexpr int value = V; };
template <int I, int N, typename Fn> __device__ static inline void qmd_for(Fn &&fn) {
    if constexpr (I < N) {
        fn(QmdInt<I>{});
        qmd_for<I + 1, N>(fn);
    }
}

// The value of v in lane B of each row of 16 lanes (DPP row_newbcast,
// gfx90a and later); the compiler folds it into the instruction that reads
// it.
template <int B> __device__ static inline float qmd_bcast(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x150 + B, 0xf,
                                                                 0xf, false));
}

#define QMD_RSRC_W3 0x00020000 // buffer resource word 3 (raw buffer, 32-bit data)

// One ring slot: the lane's chunk of a group and the dword holding the
// f16 scale of block l (gate; up for the GLU).
struct QmdSlot {
    u32x4 w, u;
    uint32_t sw, su;
};

// Bytes of LDS: the expanded row (16 lanes x (ng G + 2) entries of 8
// bytes) and its block scales (padded by a group: the stream reads one
// group ahead, and up to eight entries past a lane's row, which stay inside
// the allocation).
#define QMD_LDS_BYTES(NG, G) (16 * ((NG) * (G) + 2) * 8 + ((NG) + 1) * (G) * 4)

// The residual add + RMSNorm prologue (RN kernels): the row x' = x + rs *
// branch, as cuca_hip_add_rmsnorm's vector kernel computes it, and h =
// rms(x') with that kernel's bits.  Its sum of squares is per thread (TPR
// threads of NCH chunks of CN values: chunks li, li + TPR, ..., values in
// order), a butterfly over the thread's wave (or its group of TPR < 64
// lanes) and, for TPR > 64, the waves' sums added in wave order.  Thread
// tid here plays the kernel's threads tid, tid + 256, ...: their lane in a
// wave is tid's own, so the butterfly runs on the same partners.  x' is
// staged in LDS (over the expanded row, which is written only after the
// last read of it) for the per-thread sums.  xv holds x on entry (bv the
// branch, wv the weights) and h on exit, as the matmul reads h stored as T.
//
// Fast path, for one chunk a thread and rows of whole waves (per == 1, TPR
// >= 64: hidden 256 .. 4096 f32, 512 .. 8192 f16): the sums come straight
// from the registers, with no LDS staging and one barrier.  An f16 item is
// one chunk, so item i is the kernel's thread i, in the same lane: the
// butterfly is group_sum<64> of the item's sum.  An f32 item holds chunks
// 2i and 2i + 1, the kernel's lanes 2 (q % 32) + e of its wave i / 32 (q
// = this lane): its partners at distance 32, 16, 8, 4, 2 are this lane's
// at 16, 8, 4, 2, 1 (same e), and its last step (distance 1) adds the
// item's two sums.  Measured on MI355X (Llama-3-8B decode, batch 1): the
// LDS-staged form made the fused kernels about 2 us slower each.
template <typename T, int NI, int BT>
__device__ static inline void qmd_rms_prologue(const QmmArgs &a, float (&xv)[NI][8], const float (&bv)[NI][8],
                                               const float (&wv)[NI][8], float *vl) {
    __shared__ float rn_red[16];
    constexpr int CN = Chunk<T>::N;
    const int tid = threadIdx.x, lane = tid & (CUCA_WAVE - 1);
    const int nitems = 4 * a.nb; // 8 values an item
    const bool w0 = blockIdx.x == 0;
    const int H = a.nb * 32, nch = H / CN, tpr = a.rn_tpr, per = a.rn_per;
    const bool fast = per == 1 && tpr >= CUCA_WAVE && NI * BT * (8 / CN) >= tpr;
#pragma unroll
    for (int it = 0; it < NI; it++) {
        const int item = it * BT + tid;
        if (item < nitems) {
#pragma unroll
            for (int e = 0; e < 8; e++) {
                float v = xv[it][e];
                if (a.rn_branch) {
                    float b = bv[it][e];
                    if (a.rn_rs != 1.0f) b = b * a.rn_rs + 0.0f; // `scaled`: branch.affine(rs, 0)
                    v = Chunk<T>::as_stored(v + b);
                }
                xv[it][e] = v;
                if (!fast) vl[8 * item + e] = v;
            }
            if (w0 && a.rn_x_out) {
                T *xo = reinterpret_cast<T *>(a.rn_x_out) + 8 * (int64_t)item;
#pragma unroll
                for (int e = 0; e < 8; e++) xo[e] = to_stored<T>(xv[it][e]);
            }
        }
    }
    if (fast) {
#pragma unroll
        for (int it = 0; it < NI; it++) {
            const int item = it * BT + tid;
            if constexpr (CN == 8) {
                float ss = 0.0f;
#pragma unroll
                for (int e = 0; e < 8; e++) ss += xv[it][e] * xv[it][e];
                ss = group_sum<CUCA_WAVE>(ss);
                const int nw = item / CUCA_WAVE;
                if (lane == 0 && nw < tpr / CUCA_WAVE) rn_red[nw] = ss;
            } else {
                float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
                for (int e = 0; e < 4; e++) s0 += xv[it][e] * xv[it][e];
#pragma unroll
                for (int e = 4; e < 8; e++) s1 += xv[it][e] * xv[it][e];
                s0 = xor_add<16>(s0); s1 = xor_add<16>(s1);
                s0 = xor_add<8>(s0); s1 = xor_add<8>(s1);
                s0 = xor_add<4>(s0); s1 = xor_add<4>(s1);
                s0 = xor_add<2>(s0); s1 = xor_add<2>(s1);
                s0 = xor_add<1>(s0); s1 = xor_add<1>(s1);
                const float ws = s0 + s1;
                const int nw = item / (CUCA_WAVE / 2);
                if ((lane & 31) == 0 && nw < tpr / CUCA_WAVE) rn_red[nw] = ws;
            }
        }
        __syncthreads();
    } else { // x' staged in LDS
        __syncthreads();
        // the kernel's per-thread sums, then its butterfly
        auto thread_ss = [&](int li) {
            float ss = 0.0f;
            for (int k = 0; k < per; k++) {
                const int c = li + k * tpr;
                if (c < nch) {
#pragma unroll
                    for (int i = 0; i < CN; i++) ss += vl[c * CN + i] * vl[c * CN + i];
                }
            }
            return ss;
        };
        if (tpr <= CUCA_WAVE) {
            if (tid < CUCA_WAVE) { // wave 0: lanes below tpr are the kernel's threads
                const float ss = group_sum_rt(tid < tpr ? thread_ss(tid) : 0.0f, tpr);
                if (tid == 0) rn_red[0] = ss;
            }
        } else {
            for (int j = 0; j < 1024 / BT; j++) {
                const int li = tid + j * BT; // wave-uniform test: tpr is a multiple of 64
                if (li < tpr) {
                    const float ss = group_sum<CUCA_WAVE>(thread_ss(li));
                    if (lane == 0) rn_red[li / CUCA_WAVE] = ss;
                }
            }
        }
        __syncthreads(); // also: every read of vl is done
    }
    float s;
    if (tpr <= CUCA_WAVE) {
        s = rn_red[0];
    } else {
        s = 0.0f;
        for (int i = 0; i < tpr / CUCA_WAVE; i++) s += rn_red[i];
    }
    const float inv = 1.0f / sqrtf(s / (float)H + a.rn_eps);
#pragma unroll
    for (int it = 0; it < NI; it++) {
        const int item = it * BT + tid;
        if (item < nitems) {
#pragma unroll
            for (int e = 0; e < 8; e++) {
                float h = a.rn_w ? pin_f32(pin_f32(xv[it][e] * inv) * wv[it][e]) : pin_f32(xv[it][e] * inv);
                xv[it][e] = (float)to_stored<T>(h);
            }
            if (w0 && a.rn_h_out) {
                T *ho = reinterpret_cast<T *>(a.rn_h_out) + 8 * (int64_t)item;
#pragma unroll
                for (int e = 0; e < 8; e++) ho[e] = (T)xv[it][e];
            }
        }
    }
}

// MODE 0: plain (out[row], the LM head's cap when asked); 3: the Q|K|V
// projection with RoPE and the paged K/V store in the epilogue (qmm.hip's
// qmm_rope_kv_store).  D: ring slots; WB: waves a workgroup; NI:
// activation items (8 values) per thread, NI * 64 WB >= 4 ng G.  The grid
// is ceil(rows / (4 WB)) workgroups of 64 WB threads.  RN: the residual add
// + RMSNorm prologue.
template <typename T, int FMT, bool GLU, int ACT, int MODE, int D, int NI, int PF = 1, bool RN = false, int WB = 4>
__device__ static inline void qmd_body(const QmmArgs &a) {
    using F = QFmt<FMT>;
    constexpr int G = F::G;
    constexpr int BT = WB * CUCA_WAVE; // threads a workgroup
    extern __shared__ __attribute__((aligned(16))) unsigned char qmd_lds[];
    const int ng = a.ng, nbp = ng * G, xstr = nbp + 2;
    qmm_u2 *xe = reinterpret_cast<qmm_u2 *>(qmd_lds);
    float *xsc = reinterpret_cast<float *>(xe + 16 * xstr);
    const int tid = threadIdx.x, lt = tid & (CUCA_WAVE - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / CUCA_WAVE);
    const int r = lt >> 4, l = lt & 15;
    const int row = (blockIdx.x * WB + wave) * 4 + r;
    // a row past the matrix streams the last row; its result is not stored
    const int lrow = row < a.rows ? row : a.rows - 1;
    const uint32_t nrec = (uint32_t)((int64_t)a.rows * a.row_bytes);
    const __amdgpu_buffer_rsrc_t rw =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(a.w), 0, (int)nrec, QMD_RSRC_W3);
    const __amdgpu_buffer_rsrc_t ru =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(GLU ? a.w_up : a.w), 0, (int)nrec, QMD_RSRC_W3);
    const uint32_t rbase = (uint32_t)lrow * (uint32_t)a.row_bytes;
    const uint32_t vchunk = rbase + F::SCB + 16 * l;
    const uint32_t vscale = rbase + 4 * ((l % G) >> 1);

    // 1. The activation row's loads: item it * 256 + tid is values
    // 8 (item % 4) .. +7 of block item / 4 (zero past the row).
    const int nitems = 4 * nbp, sub = tid & 3;
    float xv[NI][8];
    // RN: the branch and the norm weights of the same values
    float bv[RN ? NI : 1][8], wv[RN ? NI : 1][8];
#pragma unroll
    for (int it = 0; it < NI; it++) {
        const int item = it * BT + tid, b = item >> 2;
        if (item < nitems && b < a.nb) {
            qmm_load8<T>(reinterpret_cast<const T *>(a.x) + (int64_t)b * 32 + sub * 8, xv[it]);
            if constexpr (RN) {
                if (a.rn_branch)
                    qmm_load8<T>(reinterpret_cast<const T *>(a.rn_branch) + (int64_t)b * 32 + sub * 8, bv[it]);
                if (a.rn_w) qmm_load8<float>(a.rn_w + (int64_t)b * 32 + sub * 8, wv[it]);
            }
        } else {
#pragma unroll
            for (int e = 0; e < 8; e++) xv[it][e] = 0.0f;
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    // 2. The ring's first D groups, issued behind the activations (loads
    // complete in order, so the quantisation below waits for its own loads
    // only) and in slot order, as the loop refills them (the loop's wait
    // counts, which merge this path with its own, then need no more than
    // the slot's own loads).  A refill past the row's last group (in the
    // round before the last) reads that group again, and is not consumed.
    QmdSlot ring[D];
    auto load = [&](QmdSlot &s, int g) {
        const int so = (g < ng ? g : ng - 1) * F::GB; // wave-uniform: the scalar offset
        s.w = __builtin_amdgcn_raw_buffer_load_b128(rw, vchunk, so, 0);
        s.sw = __builtin_amdgcn_raw_buffer_load_b32(rw, vscale, so, 0);
        if constexpr (GLU) {
            s.u = __builtin_amdgcn_raw_buffer_load_b128(ru, vchunk, so, 0);
            s.su = __builtin_amdgcn_raw_buffer_load_b32(ru, vscale, so, 0);
        }
    };
    qmd_for<0, D>([&](auto I) {
        load(ring[I.value], I.value);
        __builtin_amdgcn_sched_barrier(0);
    });
    if constexpr (RN) qmd_rms_prologue<T, NI, BT>(a, xv, bv, wv, reinterpret_cast<float *>(qmd_lds));

    // 3. Quantise (Acts::new, qmm.rs:1217-1240: the four threads of a block
    // share its maximum) and expand: per (lane, block) the f16 pair
    // (q[l], q[l+16]) and C = -K (q[l] + q[l+16]); the block scales.
    {
        const qmm_h2 negk = {(_Float16)(-F::K), (_Float16)(-F::K)};
        const bool low = sub < 2;
        const int base = 8 * (sub & 1) + (low ? 0 : 4);
#pragma unroll
        for (int it = 0; it < NI; it++) {
            const int item = it * BT + tid, b = item >> 2;
            float amax = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; e++) amax = fmaxf(amax, fabsf(xv[it][e]));
            amax = fmaxf(amax, xor_partner(amax, 1));
            amax = fmaxf(amax, xor_partner(amax, 2));
            const float d = amax / 127.0f;
            const float id = d != 0.0f ? 1.0f / d : 0.0f;
            uint32_t own[4], other[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                own[i] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(qmm_quant(xv[it][2 * i] * id),
                                                                                 qmm_quant(xv[it][2 * i + 1] * id)));
                other[i] = xor_partner_bits(own[i], 2);
            }
            if (item < nitems) {
                // threads 0/1 own elements 0-7 / 8-15, threads 2/3 16-23 /
                // 24-31; sub < 2 writes lanes 8s..8s+3, sub >= 2 lanes
                // 8s+4..8s+7 (s = sub & 1)
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const uint32_t lo = low ? own[q >> 1] : other[2 + (q >> 1)];
                    const uint32_t hi = low ? other[q >> 1] : own[2 + (q >> 1)];
                    const uint32_t xp = __builtin_amdgcn_perm(hi, lo, (q & 1) ? 0x07060302u : 0x05040100u);
                    const float cc = __builtin_amdgcn_fdot2(__builtin_bit_cast(qmm_h2, xp), negk, 0.0f, false);
                    xe[(base + q) * xstr + b] = qmm_u2{xp, __builtin_bit_cast(uint32_t, cc)};
                }
                if (sub == 0) xsc[b] = b < a.nb ? (float)(_Float16)d : 0.0f;
            }
        }
        if (tid < G) xsc[nbp + tid] = 0.0f; // the group past the row
    }
    __syncthreads();

    // 4. The stream.  Lane l's scale is block l's of the group (the odd
    // Q4_0 blocks' dw / 16); the LDS operands of the next four blocks, and
    // the next group's dx, are read one step ahead.
    const int sh = 16 * (l & 1);
    const float kmul = (FMT == 0 && (l & 1)) ? 0.0625f : 1.0f;
    const qmm_u2 *xl = xe + l * xstr;
    const float *xsl = xsc + (l % G);
    constexpr int NS = G / 4; // steps of four blocks per group
    float acc = 0.0f, accu = 0.0f;
    // the LDS operands of the current step and, with PF = 2, the next
    u32x4 cx01 = *reinterpret_cast<const u32x4 *>(xl);
    u32x4 cx23 = *reinterpret_cast<const u32x4 *>(xl + 2);
    u32x4 px01 = cx01, px23 = cx23;
    if constexpr (PF == 2) {
        px01 = *reinterpret_cast<const u32x4 *>(xl + 4);
        px23 = *reinterpret_cast<const u32x4 *>(xl + 6);
    }
    float cdx = xsl[0];
    auto consume = [&](const QmdSlot &s, int g) {
        const float sg = (qmv_h2f(s.sw >> sh) * kmul) * cdx;
        const float su = GLU ? (qmv_h2f(s.su >> sh) * kmul) * cdx : 0.0f;
        cdx = xsl[(g + 1) * G];
        qmd_for<0, NS>([&](auto S4) {
            constexpr int b0 = 4 * S4.value;
            // the operands PF steps ahead (into the next group at its end)
            const qmm_u2 *xn = xl + g * G + b0 + 4 * PF;
            const u32x4 nx01 = *reinterpret_cast<const u32x4 *>(xn);
            const u32x4 nx23 = *reinterpret_cast<const u32x4 *>(xn + 2);
            const uint32_t xp[4] = {cx01.x, cx01.z, cx23.x, cx23.z};
            const uint32_t xc[4] = {cx01.y, cx01.w, cx23.y, cx23.w};
            float pg[4], pu[4];
            qmd_for<0, 4>([&](auto Q) {
                constexpr int b = b0 + Q.value;
                const float cc = __builtin_bit_cast(float, xc[Q.value]);
                pg[Q.value] = qmm_dot(F::pair(s.w, b), xp[Q.value], cc);
                if constexpr (GLU) pu[Q.value] = qmm_dot(F::pair(s.u, b), xp[Q.value], cc);
            });
            // the dots, then the products into registers of their own, then
            // the sums: a DPP multiply waits two cycles for a register (its
            // operand or its destination) written just before it
            __builtin_amdgcn_sched_barrier(0);
            float qg[4], qu[4];
            qmd_for<0, 4>([&](auto Q) {
                constexpr int b = b0 + Q.value;
                qg[Q.value] = pg[Q.value] * qmd_bcast<b>(sg);
                if constexpr (GLU) qu[Q.value] = pu[Q.value] * qmd_bcast<b>(su);
            });
            __builtin_amdgcn_sched_barrier(0);
            qmd_for<0, 4>([&](auto Q) {
                acc = acc + qg[Q.value];
                if constexpr (GLU) accu = accu + qu[Q.value];
            });
            // pin these four blocks' arithmetic here (the chains are read
            // only at the end, so the compiler would sink it)
            asm volatile("" : "+v"(acc));
            if constexpr (GLU) asm volatile("" : "+v"(accu));
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (PF == 2) {
                cx01 = px01;
                cx23 = px23;
                px01 = nx01;
                px23 = nx23;
            } else {
                cx01 = nx01;
                cx23 = nx23;
            }
        });
    };
    const int nr = (ng + D - 1) / D;
    for (int R = 0; R + 1 < nr; R++) {
        qmd_for<0, D>([&](auto I) {
            consume(ring[I.value], R * D + I.value);
            load(ring[I.value], (R + 1) * D + I.value);
        });
    }
    const int rem = ng - (nr - 1) * D; // 1..D groups in the last round
    qmd_for<0, D>([&](auto I) {
        if (I.value < rem) consume(ring[I.value], (nr - 1) * D + I.value);
    });

    float o = qmm_hsum(acc);
    if constexpr (GLU) {
        float g = o, u = qmm_hsum(accu);
        if (a.clamp > 0.0f) { // Glu::apply's clamp (cpu.rs:364-368)
            g = fminf(g, a.clamp);
            u = fminf(fmaxf(u, -a.clamp), a.clamp);
        }
        o = (ACT == 0 ? act_silu(g) : act_gelu_tanh(g)) * u;
    } else if (MODE == 0 && a.cap_flags) { // cap_logits (cpu.rs:2603-2617)
        if (a.cap_flags & 1) o = o * a.mul1 + 0.0f;
        if (a.cap_flags & 2) o = o * a.mul2 + 0.0f;
        if (a.cap_flags & 4) o = tanhf(o * a.softcap_inv + 0.0f) * a.softcap + 0.0f;
    }
    if constexpr (MODE == 3) {
        qmm_rope_kv_store<T>(a, 0, true, 0, row, l, o);
    } else {
        if (l == 0 && row < a.rows) reinterpret_cast<T *>(a.out)[row] = to_stored<T>(o);
    }
}

#define CUCA_QMD(NAME, ...)                                                                \
    extern "C" __global__ __launch_bounds__(CUCA_BLOCK) void NAME(QmmArgs a) {             \
        qmd_body<__VA_ARGS__>(a);                                                          \
    }
// [act dtype][format][row length: n2 for k <= 4096, n8 for k <= 16384]:
// plain, SwiGLU, GeGLU-tanh, Q|K|V with RoPE and the K/V store.  Ring
// depths DP (plain) / DG (GLU, two matrices a slot) measured best at the
// Llama-3-8B decode shapes.
#define CUCA_QMD_SET(TN, T, FN, FMT, NI, DP, DG)                                           \
    CUCA_QMD(cuca_qmd_##TN##_##FN##_n##NI, T, FMT, false, 0, 0, DP, NI)                    \
    CUCA_QMD(cuca_qmd_glu_##TN##_##FN##_silu_n##NI, T, FMT, true, 0, 0, DG, NI)            \
    CUCA_QMD(cuca_qmd_glu_##TN##_##FN##_gelu_n##NI, T, FMT, true, 1, 0, DG, NI)            \
    CUCA_QMD(cuca_qmd_rope_kv_##TN##_##FN##_n##NI, T, FMT, false, 0, 3, DP, NI)
// The same with the residual add + RMSNorm prologue (_rn).
#define CUCA_QMD_RN_SET(TN, T, FN, FMT, NI, DP, DG)                                        \
    CUCA_QMD(cuca_qmd_##TN##_##FN##_n##NI##_rn, T, FMT, false, 0, 0, DP, NI, 1, true)       \
    CUCA_QMD(cuca_qmd_glu_##TN##_##FN##_silu_n##NI##_rn, T, FMT, true, 0, 0, DG, NI, 1, true) \
    CUCA_QMD(cuca_qmd_glu_##TN##_##FN##_gelu_n##NI##_rn, T, FMT, true, 1, 0, DG, NI, 1, true) \
    CUCA_QMD(cuca_qmd_rope_kv_##TN##_##FN##_n##NI##_rn, T, FMT, false, 0, 3, DP, NI, 1, true)
// The GLU as workgroups of 8 waves (32 rows; NI8 items a thread for rows
// to 4096 / 16384 values, named n2 / n8 as their 4-wave counterparts): for
// matrices of at least 32 rows per compute unit.  Every workgroup quantises
// (and, _rn, normalises) the whole activation row, so halving the
// workgroups per compute unit halves that work on each SIMD.  Measured on
// MI355X (Llama-3-8B gate/up, Q4_0, batch-1 decode step): 64.7 -> 62.4 us
// per layer with the norm in the prologue, 65.6-66.6 -> 63.5-64.8 without.
#define CUCA_QMD_W8(NAME, ...)                                                             \
    extern "C" __global__ __launch_bounds__(8 * CUCA_WAVE) void NAME(QmmArgs a) {          \
        qmd_body<__VA_ARGS__>(a);                                                          \
    }
#define CUCA_QMD_W8_SET(TN, T, FN, FMT, NI, NI8, DG)                                       \
    CUCA_QMD_W8(cuca_qmd_glu_##TN##_##FN##_silu_n##NI##w8, T, FMT, true, 0, 0, DG, NI8, 1, false, 8)   \
    CUCA_QMD_W8(cuca_qmd_glu_##TN##_##FN##_gelu_n##NI##w8, T, FMT, true, 1, 0, DG, NI8, 1, false, 8)   \
    CUCA_QMD_W8(cuca_qmd_glu_##TN##_##FN##_silu_n##NI##w8_rn, T, FMT, true, 0, 0, DG, NI8, 1, true, 8) \
    CUCA_QMD_W8(cuca_qmd_glu_##TN##_##FN##_gelu_n##NI##w8_rn, T, FMT, true, 1, 0, DG, NI8, 1, true, 8)
// The Q|K|V projection with the norm prologue as 8-wave workgroups, at any
// row count: the prologue is the larger share of its time, and halving the
// workgroups that repeat it paid even with compute units left idle (8B
// batch-1 step, 6144 rows in 192 workgroups: 61.7 -> 59.9 us per layer; the
// projection without the prologue gained nothing, so it keeps 4 waves).
// A plain matmul of at least 32 rows per compute unit (the LM head) as
// 8-wave workgroups, with or without the norm prologue (the final norm in
// front of the head): the 128256-row head at one row, Q4_0 55-59 -> 51 us
// (the decode GEMV stream took 59-60 us; Q8_0 88-89 us either way against
// its 101-103 us).
#define CUCA_QMD_W8_PLAIN(TN, T, FN, FMT, NI, NI8, DP)                                      \
    CUCA_QMD_W8(cuca_qmd_##TN##_##FN##_n##NI##w8, T, FMT, false, 0, 0, DP, NI8, 1, false, 8) \
    CUCA_QMD_W8(cuca_qmd_##TN##_##FN##_n##NI##w8_rn, T, FMT, false, 0, 0, DP, NI8, 1, true, 8)
#define CUCA_QMD_W8_QKV(TN, T, FN, FMT, NI, NI8, DP)                                        \
    CUCA_QMD_W8(cuca_qmd_rope_kv_##TN##_##FN##_n##NI##w8_rn, T, FMT, false, 0, 3, DP, NI8, 1, true, 8)
CUCA_QMD_SET(f32, float, q4_0, 0, 2, 4, 2)
CUCA_QMD_SET(f32, float, q4_0, 0, 8, 8, 2)
CUCA_QMD_SET(f32, float, q8_0, 1, 2, 8, 4)
CUCA_QMD_SET(f32, float, q8_0, 1, 8, 8, 4)
CUCA_QMD_SET(f16, _Float16, q4_0, 0, 2, 4, 2)
CUCA_QMD_SET(f16, _Float16, q4_0, 0, 8, 8, 2)
CUCA_QMD_SET(f16, _Float16, q8_0, 1, 2, 8, 4)
CUCA_QMD_SET(f16, _Float16, q8_0, 1, 8, 8, 4)
CUCA_QMD_RN_SET(f32, float, q4_0, 0, 2, 4, 2)
CUCA_QMD_RN_SET(f32, float, q4_0, 0, 8, 8, 2)
CUCA_QMD_RN_SET(f32, float, q8_0, 1, 2, 8, 4)
CUCA_QMD_RN_SET(f32, float, q8_0, 1, 8, 8, 4)
CUCA_QMD_RN_SET(f16, _Float16, q4_0, 0, 2, 4, 2)
CUCA_QMD_RN_SET(f16, _Float16, q4_0, 0, 8, 8, 2)
CUCA_QMD_RN_SET(f16, _Float16, q8_0, 1, 2, 8, 4)
CUCA_QMD_RN_SET(f16, _Float16, q8_0, 1, 8, 8, 4)
CUCA_QMD_W8_SET(f32, float, q4_0, 0, 2, 1, 2)
CUCA_QMD_W8_SET(f32, float, q4_0, 0, 8, 4, 2)
CUCA_QMD_W8_SET(f32, float, q8_0, 1, 2, 1, 4)
CUCA_QMD_W8_SET(f32, float, q8_0, 1, 8, 4, 4)
CUCA_QMD_W8_SET(f16, _Float16, q4_0, 0, 2, 1, 2)
CUCA_QMD_W8_SET(f16, _Float16, q4_0, 0, 8, 4, 2)
CUCA_QMD_W8_SET(f16, _Float16, q8_0, 1, 2, 1, 4)
CUCA_QMD_W8_SET(f16, _Float16, q8_0, 1, 8, 4, 4)
CUCA_QMD_W8_QKV(f32, float, q4_0, 0, 2, 1, 4)
CUCA_QMD_W8_QKV(f32, float, q4_0, 0, 8, 4, 8)
CUCA_QMD_W8_QKV(f32, float, q8_0, 1, 2, 1, 8)
CUCA_QMD_W8_QKV(f32, float, q8_0, 1, 8, 4, 8)
CUCA_QMD_W8_QKV(f16, _Float16, q4_0, 0, 2, 1, 4)
CUCA_QMD_W8_QKV(f16, _Float16, q4_0, 0, 8, 4, 8)
CUCA_QMD_W8_QKV(f16, _Float16, q8_0, 1, 2, 1, 8)
CUCA_QMD_W8_QKV(f16, _Float16, q8_0, 1, 8, 4, 8)
CUCA_QMD_W8_PLAIN(f32, float, q4_0, 0, 2, 1, 4)
CUCA_QMD_W8_PLAIN(f32, float, q4_0, 0, 8, 4, 8)
CUCA_QMD_W8_PLAIN(f32, float, q8_0, 1, 2, 1, 8)
CUCA_QMD_W8_PLAIN(f32, float, q8_0, 1, 8, 4, 8)
CUCA_QMD_W8_PLAIN(f16, _Float16, q4_0, 0, 2, 1, 4)
CUCA_QMD_W8_PLAIN(f16, _Float16, q4_0, 0, 8, 4, 8)
CUCA_QMD_W8_PLAIN(f16, _Float16, q8_0, 1, 2, 1, 8)
CUCA_QMD_W8_PLAIN(f16, _Float16, q8_0, 1, 8, 4, 8)
