// gemm16.hip -- the dense f16 GEMM of the prefill path on gfx950's matrix
// cores: out[t][c] = x[t] . w[c] over f16 weight rows (the dequantised copy
// cuca_qdequant_* writes) and f16 activation rows, f32 accumulation
// (v_mfma_f32_16x16x32_f16), the output rounded once to the activation
// dtype; the GLU form applies act(gate) * up to the f32 sums in registers.
//
// Replaces the float matmul the reference GPU engine runs after
// dense_dequant_kernel (moe_kernel.rs:1414-1600): the same arithmetic class
// as cuca_hip_qgemm (each operand an f16 value, products summed in f32).
//
// Tiling.  A workgroup of 4 waves computes 256 weight rows x 256 tokens (the
// GLU form: 128 gate rows and the 128 up rows of the same columns), each
// wave a 128 x 128 quarter as 8 x 8 tiles of 16 x 16 (256 accumulator
// registers).  k runs in stages of 32 values.  A stage's operands -- 256
// weight rows and 256 token rows of 64 bytes, 32 KB -- are copied from
// global memory straight into LDS (global_load_lds_dwordx4: lane L of an
// instruction writes 16 bytes at the instruction's LDS base + 16 L), four
// stages resident, each copied three stages before it is used.  Per stage a
// wave reads its 16 fragments (16 B a lane) once and issues 64 products;
// the next stage's fragments are read while this stage's products run, and
// the copies into the buffer just freed are spread between them.  One
// barrier a stage: after it every wave's copies of the next stage have
// landed and every wave has finished reading the buffer the copies refill.
//
// Split k: a call of too few tiles to fill the device (the host decides
// from the shape) runs the plain f32 form over every weight row it reads
// with k cut into equal splits (grid y), each split's sums into its own
// matrix of the workspace, and cuca_gemm16_reduce_* adds them in split
// order and applies the output (and the GLU).
//
// LDS layout: row R's 16-byte unit u sits at unit u ^ f(R), f(R) =
// (R >> 1) & 3.  Measured on MI355X with a probe of 16-byte LDS reads whose
// 16 lanes of a unit step through 64-byte rows: unswizzled, or swizzled by
// R & 3, (R >> 2) & 3 or ((R >> 1) ^ (R >> 3)) & 3, such a read takes twice
// the LDS cycles of a linear one (SQ_LDS_IDX_ACTIVE 8 against 4 a read);
// swizzled by (R >> 1) & 3 it takes the same 4 cycles as a linear read.
//
// Measured on MI355X at 4096 f16 rows (Llama-3-8B shapes), in one process
// against torch's f16 matmul (hipBLASLt): down 4096 x 14336 370-402 us
// (0.48-0.52 of the 2.5 PFLOP/s dense peak) against 326-383; q/o 4096 x
// 4096 114-124 us (0.45-0.48) against 102-103; gate+up with SwiGLU 882-884
// us (0.44), against 916-1065 for hipBLASLt's GEMM plus a separate GLU pass.
#include "common.h"
#include <type_traits>

typedef _Float16 g16_h8 __attribute__((ext_vector_type(8)));
typedef float g16_acc __attribute__((ext_vector_type(4)));

#define G16_BK 32 // k values a stage
#define G16_NB 4  // stages resident in LDS

// vmcnt(v) lgkmcnt(0) for the copy counts the pipelines wait on (4 or 8
// copies a stage, up to three stages in flight).  Any other count waits for
// every copy (vmcnt(0)): a count missing here must cost time, never let a
// stage be read before its copies have landed.
__device__ static inline void g16_wait(int v) {
    switch (v) {
    case 4: __builtin_amdgcn_s_waitcnt(0x0074); break;
    case 8: __builtin_amdgcn_s_waitcnt(0x0078); break;
    case 12: __builtin_amdgcn_s_waitcnt(0x007c); break;
    case 16: __builtin_amdgcn_s_waitcnt(0x4070); break;
    case 24: __builtin_amdgcn_s_waitcnt(0x4078); break;
    default: __builtin_amdgcn_s_waitcnt(0x0070); break; // 0
    }
}

// ACT: -1 plain, 0 SiLU, 1 GELU-tanh (the GLU form).
template <typename OutT, int ACT>
__device__ static inline void gemm16_body(const Gemm16Args &a) {
    constexpr bool GLU = ACT >= 0;
    // the four stage buffers are separate objects (rows 0..255 weights,
    // 256..511 tokens, 64 bytes each)
    __shared__ __attribute__((aligned(16))) _Float16 S0[512 * G16_BK], S1[512 * G16_BK], S2[512 * G16_BK],
        S3[512 * G16_BK];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wn = wave & 1, wm = wave >> 1;
    int r = lane & 15, u4 = lane >> 4;
    // The tile: XCD x (workgroups x, x + 8, ...) takes tiles [x per, (x + 1)
    // per) in launch order, grouped gn column tiles at a time and walked
    // token tile by token tile, so that the workgroups resident on an XCD at
    // once share weight and token rows in its L2.
    const int T = a.n_tn * a.n_tm, per = (T + 7) >> 3;
    const int L = (int)(blockIdx.x & 7) * per + (int)(blockIdx.x >> 3);
    if (L >= T) return; // uniform over the workgroup
    const int grp = L / (a.gn * a.n_tm), within = L - grp * a.gn * a.n_tm;
    const int gsz = min(a.gn, a.n_tn - grp * a.gn);
    const int tn = grp * a.gn + within % gsz, tm = within / gsz;
    const int n0 = tn * (GLU ? 128 : 256), t0 = tm * 256;
    // this workgroup's stages of the k range
    // Split y of k: a.k is the length of a split (the host makes the splits
    // equal), so stages [y nst, (y + 1) nst); its sums to output matrix y.
    const int nst = a.k / G16_BK;
    const int s0 = (int)blockIdx.y * nst;

    // Copies: wave w issues pieces c = 8 w + i (i < 8) of 16 LDS rows (pieces
    // 0..15 weights, 16..31 tokens); lane l copies row 16 c + l / 4, LDS unit
    // l % 4, from k unit (l % 4) ^ f(row).  A wave's pieces share one source
    // base, in SGPRs: wave 0 the weight tile's first 128 rows (GLU: the gate
    // rows), wave 1 its other 128 (GLU: the up rows of the same columns),
    // waves 2 and 3 the token tile; a lane adds a fixed 32-bit byte offset.
    // Rows past the matrix read the first row of the wave's base (their sums
    // are never stored); a base past the matrix falls back to the tile's.
    const _Float16 *W = reinterpret_cast<const _Float16 *>(a.w);
    const _Float16 *src;
    int lim; // rows of the wave's source that exist
    if (wave == 0) {
        src = W + (int64_t)n0 * a.ldw;
        lim = a.n - n0;
    } else if (wave == 1) {
        if (GLU) {
            src = W + (a.up_row + n0) * a.ldw;
            lim = a.n - n0;
        } else {
            const bool in = n0 + 128 < a.n;
            src = W + (int64_t)(n0 + (in ? 128 : 0)) * a.ldw;
            lim = in ? a.n - n0 - 128 : 0;
        }
    } else {
        src = reinterpret_cast<const _Float16 *>(a.x) + (int64_t)t0 * a.ldx;
        lim = a.m - t0;
    }
    const uint32_t ld = (uint32_t)(wave < 2 ? a.ldw : a.ldx);
    uint32_t off[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int R = 16 * (8 * wave + i) + (lane >> 2); // LDS row 0..511
        const int pu = (lane & 3) ^ ((R >> 1) & 3);
        int lr = wave < 2 ? R & 127 : R - 256; // the row within the wave's source
        if (lr >= lim) lr = 0;
        off[i] = 2u * ((uint32_t)lr * ld + 8u * (uint32_t)pu);
    }
    // The copies are issued from inline assembly, with the explicit waits
    // below: the compiler cannot tell the four buffers apart behind an LDS
    // DMA and would otherwise wait for every copy in flight before any LDS
    // read.  sc0: measured 3-7 % faster than the default policy.  M0 (the
    // copy's LDS base) is set by the same statement; nothing else in these
    // kernels uses M0 (clang warns that the clobber names a reserved register).
    // The base is read back from lane 0: it is uniform, and the SGPR operand
    // then needs no proof of it from the compiler.
    const uint64_t sv = (uint64_t)(uintptr_t)(src + s0 * G16_BK);
    const uint64_t bw = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(sv >> 32)) << 32) |
                        (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)sv);
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
    auto copy1 = [&](int st, _Float16 *S, int i) {
        const uint64_t base = bw + (uint64_t)st * (2 * G16_BK);
        const uint32_t dst = (uint32_t)(uintptr_t)&S[16 * (8 * wave + i) * G16_BK];
        asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1 sc0" ::"v"(off[i]), "s"(base), "s"(dst)
                     : "memory", "m0");
    };
#pragma clang diagnostic pop

    g16_acc acc[8][8];
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
        for (int j = 0; j < 8; j++) acc[i][j] = g16_acc{};
    // the wave's 16-row blocks: weights (GLU: 4 gate blocks, then the 4 up
    // blocks of the same columns) and tokens
    int arow[8], brow[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        arow[i] = GLU ? (i < 4 ? 64 * wn + 16 * i : 128 + 64 * wn + 16 * (i - 4)) : 128 * wn + 16 * i;
        brow[i] = 256 + 128 * wm + 16 * i;
    }
    // Fragment of a block at base 16 q: lane (r, u4) holds row 16 q + r,
    // k unit u4, at unit u4 ^ f(16 q + r) = u4 ^ f(r).
    const int pos = 8 * (u4 ^ ((r >> 1) & 3));
    g16_h8 fa[2][8], fb[2][8];
    auto frags = [&](const _Float16 *S, g16_h8 (&av)[8], g16_h8 (&bv)[8]) {
#pragma unroll
        for (int i = 0; i < 8; i++)
            av[i] = *reinterpret_cast<const g16_h8 *>(&S[(arow[i] + r) * G16_BK + pos]);
#pragma unroll
        for (int j = 0; j < 8; j++)
            bv[j] = *reinterpret_cast<const g16_h8 *>(&S[(brow[j] + r) * G16_BK + pos]);
    };
    // Stage st, its fragments in slot sl (read during the stage before); Sc
    // its buffer, Sn the next stage's.  FULL: the stages up to st + 4 exist.
    auto stage = [&](auto full, int st, int sl, _Float16 *Sc, _Float16 *Sn) {
        constexpr bool FULL = decltype(full)::value;
        // this wave's copies of stage st + 1 have landed (those of st + 2 and
        // st + 3 may be in flight) and its reads of Sc are done; after the
        // barrier, every wave's
        g16_wait(FULL ? 8 * (G16_NB - 2) : 8 * max(0, min(G16_NB - 2, nst - st - 2)));
        __syncthreads();
        const bool nx = FULL || st + 1 < nst;
        const bool cp = FULL || st + G16_NB < nst;
        // The products of this stage, 8 at a time, one copy after each group
        // (the scheduling barriers keep that order).  The plain form issues
        // two of the next stage's fragment reads before each group, so its
        // products start right after the barrier; the GLU form reads them
        // all first (interleaved, the compiler moves its accumulators between
        // registers inside the loop).
        if constexpr (GLU) {
            if (nx) frags(Sn, fa[sl ^ 1], fb[sl ^ 1]);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int q = 0; q < 8; q++) {
#pragma unroll
                for (int j = 0; j < 8; j++)
                    acc[q][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fa[sl][q], fb[sl][j], acc[q][j], 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
                if (cp) copy1(st + G16_NB, Sc, q);
                __builtin_amdgcn_sched_barrier(0);
            }
        } else {
#pragma unroll
            for (int q = 0; q < 8; q++) {
                if (nx) {
                    fa[sl ^ 1][q] = *reinterpret_cast<const g16_h8 *>(&Sn[(arow[q] + r) * G16_BK + pos]);
                    fb[sl ^ 1][q] = *reinterpret_cast<const g16_h8 *>(&Sn[(brow[q] + r) * G16_BK + pos]);
                }
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int j = 0; j < 8; j++)
                    acc[q][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fa[sl][q], fb[sl][j], acc[q][j], 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
                if (cp) copy1(st + G16_NB, Sc, q);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    };
    using T1 = std::integral_constant<bool, true>;
    using T0 = std::integral_constant<bool, false>;
    // (the buffers are named in every call, not picked from an array: an
    // array of LDS pointers has ended up in scratch memory)
    auto copy_stage = [&](int st, _Float16 *S) {
#pragma unroll
        for (int i = 0; i < 8; i++) copy1(st, S, i);
    };
    copy_stage(0, S0);
    if (nst > 1) copy_stage(1, S1);
    if (nst > 2) copy_stage(2, S2);
    if (nst > 3) copy_stage(3, S3);
    g16_wait(8 * max(0, min(G16_NB, nst) - 1)); // stage 0 landed
    __syncthreads();
    frags(S0, fa[0], fb[0]);
    int st = 0;
    // stage st + b: buffer b, fragment slot b & 1
    for (; st + 2 * G16_NB <= nst; st += G16_NB) {
        stage(T1{}, st, 0, S0, S1);
        stage(T1{}, st + 1, 1, S1, S2);
        stage(T1{}, st + 2, 0, S2, S3);
        stage(T1{}, st + 3, 1, S3, S0);
    }
    for (; st < nst; st += G16_NB) {
        stage(T0{}, st, 0, S0, S1);
        if (st + 1 < nst) stage(T0{}, st + 1, 1, S1, S2);
        if (st + 2 < nst) stage(T0{}, st + 2, 0, S2, S3);
        if (st + 3 < nst) stage(T0{}, st + 3, 1, S3, S0);
    }

    // Accumulator e of lane (r, u4) in tile (i, j): weight row 16 i + 4 u4 +
    // e of the wave's blocks, token 16 j + r: four consecutive columns.
    // (The lane's r and u4 computed afresh from its lane number: otherwise
    // values derived from them before the k loop are kept through it, and
    // with every register in use there one of them spills.)
    {
        const int ln = (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
        r = ln & 15;
        u4 = ln >> 4;
    }
    // (i outer: one block of columns at a time; with the tokens outer, the
    // compiler copied every tile out of the accumulators at once and spilled)
#pragma unroll
    for (int i = 0; i < (GLU ? 4 : 8); i++) {
        const int c = n0 + (GLU ? 64 * wn : 128 * wn) + 16 * i + 4 * u4;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            // (the plain form: the empty asm keeps each tile in the
            // accumulator registers until its turn, which also keeps the
            // compiler from moving tiles between registers in the k loop; the
            // GLU form allocates better without it)
            if (!GLU) asm volatile("" : "+a"(acc[i][j]));
            const int t = t0 + 128 * wm + 16 * j + r;
            if (t >= a.m) continue;
            OutT *orow = reinterpret_cast<OutT *>(a.out) + ((int64_t)blockIdx.y * a.m + t) * a.out_ld;
            float o[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                float g = acc[i][j][e];
                if (GLU) {
                    float u = acc[i + 4][j][e];
                    if (a.clamp > 0.0f) { // Glu::apply's clamp (cpu.rs:364-368)
                        g = fminf(g, a.clamp);
                        u = fminf(fmaxf(u, -a.clamp), a.clamp);
                    }
                    g = (ACT == 0 ? act_silu(g) : act_gelu_tanh(g)) * u;
                }
                o[e] = g;
            }
            if (a.vec && c + 3 < a.n) {
                if (!GLU && sizeof(OutT) == 4) { // the tile's registers as they are
                    *reinterpret_cast<f32x4 *>(orow + c) = acc[i][j];
                } else if (sizeof(OutT) == 4) {
                    *reinterpret_cast<f32x4 *>(orow + c) = f32x4{o[0], o[1], o[2], o[3]};
                } else {
                    typedef _Float16 g16_h4 __attribute__((ext_vector_type(4)));
                    *reinterpret_cast<g16_h4 *>(orow + c) =
                        g16_h4{to_stored<_Float16>(o[0]), to_stored<_Float16>(o[1]), to_stored<_Float16>(o[2]),
                               to_stored<_Float16>(o[3])};
                }
            } else if (!GLU && sizeof(OutT) == 4) {
                const f32x4 v = acc[i][j];
#pragma unroll
                for (int e = 0; e < 4; e++)
                    if (c + e < a.n) orow[c + e] = v[e];
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++)
                    if (c + e < a.n) orow[c + e] = to_stored<OutT>(o[e]);
            }
        }
    }
}

// The GLU form with 8 waves a workgroup, two a SIMD: wave w computes the
// weight half w & 1 (64 gate rows and the 64 up rows of the same columns) of
// token quarter w >> 1 (64 tokens), 8 x 4 tiles, 128 accumulators, so a
// SIMD holds two waves and one's products run while the other waits at the
// barrier or on LDS.  The same tile, tile order, LDS layout, copies (four a
// wave a stage) and stage pipeline; per stage a wave reads the next stage's
// 4 token fragments first, then after each group of 4 products the next
// stage's weight fragment of that group (in the register the group just
// used), and issues its products at raised priority.  Each output sums its
// k steps with the same instructions in the same order as the 4-wave
// kernel.  Measured on MI355X at 4096 f16 rows with the launches of the two
// forms interleaved (so that clock changes fall on both): gate+up with
// SwiGLU 843-851 -> 784-793 us (0.45 -> 0.49 of the dense peak); the plain
// form on 8 waves measured no faster (down 362-387 against 358-385 us, q/o
// 116-127 against 113-118), so plain calls keep 4 waves.  (The body is
// written for both forms; only the GLU kernels are built.)
template <typename OutT, int ACT>
__device__ static inline void gemm16_w8_body(const Gemm16Args &a) {
    constexpr bool GLU = ACT >= 0;
    __shared__ __attribute__((aligned(16))) _Float16 S0[512 * G16_BK], S1[512 * G16_BK], S2[512 * G16_BK],
        S3[512 * G16_BK];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6); // 0..7
    const int wn = wave & 1, wm = wave >> 1;                     // token quarter 0..3
    int r = lane & 15, u4 = lane >> 4;
    const int T = a.n_tn * a.n_tm, per = (T + 7) >> 3;
    const int L = (int)(blockIdx.x & 7) * per + (int)(blockIdx.x >> 3);
    if (L >= T) return; // uniform over the workgroup
    const int grp = L / (a.gn * a.n_tm), within = L - grp * a.gn * a.n_tm;
    const int gsz = min(a.gn, a.n_tn - grp * a.gn);
    const int tn = grp * a.gn + within % gsz, tm = within / gsz;
    const int n0 = tn * (GLU ? 128 : 256), t0 = tm * 256;
    const int nst = a.k / G16_BK;
    const int s0 = (int)blockIdx.y * nst;

    // Copies: wave w fills LDS rows 64 w .. 64 w + 63 in pieces of 16 rows
    // c = 4 w + i: waves 0-3 the weight tile (GLU: waves 0, 1 the gate rows,
    // 2, 3 the up rows of the same columns), waves 4-7 the token tile.  Rows
    // past the matrix read the first row of the wave's base; a base past the
    // matrix falls back to the tile's first row.
    const _Float16 *src;
    int lim; // rows of the wave's source that exist
    if (wave < 4) {
        const int rb = GLU ? 64 * (wave & 1) : 64 * wave;
        const int64_t first = GLU && wave >= 2 ? a.up_row + n0 : (int64_t)n0;
        lim = a.n - n0 - rb;
        src = reinterpret_cast<const _Float16 *>(a.w) + (first + (lim > 0 ? rb : 0)) * a.ldw;
    } else {
        const int rb = 64 * (wave - 4);
        lim = a.m - t0 - rb;
        src = reinterpret_cast<const _Float16 *>(a.x) + (int64_t)(t0 + (lim > 0 ? rb : 0)) * a.ldx;
    }
    const uint32_t ld = (uint32_t)(wave < 4 ? a.ldw : a.ldx);
    uint32_t off[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int R = 16 * (4 * wave + i) + (lane >> 2); // LDS row 0..511
        const int pu = (lane & 3) ^ ((R >> 1) & 3);
        int lr = R - 64 * wave; // the row within the wave's source
        if (lr >= lim) lr = 0;
        off[i] = 2u * ((uint32_t)lr * ld + 8u * (uint32_t)pu);
    }
    const uint64_t sv = (uint64_t)(uintptr_t)(src + s0 * G16_BK);
    const uint64_t bw = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(sv >> 32)) << 32) |
                        (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)sv);
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
    auto copy1 = [&](int st, _Float16 *S, int i) {
        const uint64_t base = bw + (uint64_t)st * (2 * G16_BK);
        const uint32_t dst = (uint32_t)(uintptr_t)&S[16 * (4 * wave + i) * G16_BK];
        asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1 sc0" ::"v"(off[i]), "s"(base), "s"(dst)
                     : "memory", "m0");
    };
#pragma clang diagnostic pop

    g16_acc acc[8][4];
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = g16_acc{};
    int arow[8], brow[4];
#pragma unroll
    for (int i = 0; i < 8; i++)
        arow[i] = GLU ? (i < 4 ? 64 * wn + 16 * i : 128 + 64 * wn + 16 * (i - 4)) : 128 * wn + 16 * i;
#pragma unroll
    for (int j = 0; j < 4; j++) brow[j] = 256 + 64 * wm + 16 * j;
    const int pos = 8 * (u4 ^ ((r >> 1) & 3));
    auto rd = [&](const _Float16 *S, int row) -> g16_h8 {
        return *reinterpret_cast<const g16_h8 *>(&S[(row + r) * G16_BK + pos]);
    };
    g16_h8 fa[8], fb[2][4];
    auto stage = [&](auto full, int st, int sl, _Float16 *Sc, _Float16 *Sn) {
        constexpr bool FULL = decltype(full)::value;
        // this wave's copies of stage st + 1 have landed and its reads of Sc
        // are done; after the barrier, every wave's
        g16_wait(FULL ? 4 * (G16_NB - 2) : 4 * max(0, min(G16_NB - 2, nst - st - 2)));
        __syncthreads();
        const bool nx = FULL || st + 1 < nst;
        const bool cp = FULL || st + G16_NB < nst;
        if (nx) {
#pragma unroll
            for (int j = 0; j < 4; j++) fb[sl ^ 1][j] = rd(Sn, brow[j]);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int q = 0; q < 8; q++) {
            __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int j = 0; j < 4; j++)
                acc[q][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fa[q], fb[sl][j], acc[q][j], 0, 0, 0);
            __builtin_amdgcn_s_setprio(0);
            __builtin_amdgcn_sched_barrier(0);
            if (nx) fa[q] = rd(Sn, arow[q]);
            if (cp && (q & 1)) copy1(st + G16_NB, Sc, q >> 1);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    using T1 = std::integral_constant<bool, true>;
    using T0 = std::integral_constant<bool, false>;
    auto copy_stage = [&](int st, _Float16 *S) {
#pragma unroll
        for (int i = 0; i < 4; i++) copy1(st, S, i);
    };
    copy_stage(0, S0);
    if (nst > 1) copy_stage(1, S1);
    if (nst > 2) copy_stage(2, S2);
    if (nst > 3) copy_stage(3, S3);
    g16_wait(4 * max(0, min(G16_NB, nst) - 1)); // stage 0 landed
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 8; i++) fa[i] = rd(S0, arow[i]);
#pragma unroll
    for (int j = 0; j < 4; j++) fb[0][j] = rd(S0, brow[j]);
    int st = 0;
    for (; st + 2 * G16_NB <= nst; st += G16_NB) {
        stage(T1{}, st, 0, S0, S1);
        stage(T1{}, st + 1, 1, S1, S2);
        stage(T1{}, st + 2, 0, S2, S3);
        stage(T1{}, st + 3, 1, S3, S0);
    }
    for (; st < nst; st += G16_NB) {
        stage(T0{}, st, 0, S0, S1);
        if (st + 1 < nst) stage(T0{}, st + 1, 1, S1, S2);
        if (st + 2 < nst) stage(T0{}, st + 2, 0, S2, S3);
        if (st + 3 < nst) stage(T0{}, st + 3, 1, S3, S0);
    }
    {
        const int ln = (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
        r = ln & 15;
        u4 = ln >> 4;
    }
    // accumulator e of lane (r, u4) in tile (i, j): weight row 16 i + 4 u4 + e
    // of the wave's blocks, token 64 wm + 16 j + r
#pragma unroll
    for (int i = 0; i < (GLU ? 4 : 8); i++) {
        const int c = n0 + (GLU ? 64 * wn : 128 * wn) + 16 * i + 4 * u4;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            if (!GLU) asm volatile("" : "+a"(acc[i][j]));
            const int t = t0 + 64 * wm + 16 * j + r;
            if (t >= a.m) continue;
            OutT *orow = reinterpret_cast<OutT *>(a.out) + ((int64_t)blockIdx.y * a.m + t) * a.out_ld;
            float o[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                float g = acc[i][j][e];
                if (GLU) {
                    float u = acc[i + 4][j][e];
                    if (a.clamp > 0.0f) { // Glu::apply's clamp (cpu.rs:364-368)
                        g = fminf(g, a.clamp);
                        u = fminf(fmaxf(u, -a.clamp), a.clamp);
                    }
                    g = (ACT == 0 ? act_silu(g) : act_gelu_tanh(g)) * u;
                }
                o[e] = g;
            }
            if (a.vec && c + 3 < a.n) {
                if (!GLU && sizeof(OutT) == 4) {
                    *reinterpret_cast<f32x4 *>(orow + c) = acc[i][j];
                } else if (sizeof(OutT) == 4) {
                    *reinterpret_cast<f32x4 *>(orow + c) = f32x4{o[0], o[1], o[2], o[3]};
                } else {
                    typedef _Float16 g16_h4 __attribute__((ext_vector_type(4)));
                    *reinterpret_cast<g16_h4 *>(orow + c) =
                        g16_h4{to_stored<_Float16>(o[0]), to_stored<_Float16>(o[1]), to_stored<_Float16>(o[2]),
                               to_stored<_Float16>(o[3])};
                }
            } else if (!GLU && sizeof(OutT) == 4) {
                const f32x4 v = acc[i][j];
#pragma unroll
                for (int e = 0; e < 4; e++)
                    if (c + e < a.n) orow[c + e] = v[e];
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++)
                    if (c + e < a.n) orow[c + e] = to_stored<OutT>(o[e]);
            }
        }
    }
}

#define CUCA_GEMM16(NAME, T, ACT)                                                          \
    extern "C" __global__ __launch_bounds__(256) void NAME(Gemm16Args a) { gemm16_body<T, ACT>(a); }
CUCA_GEMM16(cuca_gemm16_f32, float, -1)
CUCA_GEMM16(cuca_gemm16_f16, _Float16, -1)
#define CUCA_GEMM16_W8(NAME, T, ACT)                                                       \
    extern "C" __global__ __launch_bounds__(512) void NAME(Gemm16Args a) { gemm16_w8_body<T, ACT>(a); }
CUCA_GEMM16_W8(cuca_gemm16_w8_glu_f32_silu, float, 0)
CUCA_GEMM16_W8(cuca_gemm16_w8_glu_f32_gelu, float, 1)
CUCA_GEMM16_W8(cuca_gemm16_w8_glu_f16_silu, _Float16, 0)
CUCA_GEMM16_W8(cuca_gemm16_w8_glu_f16_gelu, _Float16, 1)

// The splits' f32 sums added in split order, then the output: one thread per
// output.  part [splits][m][width]: width = n, or 2 n for the GLU (gate
// columns, then up columns: the split GEMM ran over all the weight rows).
template <typename T, int ACT> __device__ static inline void gemm16_reduce_body(const Gemm16Args &a) {
    const int64_t e = (int64_t)blockIdx.x * CUCA_BLOCK + threadIdx.x;
    if (e >= (int64_t)a.m * a.n) return;
    const int t = (int)(e / a.n), c = (int)(e - (int64_t)t * a.n);
    const int64_t w = ACT >= 0 ? 2 * (int64_t)a.n : a.n;
    float g = 0.0f, u = 0.0f;
    for (int sp = 0; sp < a.splits; sp++) {
        const float *row = a.part + ((int64_t)sp * a.m + t) * w;
        g = g + row[c];
        if (ACT >= 0) u = u + row[a.n + c];
    }
    float o = g;
    if (ACT >= 0) {
        if (a.clamp > 0.0f) { // Glu::apply's clamp (cpu.rs:364-368)
            g = fminf(g, a.clamp);
            u = fminf(fmaxf(u, -a.clamp), a.clamp);
        }
        o = (ACT == 0 ? act_silu(g) : act_gelu_tanh(g)) * u;
    }
    reinterpret_cast<T *>(a.out)[(int64_t)t * a.out_ld + c] = to_stored<T>(o);
}
#define CUCA_GEMM16_RED(NAME, T, ACT)                                                      \
    extern "C" __global__ __launch_bounds__(CUCA_BLOCK) void NAME(Gemm16Args a) { gemm16_reduce_body<T, ACT>(a); }
CUCA_GEMM16_RED(cuca_gemm16_reduce_f32, float, -1)
CUCA_GEMM16_RED(cuca_gemm16_reduce_f16, _Float16, -1)
CUCA_GEMM16_RED(cuca_gemm16_reduce_glu_f32_silu, float, 0)
CUCA_GEMM16_RED(cuca_gemm16_reduce_glu_f32_gelu, float, 1)
CUCA_GEMM16_RED(cuca_gemm16_reduce_glu_f16_silu, _Float16, 0)
CUCA_GEMM16_RED(cuca_gemm16_reduce_glu_f16_gelu, _Float16, 1)
