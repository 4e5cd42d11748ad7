// qgemm.hip -- the quantized matmul for many activation rows (prefill, large
// decode batches) on gfx950's matrix cores: out[t][n] = x[t] . w[n] with
// the Q4_0 / Q8_0 weights dequantised to f16 and the activations rounded to
// f16, f32 accumulation (v_mfma_f32_32x32x16_f16).
//
// This is the reference GPU engine's arithmetic class for its dense paths
// (dense_gemv_kernel / dense_dequant_kernel, moe_kernel.rs:1414-1600: float
// products of dequantised weights and unquantised activations), not the CPU
// engine's bits (cuca_hip_qmm keeps those).  Each weight is f16(d * q) and
// each activation f16(x), one rounding each; the error is bounded by
// (2^-10 + k 2^-24) sum_i |w_i x_i| and the parity tests hold it to that.
//
// The weights are read in the packed layout of qmm.hip.  A dot product may
// sum its terms in any order, so the k index of the matrix-core operands is
// the packed layout's own order: a lane's 8 f16 of a k-step come from one
// or two packed dwords (shift, mask, an f16 bias subtracted, the block scale
// multiplied, two values at a time), and the activations are staged into
// LDS in the same order.  Slot j of a lane's 8 values is true position
// base + 16 j:
//   Q4_0: k-chunk kc = group kc/4, quarter qq = kc%4; k-step s, half h:
//         lane chunk l = 4 qq + s/2, dword t = 2 h + s%2,
//         base = 512 g + 128 t + l; dword t of chunk l holds blocks 4t..4t+3
//         (pair i = nibbles 4i and 16+4i: elements l and l+16 of block 4t+i)
//   Q8_0: k-chunk kc = group kc/2, half hh = kc%2; k-step s, half h:
//         lane chunk l = 8 hh + s, dwords 2h and 2h+1, base = 256 g + 128 h + l
//         (dword t: biased bytes of elements l, l+16 of blocks 2t, 2t+1)
//
// Workgroup: 4 waves, 128 weight rows (32 per wave) x TM tokens (TM / 32
// accumulator tiles per wave); k in chunks of 128 values (8 k-steps).  While
// a chunk computes, the next chunk's weights are loaded into registers and
// its activations copied into the other LDS buffer.  The grid is XCD-aware
// and grouped (qgemm_body).
#include "common.h"

typedef _Float16 qg_h2 __attribute__((ext_vector_type(2)));
typedef _Float16 qg_h8 __attribute__((ext_vector_type(8)));
typedef float qg_acc __attribute__((ext_vector_type(16)));
typedef uint32_t qg_u2 __attribute__((ext_vector_type(2)));

#define QG_ROWS 128       // weight rows per workgroup (32 per wave)
#define QG_KC 128         // values per k-chunk: 8 k-steps of 16

template <int FMT> struct QgFmt;
template <> struct QgFmt<0> { // Q4_0: 4 lane chunks of a 512-value group per k-chunk
    static constexpr int NW = 4, GB = 288, SCB = 32, KCG = 4;
};
template <> struct QgFmt<1> { // Q8_0: 8 lane chunks of a 256-value group per k-chunk
    static constexpr int NW = 8, GB = 272, SCB = 16, KCG = 2;
};

// The weights a lane needs for one k-chunk: its dword pair of each lane
// chunk, and the scales of its blocks (Q4_0: blocks 8h..8h+7, Q8_0: 4h..4h+3).
template <int FMT> struct QgA {
    qg_u2 w[QgFmt<FMT>::NW];
    u32x4 sc;
};

template <int FMT>
__device__ static inline void qg_load_a(const uint8_t *wrow, int kc, int h, QgA<FMT> &o) {
    using F = QgFmt<FMT>;
    const int g = kc / F::KCG, part = kc % F::KCG;
    const uint8_t *grp = wrow + (int64_t)g * F::GB;
#pragma unroll
    for (int i = 0; i < F::NW; i++) {
        const int l = part * F::NW + i;
        o.w[i] = *reinterpret_cast<const qg_u2 *>(grp + F::SCB + 16 * l + 8 * h);
    }
    if (FMT == 0) {
        o.sc = *reinterpret_cast<const u32x4 *>(grp + 16 * h);
    } else {
        const qg_u2 s2 = *reinterpret_cast<const qg_u2 *>(grp + 8 * h);
        o.sc = u32x4{s2.x, s2.y, 0u, 0u};
    }
}

__device__ static inline qg_h2 qg_pair(uint32_t u, qg_h2 bias, _Float16 d) {
    const qg_h2 p = __builtin_bit_cast(qg_h2, u) - bias;
    return p * qg_h2{d, d};
}
__device__ static inline _Float16 qg_scale(const u32x4 &sc, int i) {
    const uint32_t w = sc[i >> 1];
    return __builtin_bit_cast(_Float16, (uint16_t)((i & 1) ? (w >> 16) : (w & 0xffffu)));
}

// The A operand of k-step s (compile-time s).
template <int FMT>
__device__ static inline qg_h8 qg_dequant(const QgA<FMT> &a, int s) {
    qg_h8 o;
    if (FMT == 0) {
        const uint32_t w = a.w[s >> 1][s & 1];
        const qg_h2 bias = {(_Float16)1032.0f, (_Float16)1032.0f};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t u = ((w >> (4 * i)) & 0x000f000fu) | 0x64006400u;
            const qg_h2 p = qg_pair(u, bias, qg_scale(a.sc, (s & 1) * 4 + i));
            o[2 * i] = p.x;
            o[2 * i + 1] = p.y;
        }
    } else {
        const qg_h2 bias = {(_Float16)1152.0f, (_Float16)1152.0f};
#pragma unroll
        for (int idx = 0; idx < 2; idx++) {
            const uint32_t w = a.w[s][idx];
            const qg_h2 p0 = qg_pair(__builtin_amdgcn_perm(0x64646464u, w, 0x04020400u), bias, qg_scale(a.sc, 2 * idx));
            const qg_h2 p1 = qg_pair(__builtin_amdgcn_perm(0x64646464u, w, 0x04030401u), bias, qg_scale(a.sc, 2 * idx + 1));
            o[4 * idx + 0] = p0.x;
            o[4 * idx + 1] = p0.y;
            o[4 * idx + 2] = p1.x;
            o[4 * idx + 3] = p1.y;
        }
    }
    return o;
}

__device__ static inline void qgemm_load8f(const float *p, float (&v)[8]) {
    const f32x4 a = reinterpret_cast<const f32x4 *>(p)[0];
    const f32x4 b = reinterpret_cast<const f32x4 *>(p)[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

// The activations rewritten once per call, before the matmul: f16, in the
// slot order of the format (xp [n_ct * TM][kp], kp = 128 per k-chunk; zero
// past k and in the rows past m, up to the whole tile).  One thread per unit
// (token, k-chunk, k-step s, half h) of 8 values: the values at true
// positions base + 16 j.
template <typename T, int FMT> __device__ static inline void qgemm_prep_body(const QGemmArgs &a) {
    using F = QgFmt<FMT>;
    const int64_t u = (int64_t)blockIdx.x * CUCA_BLOCK + threadIdx.x;
    const int64_t per_row = (int64_t)a.nkc * 16;
    if (u >= (int64_t)a.mp * per_row) return;
    const int tok = (int)(u / per_row), rem = (int)(u - (int64_t)tok * per_row);
    const int kc = rem >> 4, v = rem & 15, s = v >> 1, h = v & 1;
    const int g = kc / F::KCG, part = kc % F::KCG;
    int base;
    if (FMT == 0) base = 512 * g + 128 * (2 * h + (s & 1)) + 4 * part + (s >> 1);
    else base = 256 * g + 128 * h + 8 * part + s;
    const T *row = reinterpret_cast<const T *>(a.x) + (int64_t)(tok < a.m ? tok : 0) * a.ldx;
    qg_h8 o;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int k = base + 16 * j;
        o[j] = tok < a.m && k < a.k ? (_Float16)(float)row[k] : (_Float16)0.0f;
    }
    *reinterpret_cast<qg_h8 *>(a.xp + (int64_t)tok * a.kp + (int64_t)kc * QG_KC + 8 * (2 * s + h)) = o; // xp: f16 bits
}

// The activations of one k-chunk, TM tokens x 128 f16, copied from the
// workspace straight into LDS (global_load_lds_dwordx4: lane L of a wave
// writes 16 bytes at the wave's LDS address + 16 L).  A row is 256 bytes,
// unpadded; its 16-byte unit v sits at position v ^ (row % 16), so that the
// B-operand reads of 16 rows at one unit fall in different banks.  Wave w's
// copy it fills rows 16 it + 4 w .. + 3.
// The lane's part of the source offset, lane_off = (lane / 16) kp + 8 v, is
// the same for every copy (row % 16 = (4 w + lane / 16) % 16).
template <int TM>
__device__ static inline void qg_copy_x(const QGemmArgs &a, int tok0, int kc, int wave, int lane_off,
                                        _Float16 (*xs)[QG_KC]) {
#pragma unroll
    for (int it = 0; it < TM / 16; it++) {
        const int c0 = 16 * it + 4 * wave; // wave-uniform
        const uint16_t *src = a.xp + ((int64_t)(tok0 + c0) * a.kp + (int64_t)kc * QG_KC);
        __builtin_amdgcn_global_load_lds(src + lane_off, &xs[c0][0], 16, 0, 0);
    }
}

// One k-chunk: the MFMAs over xc, while the next chunk's activations are
// copied into xn and its weights loaded into ng / nu.
template <int FMT, int TM, bool GLU>
__device__ static inline void qg_chunk(const QGemmArgs &a, const uint8_t *wg, const uint8_t *wu, int tok0, int kc,
                                       bool next, int wave, int lane, int lane_off, _Float16 (*xc)[QG_KC],
                                       _Float16 (*xn)[QG_KC],
                                       QgA<FMT> &ag, QgA<FMT> &au, qg_acc *acc, qg_acc *accu) {
    constexpr int NT = TM / 32;
    const int r = lane & 31, h = lane >> 5;
    QgA<FMT> ng, nu;
    if (next) {
        qg_load_a<FMT>(wg, kc + 1, h, ng);
        if (GLU) qg_load_a<FMT>(wu, kc + 1, h, nu);
        qg_copy_x<TM>(a, tok0, kc + 1, wave, lane_off, xn);
    }
#pragma unroll
    for (int s = 0; s < 8; s++) {
        const qg_h8 av = qg_dequant<FMT>(ag, s);
        qg_h8 uv;
        if (GLU) uv = qg_dequant<FMT>(au, s);
        const int pos = 8 * ((2 * s + h) ^ (r & 15));
#pragma unroll
        for (int i = 0; i < NT; i++) {
            const qg_h8 bv = *reinterpret_cast<const qg_h8 *>(&xc[i * 32 + r][pos]);
            acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, bv, acc[i], 0, 0, 0);
            if (GLU) accu[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(uv, bv, accu[i], 0, 0, 0);
        }
    }
    __builtin_amdgcn_s_waitcnt(0); // the copies into xn have landed
    __syncthreads();
    if (next) {
        ag = ng;
        if (GLU) au = nu;
    }
}

// SPLIT: workgroup (tile, split) takes k-chunks [split * kcs, ...) and
// writes its f32 sums to the partial rows of the workspace (qgemm_reduce
// adds the splits in order and applies the epilogue); otherwise the
// epilogue is applied here.
template <typename T, int FMT, int TM, bool GLU, int ACT, bool SPLIT, int MOE = 0>
__device__ static inline void qgemm_body(const QGemmArgs &a) {
    constexpr int NT = TM / 32;
    const int split = SPLIT ? (int)blockIdx.y : 0;
    // XCD x (workgroups x, x + 8, ...) takes row tiles x, x + 8, ... in
    // groups of 8; a group's workgroups take its row tiles in turn, token
    // tile by token tile, so that the workgroups resident on the XCD at once
    // share their weight and activation tiles in its L2
    const int id = blockIdx.x, xcd = id & 7, kq = id >> 3;
    const int n_rx = (a.n_rt - xcd + 7) >> 3; // row tiles of this XCD
    const int g = kq / (8 * a.n_ct), w = kq - g * 8 * a.n_ct;
    const int gsz = min(8, n_rx - 8 * g);
    if (gsz <= 0) return;
    const int ct = w / gsz, rt = (8 * g + (w - ct * gsz)) * 8 + xcd;
    if (ct >= a.n_ct) return;
    // routed experts: the tile's expert and pairs (uniform); tiles past the
    // last are empty
    int ex = 0, p0 = 0, np = 0;
    if (MOE) {
        ex = a.tile_e[ct];
        if (ex < 0) return;
        p0 = a.tile_p0[ct];
        np = a.tile_n[ct];
    }
    const int kc0 = split * a.kcs;
    const int kc1 = min(a.nkc, kc0 + a.kcs);
    if (kc0 >= kc1) return;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r = lane & 31, h = lane >> 5;
    const int row = rt * QG_ROWS + wave * 32 + r;
    const int tok0 = ct * TM;
    const int64_t roff = (int64_t)(row < a.rows ? row : 0) * a.row_bytes + (MOE ? (int64_t)ex * a.estride : 0);
    const uint8_t *wg = a.w + roff;
    const uint8_t *wu = GLU ? a.w_up + roff : nullptr;

    qg_acc acc[NT], accu[NT];
#pragma unroll
    for (int i = 0; i < NT; i++) {
        acc[i] = qg_acc{};
        accu[i] = qg_acc{};
    }
    // two LDS buffers, separate objects so that the compiler sees the copy
    // into one and the reads of the other do not overlap
    __shared__ __attribute__((aligned(16))) _Float16 xs0[TM][QG_KC];
    __shared__ __attribute__((aligned(16))) _Float16 xs1[TM][QG_KC];
    QgA<FMT> ag, au;
    qg_load_a<FMT>(wg, kc0, h, ag);
    if (GLU) qg_load_a<FMT>(wu, kc0, h, au);
    const int lane_off = (lane >> 4) * (int)a.kp + 8 * ((lane & 15) ^ ((4 * wave + (lane >> 4)) & 15));
    qg_copy_x<TM>(a, tok0, kc0, wave, lane_off, xs0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    for (int kc = kc0; kc < kc1; kc += 2) {
        qg_chunk<FMT, TM, GLU>(a, wg, wu, tok0, kc, kc + 1 < kc1, wave, lane, lane_off, xs0, xs1, ag, au, acc, accu);
        if (kc + 1 < kc1)
            qg_chunk<FMT, TM, GLU>(a, wg, wu, tok0, kc + 1, kc + 2 < kc1, wave, lane, lane_off, xs1, xs0, ag, au, acc, accu);
    }
    // accumulator q of lane (r, h): weight row 8 (q / 4) + 4 h + q % 4, token r.
    // The empty asm keeps a tile in the accumulator registers until its turn
    // (after the previous tile's stores): copied out all at once, the tiles
    // would set the kernel's register count.
    if (SPLIT) {
        // partial rows: [split][gate, up][m][rows] f32
#pragma unroll
        for (int i = 0; i < NT; i++) {
            asm volatile("" : "+a"(acc[i]));
            if (GLU) asm volatile("" : "+a"(accu[i]));
            const int tok = tok0 + i * 32 + r;
            if (tok >= a.m) continue;
            float *pg = a.part + ((int64_t)split * (GLU ? 2 : 1) * a.m + tok) * a.rows;
            float *pu = a.part + ((int64_t)(split * 2 + 1) * a.m + tok) * a.rows;
#pragma unroll
            for (int q = 0; q < 16; q++) {
                const int n = rt * QG_ROWS + wave * 32 + 8 * (q >> 2) + 4 * h + (q & 3);
                if (n >= a.rows) continue;
                pg[n] = acc[i][q];
                if (GLU) pu[n] = accu[i][q];
            }
        }
        return;
    }
    if (MOE) {
        // pair p0 + local of the tile: up, act(g) * u into hidden row p; down,
        // the f32 product times the pair's routing weight into scratch row p
#pragma unroll
        for (int i = 0; i < NT; i++) {
            asm volatile("" : "+a"(acc[i]));
            if (GLU) asm volatile("" : "+a"(accu[i]));
            const int local = i * 32 + r;
            if (local >= np) continue;
            const int64_t p = p0 + local;
            const float pw = MOE == 2 ? a.pair_weight[p] : 1.0f;
#pragma unroll
            for (int q = 0; q < 16; q++) {
                const int n = rt * QG_ROWS + wave * 32 + 8 * (q >> 2) + 4 * h + (q & 3);
                if (n >= a.rows) continue;
                float o = acc[i][q];
                if (GLU) {
                    float gg = o, u = accu[i][q];
                    if (a.clamp > 0.0f) { // Glu::apply's clamp (cpu.rs:364-368)
                        gg = fminf(gg, a.clamp);
                        u = fminf(fmaxf(u, -a.clamp), a.clamp);
                    }
                    o = (ACT == 0 ? act_silu(gg) : act_gelu_tanh(gg)) * u;
                }
                if (MOE == 2) reinterpret_cast<float *>(a.out)[p * a.out_ld + n] = o * pw;
                else reinterpret_cast<T *>(a.out)[p * a.out_ld + n] = to_stored<T>(o);
            }
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < NT; i++) {
        asm volatile("" : "+a"(acc[i]));
        if (GLU) asm volatile("" : "+a"(accu[i]));
        const int tok = tok0 + i * 32 + r;
        if (tok >= a.m) continue;
        T *orow = reinterpret_cast<T *>(a.out) + (int64_t)tok * a.out_ld;
#pragma unroll
        for (int q = 0; q < 16; q++) {
            const int n = rt * QG_ROWS + wave * 32 + 8 * (q >> 2) + 4 * h + (q & 3);
            if (n >= a.rows) continue;
            float o = acc[i][q];
            if (GLU) {
                float g = o, u = accu[i][q];
                if (a.clamp > 0.0f) { // Glu::apply's clamp (cpu.rs:364-368)
                    g = fminf(g, a.clamp);
                    u = fminf(fmaxf(u, -a.clamp), a.clamp);
                }
                o = (ACT == 0 ? act_silu(g) : act_gelu_tanh(g)) * u;
            }
            orow[n] = to_stored<T>(o);
        }
    }
}

// The splits' partial rows added in split order, then the epilogue: one
// thread per output.
template <typename T, bool GLU, int ACT> __device__ static inline void qgemm_reduce_body(const QGemmArgs &a) {
    const int64_t e = (int64_t)blockIdx.x * CUCA_BLOCK + threadIdx.x;
    if (e >= (int64_t)a.m * a.rows) return;
    const int tok = (int)(e / a.rows), n = (int)(e - (int64_t)tok * a.rows);
    float g = 0.0f, u = 0.0f;
    for (int sp = 0; sp < a.splits; sp++) {
        g = g + a.part[((int64_t)sp * (GLU ? 2 : 1) * a.m + tok) * a.rows + n];
        if (GLU) u = u + a.part[((int64_t)(sp * 2 + 1) * a.m + tok) * a.rows + n];
    }
    float o = g;
    if (GLU) {
        if (a.clamp > 0.0f) { // Glu::apply's clamp (cpu.rs:364-368)
            g = fminf(g, a.clamp);
            u = fminf(fmaxf(u, -a.clamp), a.clamp);
        }
        o = (ACT == 0 ? act_silu(g) : act_gelu_tanh(g)) * u;
    }
    reinterpret_cast<T *>(a.out)[(int64_t)tok * a.out_ld + n] = to_stored<T>(o);
}

// Routed experts: the token tiles of the grouped GEMM.  One workgroup:
// thread 0 walks the experts (offsets clamped into [0, max_pairs] and made
// non-decreasing, so no pair index leaves the pair arrays), giving expert e
// ceil(n_e / tm) tiles from tile ts[e] on; then every tile c < n_ct gets
// its expert (a binary search over ts), first pair and pair count, or -1
// past the last tile.
#define QG_MOE_MAX_EXPERTS 4096
__device__ static inline void qgemm_moe_plan_body(const QGemmArgs &a) {
    __shared__ int ts[QG_MOE_MAX_EXPERTS + 1], lo[QG_MOE_MAX_EXPERTS + 1];
    const int E = a.n_experts, tm = a.tm;
    if (threadIdx.x == 0) {
        int prev = 0, t = 0;
        for (int e = 0; e < E; e++) {
            int l = a.offsets[e], hh = a.offsets[e + 1];
            l = min(max(l, prev), a.max_pairs);
            hh = min(max(hh, l), a.max_pairs);
            ts[e] = t;
            lo[e] = l;
            t += (hh - l + tm - 1) / tm;
            prev = hh;
        }
        ts[E] = t;
        lo[E] = prev;
    }
    __syncthreads();
    for (int c = threadIdx.x; c < a.n_ct; c += blockDim.x) {
        if (c >= ts[E]) {
            a.tile_e[c] = -1;
            a.tile_p0[c] = 0;
            a.tile_n[c] = 0;
            continue;
        }
        int l = 0, hh = E - 1; // the last e with ts[e] <= c (experts without pairs share ts)
        while (l < hh) {
            const int mid = (l + hh + 1) >> 1;
            if (ts[mid] <= c) l = mid;
            else hh = mid - 1;
        }
        const int p0 = lo[l] + (c - ts[l]) * tm;
        const int end = lo[l + 1]; // the clamped end of expert l's pairs
        a.tile_e[c] = l;
        a.tile_p0[c] = p0;
        a.tile_n[c] = min(tm, end - p0);
    }
}

// The activation rows of the routed pairs, rewritten as qgemm_prep_body does
// into the tile layout: padded row ct * tm + i holds pair tile_p0[ct] + i of
// the tile (zero past tile_n[ct]); up reads row pair_token[p] of x (a token
// outside [0, m) gives a zero row, reported), down row p.  Tiles past the
// last are not written (the GEMM skips them).
template <typename T, int FMT> __device__ static inline void qgemm_moe_prep_body(const QGemmArgs &a) {
    using F = QgFmt<FMT>;
    const int64_t u = (int64_t)blockIdx.x * CUCA_BLOCK + threadIdx.x;
    const int64_t per_row = (int64_t)a.nkc * 16;
    if (u >= (int64_t)a.mp * per_row) return;
    const int prow = (int)(u / per_row), rem = (int)(u - (int64_t)prow * per_row);
    const int ct = prow / a.tm, i = prow - ct * a.tm;
    if (a.tile_e[ct] < 0) return;
    const int kc = rem >> 4, v = rem & 15, s = v >> 1, h = v & 1;
    const int g = kc / F::KCG, part = kc % F::KCG;
    int base;
    if (FMT == 0) base = 512 * g + 128 * (2 * h + (s & 1)) + 4 * part + (s >> 1);
    else base = 256 * g + 128 * h + 8 * part + s;
    bool valid = i < a.tile_n[ct];
    int64_t src = 0;
    if (valid) {
        const int p = a.tile_p0[ct] + i;
        if (a.moe_up) {
            const int tok = a.pair_token[p];
            if (tok < 0 || tok >= a.m) {
                valid = false;
                if (rem == 0) record_bad(a.status + CUCA_STATUS_MOE_PAIR, (uint32_t)p, (uint32_t)tok);
            } else {
                src = tok;
            }
        } else {
            src = p;
        }
    }
    const T *row = reinterpret_cast<const T *>(a.x) + src * a.ldx;
    qg_h8 o;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int k = base + 16 * j;
        o[j] = valid && k < a.k ? (_Float16)(float)row[k] : (_Float16)0.0f;
    }
    *reinterpret_cast<qg_h8 *>(a.xp + (int64_t)prow * a.kp + (int64_t)kc * QG_KC + 8 * (2 * s + h)) = o;
}

#define CUCA_QGEMM(NAME, BODY, ...)                                                        \
    extern "C" __global__ __launch_bounds__(256) void NAME(QGemmArgs a) { BODY<__VA_ARGS__>(a); }
#define CUCA_QGEMM_TM(TN, T, FN, FMT, TM)                                                  \
    CUCA_QGEMM(cuca_qgemm_##TN##_##FN##_t##TM, qgemm_body, T, FMT, TM, false, 0, false)    \
    CUCA_QGEMM(cuca_qgemm_glu_##TN##_##FN##_silu_t##TM, qgemm_body, T, FMT, TM, true, 0, false) \
    CUCA_QGEMM(cuca_qgemm_glu_##TN##_##FN##_gelu_t##TM, qgemm_body, T, FMT, TM, true, 1, false) \
    CUCA_QGEMM(cuca_qgemm_##TN##_##FN##_t##TM##_split, qgemm_body, T, FMT, TM, false, 0, true) \
    CUCA_QGEMM(cuca_qgemm_glu_##TN##_##FN##_t##TM##_split, qgemm_body, T, FMT, TM, true, 0, true)
#define CUCA_QGEMM_SET(TN, T, FN, FMT)                                                     \
    CUCA_QGEMM(cuca_qgemm_prep_##TN##_##FN, qgemm_prep_body, T, FMT)                        \
    CUCA_QGEMM_TM(TN, T, FN, FMT, 32)                                                      \
    CUCA_QGEMM_TM(TN, T, FN, FMT, 64)                                                      \
    CUCA_QGEMM_TM(TN, T, FN, FMT, 128)
CUCA_QGEMM_SET(f32, float, q4_0, 0)
CUCA_QGEMM_SET(f32, float, q8_0, 1)
CUCA_QGEMM_SET(f16, _Float16, q4_0, 0)
CUCA_QGEMM_SET(f16, _Float16, q8_0, 1)
extern "C" __global__ __launch_bounds__(256) void cuca_qgemm_moe_plan(QGemmArgs a) { qgemm_moe_plan_body(a); }
#define CUCA_QGEMM_MOE_TM(TN, T, FN, FMT, TM)                                              \
    CUCA_QGEMM(cuca_qgemm_moe_up_##TN##_##FN##_silu_t##TM, qgemm_body, T, FMT, TM, true, 0, false, 1) \
    CUCA_QGEMM(cuca_qgemm_moe_up_##TN##_##FN##_gelu_t##TM, qgemm_body, T, FMT, TM, true, 1, false, 1) \
    CUCA_QGEMM(cuca_qgemm_moe_down_##TN##_##FN##_t##TM, qgemm_body, T, FMT, TM, false, 0, false, 2)
#define CUCA_QGEMM_MOE_SET(TN, T, FN, FMT)                                                 \
    CUCA_QGEMM(cuca_qgemm_moe_prep_##TN##_##FN, qgemm_moe_prep_body, T, FMT)               \
    CUCA_QGEMM_MOE_TM(TN, T, FN, FMT, 64)                                                  \
    CUCA_QGEMM_MOE_TM(TN, T, FN, FMT, 128)
CUCA_QGEMM_MOE_SET(f32, float, q4_0, 0)
CUCA_QGEMM_MOE_SET(f32, float, q8_0, 1)
CUCA_QGEMM_MOE_SET(f16, _Float16, q4_0, 0)
CUCA_QGEMM_MOE_SET(f16, _Float16, q8_0, 1)
#define CUCA_QGEMM_RED(TN, T)                                                              \
    CUCA_QGEMM(cuca_qgemm_reduce_##TN, qgemm_reduce_body, T, false, 0)                     \
    CUCA_QGEMM(cuca_qgemm_reduce_glu_##TN##_silu, qgemm_reduce_body, T, true, 0)           \
    CUCA_QGEMM(cuca_qgemm_reduce_glu_##TN##_gelu, qgemm_reduce_body, T, true, 1)
CUCA_QGEMM_RED(f32, float)
CUCA_QGEMM_RED(f16, _Float16)

// ---------------------------------------------------------------------
// The dense f16 path for many rows: the weight dequantised once into a
// resident f16 copy (the reference GPU engine's dense_dequant_kernel,
// moe_kernel.rs:1560-1600, with f16 output), then a plain f16 GEMM (the
// library's, f32 accumulation) and, for the GLU, the epilogue below.
// ---------------------------------------------------------------------

// One thread per (weight row, group, lane chunk l): the 2 G values l and
// l + 16 of the group's G blocks, w16[row][32 b + e] = f16(d_b * q), one
// rounding (the product of an f16 scale and a small integer is exact in
// f32) -- the values qgemm's operands carry.  Blocks past k (a partial last
// group) are not written.
template <int FMT> __device__ static inline void qdequant_body(const QDequantArgs &a) {
    constexpr int G = FMT == 0 ? 16 : 8, GB = FMT == 0 ? 288 : 272, SCB = 2 * G;
    const int64_t t = (int64_t)blockIdx.x * CUCA_BLOCK + threadIdx.x;
    if (t >= (int64_t)a.n * a.ng * 16) return;
    const int l = (int)(t & 15);
    const int64_t rg = t >> 4;
    const int g = (int)(rg % a.ng);
    const int64_t row = rg / a.ng;
    const uint8_t *grp = a.w + row * a.row_bytes + (int64_t)g * GB;
    const u32x4 chunk = *reinterpret_cast<const u32x4 *>(grp + SCB + 16 * l);
    const uint16_t *sc = reinterpret_cast<const uint16_t *>(grp);
    _Float16 *dst = reinterpret_cast<_Float16 *>(a.out) + row * a.out_ld;
#pragma unroll
    for (int b = 0; b < G; b++) {
        const int blk = g * G + b;
        if (blk >= a.nb) break;
        const float d = (float)__builtin_bit_cast(_Float16, sc[b]);
        int q0, q1; // elements l and l + 16
        if (FMT == 0) {
            const uint32_t w = chunk[b >> 2];
            q0 = (int)((w >> (4 * (b & 3))) & 15u) - 8;
            q1 = (int)((w >> (16 + 4 * (b & 3))) & 15u) - 8;
        } else {
            const uint32_t w = chunk[b >> 1];
            q0 = (int)((w >> (8 * (b & 1))) & 255u) - 128;
            q1 = (int)((w >> (16 + 8 * (b & 1))) & 255u) - 128;
        }
        dst[32 * blk + l] = (_Float16)(d * (float)q0);
        dst[32 * blk + l + 16] = (_Float16)(d * (float)q1);
    }
}
extern "C" __global__ __launch_bounds__(CUCA_BLOCK) void cuca_qdequant_q4_0(QDequantArgs a) { qdequant_body<0>(a); }
extern "C" __global__ __launch_bounds__(CUCA_BLOCK) void cuca_qdequant_q8_0(QDequantArgs a) { qdequant_body<1>(a); }

// Activations rounded to f16 (RNE), the GEMM's operand: x [m][ldx] f32 ->
// xh [m][k]; eight values per thread (k % 8 == 0).
extern "C" __global__ __launch_bounds__(CUCA_BLOCK) void cuca_cvt_f16_f32(QDequantArgs a) {
    const int64_t t = (int64_t)blockIdx.x * CUCA_BLOCK + threadIdx.x;
    const int64_t per = a.k / 8;
    if (t >= (int64_t)a.m * per) return;
    const int64_t r = t / per, c = (t - r * per) * 8;
    const float *src = reinterpret_cast<const float *>(a.x) + r * a.ldx + c;
    float v[8];
    qgemm_load8f(src, v);
    f16x8 h;
#pragma unroll
    for (int i = 0; i < 8; i++) h[i] = (_Float16)v[i];
    *reinterpret_cast<f16x8 *>(reinterpret_cast<_Float16 *>(a.out) + r * a.out_ld + c) = h;
}
