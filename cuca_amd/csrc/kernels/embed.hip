// embed.hip -- GGUF Q4_0 / Q8_0 token-embedding dequant-gather on gfx950.
//
// Replaces TokenEmbedding::rows / dequant_ggml_row (quant.rs:107-198,
// 391-411) and the GPU engine's host-side RowTable gather + upload
// (quant.rs:477-501, gpu.rs:2976-2982): the quantized table stays resident
// in HBM and the gather runs on the device.
//
// One wave per token, four tokens per workgroup.  Lane l owns the 8-value
// units l, l + 64, l + 128, ... of the row (UPL units per round, one round
// for hidden <= 512 UPL); each unit is the block's f16 scale plus 4 or 8
// quant bytes, read straight from the table row with 2-byte loads (a block
// starts on an even byte; the wave's loads cover the contiguous row, so
// the L1 turns them into whole cache lines and the row crosses HBM once).
// All of a round's loads are issued before the first is used: a lane has
// 5 UPL loads in flight.  The output -- 80 to 90 % of the bytes -- is
// written with 16-byte streaming stores, consecutive lanes on consecutive
// chunks.
//
// Measured on MI355X, 16384 Q8_0 tokens of 4096 -> f16, cold caches: 34.8
// us against 38.0 for a workgroup per token with one unit per lane per
// loop trip, and 47.3 for a wave that stages the row in LDS first (the
// LDS round trip costs more than the 2-byte loads, which hit in L1).
//
// Arithmetic is the reference's: d' = f32(d) * scale, then
// f32(q) * d' (two f32 roundings, in that order); f16 output is RNE of
// that f32.  Bit-exact.

#include "common.h"

// Issue the loads of a round's units: lane unit u = u0 + lane + 64 k holds
// the block's f16 scale (dq) and the 4 (Q4_0) or 8 (Q8_0) quant bytes of its
// 8 values (w, four 16-bit words).  A lane past the row end reloads the
// last unit.
template <int QT, int UPL>
__device__ static inline void embed_load(const uint16_t *s16, int u0, int lane, int nu, uint32_t (&dq)[UPL],
                                         uint32_t (&w)[UPL][4]) {
    constexpr int BS = QT == 2 ? 18 : 34; // bytes per 32-value block
#pragma unroll
    for (int k = 0; k < UPL; k++) {
        int u = u0 + lane + CUCA_WAVE * k;
        u = u < nu ? u : nu - 1;
        const int e0 = u * 8;
        const int ob = (e0 >> 5) * BS; // byte offset of the block (even)
        const int p = e0 & 31;         // first value within the block
        dq[k] = s16[ob >> 1];
        // Q4_0: byte j holds value j (low nibble) and j + 16 (high);
        // Q8_0: 32 signed bytes
        const int q0 = (ob + 2 + (QT == 2 ? (p & 15) : p)) >> 1;
#pragma unroll
        for (int j = 0; j < 4; j++) w[k][j] = s16[q0 + j];
    }
}

// The 8 values of unit u: d' = f32(d) * scale, then f32(q) * d'.
template <int QT>
__device__ static inline void embed_dequant(int u, uint32_t dq, const uint32_t (&w)[4], float scale,
                                            float (&v)[8]) {
    const int p = (u * 8) & 31;
    const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)dq) * scale;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        if (QT == 2) {
            const int sh = p >= 16 ? 4 : 0;
            v[2 * j] = (float)((int)((w[j] >> sh) & 0xfu) - 8) * d;
            v[2 * j + 1] = (float)((int)((w[j] >> (8 + sh)) & 0xfu) - 8) * d;
        } else {
            v[2 * j] = (float)(int8_t)(w[j] & 0xffu) * d;
            v[2 * j + 1] = (float)(int8_t)(w[j] >> 8) * d;
        }
    }
}

template <typename OutT>
__device__ static inline void embed_store(OutT *orow, int u, const float (&v)[8]) {
    constexpr int CPU = 8 / Chunk<OutT>::N; // output chunks per unit
    if (CPU == 1) {
        Chunk<OutT>::store_nt(orow, u, reinterpret_cast<const float(&)[Chunk<OutT>::N]>(v));
    } else {
        Chunk<OutT>::store_nt(orow, 2 * u, reinterpret_cast<const float(&)[Chunk<OutT>::N]>(v[0]));
        Chunk<OutT>::store_nt(orow, 2 * u + 1, reinterpret_cast<const float(&)[Chunk<OutT>::N]>(v[4]));
    }
}

// An id the host could not see: a zero row, no read outside the table,
// and the id reported.
template <typename OutT>
__device__ static inline void embed_bad_id(const EmbedArgs &a, OutT *orow, int tok, uint32_t id, int lane) {
    constexpr int CPU = 8 / Chunk<OutT>::N;
    if (lane == 0) record_bad(a.status + CUCA_STATUS_EMBED_ID, (uint32_t)tok, id);
    float z[Chunk<OutT>::N];
#pragma unroll
    for (int i = 0; i < Chunk<OutT>::N; i++) z[i] = 0.0f;
    for (int c = lane; c < a.hidden / 8 * CPU; c += CUCA_WAVE) Chunk<OutT>::store_nt(orow, c, z);
}

template <int QT, typename OutT, int UPL>
__device__ static inline void embed_body(const EmbedArgs &a) {
    const int tok = blockIdx.x * (CUCA_BLOCK / CUCA_WAVE) + (int)(threadIdx.x / CUCA_WAVE);
    const int lane = threadIdx.x & (CUCA_WAVE - 1);
    if (tok >= a.n) return; // whole wave
    const int nu = a.hidden / 8;
    OutT *orow = reinterpret_cast<OutT *>(a.out) + (int64_t)tok * a.hidden;
    const uint32_t id = a.ids[tok];
    if ((int64_t)id >= a.vocab) {
        embed_bad_id<OutT>(a, orow, tok, id, lane);
        return;
    }
    const uint16_t *s16 = reinterpret_cast<const uint16_t *>(a.table + (int64_t)id * a.row_bytes);
    for (int u0 = 0; u0 < nu; u0 += CUCA_WAVE * UPL) {
        uint32_t dq[UPL], w[UPL][4];
        embed_load<QT, UPL>(s16, u0, lane, nu, dq, w);
#pragma unroll
        for (int k = 0; k < UPL; k++) {
            const int u = u0 + lane + CUCA_WAVE * k;
            float v[8];
            embed_dequant<QT>(u, dq[k], w[k], a.scale, v);
            if (u < nu) embed_store<OutT>(orow, u, v);
        }
    }
}

// rms_norm_rows (quant.rs:324-339) after the gather, for the archs whose
// looked-up rows get the scale-less norm (Hparams::norm_embeddings,
// params.rs:374-379): sum = the f64 squares of the row's f32 values summed
// in index order, inv = (f32)(1 / sqrt(sum / hidden + f64(eps))), x * inv.
//
// The wave sums the squares in its own order (per lane, then a butterfly).
// Every square is exact in f64, so any order's sum is within
// (hidden - 1) 2^-53 sum of the exact one, and the reference's sequential
// sum too: the two differ by less than B = 2.02 hidden 2^-53 sum.  inv as a
// function of the sum is monotone (every step is a correctly rounded
// monotone operation), so when inv(sum + B) and inv(sum - B), each widened
// by 2^-50 for the division and root, round to the same f32, that f32 is
// the reference's inv.  Otherwise (about 2^-17 of the rows of 4096) lane 0
// re-reads the row and sums in the reference's order.
template <int QT>
__device__ static inline float embed_norm_inv(const uint16_t *s16, double sum, int hidden, float scale,
                                              float eps, int lane) {
    const double n = (double)hidden, e = (double)eps;
    const double b = sum * (2.02 * n * 0x1p-53);
    const float lo = (float)((1.0 / __builtin_sqrt((sum + b) / n + e)) * (1.0 - 0x1p-50));
    const float hi = (float)((1.0 / __builtin_sqrt((sum - b) / n + e)) * (1.0 + 0x1p-50));
    if (lo == hi) return lo; // wave-uniform: every lane holds the same sum
    double s = 0.0;
    if (lane == 0) {
        constexpr int BS = QT == 2 ? 18 : 34;
        const uint8_t *row = reinterpret_cast<const uint8_t *>(s16);
        for (int blk = 0; blk < hidden / 32; blk++) {
            const uint8_t *p = row + blk * BS;
            const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)(p[0] | (p[1] << 8))) * scale;
            for (int j = 0; j < 32; j++) {
                int q;
                if (QT == 2) q = (int)((j < 16 ? p[2 + j] : p[2 + j - 16] >> 4) & 0xf) - 8;
                else q = (int)(int8_t)p[2 + j];
                const float x = (float)q * d;
                s = s + (double)x * (double)x;
            }
        }
    }
    s = __shfl(s, 0, CUCA_WAVE);
    return (float)(1.0 / __builtin_sqrt(s / n + e));
}

template <int QT, typename OutT, int UPL>
__device__ static inline void embed_norm_body(const EmbedArgs &a) {
    const int tok = blockIdx.x * (CUCA_BLOCK / CUCA_WAVE) + (int)(threadIdx.x / CUCA_WAVE);
    const int lane = threadIdx.x & (CUCA_WAVE - 1);
    if (tok >= a.n) return; // whole wave
    const int nu = a.hidden / 8;
    OutT *orow = reinterpret_cast<OutT *>(a.out) + (int64_t)tok * a.hidden;
    const uint32_t id = a.ids[tok];
    if ((int64_t)id >= a.vocab) {
        embed_bad_id<OutT>(a, orow, tok, id, lane);
        return;
    }
    const uint16_t *s16 = reinterpret_cast<const uint16_t *>(a.table + (int64_t)id * a.row_bytes);
    // pass 1: the squares; a row of one round keeps its values in registers
    const bool one_round = nu <= CUCA_WAVE * UPL;
    float v[UPL][8];
    double sum = 0.0;
    for (int u0 = 0; u0 < nu; u0 += CUCA_WAVE * UPL) {
        uint32_t dq[UPL], w[UPL][4];
        embed_load<QT, UPL>(s16, u0, lane, nu, dq, w);
#pragma unroll
        for (int k = 0; k < UPL; k++) {
            const int u = u0 + lane + CUCA_WAVE * k;
            embed_dequant<QT>(u, dq[k], w[k], a.scale, v[k]);
            if (u < nu) {
#pragma unroll
                for (int j = 0; j < 8; j++) sum += (double)v[k][j] * (double)v[k][j];
            }
        }
    }
#pragma unroll
    for (int off = CUCA_WAVE / 2; off >= 1; off >>= 1) sum += __shfl_xor(sum, off, CUCA_WAVE);
    const float inv = embed_norm_inv<QT>(s16, sum, a.hidden, a.scale, a.norm_eps, lane);
    // pass 2: x * inv, from registers or re-read (the row is in cache)
    for (int u0 = 0; u0 < nu; u0 += CUCA_WAVE * UPL) {
        if (!one_round) {
            uint32_t dq[UPL], w[UPL][4];
            embed_load<QT, UPL>(s16, u0, lane, nu, dq, w);
#pragma unroll
            for (int k = 0; k < UPL; k++) embed_dequant<QT>(u0 + lane + CUCA_WAVE * k, dq[k], w[k], a.scale, v[k]);
        }
#pragma unroll
        for (int k = 0; k < UPL; k++) {
            const int u = u0 + lane + CUCA_WAVE * k;
            float y[8];
#pragma unroll
            for (int j = 0; j < 8; j++) y[j] = v[k][j] * inv;
            if (u < nu) embed_store<OutT>(orow, u, y);
        }
    }
}

// The gather fused with the first block's attention norm (cpu.rs:2670-2673:
// h = rms(x, attn_norm, eps) over the block's input, which for the first
// block is the gathered row): x is stored as the plain gather stores it
// (bit-identical), and h = x * (1 / sqrt(mean(x^2) + eps)) * w is computed
// from the stored values -- what the norm kernel would read back -- in the
// norm kernel's form, each product rounded to f32 before the store rounds
// it.  The sum of squares is the wave's own order (per lane in unit order,
// then a butterfly): within the norm's bar of the reference, not its bits.
// The weights are read while the token id is in flight; a row of more than
// one round re-reads the table row (in cache) for h.
template <int QT, typename OutT, int UPL>
__device__ static inline void embed_rms_body(const EmbedArgs &a) {
    const int tok = blockIdx.x * (CUCA_BLOCK / CUCA_WAVE) + (int)(threadIdx.x / CUCA_WAVE);
    const int lane = threadIdx.x & (CUCA_WAVE - 1);
    if (tok >= a.n) return; // whole wave
    const int nu = a.hidden / 8;
    OutT *orow = reinterpret_cast<OutT *>(a.out) + (int64_t)tok * a.hidden;
    OutT *hrow = reinterpret_cast<OutT *>(a.h_out) + (int64_t)tok * a.hidden;
    const uint32_t id = a.ids[tok];
    const bool one_round = nu <= CUCA_WAVE * UPL;
    // up to 4 units per lane the weights are read up front (64 more
    // registers at 8 units would cost half the waves)
    constexpr bool PRE = UPL <= 4;
    float wv[UPL][8];
    if (PRE && one_round && a.rms_w) {
#pragma unroll
        for (int k = 0; k < UPL; k++) {
            int u = lane + CUCA_WAVE * k;
            u = u < nu ? u : 0;
            const f32x4 *wp = reinterpret_cast<const f32x4 *>(a.rms_w) + 2 * u;
            const f32x4 w0 = wp[0], w1 = wp[1];
            wv[k][0] = w0.x; wv[k][1] = w0.y; wv[k][2] = w0.z; wv[k][3] = w0.w;
            wv[k][4] = w1.x; wv[k][5] = w1.y; wv[k][6] = w1.z; wv[k][7] = w1.w;
        }
    }
    if ((int64_t)id >= a.vocab) {
        embed_bad_id<OutT>(a, orow, tok, id, lane);
        float z[Chunk<OutT>::N];
#pragma unroll
        for (int i = 0; i < Chunk<OutT>::N; i++) z[i] = 0.0f;
        constexpr int CPU = 8 / Chunk<OutT>::N;
        for (int c = lane; c < nu * CPU; c += CUCA_WAVE) Chunk<OutT>::store_nt(hrow, c, z);
        return;
    }
    const uint16_t *s16 = reinterpret_cast<const uint16_t *>(a.table + (int64_t)id * a.row_bytes);
    // a row of one round keeps its raw blocks (5 registers per unit) and
    // dequantises them again for h: the same bits as the first time
    uint32_t dq[UPL], w[UPL][4];
    float ss = 0.0f;
    for (int u0 = 0; u0 < nu; u0 += CUCA_WAVE * UPL) {
        embed_load<QT, UPL>(s16, u0, lane, nu, dq, w);
#pragma unroll
        for (int k = 0; k < UPL; k++) {
            const int u = u0 + lane + CUCA_WAVE * k;
            float v[8];
            embed_dequant<QT>(u, dq[k], w[k], a.scale, v);
            if (u < nu) {
                embed_store<OutT>(orow, u, v);
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const float x = Chunk<OutT>::as_stored(v[j]);
                    ss += x * x;
                }
            }
        }
    }
    ss = group_sum<CUCA_WAVE>(ss);
    const float inv = 1.0f / sqrtf(ss / (float)a.hidden + a.rms_eps);
    for (int u0 = 0; u0 < nu; u0 += CUCA_WAVE * UPL) {
        if (!one_round) embed_load<QT, UPL>(s16, u0, lane, nu, dq, w);
        if ((!one_round || !PRE) && a.rms_w) {
#pragma unroll
            for (int k = 0; k < UPL; k++) {
                int u = u0 + lane + CUCA_WAVE * k;
                u = u < nu ? u : 0;
                const f32x4 *wp = reinterpret_cast<const f32x4 *>(a.rms_w) + 2 * u;
                const f32x4 w0 = wp[0], w1 = wp[1];
                wv[k][0] = w0.x; wv[k][1] = w0.y; wv[k][2] = w0.z; wv[k][3] = w0.w;
                wv[k][4] = w1.x; wv[k][5] = w1.y; wv[k][6] = w1.z; wv[k][7] = w1.w;
            }
        }
#pragma unroll
        for (int k = 0; k < UPL; k++) {
            const int u = u0 + lane + CUCA_WAVE * k;
            float v[8], y[8];
            embed_dequant<QT>(u, dq[k], w[k], a.scale, v);
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = Chunk<OutT>::as_stored(v[j]);
            if (a.rms_w) {
#pragma unroll
                for (int j = 0; j < 8; j++) y[j] = pin_f32(pin_f32(v[j] * inv) * wv[k][j]);
            } else {
#pragma unroll
                for (int j = 0; j < 8; j++) y[j] = pin_f32(v[j] * inv);
            }
            if (u < nu) embed_store<OutT>(hrow, u, y);
        }
    }
}

// The fused gather for many tokens: the norm weights staged in LDS once per
// workgroup, each wave looping over a.tpw tokens.  Lane l owns the units l,
// l + 64, ... (UPL of them, one round: hidden <= 512 UPL) and keeps only
// their raw blocks between the two passes, dequantising again for h (the
// same bits as the first time).  A token's weights come from LDS, not from
// the L2 (16 KB per token at hidden 4096, as many bytes as the token's
// output), and the small register set keeps 7 waves per SIMD.
template <int QT, typename OutT, int UPL>
__device__ static inline void embed_rms_lds_body(const EmbedArgs &a) {
    extern __shared__ float wsh[]; // [hidden]
    const int lane = threadIdx.x & (CUCA_WAVE - 1), wave = threadIdx.x / CUCA_WAVE;
    const int nu = a.hidden / 8;
    const bool has_w = a.rms_w != nullptr;
    if (has_w) {
        const f32x4 *src = reinterpret_cast<const f32x4 *>(a.rms_w);
        f32x4 *dst = reinterpret_cast<f32x4 *>(wsh);
        for (int i = threadIdx.x; i < a.hidden / 4; i += CUCA_BLOCK) dst[i] = src[i];
        __syncthreads();
    }
    constexpr int WPB = CUCA_BLOCK / CUCA_WAVE;
    for (int it = 0; it < a.tpw; it++) {
        // consecutive waves of a workgroup on consecutive tokens
        const int tok = (blockIdx.x * a.tpw + it) * WPB + wave;
        if (tok >= a.n) return; // the wave's later tokens are further on
        OutT *orow = reinterpret_cast<OutT *>(a.out) + (int64_t)tok * a.hidden;
        OutT *hrow = reinterpret_cast<OutT *>(a.h_out) + (int64_t)tok * a.hidden;
        const uint32_t id = a.ids[tok];
        if ((int64_t)id >= a.vocab) {
            embed_bad_id<OutT>(a, orow, tok, id, lane);
            float z[Chunk<OutT>::N];
#pragma unroll
            for (int i = 0; i < Chunk<OutT>::N; i++) z[i] = 0.0f;
            constexpr int CPU = 8 / Chunk<OutT>::N;
            for (int c = lane; c < nu * CPU; c += CUCA_WAVE) Chunk<OutT>::store_nt(hrow, c, z);
            continue;
        }
        const uint16_t *s16 = reinterpret_cast<const uint16_t *>(a.table + (int64_t)id * a.row_bytes);
        uint32_t dq[UPL], w[UPL][4];
        embed_load<QT, UPL>(s16, 0, lane, nu, dq, w);
        float ss = 0.0f;
#pragma unroll
        for (int k = 0; k < UPL; k++) {
            const int u = lane + CUCA_WAVE * k;
            float v[8];
            embed_dequant<QT>(u, dq[k], w[k], a.scale, v);
            if (u < nu) {
                embed_store<OutT>(orow, u, v);
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const float x = Chunk<OutT>::as_stored(v[j]);
                    ss += x * x;
                }
            }
        }
        ss = group_sum<CUCA_WAVE>(ss);
        const float inv = 1.0f / sqrtf(ss / (float)a.hidden + a.rms_eps);
        // opaque to the compiler, so the second dequantisation is computed
        // again instead of keeping the first pass's 8 UPL values live
#pragma unroll
        for (int k = 0; k < UPL; k++) {
            asm volatile("" : "+v"(dq[k]));
#pragma unroll
            for (int j = 0; j < 4; j++) asm volatile("" : "+v"(w[k][j]));
        }
#pragma unroll
        for (int k = 0; k < UPL; k++) {
            const int u = lane + CUCA_WAVE * k;
            float v[8], y[8];
            embed_dequant<QT>(u, dq[k], w[k], a.scale, v);
            if (has_w) {
                const int ul = u < nu ? u : 0;
                const f32x4 w0 = reinterpret_cast<const f32x4 *>(wsh)[2 * ul];
                const f32x4 w1 = reinterpret_cast<const f32x4 *>(wsh)[2 * ul + 1];
                const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
                for (int j = 0; j < 8; j++) y[j] = pin_f32(pin_f32(Chunk<OutT>::as_stored(v[j]) * inv) * wv[j]);
            } else {
#pragma unroll
                for (int j = 0; j < 8; j++) y[j] = pin_f32(Chunk<OutT>::as_stored(v[j]) * inv);
            }
            if (u < nu) embed_store<OutT>(hrow, u, y);
        }
    }
}

// Unit u of a row as two words: its block's f16 scale (d) and its 8 quant
// bytes (q, packed; for Q4_0 the 8 bytes whose low or high nibbles hold the
// unit's values).  The 8-byte load is 2-byte aligned (a block is 18 or 34
// bytes), which global loads allow.
typedef uint32_t u32x2_a2 __attribute__((ext_vector_type(2), aligned(2)));
template <int QT>
__device__ static inline void embed_unit_load(const uint8_t *row, int u, uint32_t &d, u32x2_a2 &q) {
    constexpr int BS = QT == 2 ? 18 : 34;
    const int e0 = u * 8, ob = (e0 >> 5) * BS, p = e0 & 31;
    d = *reinterpret_cast<const uint16_t *>(row + ob);
    q = *reinterpret_cast<const u32x2_a2 *>(row + ob + 2 + (QT == 2 ? (p & 15) : p));
}
// The unit's 8 values from the packed words: the same arithmetic as
// embed_dequant (d' = f32(d) * scale, then f32(q) * d').
// (Q8_0: the 8 bytes as one vector of int8, so each conversion is one
// byte-select convert; extracted by shifts, one of them compiled to a 64-bit
// integer conversion of a dozen instructions)
template <int QT>
__device__ static inline void embed_unit_dequant(int u, uint32_t dq, u32x2_a2 q, float scale, float (&v)[8]) {
    const int p = (u * 8) & 31;
    const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)dq) * scale;
    if constexpr (QT == 2) {
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t b = (q[i >> 2] >> (8 * (i & 3))) & 0xffu;
            v[i] = (float)((int)((b >> (p >= 16 ? 4 : 0)) & 0xfu) - 8) * d;
        }
    } else {
        typedef int8_t i8x8 __attribute__((ext_vector_type(8)));
        const i8x8 b = __builtin_bit_cast(i8x8, q);
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = (float)b[i] * d;
    }
}

// A unit's 8 output values as the row holds them (f16: 16 packed bytes; f32:
// two 16-byte chunks), so that a bad id zeroes the packed words and the
// norm reads the stored values back from them.
template <typename OutT> struct EmbedOut;
template <> struct EmbedOut<_Float16> {
    u32x4 p;
    __device__ inline void set(const float (&v)[8]) {
        f16x8 h;
#pragma unroll
        for (int i = 0; i < 8; i++) h[i] = (_Float16)pin_f32(v[i]);
        p = __builtin_bit_cast(u32x4, h);
    }
    __device__ inline void zero_if(bool z) { p = z ? u32x4{0u, 0u, 0u, 0u} : p; }
    __device__ inline void store_nt(void *row, int u) const {
        __builtin_nontemporal_store(p, reinterpret_cast<u32x4 *>(row) + u);
    }
    __device__ inline void values(float (&v)[8]) const { Chunk<_Float16>::widen(p, v); }
};
template <> struct EmbedOut<float> {
    float x[8];
    __device__ inline void set(const float (&v)[8]) {
#pragma unroll
        for (int i = 0; i < 8; i++) x[i] = v[i];
    }
    __device__ inline void zero_if(bool z) {
#pragma unroll
        for (int i = 0; i < 8; i++) x[i] = z ? 0.0f : x[i];
    }
    __device__ inline void store_nt(void *row, int u) const { embed_store<float>(reinterpret_cast<float *>(row), u, x); }
    __device__ inline void values(float (&v)[8]) const {
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = x[i];
    }
};

// The fused gather for many tokens, as persistent workgroups: TPR threads
// per token (thread t owns unit t: hidden = 8 TPR), each workgroup taking
// TPW tokens it * gridDim.x + blockIdx.x (it < TPW; the launch sizes the
// grid to what the device holds at once, so every iteration of the grid
// covers a contiguous range of tokens).  A thread's 8 norm weights stay in
// registers for all its tokens, and the token ids come in one load.  The
// loop is unrolled, and the next token's unit is loaded before the current
// token's stores.  The sum of squares is the workgroup-per-token kernel's
// order (per thread, a wave butterfly, an LDS sum in wave order), so h has
// its bits; x is the plain gather's.  36 registers: 8 waves per SIMD.
// Its instruction count matters (the VALU is busy about two thirds of the
// kernel's time): the Q8_0 bytes convert as one int8 vector, a bad id zeroes
// the packed words rather than each value, the norm reads the stored values
// back from the packed words (one conversion a value), no weights is a
// weight of 1 (x * 1 == x) rather than a second code path, and the mean is
// the sum times 1 / hidden (exact: hidden is 8 TPR).  A quarter fewer
// instructions a token, the same bits: 61.0-61.4 -> 59.8-60.0 us in the
// config C step at 16384 tokens (0.69 -> 0.71 of the HBM peak), A/B in one
// process.
// Measured in the config C prefill step on MI355X (16384 Q8_0 tokens of 4096
// -> f16): 61.3-61.6 us against 65.2-65.4 for the LDS-weights wave-per-token
// kernel (0.69 against 0.65 of the HBM peak); 8 tokens per workgroup (two
// rounds of workgroups) 64.6, 4 tokens 68.5; two units per thread 65.7.
template <int QT, typename OutT, int TPR, int TPW>
__device__ static inline void embed_rms_persist_body(const EmbedArgs &a) {
    constexpr int NW = TPR / CUCA_WAVE;
    static_assert(TPW <= CUCA_WAVE, "one lane per token id");
    __shared__ float red[2][NW];
    const int t = threadIdx.x, lane = t & (CUCA_WAVE - 1), wave = t / CUCA_WAVE;
    const int G = gridDim.x;
    // (no weights: 1, and x * 1 is x exactly, so one form serves both)
    float wv[8];
    if (a.rms_w != nullptr) {
        const f32x4 *wp = reinterpret_cast<const f32x4 *>(a.rms_w) + 2 * t;
        const f32x4 w0 = wp[0], w1 = wp[1];
        wv[0] = w0.x; wv[1] = w0.y; wv[2] = w0.z; wv[3] = w0.w;
        wv[4] = w1.x; wv[5] = w1.y; wv[6] = w1.z; wv[7] = w1.w;
    } else {
#pragma unroll
        for (int j = 0; j < 8; j++) wv[j] = 1.0f;
    }
    // lane i holds the id of the workgroup's token i (tokens past n read
    // the last token's id, so every load below stays inside the table)
    uint32_t idv;
    {
        const int tk = (lane < TPW ? lane : 0) * G + (int)blockIdx.x;
        idv = a.ids[tk < a.n ? tk : a.n - 1];
    }
    auto id_at = [&](int it) -> uint32_t { return (uint32_t)__builtin_amdgcn_readlane((int)idv, it); };
    auto row_of = [&](uint32_t id) {
        return a.table + (int64_t)((int64_t)id < a.vocab ? id : 0u) * a.row_bytes;
    };
    uint32_t dq[TPW];
    u32x2_a2 q[TPW];
    embed_unit_load<QT>(row_of(id_at(0)), t, dq[0], q[0]);
#pragma unroll
    for (int it = 0; it < TPW; it++) {
        const int tok = it * G + (int)blockIdx.x;
        const uint32_t id = id_at(it);
        // (opaque until here: otherwise the byte extraction of a unit loaded
        // ahead is hoisted next to its load, which then waits for it)
        asm volatile("" : "+v"(dq[it]), "+v"(q[it]));
        if (it + 1 < TPW) embed_unit_load<QT>(row_of(id_at(it + 1)), t, dq[it + 1], q[it + 1]);
        if (tok < a.n) { // uniform over the workgroup
            OutT *orow = reinterpret_cast<OutT *>(a.out) + (int64_t)tok * a.hidden;
            OutT *hrow = reinterpret_cast<OutT *>(a.h_out) + (int64_t)tok * a.hidden;
            const bool bad = (int64_t)id >= a.vocab;
            if (bad && t == 0) record_bad(a.status + CUCA_STATUS_EMBED_ID, (uint32_t)tok, id);
            float v[8];
            embed_unit_dequant<QT>(t, dq[it], q[it], a.scale, v);
            EmbedOut<OutT> xo;
            xo.set(v);
            xo.zero_if(bad);
            xo.store_nt(orow, t);
            xo.values(v); // the stored values (zeros for a bad id)
            float ss = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; j++) ss += v[j] * v[j];
            ss = group_sum<CUCA_WAVE>(ss);
            // two slots, alternating: a wave that runs ahead writes the other
            // slot, and cannot come back to this one before every wave has
            // passed the next barrier (so has read this one)
            if (lane == 0) red[it & 1][wave] = ss;
            __syncthreads();
            ss = 0.0f;
#pragma unroll
            for (int i = 0; i < NW; i++) ss += red[it & 1][i];
            // (hidden = 8 TPR, a power of two: the sum times 1 / hidden is the
            // division's value)
            const float inv = 1.0f / sqrtf(ss * (1.0f / (8 * TPR)) + a.rms_eps);
            float y[8];
#pragma unroll
            for (int j = 0; j < 8; j++) y[j] = pin_f32(pin_f32(v[j] * inv) * wv[j]);
            EmbedOut<OutT> ho;
            ho.set(y);
            ho.zero_if(bad);
            ho.store_nt(hrow, t);
        }
    }
}

#define CUCA_EMBED_P(NAME, QT, OUT, TPR, TPW)                                              \
    extern "C" __global__ __launch_bounds__(TPR) void NAME(EmbedArgs a) {                  \
        embed_rms_persist_body<QT, OUT, TPR, TPW>(a);                                      \
    }
#define CUCA_EMBED_P_SET(NAME, QT, OUT)                                                    \
    CUCA_EMBED_P(NAME##_rms_p256_w8, QT, OUT, 256, 8)                                      \
    CUCA_EMBED_P(NAME##_rms_p256_w16, QT, OUT, 256, 16)                                    \
    CUCA_EMBED_P(NAME##_rms_p256_w32, QT, OUT, 256, 32)                                    \
    CUCA_EMBED_P(NAME##_rms_p512_w8, QT, OUT, 512, 8)                                      \
    CUCA_EMBED_P(NAME##_rms_p512_w16, QT, OUT, 512, 16)                                    \
    CUCA_EMBED_P(NAME##_rms_p512_w32, QT, OUT, 512, 32)
CUCA_EMBED_P_SET(cuca_embed_q4_0_f32, 2, float)
CUCA_EMBED_P_SET(cuca_embed_q4_0_f16, 2, _Float16)
CUCA_EMBED_P_SET(cuca_embed_q8_0_f32, 8, float)
CUCA_EMBED_P_SET(cuca_embed_q8_0_f16, 8, _Float16)

// The same with a workgroup per token: TPR threads (a power of two, 64 to
// 1024), thread t owning units t, t + TPR, ... (NU of them), the sum of
// squares a butterfly per wave and an LDS sum over the waves in wave order.
// Each thread holds one or two units, so many tokens are in flight per CU.
template <int QT, typename OutT, int TPR, int NU>
__device__ static inline void embed_rms_tpr_body(const EmbedArgs &a) {
    constexpr int NW = TPR / CUCA_WAVE;
    __shared__ float red[NW];
    const int tok = blockIdx.x;
    const int t = threadIdx.x, lane = t & (CUCA_WAVE - 1), wave = t / CUCA_WAVE;
    const int nu = a.hidden / 8;
    OutT *orow = reinterpret_cast<OutT *>(a.out) + (int64_t)tok * a.hidden;
    OutT *hrow = reinterpret_cast<OutT *>(a.h_out) + (int64_t)tok * a.hidden;
    const uint32_t id = a.ids[tok];
    // (no weights: 1, and x * 1 is x exactly, so one form serves both)
    float wv[NU][8];
#pragma unroll
    for (int k = 0; k < NU; k++) {
        if (a.rms_w) {
            int u = t + TPR * k;
            u = u < nu ? u : 0;
            const f32x4 *wp = reinterpret_cast<const f32x4 *>(a.rms_w) + 2 * u;
            const f32x4 w0 = wp[0], w1 = wp[1];
            wv[k][0] = w0.x; wv[k][1] = w0.y; wv[k][2] = w0.z; wv[k][3] = w0.w;
            wv[k][4] = w1.x; wv[k][5] = w1.y; wv[k][6] = w1.z; wv[k][7] = w1.w;
        } else {
#pragma unroll
            for (int j = 0; j < 8; j++) wv[k][j] = 1.0f;
        }
    }
    constexpr int CPU = 8 / Chunk<OutT>::N;
    if ((int64_t)id >= a.vocab) { // uniform over the workgroup
        if (t == 0) record_bad(a.status + CUCA_STATUS_EMBED_ID, (uint32_t)tok, id);
        float z[Chunk<OutT>::N];
#pragma unroll
        for (int i = 0; i < Chunk<OutT>::N; i++) z[i] = 0.0f;
        for (int c = t; c < nu * CPU; c += TPR) {
            Chunk<OutT>::store_nt(orow, c, z);
            Chunk<OutT>::store_nt(hrow, c, z);
        }
        return;
    }
    const uint16_t *s16 = reinterpret_cast<const uint16_t *>(a.table + (int64_t)id * a.row_bytes);
    uint32_t dq[NU], w[NU][4];
#pragma unroll
    for (int k = 0; k < NU; k++) {
        uint32_t d1[1], w1[1][4];
        embed_load<QT, 1>(s16, TPR * k + (t - lane), lane, nu, d1, w1);
        dq[k] = d1[0];
#pragma unroll
        for (int j = 0; j < 4; j++) w[k][j] = w1[0][j];
    }
    float v[NU][8];
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < NU; k++) {
        const int u = t + TPR * k;
        embed_dequant<QT>(u, dq[k], w[k], a.scale, v[k]);
        if (u < nu) {
            // stored, and read back from the packed words (the stored values)
            EmbedOut<OutT> xo;
            xo.set(v[k]);
            xo.store_nt(orow, u);
            xo.values(v[k]);
#pragma unroll
            for (int j = 0; j < 8; j++) ss += v[k][j] * v[k][j];
        }
    }
    ss = group_sum<CUCA_WAVE>(ss);
    if (NW > 1) {
        if (lane == 0) red[wave] = ss;
        __syncthreads();
        ss = 0.0f;
#pragma unroll
        for (int i = 0; i < NW; i++) ss += red[i];
    }
    // the mean: for a power-of-two hidden (uniform) the sum times 1 / hidden,
    // the division's value without the division's instructions
    float mean;
    if ((a.hidden & (a.hidden - 1)) == 0)
        mean = ss * __builtin_amdgcn_ldexpf(1.0f, -__builtin_ctz((unsigned)a.hidden));
    else
        mean = ss / (float)a.hidden;
    const float inv = 1.0f / sqrtf(mean + a.rms_eps);
#pragma unroll
    for (int k = 0; k < NU; k++) {
        const int u = t + TPR * k;
        float y[8];
#pragma unroll
        for (int j = 0; j < 8; j++) y[j] = pin_f32(pin_f32(v[k][j] * inv) * wv[k][j]);
        if (u < nu) embed_store<OutT>(hrow, u, y);
    }
}

#define CUCA_EMBED_TPR(NAME, QT, OUT, TPR, NU)                                             \
    extern "C" __global__ __launch_bounds__(TPR) void NAME(EmbedArgs a) {                  \
        embed_rms_tpr_body<QT, OUT, TPR, NU>(a);                                           \
    }
#define CUCA_EMBED_TPR_SET(NAME, QT, OUT)                                                  \
    CUCA_EMBED_TPR(NAME##_rms_t64, QT, OUT, 64, 1)                                         \
    CUCA_EMBED_TPR(NAME##_rms_t128, QT, OUT, 128, 1)                                       \
    CUCA_EMBED_TPR(NAME##_rms_t256, QT, OUT, 256, 1)                                       \
    CUCA_EMBED_TPR(NAME##_rms_t512, QT, OUT, 512, 1)                                       \
    CUCA_EMBED_TPR(NAME##_rms_t1024, QT, OUT, 1024, 1)                                     \
    CUCA_EMBED_TPR(NAME##_rms_t1024_c2, QT, OUT, 1024, 2)
CUCA_EMBED_TPR_SET(cuca_embed_q4_0_f32, 2, float)
CUCA_EMBED_TPR_SET(cuca_embed_q4_0_f16, 2, _Float16)
CUCA_EMBED_TPR_SET(cuca_embed_q8_0_f32, 8, float)
CUCA_EMBED_TPR_SET(cuca_embed_q8_0_f16, 8, _Float16)

#define CUCA_EMBED(NAME, BODY, QT, OUT, UPL)                                               \
    extern "C" __global__ __launch_bounds__(CUCA_BLOCK) void NAME(EmbedArgs a) {           \
        BODY<QT, OUT, UPL>(a);                                                             \
    }
#define CUCA_EMBED_LDS(NAME, QT, OUT, UPL)                                                 \
    extern "C" __global__ __launch_bounds__(CUCA_BLOCK) void NAME(EmbedArgs a) {           \
        embed_rms_lds_body<QT, OUT, UPL>(a);                                               \
    }
#define CUCA_EMBED_SET(NAME, QT, OUT)                                                      \
    CUCA_EMBED(NAME##_u1, embed_body, QT, OUT, 1)                                          \
    CUCA_EMBED(NAME##_u2, embed_body, QT, OUT, 2)                                          \
    CUCA_EMBED(NAME##_u4, embed_body, QT, OUT, 4)                                          \
    CUCA_EMBED(NAME##_u8, embed_body, QT, OUT, 8)                                          \
    CUCA_EMBED(NAME##_norm_u1, embed_norm_body, QT, OUT, 1)                                \
    CUCA_EMBED(NAME##_norm_u2, embed_norm_body, QT, OUT, 2)                                \
    CUCA_EMBED(NAME##_norm_u4, embed_norm_body, QT, OUT, 4)                                \
    CUCA_EMBED(NAME##_norm_u8, embed_norm_body, QT, OUT, 8)                                \
    CUCA_EMBED(NAME##_rms_u1, embed_rms_body, QT, OUT, 1)                                  \
    CUCA_EMBED(NAME##_rms_u2, embed_rms_body, QT, OUT, 2)                                  \
    CUCA_EMBED(NAME##_rms_u4, embed_rms_body, QT, OUT, 4)                                  \
    CUCA_EMBED(NAME##_rms_u8, embed_rms_body, QT, OUT, 8)                                  \
    CUCA_EMBED_LDS(NAME##_rms_lds_u2, QT, OUT, 2)                                          \
    CUCA_EMBED_LDS(NAME##_rms_lds_u4, QT, OUT, 4)                                          \
    CUCA_EMBED_LDS(NAME##_rms_lds_u8, QT, OUT, 8)

CUCA_EMBED_SET(cuca_embed_q4_0_f32, 2, float)
CUCA_EMBED_SET(cuca_embed_q4_0_f16, 2, _Float16)
CUCA_EMBED_SET(cuca_embed_q8_0_f32, 8, float)
CUCA_EMBED_SET(cuca_embed_q8_0_f16, 8, _Float16)
