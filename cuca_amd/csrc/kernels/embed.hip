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

template <int QT, typename OutT, int UPL>
__device__ static inline void embed_body(const EmbedArgs &a) {
    constexpr int BS = QT == 2 ? 18 : 34;     // bytes per 32-value block
    constexpr int CPU = 8 / Chunk<OutT>::N;   // output chunks per unit
    const int tok = blockIdx.x * (CUCA_BLOCK / CUCA_WAVE) + (int)(threadIdx.x / CUCA_WAVE);
    const int lane = threadIdx.x & (CUCA_WAVE - 1);
    if (tok >= a.n) return; // whole wave
    const int nu = a.hidden / 8;
    OutT *orow = reinterpret_cast<OutT *>(a.out) + (int64_t)tok * a.hidden;
    const uint32_t id = a.ids[tok];
    if ((int64_t)id >= a.vocab) {
        // The host could not see this id; write a zero row, never read
        // outside the table, and report it.
        if (lane == 0) record_bad(a.status + CUCA_STATUS_EMBED_ID, (uint32_t)tok, id);
        float z[Chunk<OutT>::N];
#pragma unroll
        for (int i = 0; i < Chunk<OutT>::N; i++) z[i] = 0.0f;
        for (int c = lane; c < nu * CPU; c += CUCA_WAVE) Chunk<OutT>::store_nt(orow, c, z);
        return;
    }
    const uint16_t *s16 = reinterpret_cast<const uint16_t *>(a.table + (int64_t)id * a.row_bytes);
    for (int u0 = 0; u0 < nu; u0 += CUCA_WAVE * UPL) {
        uint32_t dq[UPL], w[UPL][4];
#pragma unroll
        for (int k = 0; k < UPL; k++) {
            int u = u0 + lane + CUCA_WAVE * k;
            u = u < nu ? u : nu - 1; // a lane past the row end reloads the last unit
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
#pragma unroll
        for (int k = 0; k < UPL; k++) {
            const int u = u0 + lane + CUCA_WAVE * k;
            const int p = (u * 8) & 31;
            const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)dq[k]) * a.scale;
            float v[8];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                if (QT == 2) {
                    const int sh = p >= 16 ? 4 : 0;
                    v[2 * j] = (float)((int)((w[k][j] >> sh) & 0xfu) - 8) * d;
                    v[2 * j + 1] = (float)((int)((w[k][j] >> (8 + sh)) & 0xfu) - 8) * d;
                } else {
                    v[2 * j] = (float)(int8_t)(w[k][j] & 0xffu) * d;
                    v[2 * j + 1] = (float)(int8_t)(w[k][j] >> 8) * d;
                }
            }
            if (u < nu) {
                if (CPU == 1) {
                    Chunk<OutT>::store_nt(orow, u, reinterpret_cast<const float(&)[Chunk<OutT>::N]>(v));
                } else {
                    Chunk<OutT>::store_nt(orow, 2 * u, reinterpret_cast<const float(&)[Chunk<OutT>::N]>(v[0]));
                    Chunk<OutT>::store_nt(orow, 2 * u + 1, reinterpret_cast<const float(&)[Chunk<OutT>::N]>(v[4]));
                }
            }
        }
    }
}

#define CUCA_EMBED(NAME, QT, OUT, UPL)                                                     \
    extern "C" __global__ __launch_bounds__(CUCA_BLOCK) void NAME(EmbedArgs a) {           \
        embed_body<QT, OUT, UPL>(a);                                                       \
    }
#define CUCA_EMBED_SET(NAME, QT, OUT)                                                      \
    CUCA_EMBED(NAME##_u1, QT, OUT, 1)                                                      \
    CUCA_EMBED(NAME##_u2, QT, OUT, 2)                                                      \
    CUCA_EMBED(NAME##_u4, QT, OUT, 4)                                                      \
    CUCA_EMBED(NAME##_u8, QT, OUT, 8)

CUCA_EMBED_SET(cuca_embed_q4_0_f32, 2, float)
CUCA_EMBED_SET(cuca_embed_q4_0_f16, 2, _Float16)
CUCA_EMBED_SET(cuca_embed_q8_0_f32, 8, float)
CUCA_EMBED_SET(cuca_embed_q8_0_f16, 8, _Float16)
