// embed.hip -- GGUF Q4_0 / Q8_0 token-embedding dequant-gather on gfx950.
//
// Replaces TokenEmbedding::rows / dequant_ggml_row (quant.rs:107-198,
// 391-411) and the GPU engine's host-side RowTable gather + upload
// (quant.rs:477-501, gpu.rs:2976-2982): the quantized table stays resident
// in HBM and the gather runs on the device.
//
// One workgroup per token.  Every lane produces one 16-byte output chunk
// (4 f32 or 8 f16 values, one global_store_dwordx4; consecutive lanes write
// consecutive chunks, so the output -- 80 to 90 % of the bytes -- is fully
// coalesced) from its block's f16 scale and its 2 to 8 quant bytes, read
// straight from the table row with 2-byte loads (a block starts on an even
// byte; the wave's loads cover the contiguous row, so the L1 turns them into
// whole cache lines and the row crosses HBM once).  Staging the row through
// LDS first (one 16-byte load per lane, a barrier, then LDS reads) measured
// slower on MI355X -- 16.0 vs 14.4 us per 4096 tokens of Q8_0 -> f16 and
// 38.8 vs 36.9 us per 16384, cold caches -- because the barrier serializes
// the two phases of every workgroup while the direct loads hit in L1.
//
// Arithmetic is the reference's: d' = f32(d) * scale, then
// f32(q) * d' (two f32 roundings, in that order); f16 output is RNE of
// that f32.  Bit-exact.

#include "common.h"

template <int QT, typename OutT>
__device__ static inline void embed_body(const EmbedArgs &a) {
    constexpr int N = Chunk<OutT>::N;
    constexpr int BS = QT == 2 ? 18 : 34; // bytes per 32-value block
    const int tok = blockIdx.x;
    const int nch = a.hidden / N;
    void *orow = reinterpret_cast<OutT *>(a.out) + (int64_t)tok * a.hidden;
    const uint32_t id = a.ids[tok];
    if ((int64_t)id >= a.vocab) {
        // The host could not see this id; write a zero row, never read
        // outside the table, and report it.
        if (threadIdx.x == 0) record_bad(a.status + CUCA_STATUS_EMBED_ID, (uint32_t)tok, id);
        float z[N];
#pragma unroll
        for (int i = 0; i < N; i++) z[i] = 0.0f;
        for (int c = threadIdx.x; c < nch; c += blockDim.x) Chunk<OutT>::store(orow, c, z);
        return;
    }
    const uint16_t *s16 = reinterpret_cast<const uint16_t *>(a.table + (int64_t)id * a.row_bytes);
    for (int c = threadIdx.x; c < nch; c += blockDim.x) {
        const int e0 = c * N;
        const int ob = (e0 >> 5) * BS;  // byte offset of the block (even)
        const int p = e0 & 31;          // first value within the block
        const float d = (float)__builtin_bit_cast(_Float16, s16[ob >> 1]) * a.scale;
        float v[N];
        if (QT == 2) {
            // Q4_0: byte j holds value j (low nibble) and j + 16 (high).
            const int q0 = (ob + 2 + (p & 15)) >> 1;
            const int sh = p >= 16 ? 4 : 0;
#pragma unroll
            for (int j = 0; j < N / 2; j++) {
                const uint32_t w = s16[q0 + j];
                v[2 * j] = (float)((int)((w >> sh) & 0xfu) - 8) * d;
                v[2 * j + 1] = (float)((int)((w >> (8 + sh)) & 0xfu) - 8) * d;
            }
        } else {
            // Q8_0: 32 signed bytes.
            const int q0 = (ob + 2 + p) >> 1;
#pragma unroll
            for (int j = 0; j < N / 2; j++) {
                const uint32_t w = s16[q0 + j];
                v[2 * j] = (float)(int8_t)(w & 0xffu) * d;
                v[2 * j + 1] = (float)(int8_t)(w >> 8) * d;
            }
        }
        Chunk<OutT>::store(orow, c, v);
    }
}

#define CUCA_EMBED(NAME, QT, OUT)                                                          \
    extern "C" __global__ __launch_bounds__(CUCA_BLOCK) void NAME(EmbedArgs a) {           \
        embed_body<QT, OUT>(a);                                                            \
    }

CUCA_EMBED(cuca_embed_q4_0_f32, 2, float)
CUCA_EMBED(cuca_embed_q4_0_f16, 2, _Float16)
CUCA_EMBED(cuca_embed_q8_0_f32, 8, float)
CUCA_EMBED(cuca_embed_q8_0_f16, 8, _Float16)
