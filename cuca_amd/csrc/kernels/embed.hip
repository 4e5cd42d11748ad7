// embed.hip -- GGUF Q4_0 / Q8_0 token-embedding dequant-gather on gfx950.
//
// Replaces TokenEmbedding::rows / dequant_ggml_row (quant.rs:107-198,
// 391-411) and the GPU engine's host-side RowTable gather + upload
// (quant.rs:477-501, gpu.rs:2976-2982): the quantized table stays resident
// in HBM and the gather runs on the device.
//
// One workgroup per token.  The token's row (row_bytes = 18 or 34 B per 32
// values) is staged into LDS with 16-byte loads -- one coalesced pass over
// the row, since every row of a hidden size that is a multiple of 256
// starts on a 16-byte boundary -- then every lane decodes one 16-byte output
// chunk (4 f32 or 8 f16) from LDS: the block's f16 scale `d` and the
// chunk's nibble/int8 bytes (ds_read_u16: block starts are only 2-byte
// aligned), and writes it with one global_store_dwordx4.  Consecutive lanes
// write consecutive chunks, so the output -- 90 % of the bytes -- is fully
// coalesced.
//
// Arithmetic is the reference's: d' = f32(d) * scale, then
// f32(q) * d' (two f32 roundings, in that order); f16 output is RNE of
// that f32.  Bit-exact.

#include "common.h"

template <int QT, typename OutT, bool AL16>
__device__ static inline void embed_body(const EmbedArgs &a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t embed_lds[];
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
    const uint8_t *row = a.table + (int64_t)id * a.row_bytes;
    if (AL16) {
        const int n16 = (int)(a.row_bytes >> 4);
        for (int i = threadIdx.x; i < n16; i += blockDim.x)
            reinterpret_cast<u32x4 *>(embed_lds)[i] = reinterpret_cast<const u32x4 *>(row)[i];
    } else {
        const int n2 = (int)(a.row_bytes >> 1);
        for (int i = threadIdx.x; i < n2; i += blockDim.x)
            reinterpret_cast<uint16_t *>(embed_lds)[i] = reinterpret_cast<const uint16_t *>(row)[i];
    }
    __syncthreads();
    const uint16_t *s16 = reinterpret_cast<const uint16_t *>(embed_lds);
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

#define CUCA_EMBED(NAME, QT, OUT, AL)                                                      \
    extern "C" __global__ __launch_bounds__(CUCA_BLOCK) void NAME(EmbedArgs a) {           \
        embed_body<QT, OUT, AL>(a);                                                        \
    }

CUCA_EMBED(cuca_embed_q4_0_f32_a16, 2, float, true)
CUCA_EMBED(cuca_embed_q4_0_f32_a2, 2, float, false)
CUCA_EMBED(cuca_embed_q4_0_f16_a16, 2, _Float16, true)
CUCA_EMBED(cuca_embed_q4_0_f16_a2, 2, _Float16, false)
CUCA_EMBED(cuca_embed_q8_0_f32_a16, 8, float, true)
CUCA_EMBED(cuca_embed_q8_0_f32_a2, 8, float, false)
CUCA_EMBED(cuca_embed_q8_0_f16_a16, 8, _Float16, true)
CUCA_EMBED(cuca_embed_q8_0_f16_a2, 8, _Float16, false)
