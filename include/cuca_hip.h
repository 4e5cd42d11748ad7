/*
 * cuca_hip.h -- C ABI of the MI355X (gfx950) per-layer ops of the
 * provider-local GGUF engine of nassor/cuca 0.10.0.
 *
 * This is the drop-in boundary.  Each op replaces one op site of the
 * reference's layer loop (paths relative to src/provider/local/model/):
 *
 *   cuca_hip_embed_gguf    TokenEmbedding::rows           quant.rs:391-411
 *                          (GPU engine: RowTable::rows +  quant.rs:477-501,
 *                           upload in forward_stage)      gpu.rs:2976-2982, 4589-4598
 *   cuca_hip_embed_gguf_   the same + norm_embeddings     params.rs:374-379,
 *     norm                 (rms_norm_rows)                quant.rs:324-339
 *   cuca_hip_embed_gguf_   the gather + the first block's cpu.rs:2670-2673
 *     rms                  attention norm
 *   cuca_hip_add_rmsnorm   rms / residual add in block    cpu.rs:2650-2711, 3652
 *                          GPU rms, attn_tail, ffn_half,  gpu.rs:5420-5483, 5883-5896
 *                          ffn_tail
 *   cuca_hip_glu           activate(gate) * up, Glu::apply cpu.rs:342-371, 3554-3566, 3644
 *                          GPU activate / gelu            gpu.rs:5899-5913
 *   cuca_hip_glu_ragged    the same over expert-grouped   cpu.rs:3599-3642, moe.rs:39-94,
 *                          rows (MoE up epilogue)         moe_kernel.rs:1265-1288
 *   cuca_hip_rope          apply_rope / rotate_calls,     cpu.rs:2837-2871, 2996-3026,
 *                          with the per-head QK-norm      3040-3055, 3672-3688
 *                          GPU rope                       gpu.rs:5922-5964
 *   cuca_hip_rope_full,    the same with the full-width   cpu.rs:2838-2843, 3042-3045,
 *   _rope_store_kv_full    QK-norm (qk_norm_full)         gpu.rs:5233-5236
 *   cuca_hip_rope_tables   RopeSpec::tables (host)        rope.rs:118-151, mod.rs:460-472
 *   cuca_hip_rope_store_kv QK-norm + RoPE + the paged     cpu.rs:3028-3097,
 *                          K/V store of store_kv          cpu/paged_attn.rs:370-400
 *                          GPU k/v branch, KvPool::write  gpu.rs:5266-5285, 1786-1806
 *   cuca_hip_kv_slots      block-table positions -> pool  paged.rs:9-16, gpu.rs:1940-1975
 *                          rows (host)
 *   cuca_hip_attend_rows   attention of a sequence's rows cpu/paged_attn.rs:177-213,
 *                          over its paged cache (prefill) paged_kernel.rs:6-8
 *   cuca_hip_attend_       the latent (MLA) form          cpu/paged_attn.rs:215-251,
 *     latent_rows                                         paged_kernel.rs:21-31
 *   cuca_hip_paged_decode  paged decode attention         paged_kernel.rs:92-282,
 *                          (+ _workspace, host)           cpu/paged_attn.rs:105-290
 *   cuca_hip_qmm           QmmWeight::forward_rows        qmm.rs:1810-1838
 *   cuca_hip_qmm_glu       gate/up qmm + Glu::apply       cpu.rs:342-371, 3554-3566
 *   cuca_hip_qmm_rope_     Q|K|V qmm + store_kv (RoPE,    cpu.rs:3028-3097,
 *     store_kv             paged K/V store)               gpu.rs:5266-5285
 *   cuca_hip_add_rmsnorm_  the block's residual add +     cpu.rs:2650-2711, 342-371,
 *     qmm(_glu, _rope_     rms, then the next projection  3028-3097; gpu.rs:5420-5483
 *     store_kv)            (one launch at one row)
 *   cuca_hip_qgemm(_glu)   dense_dequant + matmul (GPU)   moe_kernel.rs:1414-1600
 *   cuca_hip_qweight_      dense_dequant_kernel, then     moe_kernel.rs:1560-1600,
 *     dequant, _gemm_w16   the dense matmul (GPU engine)  1414-1500
 *   cuca_hip_qweight_pack  (the weight upload)            qmm.rs:1763-1783
 *   cuca_hip_moe_up/down/  expert_sum, CpuExpert          cpu.rs:373-419, 3599-3642
 *            _sum          (GPU moe_up/moe_down/moe_sum)  moe_kernel.rs:1163-1385
 *   cuca_hip_moe_up/down_  the same as grouped GEMMs on   moe_kernel.rs:1163-1300
 *     qgemm                the matrix cores (prefill)
 *   cuca_hip_lm_head       head + cap_logits              cpu.rs:2588-2617
 *   cuca_hip_lm_head_      head_indexed + cap_logits      cpu.rs:2603-2606,
 *     indexed              (forward_indexed)              qmm.rs:1818-1843
 *   cuca_hip_argmax        greedy                         sampler.rs:44-56
 *   cuca_hip_top_k         select_top_k                   sampler.rs:254-286
 *
 * Conventions
 * - A context owns one device, one HIP stream (or borrows the caller's),
 *   the loaded gfx950 code object and a device status word.  A context is
 *   not thread-safe: one per engine thread, as the reference runs every model
 *   call on its single engine thread (local/mod.rs:2478).
 * - Every buffer argument is a device pointer the caller owns (allocated
 *   with cuca_hip_malloc or any other HIP allocator on the context's
 *   device).  Ops never allocate, never synchronize and never retain a
 *   pointer after they return, except inside a captured graph.
 * - Ops are asynchronous on the context's stream; call cuca_hip_stream_sync
 *   before reading results on the host.
 * - Activations are f32 or f16 (cuca_dtype); arithmetic is always f32,
 *   and f16 results are rounded once, to nearest-even.
 * - Errors: every entry point returns a cuca_status; a message is kept for
 *   cuca_hip_last_error.  Argument errors are caught on the host before any
 *   launch.  Values only the device sees (token ids, positions) are checked
 *   by the kernels, which skip the bad row and record it in the status word
 *   that cuca_hip_check_device (a blocking call) reports.
 */
#ifndef CUCA_HIP_H
#define CUCA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CUCA_HIP_ABI_VERSION 1

typedef struct cuca_hip_ctx cuca_hip_ctx;
typedef struct cuca_hip_graph cuca_hip_graph;

/* The reference maps its errors to CucaError::Provider(Local, msg)
 * (model/mod.rs:222-228); a binding maps every non-OK status the same way,
 * with cuca_hip_last_error as the message. */
typedef enum {
    CUCA_OK = 0,
    CUCA_INVALID_ARG = 1,  /* shape, type, alignment or pointer error      */
    CUCA_OUT_OF_RANGE = 2, /* token id >= vocab, position outside the table */
    CUCA_HIP_ERROR = 3,    /* a HIP runtime call failed                     */
    CUCA_NOT_GFX950 = 4,   /* the device is not an MI355X-class gfx950      */
    CUCA_UNSUPPORTED = 5   /* a valid request this build has no kernel for  */
} cuca_status;

typedef enum { CUCA_F32 = 0, CUCA_F16 = 1 } cuca_dtype;

/* ggml type ids (gguf/dtype.rs:195-250). */
typedef enum { CUCA_GGML_Q4_0 = 2, CUCA_GGML_Q8_0 = 8 } cuca_ggml_type;

/* Act (arch.rs:101-106). */
typedef enum { CUCA_ACT_SILU = 0, CUCA_ACT_GELU_TANH = 1 } cuca_act;

/* RopeKind (rope.rs:28-36), llama.cpp's rope type values. */
typedef enum { CUCA_ROPE_NORM = 0, CUCA_ROPE_NEOX = 2 } cuca_rope_kind;

/* ------------------------------------------------------------------ */
/* Context, memory, stream                                              */
/* ------------------------------------------------------------------ */

/* Open `device`, check it is gfx950, create a stream of default priority
 * and load the kernels.  Replaces the device open of GpuTransformer::load
 * (gpu.rs:2597, adapter log gpu.rs:403-420). */
cuca_status cuca_hip_ctx_create(int device, cuca_hip_ctx **out);
void cuca_hip_ctx_destroy(cuca_hip_ctx *ctx);

/* The last error message of `ctx`, or of the calling thread when ctx is
 * NULL (context creation failures).  Never NULL; "" when there is none. */
const char *cuca_hip_last_error(const cuca_hip_ctx *ctx);

/* Run the context's work on `stream` (a hipStream_t of the same device,
 * e.g. the caller's framework stream); NULL returns to the context's own. */
cuca_status cuca_hip_set_stream(cuca_hip_ctx *ctx, void *stream);
/* The hipStream_t ops are issued on. */
void *cuca_hip_get_stream(const cuca_hip_ctx *ctx);
int cuca_hip_device(const cuca_hip_ctx *ctx);

cuca_status cuca_hip_malloc(cuca_hip_ctx *ctx, size_t bytes, void **out);
cuca_status cuca_hip_free(cuca_hip_ctx *ctx, void *ptr);
cuca_status cuca_hip_memcpy_h2d_async(cuca_hip_ctx *ctx, void *dst, const void *src, size_t bytes);
cuca_status cuca_hip_memcpy_d2h_async(cuca_hip_ctx *ctx, void *dst, const void *src, size_t bytes);
cuca_status cuca_hip_memcpy_d2d_async(cuca_hip_ctx *ctx, void *dst, const void *src, size_t bytes);
cuca_status cuca_hip_stream_sync(cuca_hip_ctx *ctx);

/* Synchronize, then report (and clear) what the kernels recorded in the
 * status word: CUCA_OUT_OF_RANGE with the first bad row in the message
 * ("token id {id} outside the embedding table of {rows} rows", as
 * quant.rs:395-400, a RoPE position outside its table, or a K/V slot outside
 * its pool). */
cuca_status cuca_hip_check_device(cuca_hip_ctx *ctx);

/* Self-test of the kernels' wave reductions (no counterpart in the
 * reference): for input[n] (n a positive multiple of 256) writes out[12 * n],
 * for each group size 2, 4, ..., 64 the sum of each value's aligned group
 * as the kernels compute it (DPP, swizzle and permlane partners) and as the
 * __shfl_xor butterfly computes it; the two must agree bit for bit. */
cuca_status cuca_hip_selftest_group_sum(cuca_hip_ctx *ctx, const float *input, int64_t n, float *out);

/* ------------------------------------------------------------------ */
/* Ops                                                                  */
/* ------------------------------------------------------------------ */

/* Token-embedding dequant-gather (TokenEmbedding::rows, quant.rs:391-411;
 * dequant_ggml_row Q4_0/Q8_0, quant.rs:107-198).
 *   table : [vocab, hidden/32 blocks] of ggml_type, resident on the device
 *   ids   : device u32[n]
 *   out   : device [n, hidden] of out_dtype
 * out[t, :] = dequant_row(table row ids[t]) with `scale` folded into each
 * block's f16 scale first (bit-exact with the reference; f16 output is the
 * f32 value rounded to nearest-even).  hidden must be a multiple of 32.
 * An id >= vocab writes a zero row and is reported by cuca_hip_check_device. */
cuca_status cuca_hip_embed_gguf(cuca_hip_ctx *ctx, const void *table, uint32_t ggml_type,
                                int64_t vocab, int64_t hidden, const uint32_t *ids,
                                int64_t n, float scale, void *out, cuca_dtype out_dtype);

/* cuca_hip_embed_gguf followed by the scale-less norm of the archs with
 * embd_norm (Hparams::norm_embeddings, params.rs:374-379 -> rms_norm_rows,
 * quant.rs:324-339; run right after the gather in forward_stage,
 * cpu.rs:1881-1882, gpu.rs:2976-2981), in the same pass over the row:
 *   sum = f64 squares of the row's f32 values (after `scale`), index order
 *   inv = (f32)(1 / sqrt(sum / hidden + f64(norm_eps)))
 *   out[t, :] = row * inv (f32; f16 output rounds that once)
 * Bit-exact with the reference: the device sums in its own order and
 * proves from an error bound that the f32 inv is the sequential sum's, and
 * re-sums in index order the rare row where it cannot. */
cuca_status cuca_hip_embed_gguf_norm(cuca_hip_ctx *ctx, const void *table, uint32_t ggml_type,
                                     int64_t vocab, int64_t hidden, const uint32_t *ids,
                                     int64_t n, float scale, float norm_eps, void *out,
                                     cuca_dtype out_dtype);

/* The gather fused with the first block's attention norm: TokenEmbedding::rows
 * (quant.rs:391-411) into x_out, then h = rms(x, w, eps) (Transformer::block's
 * first step, cpu.rs:2670-2673, whose input for the first block is the
 * gathered rows) into h_out, in one pass.  x_out is bit-identical to
 * cuca_hip_embed_gguf's output; h is computed from x as stored, as
 * cuca_hip_add_rmsnorm with branch == NULL would, and meets the same bar
 * (the sum of squares is summed in this kernel's own order).  w == NULL is
 * the weightless norm.  x_out, h_out: [n, hidden] of out_dtype, 16-byte
 * aligned; w: f32[hidden], 16-byte aligned.  Bad ids: as cuca_hip_embed_gguf,
 * with zero rows in both outputs. */
cuca_status cuca_hip_embed_gguf_rms(cuca_hip_ctx *ctx, const void *table, uint32_t ggml_type,
                                    int64_t vocab, int64_t hidden, const uint32_t *ids, int64_t n,
                                    float scale, const float *w, float eps, void *x_out,
                                    void *h_out, cuca_dtype out_dtype);

/* Fused residual add + RMSNorm (Transformer::block, cpu.rs:2650-2711, with
 * rms = candle_nn::ops::rms_norm, cpu.rs:3652; GPU attn_tail / ffn_half /
 * ffn_tail, gpu.rs:5420-5483):
 *   b  = w_post ? rms(branch, w_post, post_eps) : branch   (Gemma sandwich)
 *   x' = branch ? x + residual_scale * b : x              -> x_out (nullable)
 *   h  = rms(x' as stored, w, eps)                         -> h_out
 * rms(v, w, eps) = v / sqrt(mean(v^2) + eps) * w; w == NULL is the
 * weightless norm.  All of x, branch, x_out, h_out are [rows, hidden] of
 * `dtype`; x_out may alias x; w and w_post are f32[hidden].  With branch ==
 * NULL this is the plain `rms(x, w, eps)`. */
cuca_status cuca_hip_add_rmsnorm(cuca_hip_ctx *ctx, const void *x, const void *branch,
                                 const float *w, const float *w_post, float eps,
                                 float post_eps, float residual_scale, int64_t rows,
                                 int64_t hidden, void *x_out, void *h_out, cuca_dtype dtype);

/* Gated activation (Glu::apply, cpu.rs:362-371; activate, cpu.rs:3644;
 * FfnWeights::forward GateUp::{Split, Fused}, cpu.rs:319-330, 3554-3566):
 *   g = clamp > 0 ? min(g, clamp) : g,  u = clamp > 0 ? clamp(u, -clamp, clamp) : u
 *   out[r, j] = act(g[r, j]) * u[r, j]
 * Row r of gate/up/out starts at r * gate_ld / up_ld / out_ld elements, so
 * the fused [gate | up] projection is gate = y, up = y + ff, ld = 2 * ff.
 * SiLU g / (1 + e^-g); GELU-tanh 0.5 g (1 + tanh(sqrt(2/pi) (g + 0.044715 g^3))). */
cuca_status cuca_hip_glu(cuca_hip_ctx *ctx, const void *gate, int64_t gate_ld,
                         const void *up, int64_t up_ld, int64_t rows, int64_t ff,
                         cuca_act act, float clamp, void *out, int64_t out_ld,
                         cuca_dtype dtype);

/* The gated activation over MoE rows grouped by expert (route_with's
 * per-expert grouping, moe.rs:39-94; expert_sum, cpu.rs:3599-3642; the
 * reference fuses the same activation into up_kernel's epilogue,
 * moe_kernel.rs:1265-1288).  expert_offsets is a DEVICE int32[n_experts + 1]
 * prefix sum: expert e owns rows [offsets[e], offsets[e+1]).  The row count
 * is read on the device (offsets[n_experts], capped at max_rows), so routing
 * done on the device needs no host round trip and the call can be captured
 * in a graph.  Rows past the count are not touched. */
cuca_status cuca_hip_glu_ragged(cuca_hip_ctx *ctx, const void *gate, int64_t gate_ld,
                                const void *up, int64_t up_ld,
                                const int32_t *expert_offsets, int32_t n_experts,
                                int64_t max_rows, int64_t ff, cuca_act act, float clamp,
                                void *out, int64_t out_ld, cuca_dtype dtype);

/* Rotary embedding on Q and K in place (apply_rope, cpu.rs:3672-3688 ->
 * candle rope (NEOX) / rope_i (NORM); rotate_calls, cpu.rs:2996-3026; GPU
 * rope, gpu.rs:5922-5964), with the optional per-head QK-norm fused in
 * front (cpu.rs:2840-2864 for Q, 3040-3055 for K).
 *   q : [rows, nq, head_dim] with row stride q_ld elements (>= nq*head_dim)
 *   k : [rows, nk, head_dim] with row stride k_ld (k may be NULL when nk = 0)
 *   cos, sin : f32 [table_rows, n_dims/2] (cuca_hip_rope_tables)
 *   positions: device int32[rows], each < table_rows
 * For every head: v = q_norm_w ? rms(head, q_norm_w[head_dim], eps) : head,
 * then pair i of the first n_dims values (NORM: 2i, 2i+1; NEOX: i, i+n/2):
 *   a' = a*c - b*s,  b' = a*s + b*c        (rope.rs:158-171)
 * with each product rounded separately (no FMA): without QK-norm the result
 * is bit-identical to the reference's f32 rotation.  Values past n_dims pass
 * through (normalized when a norm weight is given).  k_norm_w applies to K. */
cuca_status cuca_hip_rope(cuca_hip_ctx *ctx, void *q, int64_t q_ld, void *k, int64_t k_ld,
                          int64_t rows, int32_t nq, int32_t nk, int32_t head_dim,
                          int32_t n_dims, cuca_rope_kind kind, const float *cos,
                          const float *sin, int64_t table_rows, const int32_t *positions,
                          const float *q_norm_w, const float *k_norm_w, float eps,
                          cuca_dtype dtype);

/* cuca_hip_rope with the full-width QK-norm of the qk_norm_full archs
 * (OLMo 2; cpu.rs:2838-2843 for Q, 3042-3045 for K; GPU gpu.rs:5233-5236):
 * q_norm_w is f32 [nq * head_dim] and normalises a row's whole Q projection,
 * k_norm_w [nk * head_dim] its whole K projection, before the heads are
 * split and rotated:
 *   q' = q / sqrt(mean over the nq * head_dim values + eps) * q_norm_w
 * in f32, then the rotation as cuca_hip_rope (no rounding in between).
 * Needs the vector layout (head_dim and n_dims in whole 16-byte chunks per
 * lane, 16-byte aligned rows, tables and weights) and at most 4096 head
 * lanes per row; CUCA_UNSUPPORTED otherwise. */
cuca_status cuca_hip_rope_full(cuca_hip_ctx *ctx, void *q, int64_t q_ld, void *k, int64_t k_ld,
                               int64_t rows, int32_t nq, int32_t nk, int32_t head_dim,
                               int32_t n_dims, cuca_rope_kind kind, const float *cos,
                               const float *sin, int64_t table_rows, const int32_t *positions,
                               const float *q_norm_w, const float *k_norm_w, float eps,
                               cuca_dtype dtype);

/* Positions per paged K/V block (paged.rs:45, BLOCK_SIZE), and the block
 * table entry of a released block (paged.rs:49, NO_BLOCK). */
#define CUCA_KV_BLOCK 16
#define CUCA_NO_BLOCK 0xffffffffu

/* cuca_hip_rope fused with the paged K/V store of a K/V-owning layer
 * (store_kv, cpu.rs:3028-3097 -> store_rows, cpu/paged_attn.rs:370-400;
 * GPU: the k/v branch of gpu.rs:5266-5285 -> KvPool::write,
 * gpu.rs:1786-1806).  One launch:
 *   Q: QK-norm (q_norm_w) and rotation in place, as cuca_hip_rope;
 *   K: QK-norm (k_norm_w) and rotation, written to pool_k only (the k
 *      buffer is read, not written);
 *   V: rms(v, no weight, eps) when v_norm (gpu.rs:5277), written to pool_v.
 * The pools are [n_blocks, nk, CUCA_KV_BLOCK, head_dim] in the activation
 * dtype (paged_attn.rs:1-38): row r of the call goes to pool row
 *   slots[r] = block * CUCA_KV_BLOCK + position % CUCA_KV_BLOCK
 * of each KV head, i.e. element ((block*nk + h)*16 + slot%16)*head_dim.
 * slots: device int32[rows] (cuca_hip_kv_slots builds them from a block
 * table).  A slot outside [0, n_blocks*16) or a position outside the table
 * leaves the row untouched and is reported by cuca_hip_check_device. */
cuca_status cuca_hip_rope_store_kv(cuca_hip_ctx *ctx, void *q, int64_t q_ld, const void *k,
                                   int64_t k_ld, const void *v, int64_t v_ld, int64_t rows,
                                   int32_t nq, int32_t nk, int32_t head_dim, int32_t n_dims,
                                   cuca_rope_kind kind, const float *cos, const float *sin,
                                   int64_t table_rows, const int32_t *positions,
                                   const float *q_norm_w, const float *k_norm_w, int32_t v_norm,
                                   float eps, void *pool_k, void *pool_v, int64_t n_blocks,
                                   const int32_t *slots, cuca_dtype dtype);

/* cuca_hip_rope_store_kv with the full-width QK-norm of cuca_hip_rope_full
 * (q_norm_w [nq * head_dim], k_norm_w [nk * head_dim]); V's weightless norm
 * (v_norm) stays per head, as gpu.rs:5277 runs it. */
cuca_status cuca_hip_rope_store_kv_full(cuca_hip_ctx *ctx, void *q, int64_t q_ld, const void *k,
                                        int64_t k_ld, const void *v, int64_t v_ld, int64_t rows,
                                        int32_t nq, int32_t nk, int32_t head_dim, int32_t n_dims,
                                        cuca_rope_kind kind, const float *cos, const float *sin,
                                        int64_t table_rows, const int32_t *positions,
                                        const float *q_norm_w, const float *k_norm_w,
                                        int32_t v_norm, float eps, void *pool_k, void *pool_v,
                                        int64_t n_blocks, const int32_t *slots, cuca_dtype dtype);

/* Host-side: the pool slots of cache indices start..start+t of a sequence
 * whose block table is table[table_len] (position p -> block table[p/16],
 * row p%16, paged.rs:9-16; the write runs of gpu.rs:1940-1975).  Fails with
 * CUCA_OUT_OF_RANGE, as check_range does (paged_attn.rs:42-65), when a
 * position has no block: past the table, a released block (0xffffffff,
 * NO_BLOCK) or an id outside the pool of n_blocks. */
cuca_status cuca_hip_kv_slots(const uint32_t *table, int64_t table_len, int64_t start, int64_t t,
                              int64_t n_blocks, int32_t *slots_out);

/* Paged decode attention: one query row per sequence over its keys, read in
 * place from the pools cuca_hip_rope_store_kv fills (the GPU engine's
 * paged_attention_decode, paged_kernel.rs:92-282, on a step's stacked
 * rows, gpu.rs:6002-6011; the CPU's attend_paged_rows for one row,
 * cpu/paged_attn.rs:105-290).
 *   q      : [rows][q_ld] of dtype, n_head heads of head_dim at the start
 *            of each row (q_ld = n_head * head_dim when packed; a fused QKV
 *            projection's row otherwise); rows 4-byte aligned
 *   pools  : [n_blocks, n_kv, 16, head_dim] of dtype
 *   tables : device u32 [rows, max_blocks] block ids; ranges: device int32
 *            [rows, 2] = (lo, hi) key positions relative to the table (the
 *            reference's BlockRead::Decode table and range)
 *   out    : [rows, n_head, head_dim] of dtype
 * Query head h reads KV head h / (n_head / n_kv); out = softmax(q.k * scale)
 * . v over positions lo..hi-1, f32 throughout.  The keys are split into
 * fixed chunks of 64 positions, merged in chunk order, so a row's result
 * does not depend on the other rows of the call.  workspace: device, 16-byte
 * aligned, at least cuca_hip_paged_decode_workspace bytes (the ops never
 * allocate).  An empty range, a range past the table or a position whose
 * block id is >= n_blocks is reported by cuca_hip_check_device (the row's
 * output is then unspecified; zeros for a bad range). */
cuca_status cuca_hip_paged_decode_workspace(int64_t rows, int32_t n_head, int32_t head_dim,
                                            int64_t max_blocks, size_t *bytes);
cuca_status cuca_hip_paged_decode(cuca_hip_ctx *ctx, const void *q, int64_t q_ld,
                                  const void *pool_k, const void *pool_v, int64_t n_blocks,
                                  const uint32_t *tables,
                                  int64_t max_blocks, const int32_t *ranges, int64_t rows,
                                  int32_t n_head, int32_t n_kv, int32_t head_dim, float scale,
                                  void *workspace, size_t workspace_bytes, void *out,
                                  cuca_dtype dtype);

/* Attention of many query rows of ONE sequence over its paged cache: a
 * prefill chunk, or speculative verification rows (attend_paged_rows,
 * cpu/paged_attn.rs:177-213, 257-309; the GPU engine gathers the blocks and
 * multiplies, paged_kernel.rs:6-8).
 *   q      : [rows][q_ld] of dtype, n_head heads of head_dim at the start
 *            of each row, rows aligned to the element
 *   pools  : [n_blocks, n_kv, 16, head_dim] of dtype (pool_v NULL is an error)
 *   table  : device u32 [max_blocks], the sequence's block table
 *   ranges : device int32 [rows, 2] = (lo, hi): row r attends to positions
 *            lo..hi-1 of the table (causal prefill: hi = its position + 1)
 *   out    : [rows][out_ld] of dtype, n_head heads of head_dim
 * Query head h reads KV head h / (n_head / n_kv); out = softmax(q.k *
 * scale) . v over the row's positions, block by block with a running
 * maximum, f32 throughout (f16 pools: exact f16 products on the matrix
 * cores).  A row's result does not depend on the other rows of the call.
 * An empty range, a range past the table, or a position of a range whose
 * block id is >= n_blocks, is reported by cuca_hip_check_device, the row's
 * output then zeros.  No workspace. */
cuca_status cuca_hip_attend_rows(cuca_hip_ctx *ctx, const void *q, int64_t q_ld, const void *pool_k,
                                 const void *pool_v, int64_t n_blocks, const uint32_t *table,
                                 int64_t max_blocks, const int32_t *ranges, int64_t rows, int32_t n_head,
                                 int32_t n_kv, int32_t head_dim, float scale, void *out, int64_t out_ld,
                                 cuca_dtype dtype);

/* The latent (multi-head latent attention) form: one pool of head_dim
 * columns per position (n_kv 1) whose first v_width columns are also the
 * value (attend_latent_rows, cpu/paged_attn.rs:215-251; the GPU decode's
 * PagedCall::v_width, paged_kernel.rs:21-31).  out: [rows][out_ld], n_head
 * heads of v_width.  v_width 0 or above head_dim is CUCA_INVALID_ARG
 * ("attention: bad latent value width", as the reference). */
cuca_status cuca_hip_attend_latent_rows(cuca_hip_ctx *ctx, const void *q, int64_t q_ld, const void *pool,
                                        int64_t n_blocks, const uint32_t *table, int64_t max_blocks,
                                        const int32_t *ranges, int64_t rows, int32_t n_head,
                                        int32_t head_dim, int32_t v_width, float scale, void *out,
                                        int64_t out_ld, cuca_dtype dtype);

/* No counterpart in the reference.  cuca_hip_paged_decode without a
 * workspace, for callers that cannot allocate (code under HIP graph capture,
 * serving loops or harnesses that forbid hipMalloc): the split pass's
 * partials go to a library-owned device array of CUCA_NOALLOC_SCRATCH_BYTES,
 * one per GPU, held from the first context on that GPU until the process
 * ends.  The call allocates nothing; the caller passes the inputs and the
 * output, as to cuca_hip_paged_decode, and gets the same bits.  A call whose
 * partials need more than the maximum -- rows * n_head * parts * (head_dim +
 * 2) * 4 bytes, parts = ceil(max_blocks * 16 / part length), the part length
 * 64 to 256 positions by dtype, head_dim and group -- fails with
 * CUCA_INVALID_ARG before any launch.  Nothing in the array has to start at
 * zero (every partial a merge reads is written by the same call's split);
 * it keeps the last call's contents.  Every call on one GPU shares the
 * array: calls that overlap on one GPU (other streams, other contexts or
 * threads) race and must be ordered by the caller. */
#define CUCA_NOALLOC_SCRATCH_BYTES (64u << 20)
cuca_status cuca_hip_paged_decode_noalloc(cuca_hip_ctx *ctx, const void *q, int64_t q_ld,
                                          const void *pool_k, const void *pool_v, int64_t n_blocks,
                                          const uint32_t *tables, int64_t max_blocks,
                                          const int32_t *ranges, int64_t rows, int32_t n_head,
                                          int32_t n_kv, int32_t head_dim, float scale, void *out,
                                          cuca_dtype dtype);

/* ------------------------------------------------------------------ */
/* Quantized matmul (the CPU engine's QmmWeight, qmm.rs)               */
/* ------------------------------------------------------------------ */

/* A quantized [n, k] weight (y = x w^T) as the GGUF file stores it, Q4_0 or
 * Q8_0, is repacked once on the device into the kernels' layout (groups of
 * 16 (Q4_0) or 8 (Q8_0) blocks: the group's f16 scales, then one 16-byte
 * chunk per lane holding that lane's quants of every block of the group;
 * the same bytes as the file, reordered).  The reference reads the file
 * bytes in place (QmmWeight::from_raw, qmm.rs:1763-1783); its GPU engine
 * repacks into its own word order too (moe_kernel.rs DenseLayout).
 * cuca_hip_qweight_bytes: the packed size.  cuca_hip_qweight_pack: gguf
 * (device, [n][k/32 blocks]) -> packed (device, 16-byte aligned). */
cuca_status cuca_hip_qweight_bytes(uint32_t ggml_type, int64_t n, int64_t k, size_t *bytes);
cuca_status cuca_hip_qweight_pack(cuca_hip_ctx *ctx, const void *gguf, uint32_t ggml_type, int64_t n,
                                  int64_t k, void *packed);

/* QmmWeight::forward_rows (qmm.rs:1810-1838), bit for bit: out[j][r] =
 * x[j] . w[r] for the first `rows` weight rows, with the reference CPU
 * engine's arithmetic (qmm.rs:14-45): x quantised to Q8_0 per 32 values,
 * sixteen f32 lanes each summing (f32)(exact integer pair dot) * (dw * dx)
 * over the blocks in order, reduced by the fixed tree of hsum.  A row's
 * result does not depend on m or on the other rows.
 *   w   : packed weight (cuca_hip_qweight_pack) of n rows of k values
 *   x   : [m][ldx] of dtype (f16 is widened exactly); 16-byte aligned rows
 *   out : [m][out_ld] of dtype (f32: the reference's bits; f16: rounded once)
 * rows outside 1..n is an error ("qmm: {rows} weight rows of {n}"). */
cuca_status cuca_hip_qmm(cuca_hip_ctx *ctx, const void *w, uint32_t ggml_type, int64_t n, int64_t k,
                         const void *x, int64_t ldx, int64_t m, int64_t rows, void *out, int64_t out_ld,
                         cuca_dtype dtype);

/* The fused Q|K|V projection of a K/V-owning layer with RoPE and the paged
 * K/V store in its epilogue: cuca_hip_qmm over w = the Q, K and V rows
 * ((nq + 2 nk) * head_dim rows of k values, Q heads first), then what
 * cuca_hip_rope_store_kv does to its output (store_kv, cpu.rs:3028-3097),
 * in one launch and with the same bits:
 *   Q heads: rotated, written to q_out [m][q_ld] (the first nq * head_dim
 *            values of each row);
 *   K heads: rotated, written to pool_k at pool row slots[j] of their KV
 *            head; V heads: written to pool_v there (pools as
 *            cuca_hip_rope_store_kv's, [n_blocks, nk, 16, head_dim]).
 * Only NORM RoPE (adjacent pairs, Llama-family) and no QK-norm: a pair's two
 * rows then belong to one workgroup (CUCA_UNSUPPORTED for NEOX).  A row whose
 * position or slot is bad keeps Q unrotated and stores no K/V, and is
 * reported by cuca_hip_check_device. */
cuca_status cuca_hip_qmm_rope_store_kv(cuca_hip_ctx *ctx, const void *w, uint32_t ggml_type, int64_t k,
                                       const void *x, int64_t ldx, int64_t m, int32_t nq, int32_t nk,
                                       int32_t head_dim, int32_t n_dims, cuca_rope_kind kind,
                                       const float *cos, const float *sin, int64_t table_rows,
                                       const int32_t *positions, void *q_out, int64_t q_ld,
                                       void *pool_k, void *pool_v, int64_t n_blocks,
                                       const int32_t *slots, cuca_dtype dtype);

/* The dense FFN's gate and up projections with the gated activation fused in
 * (FfnWeights::forward GateUp::Split + Glu::apply, cpu.rs:342-371,
 * 3554-3566; the reference GPU engine fuses the same act * up into its
 * up_kernel, moe_kernel.rs:1163-1288):
 *   out[j][f] = act(min(g, clamp)) * clamp(u, -clamp, clamp)   (clamp > 0)
 *             = act(g) * u                                     (clamp <= 0)
 * g = qmm(gate)[j][f], u = qmm(up)[j][f] with cuca_hip_qmm's bits; the
 * activation as cuca_hip_glu.  gate, up: packed [ff][k]; out [m][out_ld]. */
cuca_status cuca_hip_qmm_glu(cuca_hip_ctx *ctx, const void *gate, const void *up, uint32_t ggml_type,
                             int64_t ff, int64_t k, const void *x, int64_t ldx, int64_t m, cuca_act act,
                             float clamp, void *out, int64_t out_ld, cuca_dtype dtype);

/* The residual add + RMSNorm fused into the projection that reads it (a
 * block's attention norm before the Q|K|V projection, its FFN norm before
 * gate/up: Transformer::block, cpu.rs:2650-2711; GPU attn_tail / ffn_half,
 * gpu.rs:5420-5483), with the bits of the two calls it replaces:
 *   cuca_hip_add_rmsnorm(x, branch, norm_w, NULL, eps, eps, residual_scale,
 *                        m, k, x_out, h_out, dtype)
 *   then cuca_hip_qmm / _qmm_glu / _qmm_rope_store_kv on h_out (ldx = k).
 * At one activation row the matmul's workgroups each compute the norm of the
 * row themselves (workgroup 0 also writes x_out and h_out), so the norm costs
 * no launch of its own; otherwise the two calls run in turn.  x, branch,
 * x_out, h_out: [m][k] of dtype, k the hidden size; branch and norm_w
 * (f32[k]) nullable, x_out nullable; the Gemma post-norm (w_post) is not
 * offered here.  x_out and h_out must not overlap x, branch or each other
 * (CUCA_INVALID_ARG): the norm's outputs are written while other workgroups
 * still read its inputs.  Other arguments and errors as the matmul's. */
cuca_status cuca_hip_add_rmsnorm_qmm(cuca_hip_ctx *ctx, const void *x, const void *branch,
                                     const float *norm_w, float eps, float residual_scale,
                                     void *x_out, void *h_out, const void *w, uint32_t ggml_type,
                                     int64_t n, int64_t k, int64_t m, int64_t rows, void *out,
                                     int64_t out_ld, cuca_dtype dtype);
cuca_status cuca_hip_add_rmsnorm_qmm_glu(cuca_hip_ctx *ctx, const void *x, const void *branch,
                                         const float *norm_w, float eps, float residual_scale,
                                         void *x_out, void *h_out, const void *gate, const void *up,
                                         uint32_t ggml_type, int64_t ff, int64_t k, int64_t m,
                                         cuca_act act, float clamp, void *out, int64_t out_ld,
                                         cuca_dtype dtype);
cuca_status cuca_hip_add_rmsnorm_qmm_rope_store_kv(cuca_hip_ctx *ctx, const void *x,
                                                   const void *branch, const float *norm_w,
                                                   float eps, float residual_scale, void *x_out,
                                                   void *h_out, const void *w, uint32_t ggml_type,
                                                   int64_t k, int64_t m, int32_t nq, int32_t nk,
                                                   int32_t head_dim, int32_t n_dims,
                                                   cuca_rope_kind kind, const float *cos,
                                                   const float *sin, int64_t table_rows,
                                                   const int32_t *positions, void *q_out,
                                                   int64_t q_ld, void *pool_k, void *pool_v,
                                                   int64_t n_blocks, const int32_t *slots,
                                                   cuca_dtype dtype);

/* The quantized matmul for many activation rows (prefill, large decode
 * batches) on the matrix cores: out[j][r] = x[j] . w[r] with each weight
 * dequantised to f16 (f16(d * q), one rounding), each activation rounded to
 * f16 and f32 accumulation.  This is the arithmetic class of the reference
 * GPU engine's dense paths (dense_gemv_kernel / dense_dequant_kernel,
 * moe_kernel.rs:1414-1600: float products of dequantised weights and
 * unquantised activations), not the CPU engine's bits (cuca_hip_qmm): the
 * error against the exact product is at most (2^-10 + k 2^-24) sum |w x|.
 * Same packed weights, shapes and errors as cuca_hip_qmm / _qmm_glu
 * ("qgemm: ..."); activations and outputs need no alignment; |d q| and |x|
 * within f16's range.
 * The workspace (device, 16-byte aligned) holds the activations rewritten as
 * f16 in the kernel's order (rows padded with zeros to a whole tile of 32,
 * 64 or 128 rows) and, for small grids, the f32 sums of a split
 * of k that a second launch adds in a fixed order (deterministic for a
 * given shape, device and workspace size; the split changes the summation
 * order, within the same bound); cuca_hip_qgemm_workspace gives the bytes
 * for n weight rows, k
 * values and m activation rows (glu != 0 for cuca_hip_qgemm_glu); a smaller
 * one that still holds the activations is used without splitting. */
cuca_status cuca_hip_qgemm_workspace(uint32_t ggml_type, int64_t n, int64_t k, int64_t m, int32_t glu, size_t *bytes);
cuca_status cuca_hip_qgemm(cuca_hip_ctx *ctx, const void *w, uint32_t ggml_type, int64_t n, int64_t k, const void *x,
                           int64_t ldx, int64_t m, int64_t rows, void *workspace, size_t workspace_bytes, void *out,
                           int64_t out_ld, cuca_dtype dtype);
cuca_status cuca_hip_qgemm_glu(cuca_hip_ctx *ctx, const void *gate, const void *up, uint32_t ggml_type, int64_t ff,
                               int64_t k, const void *x, int64_t ldx, int64_t m, cuca_act act, float clamp,
                               void *workspace, size_t workspace_bytes, void *out, int64_t out_ld, cuca_dtype dtype);

/* The dense f16 path for many activation rows (prefill): the reference GPU
 * engine's dense_dequant_kernel + matmul (moe_kernel.rs:1414-1600), shaped
 * for MI355X's 288 GB: the weight is dequantised once into a resident f16
 * copy (2 bytes a value: 16 GB for an 8B model, next to the Q4_0 weights
 * the decode kernels read), and each call is one f16 GEMM on the matrix
 * cores (the library's own kernel, f32 accumulation).  The arithmetic class
 * of cuca_hip_qgemm (weights f16(d * q), activations f16(x), one rounding
 * each), held to the same bound.
 *   cuca_hip_qweight_dequant: packed (cuca_hip_qweight_pack) [n, k] ->
 *     w16 f16 [n][k] row-major, f16(d * q) per value.
 *   cuca_hip_gemm_w16: out[m][rows] = x[m] . w16[0..rows)^T; x and out of
 *     dtype (f32 rows are rounded to f16 into the workspace first).
 *   cuca_hip_gemm_w16_glu: w16 [2 ff][k] = the gate rows, then the up rows
 *     (one GEMM); out[m][ff] = act(gate) * up with Glu::apply's clamp, from
 *     the f32 sums in registers.
 * workspace: device, 16-byte aligned, cuca_hip_gemm_w16_workspace bytes
 * (n = the output width: rows, or ff for the GLU): the f32 activations
 * rounded to f16, so 0 bytes (and workspace may be NULL) for f16 calls.
 * k and ldx below 2^22.  Not for a few rows: decode batches take
 * cuca_hip_qmm / cuca_hip_qgemm on the packed weight. */
cuca_status cuca_hip_qweight_dequant(cuca_hip_ctx *ctx, const void *packed, uint32_t ggml_type, int64_t n,
                                     int64_t k, void *w16);
cuca_status cuca_hip_gemm_w16_workspace(int64_t n, int64_t k, int64_t m, int32_t glu, cuca_dtype dtype,
                                        size_t *bytes);
cuca_status cuca_hip_gemm_w16(cuca_hip_ctx *ctx, const void *w16, int64_t n, int64_t k, const void *x,
                              int64_t ldx, int64_t m, int64_t rows, void *workspace,
                              size_t workspace_bytes, void *out, int64_t out_ld, cuca_dtype dtype);
cuca_status cuca_hip_gemm_w16_glu(cuca_hip_ctx *ctx, const void *w16, int64_t ff, int64_t k, const void *x,
                                  int64_t ldx, int64_t m, cuca_act act, float clamp, void *workspace,
                                  size_t workspace_bytes, void *out, int64_t out_ld, cuca_dtype dtype);

/* The end of a step (Transformer::finish / head / cap_logits,
 * cpu.rs:2495-2617; the final norm is cuca_hip_add_rmsnorm).
 * cuca_hip_lm_head: the LM head's quantized matmul (cuca_hip_qmm's bits)
 * with cap_logits fused into its epilogue, in candle's affine form:
 *   v = v * f32(1 / logit_scale) + 0   (logit_scale != 1)
 *   v = v * logit_mult + 0             (logit_mult != 1)
 *   v = tanh(v * f32(1 / softcap) + 0) * softcap + 0   (softcap > 0)
 * Without a soft-cap the logits are the reference's bits; tanh is the
 * device's (within 2 ulp).  rows: the first `rows` vocabulary entries
 * (head_rows, cpu.rs:2597-2601). */
cuca_status cuca_hip_lm_head(cuca_hip_ctx *ctx, const void *w, uint32_t ggml_type, int64_t vocab, int64_t n_embd,
                             const void *x, int64_t ldx, int64_t m, int64_t rows, float logit_scale,
                             float logit_mult, float softcap, void *logits, int64_t logits_ld, cuca_dtype dtype);

/* The LM head over chosen vocabulary entries only (head_indexed,
 * cpu.rs:2603-2606: QMatMul::forward_indexed, qmm.rs:1818-1843, then
 * cap_logits): logits[t][j] is the full head's logit of entry ids[j] for
 * row t -- the same bits as cuca_hip_lm_head's column ids[j] -- for
 * j < n_ids (any order, repeats allowed).  ids: device u32 [n_ids].  The
 * chosen packed rows are gathered into the workspace (device, 16-byte
 * aligned, cuca_hip_lm_head_indexed_workspace bytes: n_ids packed rows)
 * and run as a row prefix.  An id >= vocab is reported by
 * cuca_hip_check_device ("weight row ... out of range", as the reference's
 * error), its column then the logit of a zero row. */
cuca_status cuca_hip_lm_head_indexed_workspace(uint32_t ggml_type, int64_t n_embd, int64_t n_ids, size_t *bytes);
cuca_status cuca_hip_lm_head_indexed(cuca_hip_ctx *ctx, const void *w, uint32_t ggml_type, int64_t vocab,
                                     int64_t n_embd, const void *x, int64_t ldx, int64_t m, const uint32_t *ids,
                                     int64_t n_ids, float logit_scale, float logit_mult, float softcap,
                                     void *workspace, size_t workspace_bytes, void *logits, int64_t logits_ld,
                                     cuca_dtype dtype);

/* Sampling's scans over the vocabulary on the device (sampler.rs), so a
 * step reads back an id or k candidates per row instead of the logits.
 * cuca_hip_argmax: greedy (sampler.rs:44-56) per row: the first maximum
 *   (NaN never wins; a row without a value above -inf gives 0).
 * cuca_hip_top_k: select_top_k (sampler.rs:254-286) per row: after
 *   l / temperature, the k best finite logits, best first by
 *   (f32 total order desc, id asc) -- those of a full sort -- into
 *   out_logits / out_ids ([rows][k]; the scaled logits), their count
 *   (min(k, finite logits)) into out_count[rows].  The host continues
 *   warp_candidates / sample (softmax, top-p, the SplitMix64 draw) on them.
 *   k is at most CUCA_TOP_K_MAX. */
#define CUCA_TOP_K_MAX 1024

/* Host-side: the rest of sample() after select_top_k (sampler.rs:166-185,
 * 308-334) over one row's candidates from cuca_hip_top_k (best first):
 * p = exp(l - l[0]) / sum, zeros dropped (none left: `fallback`, the row's
 * greedy id), cut_top_p, then one SplitMix64 draw (*rng_state advances) --
 * the reference's bits with the platform libm's expf.  No GPU is used. */
cuca_status cuca_hip_sample_candidates(const float *logits, const uint32_t *ids, int32_t count, float top_p,
                                       uint32_t fallback, uint64_t *rng_state, uint32_t *out_id);
cuca_status cuca_hip_argmax(cuca_hip_ctx *ctx, const void *logits, int64_t ld, int64_t rows, int64_t vocab,
                            cuca_dtype dtype, uint32_t *ids);
cuca_status cuca_hip_top_k(cuca_hip_ctx *ctx, const void *logits, int64_t ld, int64_t rows, int64_t vocab,
                           cuca_dtype dtype, int32_t k, float temperature, float *out_logits, uint32_t *out_ids,
                           int32_t *out_count);

/* The decode GEMV in two steps, for callers that quantise an activation
 * once for several matrices (Q, K and V of one row; gate and up):
 * cuca_hip_q8_acts: Acts::new (qmm.rs:1272-1343) on the device: x [m][ldx]
 *   -> quants int8 [m][k] (element order) and scales f32 [m][k/32] (the
 *   f16-rounded block scales); quants 16-byte aligned, k a multiple of 32.
 * cuca_hip_qmv / cuca_hip_qmv_glu: cuca_hip_qmm / _qmm_glu on those, the
 *   same bits, for m = 1 or 2 rows whose row length fits the kernel's LDS
 *   (up to 14336 values for one row, 6144 for two; CUCA_UNSUPPORTED
 *   otherwise).
 * cuca_hip_qmm, _qmm_glu and _lm_head use the same kernel by themselves for
 * one or two rows of a tall matrix (at least 32 four-row tasks per CU: the
 * LM head), each workgroup quantising the rows itself; the MoE calls use it
 * from two tokens' pairs up. */
cuca_status cuca_hip_q8_acts(cuca_hip_ctx *ctx, const void *x, int64_t ldx, int64_t m, int64_t k, cuca_dtype dtype,
                             int8_t *quants, float *scales);
cuca_status cuca_hip_qmv(cuca_hip_ctx *ctx, const void *w, uint32_t ggml_type, int64_t n, int64_t k,
                         const int8_t *quants, const float *scales, int64_t m, int64_t rows, void *out, int64_t out_ld,
                         cuca_dtype dtype);
cuca_status cuca_hip_qmv_glu(cuca_hip_ctx *ctx, const void *gate, const void *up, uint32_t ggml_type, int64_t ff,
                             int64_t k, const int8_t *quants, const float *scales, int64_t m, cuca_act act, float clamp,
                             void *out, int64_t out_ld, cuca_dtype dtype);

/* Routed experts (MoE), the CPU engine's expert_sum (cpu.rs:3599-3642)
 * with CpuExpert::forward / add_picks (cpu.rs:373-419), split as the
 * reference GPU engine splits it (MoeKernels::moe_up / moe_down / moe_sum,
 * moe_kernel.rs:1163-1385).  Routing (moe.rs:39-94) is the caller's: the
 * (token, expert) pairs are grouped by expert, expert e owning pairs
 * [offsets[e], offsets[e+1]) in token order (device int32[n_experts + 1],
 * read on the device; the pair arrays hold max_pairs entries).  The
 * experts' packed matrices (cuca_hip_qweight_pack) lie expert_stride bytes
 * apart (a pool, as the reference GPU engine's expert slots).
 *
 * moe_up: hidden[p] = act(gate_e . x[pair_token[p]]) * (up_e . x[...]), the
 *   products bit-exact with cuca_hip_qmm, the activation and clamp as
 *   cuca_hip_glu.  hidden: [max_pairs][hidden_ld] of dtype.  A pair token
 *   outside [0, n_tokens) is skipped and reported by cuca_hip_check_device.
 * moe_down: scratch[p] = (down_e . hidden[p]) * pair_weight[p] (f32; the
 *   product of add_picks, cpu.rs:400-417).
 * moe_sum: out[t] = sum over i < n_used of scratch[token_pairs[t][i]], in
 *   f32 from 0, in the given order (ascending expert order, as expert_sum
 *   adds); entries < 0 are skipped. */
cuca_status cuca_hip_moe_up(cuca_hip_ctx *ctx, const void *gate, const void *up, int64_t expert_stride,
                            uint32_t ggml_type, int64_t ff, int64_t n_embd, int32_t n_experts, const void *x,
                            int64_t ldx, int64_t n_tokens, const int32_t *offsets, const int32_t *pair_token,
                            int64_t max_pairs, cuca_act act, float clamp, void *hidden, int64_t hidden_ld,
                            cuca_dtype dtype);
cuca_status cuca_hip_moe_down(cuca_hip_ctx *ctx, const void *down, int64_t expert_stride, uint32_t ggml_type,
                              int64_t n_embd, int64_t ff, int32_t n_experts, const void *hidden,
                              int64_t hidden_ld, const int32_t *offsets, const float *pair_weight,
                              int64_t max_pairs, float *scratch, int64_t scratch_ld, cuca_dtype dtype);
cuca_status cuca_hip_moe_sum(cuca_hip_ctx *ctx, const float *scratch, int64_t scratch_ld, int64_t max_pairs,
                             const int32_t *token_pairs, int32_t n_used, int64_t n_tokens, int64_t n_embd,
                             void *out, int64_t out_ld, cuca_dtype dtype);

/* Routed experts at prefill on the matrix cores: moe_up / moe_down as one
 * grouped GEMM launch each over the expert-sorted pairs, in the arithmetic
 * class of cuca_hip_qgemm (the reference GPU engine's MoE kernels,
 * moe_kernel.rs:1163-1300, with f32 sums of products of f16(d * q) weights
 * and f16 activations), not the CPU engine's bits (cuca_hip_moe_up/_down):
 *   up:   hidden[p] = act(gate_e . x[pair_token[p]]) * (up_e . x[...]),
 *         the GLU applied to the f32 sums, Glu::apply's clamp;
 *   down: scratch[p] = (down_e . hidden[p]) * pair_weight[p], f32.
 * Each product is within (2^-10 + k 2^-24) sum |w x| of the exact one.
 * Arguments as cuca_hip_moe_up / _down (expert e's pairs are
 * [offsets[e], offsets[e + 1]), read on the device, clamped into
 * [0, max_pairs] and made non-decreasing; a pair token outside
 * [0, n_tokens) gives a zero activation row and is reported by
 * cuca_hip_check_device), plus a device workspace (16-byte aligned) of
 * cuca_hip_moe_qgemm_workspace bytes for k = n_embd (up) or ff (down),
 * n_experts and max_pairs.  Up to 4096 experts.  moe_sum then adds the
 * scratch rows as for the other path.  For a few pairs per expert the
 * GEMV path (cuca_hip_moe_up/_down) is the faster one. */
cuca_status cuca_hip_moe_qgemm_workspace(uint32_t ggml_type, int64_t k, int32_t n_experts, int64_t max_pairs,
                                         size_t *bytes);
cuca_status cuca_hip_moe_up_qgemm(cuca_hip_ctx *ctx, const void *gate, const void *up, int64_t expert_stride,
                                  uint32_t ggml_type, int64_t ff, int64_t n_embd, int32_t n_experts, const void *x,
                                  int64_t ldx, int64_t n_tokens, const int32_t *offsets, const int32_t *pair_token,
                                  int64_t max_pairs, cuca_act act, float clamp, void *workspace,
                                  size_t workspace_bytes, void *hidden, int64_t hidden_ld, cuca_dtype dtype);
cuca_status cuca_hip_moe_down_qgemm(cuca_hip_ctx *ctx, const void *down, int64_t expert_stride, uint32_t ggml_type,
                                    int64_t n_embd, int64_t ff, int32_t n_experts, const void *hidden,
                                    int64_t hidden_ld, const int32_t *offsets, const float *pair_weight,
                                    int64_t max_pairs, void *workspace, size_t workspace_bytes, float *scratch,
                                    int64_t scratch_ld, cuca_dtype dtype);

/* RopeSpec (rope.rs:62-79). yarn_ext_factor == 0 disables YaRN. */
typedef struct {
    int32_t kind;         /* cuca_rope_kind (not used by the tables)   */
    int32_t n_dims;       /* rotated leading dims, even                 */
    double base;          /* frequency base (theta)                     */
    double freq_scale;    /* 1 / scaling factor; 1.0 when unscaled      */
    double yarn_ext_factor, yarn_beta_fast, yarn_beta_slow;
    int64_t yarn_n_ctx_orig;
    double attn_factor;   /* multiplier on cos and sin; 1.0 when plain  */
} cuca_rope_spec;

/* Host-side RopeSpec::tables (rope.rs:118-151): cos/sin [positions, n_dims/2]
 * computed in f64 with the platform libm and rounded to f32, bit-identical
 * to the reference's tables.  factors: NULL or n_dims/2 positive divisors
 * (rope_factors, mod.rs:420-458).  Writes host memory; upload once. */
cuca_status cuca_hip_rope_tables(const cuca_rope_spec *spec, const float *factors,
                                 int64_t positions, float *cos_out, float *sin_out);

/* ------------------------------------------------------------------ */
/* Graphs (decode) and timing                                           */
/* ------------------------------------------------------------------ */

/* Capture every op issued on the context's stream between begin and end
 * into an executable graph (the per-layer launches of a decode step).  The
 * captured ops keep the pointers and scalars they were called with; replay
 * with cuca_hip_graph_launch after refreshing the buffers' contents. */
cuca_status cuca_hip_graph_begin(cuca_hip_ctx *ctx);
cuca_status cuca_hip_graph_end(cuca_hip_ctx *ctx, cuca_hip_graph **out);
cuca_status cuca_hip_graph_launch(cuca_hip_ctx *ctx, cuca_hip_graph *graph);
void cuca_hip_graph_destroy(cuca_hip_graph *graph);

/* Elapsed milliseconds of the work issued on the context's stream between
 * cuca_hip_timer_start and cuca_hip_timer_stop (HIP events; blocks until
 * the stop event completes). */
cuca_status cuca_hip_timer_start(cuca_hip_ctx *ctx);
cuca_status cuca_hip_timer_stop(cuca_hip_ctx *ctx, float *ms);

/* Per-kernel timing, the device-side counterpart of the engine's
 * ServingCounters (engine/mod.rs:566-612, per-forward step_ns): between
 * profile_start and profile_stop the first `max_launches` kernels the ops
 * launch carry start/stop events on the kernel itself
 * (hipExtModuleLaunchKernel), so their durations exclude dispatch gaps.
 * profile_stop synchronizes and writes up to `max` records, in launch order.
 * Not available during a graph capture. */
typedef struct {
    const char *kernel; /* the kernel's symbol in the code object (static) */
    float ms;
} cuca_hip_kernel_time;

cuca_status cuca_hip_profile_start(cuca_hip_ctx *ctx, int32_t max_launches);
cuca_status cuca_hip_profile_stop(cuca_hip_ctx *ctx, cuca_hip_kernel_time *out, int32_t max,
                                  int32_t *count);

#ifdef __cplusplus
}
#endif
#endif
