/*
 * cuca_oracle.h -- CPU restatement of the reference engine's per-layer
 * non-matmul ops (nassor/cuca 0.10.0, provider-local).
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker and the
 * CPU-baseline timer.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it.  The product path (cuca_amd/, libcuca_hip.so)
 * never links, loads or falls back to it.
 *
 * Every function cites the reference file:line it restates.  Paths are
 * relative to the reference crate root (src/provider/local/model/...).
 *
 * Arithmetic contract: compiled with -ffp-contract=off so that every f32
 * product and sum is rounded on its own, as Rust (which never contracts)
 * and candle's scalar CPU kernels do.  f16 values are widened exactly and
 * results are rounded once, to nearest-even, on output.
 */
#ifndef CUCA_ORACLE_H
#define CUCA_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { OR_F32 = 0, OR_F16 = 1 };          /* element type of activations   */
enum { OR_Q4_0 = 2, OR_Q8_0 = 8 };        /* ggml type ids (gguf/dtype.rs) */
enum { OR_SILU = 0, OR_GELU_TANH = 1 };   /* arch.rs:101-106 Act          */
enum { OR_ROPE_NORM = 0, OR_ROPE_NEOX = 2 }; /* rope.rs:28-36 RopeKind    */

/* IEEE binary16 <-> binary32 (the `half` crate's to_f32 is exact;
 * the f32 -> f16 direction rounds to nearest, ties to even). */
float oracle_f16_to_f32(uint16_t h);
uint16_t oracle_f32_to_f16(float f);
void oracle_f16_to_f32_n(const uint16_t *h, float *f, int64_t n);
void oracle_f32_to_f16_n(const float *f, uint16_t *h, int64_t n);
/* The _n conversions use the x86 F16C instructions when the CPU has them
 * (oracle_has_f16c), the scalar restatement otherwise; the _soft_n forms are
 * always the scalar restatement. */
void oracle_f16_to_f32_soft_n(const uint16_t *h, float *f, int64_t n);
void oracle_f32_to_f16_soft_n(const float *f, uint16_t *h, int64_t n);
int oracle_has_f16c(void);

/* Bytes per row of `hidden` values of a Q4_0 / Q8_0 tensor, or -1 when the
 * row is not a whole number of 32-value blocks (quant.rs:110-118). */
int64_t oracle_row_bytes(uint32_t ggml_type, int64_t hidden);

/* dequant_row for Q4_0 / Q8_0 (quant.rs:107-198).  Returns 0, or -1 when
 * `nbytes` is not exactly n/32 blocks. */
int oracle_dequant_row(uint32_t ggml_type, const uint8_t *bytes, int64_t nbytes,
                       float scale, float *out, int64_t n);

/* TokenEmbedding::rows (quant.rs:391-411): out[n_tok, hidden] in `out_dtype`.
 * Returns 0; -1 for a bad row geometry; -2 for an id >= vocab, whose index
 * is stored in *bad_index (the reference's "token id {id} outside the
 * embedding table" error, quant.rs:395-400).  Rows are split over
 * `nthreads` threads (1 = the reference's scalar loop). */
int oracle_embed(const uint8_t *table, uint32_t ggml_type, int64_t vocab,
                 int64_t hidden, const uint32_t *ids, int64_t n_tok, float scale,
                 void *out, int out_dtype, int nthreads, int64_t *bad_index);

/* rms_norm_rows (quant.rs:324-339), applied by Hparams::norm_embeddings
 * (params.rs:374-379) to the looked-up rows of archs with embd_norm
 * (arch.rs:229-231): per row of row_len f32 values, in place,
 *   sum  = sum of f64(x) * f64(x), in index order, from 0
 *   inv  = (f32)(1 / sqrt(sum / row_len + f64(eps)))
 *   x    = x * inv (f32). */
void oracle_rms_norm_rows(float *rows, int64_t n_rows, int64_t row_len, float eps);

/* oracle_embed, then (norm != 0) rms_norm_rows on each f32 row before the
 * output rounding (forward_stage: rows(tokens, embd_scale) then
 * norm_embeddings, cpu.rs:1881-1882, gpu.rs:2976-2981). */
int oracle_embed_norm(const uint8_t *table, uint32_t ggml_type, int64_t vocab,
                      int64_t hidden, const uint32_t *ids, int64_t n_tok, float scale,
                      int norm, float norm_eps, void *out, int out_dtype, int nthreads,
                      int64_t *bad_index);

/* Fused residual add + RMSNorm, restating Transformer::block
 * (cpu.rs:2650-2711) with candle's rms_norm (cpu.rs:3652):
 *   b'  = w_post ? rms(branch, w_post, post_eps) : branch
 *   b'' = residual_scale == 1 ? b' : b' * residual_scale + 0   (affine)
 *   x'  = branch ? x + b'' : x           (stored in dtype -> x_out)
 *   h   = rms(x' as stored, w, eps)      (w == NULL: weightless norm)
 * rms(v, w, eps) = v / sqrt(sum(v*v)/H + eps) * w, sum in f32 in index
 * order.  x_out may be NULL (then x' is not written) or alias x. */
void oracle_add_rmsnorm(const void *x, const void *branch, const float *w,
                        const float *w_post, float eps, float post_eps,
                        float residual_scale, int64_t rows, int64_t hidden,
                        void *x_out, void *h_out, int dtype, int nthreads);

/* Glu::apply (cpu.rs:342-371) with activate (cpu.rs:3644-3649):
 *   g = clamp > 0 ? min(g, clamp) : g;  u = clamp > 0 ? clamp(u, -c, c) : u
 *   out = act(g) * u
 * SiLU v/(1+exp(-v)); GELU-tanh 0.5*v*(1+tanh(sqrt(2/pi)*v*(1+0.044715*v*v))).
 * Row r of gate/up/out starts at r*gate_ld / r*up_ld / r*out_ld elements. */
void oracle_glu(const void *gate, int64_t gate_ld, const void *up, int64_t up_ld,
                int64_t rows, int64_t ff, int act, float clamp, void *out,
                int64_t out_ld, int dtype, int nthreads);

/* RopeSpec::tables (rope.rs:118-151) in f64 with the platform libm, rounded
 * to f32.  yarn_ext_factor == 0 disables YaRN.  factors: NULL or n_dims/2
 * per-pair divisors.  cos/sin: [positions, n_dims/2]. */
void oracle_rope_tables(int n_dims, double base, double freq_scale,
                        double yarn_ext_factor, double yarn_beta_fast,
                        double yarn_beta_slow, int64_t yarn_n_ctx_orig,
                        double attn_factor, const float *factors,
                        int64_t positions, float *cos_out, float *sin_out);

/* apply_rope (cpu.rs:3672-3688, candle rope/rope_i) on x[rows, heads, d]
 * in place, with an optional per-head RMSNorm first (QK-norm,
 * cpu.rs:2840-2864, 3040-3055):
 *   norm_w != NULL: v = rms(head, norm_w[head_dim], eps)
 *   pair (a, b) of the first n_dims values (NORM: 2i,2i+1; NEOX: i,i+n/2):
 *     a' = a*c - b*s;  b' = a*s + b*c     (rope.rs:158-171)
 * c, s = cos/sin[positions[row], i].  Row r starts at r*ld elements. */
void oracle_rope(void *x, int64_t ld, int64_t rows, int heads, int head_dim,
                 int n_dims, int kind, const float *cos_t, const float *sin_t,
                 const int32_t *positions, const float *norm_w, float eps,
                 int dtype, int nthreads);

/* oracle_rope with the full-width QK-norm of the qk_norm_full archs (OLMo 2,
 * cpu.rs:2838-2843 for Q, 3042-3045 for K): rms over each row's whole
 * heads * head_dim projection with norm_w [heads * head_dim] (f32, as
 * rms_row), then every head rotated from those f32 values, one rounding on
 * output. */
void oracle_rope_full(void *x, int64_t ld, int64_t rows, int heads, int head_dim,
                      int n_dims, int kind, const float *cos_t, const float *sin_t,
                      const int32_t *positions, const float *norm_w, float eps,
                      int dtype, int nthreads);

/* Paged K/V pools (cpu/paged_attn.rs:1-38): [n_blocks][n_kv][16][d]
 * elements of `dtype` (1 = f16, else f32); position p of a sequence is row
 * p % 16 of block table[p / 16] (paged.rs:9-16), KV head kvh of it starts at
 * ((block * n_kv + kvh) * 16 + p % 16) * d (row_offset, :33-38).
 *
 * store_rows (:370-400): positions start..start+rows of src [n_kv][rows][d]
 * into the pool.  gather (:340-362): positions lo..hi of the pool into
 * out [n_kv][hi-lo][d].  Both check the range first as check_range does
 * (:42-65) and return -1, writing nothing, when a position has no block
 * (past the table, 0xffffffff, or an id >= n_blocks); 0 otherwise. */
int oracle_store_rows(const uint32_t *table, int64_t table_len, int64_t start, int64_t rows,
                      const void *src, void *pool, int64_t n_blocks, int n_kv, int d,
                      int dtype);
int oracle_gather(const uint32_t *table, int64_t table_len, int64_t lo, int64_t hi,
                  const void *pool, void *out, int64_t n_blocks, int n_kv, int d, int dtype);

/* attend_paged_rows (cpu/paged_attn.rs:105-290, attend_head :115-176) for
 * `rows` query rows, each with its own block table tables[row][max_blocks]
 * and key range ranges[row] = (lo, hi):
 *   q   : [rows][n_head][d], pools [n_blocks][n_kv][16][d], out [rows][n_head][d]
 *         (dtype 1 = f16, else f32; f16 values are widened, out rounded once)
 * Query head h reads KV head h / (n_head / n_kv).  Per block of the range:
 * scores dot(q, k) * scale (dot: eight lanes, paged_attn.rs:67-82), the
 * block maximum, the running sum and accumulator rescaled by
 * exp(max - block_max) when it grows, then p = exp(s - max), sum += p,
 * acc += p * v; out = acc / sum.  Returns -1, computing nothing, when a row's
 * range is empty or a position in it has no block (check_range); else 0. */
int oracle_paged_attention(const void *q, int64_t rows, int n_head, int n_kv, int d,
                           const uint32_t *tables, int64_t max_blocks, const int32_t *ranges,
                           const void *pool_k, const void *pool_v, int64_t n_blocks, float scale,
                           void *out, int dtype, int nthreads);

/* Quantized matmul of the CPU engine, QmmWeight (qmm.rs), for Q4_0 and Q8_0
 * weights (formats without minima, one entry per block).
 *
 * oracle_q8_acts restates Acts::new / quantise_block (qmm.rs:1217-1343) for
 * MIN_NONE: per 32-value block of each of the m rows of x (f32, or f16
 * widened): amax = max |v| (NaN ignored), d = amax / 127, id = d != 0 ?
 * 1 / d : 0, scale = f16(d) widened, q[e] = i8(round_away(v[e] * id))
 * (saturating, NaN -> 0).  q: [m][k] int8 in element order; scales: [m][k/32].
 *
 * oracle_qmm restates QmmWeight::forward_rows (qmm.rs:1810-1838) through the
 * definition the reference's own test states (qmm/tests.rs:151-191, module
 * docs qmm.rs:29-45): out[j][r] for weight rows r < rows is sixteen f32
 * lanes; lane l adds, block by block in row order,
 *     (float)(w[l]*q[l] + w[l+16]*q[l+16]) * (dw * dx)
 * (the exact integer pair sum, times the rounded product of the two f32
 * scales, product and sum each rounded), and the lanes are reduced by hsum
 * (qmm.rs:1345-1353): h[i] = a[i] + a[i+8], then
 * ((h0+h4)+(h1+h5))+((h2+h6)+(h3+h7)).  Q4_0 weight quants are nibble-8
 * (element i low nibble of byte i, element i+16 its high nibble,
 * qmm.rs:240-263); Q8_0 quants are the signed bytes (qmm.rs:404-426); dw is
 * the block's f16 scale.  w: GGUF bytes [n][k/32 blocks]; x: [m][ld] of
 * dtype; out: [m][rows] f32.  Returns 0, or -1 for a bad shape (k not a
 * multiple of 32, rows outside 1..n). */
void oracle_q8_acts(const void *x, int64_t ld, int64_t m, int64_t k, int dtype,
                    int8_t *q, float *scales);
int oracle_qmm(const uint8_t *w, uint32_t ggml_type, int64_t n, int64_t k,
               const void *x, int64_t ld, int64_t m, int64_t rows, float *out,
               int dtype, int nthreads);

/* The end of a step: cap_logits and the sampler.
 * oracle_cap_logits restates cap_logits (cpu.rs:2603-2617) with candle's
 * affine (v * f32(mul) + f32(add)) and tanhf, in place.
 * oracle_greedy restates greedy (sampler.rs:44-56).
 * oracle_splitmix64 / oracle_next_f32 restate SplitMix64 (sampler.rs:18-35).
 * oracle_select_top_k: select_top_k (sampler.rs:254-286) by its definition,
 * the k best finite logits / temperature of a full sort by by_logit_desc
 * (sampler.rs:58-60, its test sampler.rs:578-596); returns the count.
 * oracle_sample restates sample (sampler.rs:308-334) with warp_candidates
 * (:159-252) and cut_top_p (:288-300); logits are scaled in place. */
void oracle_cap_logits(float *v, int64_t n, float logit_scale, float logit_mult, float softcap);
uint32_t oracle_greedy(const float *logits, int64_t n);
uint64_t oracle_splitmix64(uint64_t *state);
float oracle_next_f32(uint64_t *state);
int64_t oracle_select_top_k(const float *logits, int64_t n, float temperature, int64_t k,
                            float *out_logits, uint32_t *out_ids);
uint32_t oracle_sample(float *logits, int64_t n, float temperature, int64_t top_k, float top_p,
                       uint64_t *rng);

#ifdef __cplusplus
}
#endif
#endif
