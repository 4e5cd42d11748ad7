/*
 * kernel_args.h -- by-value argument blocks of the gfx950 kernels.
 *
 * Shared by the host runtime (runtime.cpp, which packs one block per
 * hipModuleLaunchKernel call) and the device code (the kernels/ sources, where each
 * kernel takes its block as its only parameter).  Plain C layout only.
 */
#ifndef CUCA_KERNEL_ARGS_H
#define CUCA_KERNEL_ARGS_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Device status words, one per kind of bad input the kernels can meet.
 * Each holds (row << 32 | value) of the smallest bad row seen, or all
 * ones.  The host resets them after reading (cuca_hip_check_device). */
enum {
    CUCA_STATUS_EMBED_ID = 0,
    CUCA_STATUS_ROPE_POS = 1,
    CUCA_STATUS_KV_SLOT = 2,
    CUCA_STATUS_KV_RANGE = 3, /* attention: a key position without a block, or a bad range */
    CUCA_STATUS_MOE_PAIR = 4, /* MoE: a pair whose token is outside the activation rows */
    CUCA_STATUS_HEAD_ROW = 5, /* indexed LM head: a vocabulary id past the head's rows */
    CUCA_STATUS_WORDS = 6
};

typedef struct {
    const uint8_t *table;   /* [vocab, row_bytes]                          */
    const uint32_t *ids;    /* [n]                                         */
    void *out;              /* [n, hidden] f32 or f16                      */
    unsigned long long *status;
    int64_t vocab;
    int64_t row_bytes;
    int32_t hidden;
    int32_t n;
    float scale;
    float norm_eps;         /* the _norm kernels: rms_norm_rows' eps       */
    void *h_out;            /* the _rms kernels: [n, hidden] rms(x, w)     */
    const float *rms_w;     /* the _rms kernels: [hidden] or NULL          */
    float rms_eps;          /* the _rms kernels                            */
    int32_t tpw;            /* the _rms_lds kernels: tokens per wave; a
                               workgroup of 4 waves covers 4 tpw tokens   */
} EmbedArgs;

/* Self-test of the wave reductions (cuca_selftest_group_sum): out holds 12
 * arrays of n: for each group size 2, 4, ..., 64 the library's group_sum,
 * then the __shfl_xor butterfly, of in[i] over its aligned group. */
typedef struct {
    const float *in;
    float *out;
    int64_t n;
} SelftestArgs;

typedef struct {
    const void *x;          /* [rows, hidden]                              */
    const void *branch;     /* [rows, hidden] or NULL                      */
    const float *w;         /* [hidden] or NULL                            */
    const float *w_post;    /* [hidden] or NULL                            */
    void *x_out;            /* [rows, hidden] or NULL                      */
    void *h_out;            /* [rows, hidden]                              */
    int64_t rows;
    int32_t hidden;
    float eps;
    float post_eps;
    float rs;               /* residual scale                              */
} NormArgs;

typedef struct {
    const void *gate;
    const void *up;
    void *out;
    const int32_t *offsets; /* ragged: device [n_experts + 1] or NULL      */
    int64_t rows;           /* dense: rows; ragged: max_rows               */
    int64_t gate_ld, up_ld, out_ld; /* row strides in elements             */
    int32_t ff;
    int32_t blocks_per_row;
    int32_t n_experts;
    float clamp;            /* > 0: clamp gate from above, up to +-clamp   */
} GluArgs;
#define CUCA_GLU_NT_BLOCK 64 /* threads of a streaming (_nt) GLU workgroup */

typedef struct {
    void *q;                /* [rows, nq, d] with row stride q_ld           */
    void *k;                /* [rows, nk, d] with row stride k_ld           */
    const float *cos_t;     /* [table_rows, n_dims / 2]                     */
    const float *sin_t;
    const int32_t *pos;     /* [rows]                                       */
    const float *q_norm_w;  /* [d] or NULL                                  */
    const float *k_norm_w;  /* [d] or NULL                                  */
    unsigned long long *status;
    int64_t q_ld, k_ld;
    int64_t table_rows;
    int32_t rows;
    int32_t nq, nk;
    int32_t head_dim;
    int32_t n_dims;
    int32_t tph_log2;       /* log2(threads per head), vector kernels       */
    float eps;
    int32_t kind;           /* generic kernel: 0 NORM, 2 NEOX               */
    /* paged K/V store (the _kv kernels; zero otherwise): K heads are
     * written to pool_k and V heads to pool_v instead of in place, row r
     * to pool row slots[r] = block * 16 + position % 16 of a
     * [n_blocks, nk, 16, d] pool                                            */
    const void *v;          /* [rows, nk, d] with row stride v_ld           */
    void *pool_k;
    void *pool_v;
    const int32_t *slots;   /* [rows]                                       */
    int64_t v_ld;
    int64_t n_slots;        /* n_blocks * 16                                */
    int32_t nv;             /* V heads: nk for the store, else 0            */
    int32_t v_norm;         /* weightless RMSNorm of V before the store     */
} RopeArgs;

/* Paged decode attention: split pass (partials over `part_positions` key
 * positions each) and merge pass (one wave per row and query head).
 * part: [rows, n_head, max_parts, head_dim + 2] f32 partials (value
 * accumulator, maximum, sum).  CUCA_ATTN_MIN_PART bounds part_positions
 * from below (it sizes the workspace). */
#define CUCA_ATTN_MIN_PART 64
typedef struct {
    const void *q;          /* [rows][q_ld]: n_head heads of d per row      */
    const void *pool_k;     /* [n_blocks, n_kv, 16, d]                      */
    const void *pool_v;
    const uint32_t *tables; /* [rows, max_blocks]                           */
    const int32_t *ranges;  /* [rows, 2]: lo, hi relative to the table      */
    float *part;
    void *out;              /* [rows, n_head, d]                            */
    unsigned long long *status;
    int64_t q_ld;           /* row stride of q in elements                  */
    int64_t n_blocks;
    int32_t rows, n_head, n_kv, head_dim;
    int32_t max_blocks, max_parts;
    int32_t part_positions; /* key positions per partial                    */
    float scale;
    int32_t direct;         /* one part a row: the split writes out itself  */
    int32_t pad_;
} AttnArgs;

/* Packed weight rows gathered by index (the indexed LM head): dst row j =
 * src row ids[j] (row_bytes each, a multiple of 16), zeros for an id past
 * n_src (recorded). */
typedef struct {
    const uint8_t *src;
    const uint32_t *ids;
    uint8_t *dst;
    unsigned long long *status;
    int64_t n_src;
    int64_t row_bytes;
    int32_t n;
    int32_t pad_;
} RowGatherArgs;

/* Paged attention of many query rows of one sequence (attn_rows.hip): row
 * r of q attends to the positions ranges[r] = [lo, hi) of the sequence's
 * block table.  Values: pool_v, or (pool_v NULL, the latent form) the first
 * v_width columns of the key rows themselves. */
typedef struct {
    const void *q;          /* [rows][q_ld]: n_head heads of head_dim        */
    const void *pool_k;     /* [n_blocks, n_kv, 16, head_dim]                */
    const void *pool_v;     /* the same, or NULL (values = key prefix)       */
    const uint32_t *table;  /* [max_blocks]                                  */
    const int32_t *ranges;  /* [rows, 2]                                     */
    void *out;              /* [rows][out_ld]: n_head heads of v_width       */
    unsigned long long *status;
    int64_t q_ld, out_ld;   /* row strides in elements                       */
    int64_t n_blocks;
    int32_t rows, n_head, n_kv, head_dim, v_width, max_blocks;
    float scale;
    int32_t pad_;
} AttnRowsArgs;

/* Quantized matmul (qmm.hip): packed weights [n][ng][GB] (see there),
 * activations x [m][ldx], out [m][out_ld] in the activation type.  The
 * grid is nrb8 * ntile workgroups (nrb8 = nrb rounded up to a multiple of
 * 8); workgroup id -> (row block, activation tile) is XCD-aware. */
typedef struct {
    const uint8_t *w;       /* packed weight (gate for the GLU kernels)     */
    const uint8_t *w_up;    /* packed up weight (GLU kernels) or NULL       */
    const void *x;          /* [m][ldx]                                      */
    void *out;              /* [m][out_ld]                                   */
    int64_t ldx, out_ld;    /* row strides in elements                       */
    int64_t row_bytes;      /* packed bytes per weight row (ng * GB)         */
    int32_t rows;           /* weight rows computed (<= n)                   */
    int32_t m;              /* activation rows                               */
    int32_t nb;             /* blocks per row (k / 32)                       */
    int32_t ng;             /* groups per row                                */
    int32_t nrb;            /* row blocks of 16 rows                         */
    int32_t ntile;          /* activation tiles                              */
    float clamp;            /* GLU: > 0 clamps gate from above, up to +-clamp */
    int32_t n_tokens;       /* MoE up: rows of x (pair tokens are checked)   */
    /* MoE (moe_up / moe_down kernels): pairs grouped by expert, expert e
     * owning pairs [offsets[e], offsets[e+1]); an activation tile is MT
     * pairs of one expert; the expert's packed matrices start at
     * w + e * w_estride (and w_up + e * w_estride).                          */
    const int32_t *offsets;     /* [n_experts + 1], on the device            */
    const int32_t *pair_token;  /* moe_up: token (row of x) of each pair     */
    const float *pair_weight;   /* moe_down: routing weight of each pair     */
    unsigned long long *status;
    int64_t w_estride;          /* bytes between experts' packed matrices    */
    int32_t n_experts;
    int32_t max_pairs;          /* capacity of the pair arrays               */
    /* LM head epilogue (plain kernels; cap_flags 0 = none): bit 1 scales
     * by mul1 = f32(1 / logit_scale), bit 2 by mul2 = logit_mult, bit 4
     * soft-caps: tanh(v * softcap_inv) * softcap; each step adds +0 as
     * candle's affine does (cpu.rs:2603-2617).                              */
    int32_t cap_flags;
    float mul1, mul2, softcap_inv, softcap;
    int32_t pad2_;
    /* Q|K|V projection with RoPE and the paged K/V store in the epilogue
     * (qmm_rope_kv kernels): weight rows [0, nq * d) are the Q heads, then
     * nk K heads and nk V heads of d rows; Q is rotated into out, K rotated
     * and V copied into the pools [n_blocks, nk, 16, d] at slots[j].       */
    const float *cos_t, *sin_t;     /* [table_rows, n_dims / 2]              */
    const int32_t *pos, *slots;     /* [m]                                   */
    void *pool_k, *pool_v;
    int64_t table_rows, n_slots;
    int32_t nq, nk, head_dim, n_dims;
    /* residual add + RMSNorm in the prologue (qmd *_rn kernels, one row):
     * x' = x + rs * branch (branch nullable) -> rn_x_out, h = rms(x', rn_w,
     * eps) -> rn_h_out (both written by workgroup 0, either nullable), and
     * the matmul runs on h.  The sum of squares follows the add_rmsnorm
     * vector kernel of rn_tpr threads x rn_per chunks per row.             */
    const void *rn_branch;
    const float *rn_w;
    void *rn_x_out, *rn_h_out;
    float rn_eps, rn_rs;
    int32_t rn_tpr, rn_per;
} QmmArgs;

/* The quantized matmul on the matrix cores (qgemm.hip): out[t][n] =
 * x[t] . w[n] over f16 weights f16(d * q) and f16 activations, f32
 * accumulation; workgroups of 128 weight rows x TM tokens. */
typedef struct {
    const uint8_t *w, *w_up;    /* packed weights (gate/up for GLU)          */
    const void *x;              /* [m][ldx] f32 or f16                       */
    uint16_t *xp;               /* workspace: x in slot order [mp][kp] f16,  */
                                /* mp = n_ct * tile tokens, rows past m zero */
    float *part;                /* workspace: split sums [splits][g,u][m][rows] */
    void *out;                  /* [m][out_ld]                               */
    int64_t ldx, out_ld, row_bytes, kp;
    int32_t rows, m, k, nkc, n_rt, n_ct, kcs, splits;
    float clamp;
    int32_t mp;
    /* routed experts (the qgemm_moe kernels): expert e's packed matrices at
     * w (w_up) + e * estride; token tile ct holds pairs [tile_p0[ct],
     * tile_p0[ct] + tile_n[ct]) of expert tile_e[ct] (-1 past the last
     * tile), written by cuca_moe_plan from offsets; up: activation row of
     * pair p = x[pair_token[p]] (m = n_tokens), out = hidden [pairs][out_ld];
     * down: activation row = x[p] (m = max_pairs), out = f32 scratch
     * [pairs][out_ld] times pair_weight[p].                                */
    const int32_t *offsets, *pair_token;
    const float *pair_weight;
    int32_t *tile_e, *tile_p0, *tile_n;
    unsigned long long *status;
    int64_t estride;
    int32_t n_experts, max_pairs, tm, moe_up;
} QGemmArgs;

/* The dense f16 path's conversions (qgemm.hip): cuca_qdequant_* (packed w
 * [n][ng][GB], row_bytes each -> out f16 [n][out_ld]) and cuca_cvt_f16_f32
 * (x [m][ldx] f32 -> out f16 [m][out_ld], k values a row). */
typedef struct {
    const uint8_t *w;
    const void *x;
    void *out;
    int64_t row_bytes, ldx, out_ld;
    int64_t n;
    int32_t m, k, nb, ng;
    float clamp;
    int32_t pad_;
} QDequantArgs;

/* The dense f16 GEMM (gemm16.hip): out [m][out_ld] = x [m][ldx] . w^T over
 * f16 weight rows [.][ldw]; the GLU form reads gate rows from 0 and up rows
 * from up_row and writes act(gate) * up.  Tiles of 256 (GLU 128) output
 * columns x 256 rows; k a multiple of 32; ldw, ldx < 2^22. */
typedef struct {
    const void *w;
    const void *x;
    void *out;
    int64_t ldw, ldx, out_ld;
    int64_t up_row;
    int32_t n, m, k;        /* output columns, rows, k                      */
    int32_t n_tn, n_tm, gn; /* column tiles, row tiles, tile-order group    */
    int32_t vec;            /* out_ld % 4 == 0: four-column stores          */
    float clamp;            /* GLU: > 0 clamps gate from above, up to +-    */
    /* split k (grid y = splits): k is then the length of one split, and
     * split s takes k values from s k on and writes its sums to output
     * matrix s (out + s m out_ld).  cuca_gemm16_reduce_* adds the splits'
     * part [splits][m][n or 2 n] in order and applies the output (n, out,
     * out_ld, clamp as for the GEMM). */
    float *part;
    int32_t splits, pad_;
} Gemm16Args;

/* Activation quantisation for the decode GEMV (Acts::new, qmm.rs:1272-1343):
 * x [m][ldx] -> quants [m][q_ld] int8 (element order) and scales [m][nb]. */
typedef struct {
    const void *x;
    int8_t *quants;
    float *scales;
    int64_t ldx, q_ld;
    int32_t m, nb;
} Q8ActsArgs;

/* The decode GEMV (qmv.hip): tiles of MT <= 4 activation rows held in LDS
 * for the whole row length, either quantised already (quants / scales) or
 * quantised by the workgroup from x; tasks of 4 weight rows per wave.
 * Epilogue as QmmArgs (GLU, cap).  MoE (modes 1 / 2): workgroup (tile,
 * split) takes tile `tile` of the expert order and row tasks
 * [split * tps, (split + 1) * tps) of the expert's matrix. */
typedef struct {
    const uint8_t *w, *w_up;    /* packed weights (gate/up for GLU)          */
    const int8_t *quants;       /* mode 0: [m][q_ld]                         */
    const float *scales;        /* mode 0: [m][nb]                           */
    const void *x;              /* modes 1-3: activation rows [.][ldx]       */
    void *out;                  /* [m or pairs][out_ld]                      */
    const int32_t *offsets;     /* MoE: [n_experts + 1]                      */
    const int32_t *pair_token;  /* MoE up: [max_pairs]                       */
    const float *pair_weight;   /* MoE down: [max_pairs]                     */
    unsigned long long *status;
    int64_t q_ld, out_ld, row_bytes, ldx, w_estride;
    int32_t rows, m, nb, ng, nbp, ntask;
    int32_t n_experts, max_pairs, n_tokens, splits, tps;
    float clamp;
    int32_t cap_flags;
    float mul1, mul2, softcap_inv, softcap;
} QmvArgs;

/* Greedy argmax and top-k over logits rows (sampler.rs greedy and
 * select_top_k).  top-k: keys are logit / temperature; the k best finite
 * ones in (logit desc, id asc) order go to out_logits / out_ids, their
 * count to out_count.  A row is split into `slices` of slice_len values;
 * with more than one, the slices' results go to cand (argmax: one (value
 * bits << 32 | id) per slice; top-k: up to k composites per slice, their
 * count in cand_count) and a merge launch finishes the row. */
#define CUCA_PICK_CAP 7680        /* top-k composites a workgroup holds in LDS */
#define CUCA_PICK_MAX_SLICES 256  /* slices per row                           */

typedef struct {
    const void *logits;     /* [rows][ld] f32 or f16                          */
    float *out_logits;      /* [rows][k]                                      */
    uint32_t *out_ids;      /* [rows][k] (argmax: [rows])                     */
    int32_t *out_count;     /* [rows]                                         */
    unsigned long long *cand; /* [rows][slices][k] (argmax: [rows][slices])   */
    int32_t *cand_count;    /* [rows][slices]                                 */
    int64_t ld;
    int32_t rows, vocab, k;
    float temperature;
    int32_t slices, slice_len;
    int32_t mode;           /* 0: whole rows, final; 1: slices to cand        */
    int32_t pad_;
} PickArgs;

/* MoE expert sum: out[t] = sum over i < n_used of scratch[pairs[t][i]]
 * (pairs in ascending expert order, -1 = none), f32 in order from 0. */
typedef struct {
    const float *scratch;   /* [pairs][scratch_ld] f32                       */
    const int32_t *pairs;   /* [n_tokens][n_used]                            */
    void *out;              /* [n_tokens][out_ld]                            */
    int64_t scratch_ld, out_ld;
    int32_t n_tokens, n_used, n_embd, max_pairs;
} MoeSumArgs;

typedef struct {
    const uint8_t *src;     /* GGUF rows [n][nb * block bytes]               */
    uint8_t *dst;           /* packed [n][ng][GB]                            */
    int32_t n, nb, ng, pad_;
} QPackArgs;

#ifdef __cplusplus
}
#endif
#endif
