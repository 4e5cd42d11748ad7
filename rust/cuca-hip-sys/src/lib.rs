//! Raw bindings of `include/cuca_hip.h` (C ABI version 1): the MI355X
//! (gfx950) per-layer ops of provider-local -- the Q4_0/Q8_0 embedding
//! gather, residual add + RMSNorm, SwiGLU/GeGLU, RoPE with QK-norm and the
//! paged K/V store, paged decode attention, the quantized matmuls, the LM
//! head and sampling scans -- and the context, memory, graph and timing
//! plumbing around them.  Every function mirrors the header one to one
//! (`tests/test_rust_binding.py` checks names, argument types and struct
//! layouts against it); the header documents each call.  `safe` wraps the
//! calls the engine's layer loop makes.
#![allow(non_camel_case_types)]

use std::os::raw::{c_char, c_int, c_void};

pub mod safe;

pub const CUCA_HIP_ABI_VERSION: c_int = 1;

/// Opaque context: one device, its stream and the loaded code object.
#[repr(C)]
pub struct cuca_hip_ctx {
    _private: [u8; 0],
}

/// Opaque executable graph of captured launches.
#[repr(C)]
pub struct cuca_hip_graph {
    _private: [u8; 0],
}

pub type cuca_status = c_int;
pub const CUCA_OK: cuca_status = 0;
pub const CUCA_INVALID_ARG: cuca_status = 1;
pub const CUCA_OUT_OF_RANGE: cuca_status = 2;
pub const CUCA_HIP_ERROR: cuca_status = 3;
pub const CUCA_NOT_GFX950: cuca_status = 4;
pub const CUCA_UNSUPPORTED: cuca_status = 5;

pub type cuca_dtype = c_int;
pub const CUCA_F32: cuca_dtype = 0;
pub const CUCA_F16: cuca_dtype = 1;

/// ggml type ids (gguf/dtype.rs:195-250).
pub const CUCA_GGML_Q4_0: u32 = 2;
pub const CUCA_GGML_Q8_0: u32 = 8;

/// Act (arch.rs:101-106).
pub type cuca_act = c_int;
pub const CUCA_ACT_SILU: cuca_act = 0;
pub const CUCA_ACT_GELU_TANH: cuca_act = 1;

/// RopeKind (rope.rs:28-36), llama.cpp's rope type values.
pub type cuca_rope_kind = c_int;
pub const CUCA_ROPE_NORM: cuca_rope_kind = 0;
pub const CUCA_ROPE_NEOX: cuca_rope_kind = 2;

/// Positions per paged K/V block (paged.rs:45) and a released block's entry
/// (paged.rs:49).
pub const CUCA_KV_BLOCK: i64 = 16;
pub const CUCA_NO_BLOCK: u32 = 0xffff_ffff;
/// Largest k of cuca_hip_top_k.
pub const CUCA_TOP_K_MAX: i32 = 1024;
/// The per-GPU scratch of cuca_hip_paged_decode_noalloc, in bytes.
pub const CUCA_NOALLOC_SCRATCH_BYTES: usize = 64 << 20;

/// RopeSpec (rope.rs:62-79); yarn_ext_factor == 0 disables YaRN.
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct cuca_rope_spec {
    pub kind: i32,
    pub n_dims: i32,
    pub base: f64,
    pub freq_scale: f64,
    pub yarn_ext_factor: f64,
    pub yarn_beta_fast: f64,
    pub yarn_beta_slow: f64,
    pub yarn_n_ctx_orig: i64,
    pub attn_factor: f64,
}

/// One kernel's duration from cuca_hip_profile_stop.
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct cuca_hip_kernel_time {
    pub kernel: *const c_char,
    pub ms: f32,
}

extern "C" {
    pub fn cuca_hip_ctx_create(device: c_int, out: *mut *mut cuca_hip_ctx) -> cuca_status;
    pub fn cuca_hip_ctx_destroy(ctx: *mut cuca_hip_ctx);
    pub fn cuca_hip_last_error(ctx: *const cuca_hip_ctx) -> *const c_char;
    pub fn cuca_hip_set_stream(ctx: *mut cuca_hip_ctx, stream: *mut c_void) -> cuca_status;
    pub fn cuca_hip_get_stream(ctx: *const cuca_hip_ctx) -> *mut c_void;
    pub fn cuca_hip_device(ctx: *const cuca_hip_ctx) -> c_int;
    pub fn cuca_hip_malloc(
        ctx: *mut cuca_hip_ctx,
        bytes: usize,
        out: *mut *mut c_void,
    ) -> cuca_status;
    pub fn cuca_hip_free(ctx: *mut cuca_hip_ctx, ptr: *mut c_void) -> cuca_status;
    pub fn cuca_hip_memcpy_h2d_async(
        ctx: *mut cuca_hip_ctx,
        dst: *mut c_void,
        src: *const c_void,
        bytes: usize,
    ) -> cuca_status;
    pub fn cuca_hip_memcpy_d2h_async(
        ctx: *mut cuca_hip_ctx,
        dst: *mut c_void,
        src: *const c_void,
        bytes: usize,
    ) -> cuca_status;
    pub fn cuca_hip_memcpy_d2d_async(
        ctx: *mut cuca_hip_ctx,
        dst: *mut c_void,
        src: *const c_void,
        bytes: usize,
    ) -> cuca_status;
    pub fn cuca_hip_stream_sync(ctx: *mut cuca_hip_ctx) -> cuca_status;
    pub fn cuca_hip_check_device(ctx: *mut cuca_hip_ctx) -> cuca_status;
    pub fn cuca_hip_selftest_group_sum(
        ctx: *mut cuca_hip_ctx,
        input: *const f32,
        n: i64,
        out: *mut f32,
    ) -> cuca_status;
    pub fn cuca_hip_embed_gguf(
        ctx: *mut cuca_hip_ctx,
        table: *const c_void,
        ggml_type: u32,
        vocab: i64,
        hidden: i64,
        ids: *const u32,
        n: i64,
        scale: f32,
        out: *mut c_void,
        out_dtype: cuca_dtype,
    ) -> cuca_status;
    pub fn cuca_hip_embed_gguf_norm(
        ctx: *mut cuca_hip_ctx,
        table: *const c_void,
        ggml_type: u32,
        vocab: i64,
        hidden: i64,
        ids: *const u32,
        n: i64,
        scale: f32,
        norm_eps: f32,
        out: *mut c_void,
        out_dtype: cuca_dtype,
    ) -> cuca_status;
    pub fn cuca_hip_embed_gguf_rms(
        ctx: *mut cuca_hip_ctx,
        table: *const c_void,
        ggml_type: u32,
        vocab: i64,
        hidden: i64,
        ids: *const u32,
        n: i64,
        scale: f32,
        w: *const f32,
        eps: f32,
        x_out: *mut c_void,
        h_out: *mut c_void,
        out_dtype: cuca_dtype,
    ) -> cuca_status;
    pub fn cuca_hip_add_rmsnorm(
        ctx: *mut cuca_hip_ctx,
        x: *const c_void,
        branch: *const c_void,
        w: *const f32,
        w_post: *const f32,
        eps: f32,
        post_eps: f32,
        residual_scale: f32,
        rows: i64,
        hidden: i64,
        x_out: *mut c_void,
        h_out: *mut c_void,
        dtype: cuca_dtype,
    ) -> cuca_status;
    pub fn cuca_hip_glu(
        ctx: *mut cuca_hip_ctx,
        gate: *const c_void,
        gate_ld: i64,
        up: *const c_void,
        up_ld: i64,
        rows: i64,
        ff: i64,
        act: cuca_act,
        clamp: f32,
        out: *mut c_void,
        out_ld: i64,
        dtype: cuca_dtype,
    ) -> cuca_status;
    pub fn cuca_hip_glu_ragged(
        ctx: *mut cuca_hip_ctx,
        gate: *const c_void,
        gate_ld: i64,
        up: *const c_void,
        up_ld: i64,
        expert_offsets: *const i32,
        n_experts: i32,
        max_rows: i64,
        ff: i64,
        act: cuca_act,
        clamp: f32,
        out: *mut c_void,
        out_ld: i64,
        dtype: cuca_dtype,
    ) -> cuca_status;
    pub fn cuca_hip_rope(
        ctx: *mut cuca_hip_ctx,
        q: *mut c_void,
        q_ld: i64,
        k: *mut c_void,
        k_ld: i64,
        rows: i64,
        nq: i32,
        nk: i32,
        head_dim: i32,
        n_dims: i32,
        kind: cuca_rope_kind,
        cos: *const f32,
        sin: *const f32,
        table_rows: i64,
        positions: *const i32,
        q_norm_w: *const f32,
        k_norm_w: *const f32,
        eps: f32,
        dtype: cuca_dtype,
    ) -> cuca_status;
    pub fn cuca_hip_rope_full(
        ctx: *mut cuca_hip_ctx,
        q: *mut c_void,
        q_ld: i64,
        k: *mut c_void,
        k_ld: i64,
        rows: i64,
        nq: i32,
        nk: i32,
        head_dim: i32,
        n_dims: i32,
        kind: cuca_rope_kind,
        cos: *const f32,
        sin: *const f32,
        table_rows: i64,
        positions: *const i32,
        q_norm_w: *const f32,
        k_norm_w: *const f32,
        eps: f32,
        dtype: cuca_dtype,
    ) -> cuca_status;
    pub fn cuca_hip_rope_store_kv(
        ctx: *mut cuca_hip_ctx,
        q: *mut c_void,
        q_ld: i64,
        k: *const c_void,
        k_ld: i64,
        v: *const c_void,
        v_ld: i64,
        rows: i64,
        nq: i32,
        nk: i32,
        head_dim: i32,
        n_dims: i32,
        kind: cuca_rope_kind,
        cos: *const f32,
        sin: *const f32,
        table_rows: i64,
        positions: *const i32,
        q_norm_w: *const f32,
        k_norm_w: *const f32,
        v_norm: i32,
        eps: f32,
        pool_k: *mut c_void,
        pool_v: *mut c_void,
        n_blocks: i64,
        slots: *const i32,
        dtype: cuca_dtype,
    ) -> cuca_status;
    pub fn cuca_hip_rope_store_kv_full(
        ctx: *mut cuca_hip_ctx,
        q: *mut c_void,
        q_ld: i64,
        k: *const c_void,
        k_ld: i64,
        v: *const c_void,
        v_ld: i64,
        rows: i64,
        nq: i32,
        nk: i32,
        head_dim: i32,
        n_dims: i32,
        kind: cuca_rope_kind,
        cos: *const f32,
        sin: *const f32,
        table_rows: i64,
        positions: *const i32,
        q_norm_w: *const f32,
        k_norm_w: *const f32,
        v_norm: i32,
        eps: f32,
        pool_k: *mut c_void,
        pool_v: *mut c_void,
        n_blocks: i64,
        slots: *const i32,
        dtype: cuca_dtype,
    ) -> cuca_status;
    pub fn cuca_hip_kv_slots(
        table: *const u32,
        table_len: i64,
        start: i64,
        t: i64,
        n_blocks: i64,
        slots_out: *mut i32,
    ) -> cuca_status;
    pub fn cuca_hip_paged_decode_workspace(
        rows: i64,
        n_head: i32,
        head_dim: i32,
        max_blocks: i64,
        bytes: *mut usize,
    ) -> cuca_status;
    pub fn cuca_hip_paged_decode(
        ctx: *mut cuca_hip_ctx,
        q: *const c_void,
        q_ld: i64,
        pool_k: *const c_void,
        pool_v: *const c_void,
        n_blocks: i64,
        tables: *const u32,
        max_blocks: i64,
        ranges: *const i32,
        rows: i64,
        n_head: i32,
        n_kv: i32,
        head_dim: i32,
        scale: f32,
        workspace: *mut c_void,
        workspace_bytes: usize,
        out: *mut c_void,
        dtype: cuca_dtype,
    ) -> cuca_status;
    pub fn cuca_hip_attend_rows(
        ctx: *mut cuca_hip_ctx,
        q: *const c_void,
        q_ld: i64,
        pool_k: *const c_void,
        pool_v: *const c_void,
        n_blocks: i64,
        table: *const u32,
        max_blocks: i64,
        ranges: *const i32,
        rows: i64,
        n_head: i32,
        n_kv: i32,
        head_dim: i32,
        scale: f32,
        out: *mut c_void,
        out_ld: i64,
        dtype: cuca_dtype,
    ) -> cuca_status;
    pub fn cuca_hip_attend_latent_rows(
        ctx: *mut cuca_hip_ctx,
        q: *const c_void,
        q_ld: i64,
        pool: *const c_void,
        n_blocks: i64,
        table: *const u32,
        max_blocks: i64,
        ranges: *const i32,
        rows: i64,
        n_head: i32,
        head_dim: i32,
        v_width: i32,
        scale: f32,
        out: *mut c_void,
        out_ld: i64,
        dtype: cuca_dtype,
    ) -> cuca_status;
    pub fn cuca_hip_paged_decode_noalloc(
        ctx: *mut cuca_hip_ctx,
        q: *const c_void,
        q_ld: i64,
        pool_k: *const c_void,
        pool_v: *const c_void,
        n_blocks: i64,
        tables: *const u32,
        max_blocks: i64,
        ranges: *const i32,
        rows: i64,
        n_head: i32,
        n_kv: i32,
        head_dim: i32,
        scale: f32,
        out: *mut c_void,
        dtype: cuca_dtype,
    ) -> cuca_status;
    pub fn cuca_hip_qweight_bytes(ggml_type: u32, n: i64, k: i64, bytes: *mut usize) -> cuca_status;
    pub fn cuca_hip_qweight_pack(
        ctx: *mut cuca_hip_ctx,
        gguf: *const c_void,
        ggml_type: u32,
        n: i64,
        k: i64,
        packed: *mut c_void,
    ) -> cuca_status;
    pub fn cuca_hip_qmm(
        ctx: *mut cuca_hip_ctx,
        w: *const c_void,
        ggml_type: u32,
        n: i64,
        k: i64,
        x: *const c_void,
        ldx: i64,
        m: i64,
        rows: i64,
        out: *mut c_void,
        out_ld: i64,
        dtype: cuca_dtype,
    ) -> cuca_status;
    pub fn cuca_hip_qmm_rope_store_kv(
        ctx: *mut cuca_hip_ctx,
        w: *const c_void,
        ggml_type: u32,
        k: i64,
        x: *const c_void,
        ldx: i64,
        m: i64,
        nq: i32,
        nk: i32,
        head_dim: i32,
        n_dims: i32,
        kind: cuca_rope_kind,
        cos: *const f32,
        sin: *const f32,
        table_rows: i64,
        positions: *const i32,
        q_out: *mut c_void,
        q_ld: i64,
        pool_k: *mut c_void,
        pool_v: *mut c_void,
        n_blocks: i64,
        slots: *const i32,
        dtype: cuca_dtype,
    ) -> cuca_status;
    pub fn cuca_hip_qmm_glu(
        ctx: *mut cuca_hip_ctx,
        gate: *const c_void,
        up: *const c_void,
        ggml_type: u32,
        ff: i64,
        k: i64,
        x: *const c_void,
        ldx: i64,
        m: i64,
        act: cuca_act,
        clamp: f32,
        out: *mut c_void,
        out_ld: i64,
        dtype: cuca_dtype,
    ) -> cuca_status;
    pub fn cuca_hip_add_rmsnorm_qmm(
        ctx: *mut cuca_hip_ctx,
        x: *const c_void,
        branch: *const c_void,
        norm_w: *const f32,
        eps: f32,
        residual_scale: f32,
        x_out: *mut c_void,
        h_out: *mut c_void,
        w: *const c_void,
        ggml_type: u32,
        n: i64,
        k: i64,
        m: i64,
        rows: i64,
        out: *mut c_void,
        out_ld: i64,
        dtype: cuca_dtype,
    ) -> cuca_status;
    pub fn cuca_hip_add_rmsnorm_qmm_glu(
        ctx: *mut cuca_hip_ctx,
        x: *const c_void,
        branch: *const c_void,
        norm_w: *const f32,
        eps: f32,
        residual_scale: f32,
        x_out: *mut c_void,
        h_out: *mut c_void,
        gate: *const c_void,
        up: *const c_void,
        ggml_type: u32,
        ff: i64,
        k: i64,
        m: i64,
        act: cuca_act,
        clamp: f32,
        out: *mut c_void,
        out_ld: i64,
        dtype: cuca_dtype,
    ) -> cuca_status;
    pub fn cuca_hip_add_rmsnorm_qmm_rope_store_kv(
        ctx: *mut cuca_hip_ctx,
        x: *const c_void,
        branch: *const c_void,
        norm_w: *const f32,
        eps: f32,
        residual_scale: f32,
        x_out: *mut c_void,
        h_out: *mut c_void,
        w: *const c_void,
        ggml_type: u32,
        k: i64,
        m: i64,
        nq: i32,
        nk: i32,
        head_dim: i32,
        n_dims: i32,
        kind: cuca_rope_kind,
        cos: *const f32,
        sin: *const f32,
        table_rows: i64,
        positions: *const i32,
        q_out: *mut c_void,
        q_ld: i64,
        pool_k: *mut c_void,
        pool_v: *mut c_void,
        n_blocks: i64,
        slots: *const i32,
        dtype: cuca_dtype,
    ) -> cuca_status;
    pub fn cuca_hip_qgemm_workspace(
        ggml_type: u32,
        n: i64,
        k: i64,
        m: i64,
        glu: i32,
        bytes: *mut usize,
    ) -> cuca_status;
    pub fn cuca_hip_qgemm(
        ctx: *mut cuca_hip_ctx,
        w: *const c_void,
        ggml_type: u32,
        n: i64,
        k: i64,
        x: *const c_void,
        ldx: i64,
        m: i64,
        rows: i64,
        workspace: *mut c_void,
        workspace_bytes: usize,
        out: *mut c_void,
        out_ld: i64,
        dtype: cuca_dtype,
    ) -> cuca_status;
    pub fn cuca_hip_qgemm_glu(
        ctx: *mut cuca_hip_ctx,
        gate: *const c_void,
        up: *const c_void,
        ggml_type: u32,
        ff: i64,
        k: i64,
        x: *const c_void,
        ldx: i64,
        m: i64,
        act: cuca_act,
        clamp: f32,
        workspace: *mut c_void,
        workspace_bytes: usize,
        out: *mut c_void,
        out_ld: i64,
        dtype: cuca_dtype,
    ) -> cuca_status;
    pub fn cuca_hip_qweight_dequant(
        ctx: *mut cuca_hip_ctx,
        packed: *const c_void,
        ggml_type: u32,
        n: i64,
        k: i64,
        w16: *mut c_void,
    ) -> cuca_status;
    pub fn cuca_hip_gemm_w16_workspace(
        n: i64,
        k: i64,
        m: i64,
        glu: i32,
        dtype: cuca_dtype,
        bytes: *mut usize,
    ) -> cuca_status;
    pub fn cuca_hip_gemm_w16(
        ctx: *mut cuca_hip_ctx,
        w16: *const c_void,
        n: i64,
        k: i64,
        x: *const c_void,
        ldx: i64,
        m: i64,
        rows: i64,
        workspace: *mut c_void,
        workspace_bytes: usize,
        out: *mut c_void,
        out_ld: i64,
        dtype: cuca_dtype,
    ) -> cuca_status;
    pub fn cuca_hip_gemm_w16_glu(
        ctx: *mut cuca_hip_ctx,
        w16: *const c_void,
        ff: i64,
        k: i64,
        x: *const c_void,
        ldx: i64,
        m: i64,
        act: cuca_act,
        clamp: f32,
        workspace: *mut c_void,
        workspace_bytes: usize,
        out: *mut c_void,
        out_ld: i64,
        dtype: cuca_dtype,
    ) -> cuca_status;
    pub fn cuca_hip_lm_head(
        ctx: *mut cuca_hip_ctx,
        w: *const c_void,
        ggml_type: u32,
        vocab: i64,
        n_embd: i64,
        x: *const c_void,
        ldx: i64,
        m: i64,
        rows: i64,
        logit_scale: f32,
        logit_mult: f32,
        softcap: f32,
        logits: *mut c_void,
        logits_ld: i64,
        dtype: cuca_dtype,
    ) -> cuca_status;
    pub fn cuca_hip_lm_head_indexed_workspace(
        ggml_type: u32,
        n_embd: i64,
        n_ids: i64,
        bytes: *mut usize,
    ) -> cuca_status;
    pub fn cuca_hip_lm_head_indexed(
        ctx: *mut cuca_hip_ctx,
        w: *const c_void,
        ggml_type: u32,
        vocab: i64,
        n_embd: i64,
        x: *const c_void,
        ldx: i64,
        m: i64,
        ids: *const u32,
        n_ids: i64,
        logit_scale: f32,
        logit_mult: f32,
        softcap: f32,
        workspace: *mut c_void,
        workspace_bytes: usize,
        logits: *mut c_void,
        logits_ld: i64,
        dtype: cuca_dtype,
    ) -> cuca_status;
    pub fn cuca_hip_sample_candidates(
        logits: *const f32,
        ids: *const u32,
        count: i32,
        top_p: f32,
        fallback: u32,
        rng_state: *mut u64,
        out_id: *mut u32,
    ) -> cuca_status;
    pub fn cuca_hip_argmax(
        ctx: *mut cuca_hip_ctx,
        logits: *const c_void,
        ld: i64,
        rows: i64,
        vocab: i64,
        dtype: cuca_dtype,
        ids: *mut u32,
    ) -> cuca_status;
    pub fn cuca_hip_top_k(
        ctx: *mut cuca_hip_ctx,
        logits: *const c_void,
        ld: i64,
        rows: i64,
        vocab: i64,
        dtype: cuca_dtype,
        k: i32,
        temperature: f32,
        out_logits: *mut f32,
        out_ids: *mut u32,
        out_count: *mut i32,
    ) -> cuca_status;
    pub fn cuca_hip_q8_acts(
        ctx: *mut cuca_hip_ctx,
        x: *const c_void,
        ldx: i64,
        m: i64,
        k: i64,
        dtype: cuca_dtype,
        quants: *mut i8,
        scales: *mut f32,
    ) -> cuca_status;
    pub fn cuca_hip_qmv(
        ctx: *mut cuca_hip_ctx,
        w: *const c_void,
        ggml_type: u32,
        n: i64,
        k: i64,
        quants: *const i8,
        scales: *const f32,
        m: i64,
        rows: i64,
        out: *mut c_void,
        out_ld: i64,
        dtype: cuca_dtype,
    ) -> cuca_status;
    pub fn cuca_hip_qmv_glu(
        ctx: *mut cuca_hip_ctx,
        gate: *const c_void,
        up: *const c_void,
        ggml_type: u32,
        ff: i64,
        k: i64,
        quants: *const i8,
        scales: *const f32,
        m: i64,
        act: cuca_act,
        clamp: f32,
        out: *mut c_void,
        out_ld: i64,
        dtype: cuca_dtype,
    ) -> cuca_status;
    pub fn cuca_hip_moe_up(
        ctx: *mut cuca_hip_ctx,
        gate: *const c_void,
        up: *const c_void,
        expert_stride: i64,
        ggml_type: u32,
        ff: i64,
        n_embd: i64,
        n_experts: i32,
        x: *const c_void,
        ldx: i64,
        n_tokens: i64,
        offsets: *const i32,
        pair_token: *const i32,
        max_pairs: i64,
        act: cuca_act,
        clamp: f32,
        hidden: *mut c_void,
        hidden_ld: i64,
        dtype: cuca_dtype,
    ) -> cuca_status;
    pub fn cuca_hip_moe_down(
        ctx: *mut cuca_hip_ctx,
        down: *const c_void,
        expert_stride: i64,
        ggml_type: u32,
        n_embd: i64,
        ff: i64,
        n_experts: i32,
        hidden: *const c_void,
        hidden_ld: i64,
        offsets: *const i32,
        pair_weight: *const f32,
        max_pairs: i64,
        scratch: *mut f32,
        scratch_ld: i64,
        dtype: cuca_dtype,
    ) -> cuca_status;
    pub fn cuca_hip_moe_qgemm_workspace(
        ggml_type: u32,
        k: i64,
        n_experts: i32,
        max_pairs: i64,
        bytes: *mut usize,
    ) -> cuca_status;
    pub fn cuca_hip_moe_up_qgemm(
        ctx: *mut cuca_hip_ctx,
        gate: *const c_void,
        up: *const c_void,
        expert_stride: i64,
        ggml_type: u32,
        ff: i64,
        n_embd: i64,
        n_experts: i32,
        x: *const c_void,
        ldx: i64,
        n_tokens: i64,
        offsets: *const i32,
        pair_token: *const i32,
        max_pairs: i64,
        act: cuca_act,
        clamp: f32,
        workspace: *mut c_void,
        workspace_bytes: usize,
        hidden: *mut c_void,
        hidden_ld: i64,
        dtype: cuca_dtype,
    ) -> cuca_status;
    pub fn cuca_hip_moe_down_qgemm(
        ctx: *mut cuca_hip_ctx,
        down: *const c_void,
        expert_stride: i64,
        ggml_type: u32,
        n_embd: i64,
        ff: i64,
        n_experts: i32,
        hidden: *const c_void,
        hidden_ld: i64,
        offsets: *const i32,
        pair_weight: *const f32,
        max_pairs: i64,
        workspace: *mut c_void,
        workspace_bytes: usize,
        scratch: *mut f32,
        scratch_ld: i64,
        dtype: cuca_dtype,
    ) -> cuca_status;
    pub fn cuca_hip_moe_sum(
        ctx: *mut cuca_hip_ctx,
        scratch: *const f32,
        scratch_ld: i64,
        max_pairs: i64,
        token_pairs: *const i32,
        n_used: i32,
        n_tokens: i64,
        n_embd: i64,
        out: *mut c_void,
        out_ld: i64,
        dtype: cuca_dtype,
    ) -> cuca_status;
    pub fn cuca_hip_rope_tables(
        spec: *const cuca_rope_spec,
        factors: *const f32,
        positions: i64,
        cos_out: *mut f32,
        sin_out: *mut f32,
    ) -> cuca_status;
    pub fn cuca_hip_graph_begin(ctx: *mut cuca_hip_ctx) -> cuca_status;
    pub fn cuca_hip_graph_end(ctx: *mut cuca_hip_ctx, out: *mut *mut cuca_hip_graph) -> cuca_status;
    pub fn cuca_hip_graph_launch(ctx: *mut cuca_hip_ctx, graph: *mut cuca_hip_graph) -> cuca_status;
    pub fn cuca_hip_graph_destroy(graph: *mut cuca_hip_graph);
    pub fn cuca_hip_timer_start(ctx: *mut cuca_hip_ctx) -> cuca_status;
    pub fn cuca_hip_timer_stop(ctx: *mut cuca_hip_ctx, ms: *mut f32) -> cuca_status;
    pub fn cuca_hip_profile_start(ctx: *mut cuca_hip_ctx, max_launches: i32) -> cuca_status;
    pub fn cuca_hip_profile_stop(
        ctx: *mut cuca_hip_ctx,
        out: *mut cuca_hip_kernel_time,
        max: i32,
        count: *mut i32,
    ) -> cuca_status;
}
