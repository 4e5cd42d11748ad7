//! Safe wrapper over the raw bindings, for the calls the engine's layer loop
//! makes (the op sites of `model/gpu.rs`).  The raw calls cannot see the
//! size of a device buffer, so every method here checks each buffer's
//! length against the shape it is given before it calls into the library;
//! buffers are freed on drop, and every non-OK status becomes a [`HipError`]
//! carrying the library's message.  The engine maps that to its own error
//! exactly as the reference maps candle's (model/mod.rs:222-228):
//!
//! ```ignore
//! ctx.add_rmsnorm(...).map_err(|e| CucaError::Provider(ProviderKind::Local, e.to_string()))?;
//! ```
//!
//! A [`Context`] is not `Send` or `Sync`: one per engine thread, as the
//! reference runs every model call on its single engine thread
//! (local/mod.rs:2478).  Ops are asynchronous on the context's stream;
//! [`Context::sync`] or a download waits for them.

use std::ffi::CStr;
use std::fmt;
use std::marker::PhantomData;
use std::os::raw::c_void;
use std::ptr;
use std::rc::Rc;

use crate::*;

/// A failed call: the `cuca_status` and the library's message.
#[derive(Clone, Debug, PartialEq, Eq)]
pub struct HipError {
    pub status: cuca_status,
    pub message: String,
}

impl fmt::Display for HipError {
    fn fmt(&self, f: &mut fmt::Formatter<'_>) -> fmt::Result {
        write!(f, "{} (cuca_hip status {})", self.message, self.status)
    }
}

impl std::error::Error for HipError {}

pub type Result<T> = std::result::Result<T, HipError>;

fn arg_error(message: String) -> HipError {
    HipError { status: CUCA_INVALID_ARG, message }
}

fn message(ctx: *const cuca_hip_ctx) -> String {
    // SAFETY: cuca_hip_last_error never returns NULL; the string lives until
    // the next call on the context (or thread), and is copied here.
    unsafe { CStr::from_ptr(cuca_hip_last_error(ctx)).to_string_lossy().into_owned() }
}

/// The activation element types: f32, and f16 carried as its bits (the
/// engine's `half::f16` is a transparent u16).
pub trait Elem: Copy + 'static {
    const DTYPE: cuca_dtype;
}

impl Elem for f32 {
    const DTYPE: cuca_dtype = CUCA_F32;
}

#[repr(transparent)]
#[derive(Clone, Copy, Debug, Default, PartialEq, Eq)]
pub struct F16Bits(pub u16);

impl Elem for F16Bits {
    const DTYPE: cuca_dtype = CUCA_F16;
}

/// The context handle, destroyed when the last of the context, its buffers
/// and its graphs is dropped (they hold it), so a buffer is never freed on
/// a destroyed context.
struct CtxInner {
    raw: *mut cuca_hip_ctx,
}

impl Drop for CtxInner {
    fn drop(&mut self) {
        // SAFETY: raw came from cuca_hip_ctx_create and nothing uses it after.
        unsafe { cuca_hip_ctx_destroy(self.raw) }
    }
}

/// A device allocation of `len` values of `T`, freed on drop.
pub struct DeviceBuffer<T: Copy> {
    ptr: *mut c_void,
    len: usize,
    ctx: Rc<CtxInner>,
    _t: PhantomData<T>,
}

impl<T: Copy> DeviceBuffer<T> {
    pub fn len(&self) -> usize {
        self.len
    }
    pub fn is_empty(&self) -> bool {
        self.len == 0
    }
    pub fn as_ptr(&self) -> *const c_void {
        self.ptr
    }
    pub fn as_mut_ptr(&mut self) -> *mut c_void {
        self.ptr
    }
    fn need(&self, what: &str, n: usize) -> Result<()> {
        if self.len < n {
            return Err(arg_error(format!("{what}: buffer of {} values, {n} needed", self.len)));
        }
        Ok(())
    }
}

impl<T: Copy> Drop for DeviceBuffer<T> {
    fn drop(&mut self) {
        if !self.ptr.is_null() {
            // SAFETY: ptr came from cuca_hip_malloc on this context, which
            // the buffer keeps alive.
            unsafe {
                cuca_hip_free(self.ctx.raw, self.ptr);
            }
        }
    }
}

/// One device, its stream and the loaded kernels.
pub struct Context {
    inner: Rc<CtxInner>,
    raw: *mut cuca_hip_ctx,
}

/// An executable graph of captured launches (a decode step's per-layer ops).
pub struct Graph {
    raw: *mut cuca_hip_graph,
    ctx: Rc<CtxInner>,
}

impl Graph {
    /// Replay the captured launches, with the pointers and scalars they were
    /// captured with (refresh the buffers' contents first).
    pub fn launch(&self) -> Result<()> {
        // SAFETY: both handles are live; the graph is destroyed only on drop.
        let st = unsafe { cuca_hip_graph_launch(self.ctx.raw, self.raw) };
        if st != CUCA_OK {
            return Err(HipError { status: st, message: message(self.ctx.raw) });
        }
        Ok(())
    }
}

impl Drop for Graph {
    fn drop(&mut self) {
        // SAFETY: raw came from cuca_hip_graph_end.
        unsafe { cuca_hip_graph_destroy(self.raw) }
    }
}

/// The Q and K (and, for the store, V) heads of one attention call, with
/// the rotation and the optional QK-norm.
pub struct RopeCall<'a> {
    pub rows: i64,
    pub nq: i32,
    pub nk: i32,
    pub head_dim: i32,
    pub n_dims: i32,
    pub kind: cuca_rope_kind,
    /// f32 [table_rows, n_dims / 2] each (cuca_hip_rope_tables, uploaded once)
    pub cos: &'a DeviceBuffer<f32>,
    pub sin: &'a DeviceBuffer<f32>,
    /// int32 [rows]
    pub positions: &'a DeviceBuffer<i32>,
    /// per-head weights [head_dim], or with `qk_norm_full` [nq * head_dim] /
    /// [nk * head_dim] over the whole projection (OLMo 2, OLMoE)
    pub q_norm: Option<&'a DeviceBuffer<f32>>,
    pub k_norm: Option<&'a DeviceBuffer<f32>>,
    pub qk_norm_full: bool,
    pub eps: f32,
}

impl Context {
    /// Open `device` (it must be a gfx950).
    pub fn new(device: i32) -> Result<Self> {
        let mut raw = ptr::null_mut();
        // SAFETY: out-pointer to a local.
        let st = unsafe { cuca_hip_ctx_create(device, &mut raw) };
        if st != CUCA_OK {
            return Err(HipError { status: st, message: message(ptr::null()) });
        }
        Ok(Context { inner: Rc::new(CtxInner { raw }), raw })
    }

    fn check(&self, st: cuca_status) -> Result<()> {
        if st == CUCA_OK {
            Ok(())
        } else {
            Err(HipError { status: st, message: message(self.raw) })
        }
    }

    pub fn raw(&self) -> *mut cuca_hip_ctx {
        self.raw
    }

    pub fn alloc<T: Copy>(&self, len: usize) -> Result<DeviceBuffer<T>> {
        let mut p = ptr::null_mut();
        let bytes = len
            .checked_mul(std::mem::size_of::<T>())
            .ok_or_else(|| arg_error("allocation size overflows".into()))?;
        // SAFETY: out-pointer to a local.
        self.check(unsafe { cuca_hip_malloc(self.raw, bytes, &mut p) })?;
        Ok(DeviceBuffer { ptr: p, len, ctx: Rc::clone(&self.inner), _t: PhantomData })
    }

    /// A device copy of `host` (waits for the copy).
    pub fn upload<T: Copy>(&self, host: &[T]) -> Result<DeviceBuffer<T>> {
        let buf = self.alloc::<T>(host.len())?;
        let bytes = std::mem::size_of_val(host);
        // SAFETY: the buffer holds host.len() values; sync before host goes away.
        self.check(unsafe { cuca_hip_memcpy_h2d_async(self.raw, buf.ptr, host.as_ptr().cast(), bytes) })?;
        self.sync()?;
        Ok(buf)
    }

    /// Copy `buf` into `host` (waits for the copy and the work before it).
    pub fn download<T: Copy>(&self, buf: &DeviceBuffer<T>, host: &mut [T]) -> Result<()> {
        buf.need("download", host.len())?;
        let bytes = std::mem::size_of_val(host);
        // SAFETY: both sides hold host.len() values; sync before returning.
        self.check(unsafe { cuca_hip_memcpy_d2h_async(self.raw, host.as_mut_ptr().cast(), buf.ptr, bytes) })?;
        self.sync()
    }

    pub fn sync(&self) -> Result<()> {
        // SAFETY: live context.
        self.check(unsafe { cuca_hip_stream_sync(self.raw) })
    }

    /// Wait, then report what the kernels found in their inputs: a token id
    /// outside the table ("token id {id} outside the embedding table of
    /// {rows} rows", quant.rs:395-400), a position outside the RoPE table, a
    /// K/V slot outside its pool, an attention range without blocks.
    pub fn check_device(&self) -> Result<()> {
        // SAFETY: live context.
        self.check(unsafe { cuca_hip_check_device(self.raw) })
    }

    /// TokenEmbedding::rows (quant.rs:391-411), then, with `norm_eps`,
    /// norm_embeddings' rms_norm_rows (params.rs:374-379): out [n, hidden].
    #[allow(clippy::too_many_arguments)]
    pub fn embed<T: Elem>(
        &self,
        table: &DeviceBuffer<u8>,
        ggml_type: u32,
        vocab: i64,
        hidden: i64,
        ids: &DeviceBuffer<u32>,
        scale: f32,
        norm_eps: Option<f32>,
        out: &mut DeviceBuffer<T>,
    ) -> Result<()> {
        let block = match ggml_type {
            CUCA_GGML_Q4_0 => 18,
            CUCA_GGML_Q8_0 => 34,
            _ => return Err(HipError { status: CUCA_UNSUPPORTED, message: format!("ggml type {ggml_type}") }),
        };
        if hidden <= 0 || hidden % 32 != 0 || vocab <= 0 {
            return Err(arg_error(format!("token embedding: {vocab} rows of {hidden}")));
        }
        let n = ids.len();
        table.need("embedding table", (vocab * hidden / 32 * block) as usize)?;
        out.need("embedding output", n * hidden as usize)?;
        // SAFETY: every buffer holds what the shape names.
        self.check(unsafe {
            match norm_eps {
                None => cuca_hip_embed_gguf(
                    self.raw, table.ptr, ggml_type, vocab, hidden, ids.as_ptr().cast(), n as i64, scale, out.ptr,
                    T::DTYPE,
                ),
                Some(eps) => cuca_hip_embed_gguf_norm(
                    self.raw, table.ptr, ggml_type, vocab, hidden, ids.as_ptr().cast(), n as i64, scale, eps,
                    out.ptr, T::DTYPE,
                ),
            }
        })
    }

    /// The fused residual add + RMSNorm of Transformer::block
    /// (cpu.rs:2650-2711): x' = x + rs * [rms(branch, w_post)], h = rms(x',
    /// w).  `x_out` None writes no x' (and may not alias x here: pass the
    /// same buffer through the raw call for the in-place form).
    #[allow(clippy::too_many_arguments)]
    pub fn add_rmsnorm<T: Elem>(
        &self,
        x: &DeviceBuffer<T>,
        branch: Option<&DeviceBuffer<T>>,
        w: Option<&DeviceBuffer<f32>>,
        w_post: Option<&DeviceBuffer<f32>>,
        eps: f32,
        post_eps: f32,
        residual_scale: f32,
        rows: i64,
        hidden: i64,
        x_out: Option<&mut DeviceBuffer<T>>,
        h_out: &mut DeviceBuffer<T>,
    ) -> Result<()> {
        let n = (rows * hidden) as usize;
        x.need("x", n)?;
        h_out.need("h", n)?;
        if let Some(b) = branch {
            b.need("branch", n)?;
        }
        for (what, v) in [("w", w), ("w_post", w_post)] {
            if let Some(v) = v {
                v.need(what, hidden as usize)?;
            }
        }
        let xo = match x_out {
            Some(b) => {
                b.need("x_out", n)?;
                b.ptr
            }
            None => ptr::null_mut(),
        };
        // SAFETY: every buffer holds rows x hidden (weights: hidden) values.
        self.check(unsafe {
            cuca_hip_add_rmsnorm(
                self.raw,
                x.ptr,
                branch.map_or(ptr::null(), |b| b.as_ptr()),
                w.map_or(ptr::null(), |b| b.as_ptr().cast()),
                w_post.map_or(ptr::null(), |b| b.as_ptr().cast()),
                eps,
                post_eps,
                residual_scale,
                rows,
                hidden,
                xo,
                h_out.ptr,
                T::DTYPE,
            )
        })
    }

    /// Glu::apply over the fused [gate | up] projection y [rows, 2 ff]
    /// (FfnWeights::forward, cpu.rs:3554-3566): out [rows, ff].
    pub fn glu_fused<T: Elem>(
        &self,
        y: &DeviceBuffer<T>,
        rows: i64,
        ff: i64,
        act: cuca_act,
        clamp: f32,
        out: &mut DeviceBuffer<T>,
    ) -> Result<()> {
        y.need("gate|up", (rows * 2 * ff) as usize)?;
        out.need("out", (rows * ff) as usize)?;
        let up = (y.ptr as usize + ff as usize * std::mem::size_of::<T>()) as *const c_void;
        // SAFETY: y holds rows x 2 ff values, out rows x ff.
        self.check(unsafe {
            cuca_hip_glu(self.raw, y.ptr, 2 * ff, up, 2 * ff, rows, ff, act, clamp, out.ptr, ff, T::DTYPE)
        })
    }

    /// The same over MoE rows grouped by expert (device int32 offsets
    /// [n_experts + 1]); gate / up / out hold max_rows x ff values.
    #[allow(clippy::too_many_arguments)]
    pub fn glu_ragged<T: Elem>(
        &self,
        gate: &DeviceBuffer<T>,
        up: &DeviceBuffer<T>,
        offsets: &DeviceBuffer<i32>,
        max_rows: i64,
        ff: i64,
        act: cuca_act,
        clamp: f32,
        out: &mut DeviceBuffer<T>,
    ) -> Result<()> {
        let n = (max_rows * ff) as usize;
        gate.need("gate", n)?;
        up.need("up", n)?;
        out.need("out", n)?;
        let n_experts = offsets.len() as i32 - 1;
        // SAFETY: as checked above; the row count is read on the device and
        // capped at max_rows.
        self.check(unsafe {
            cuca_hip_glu_ragged(
                self.raw, gate.ptr, ff, up.ptr, ff, offsets.as_ptr().cast(), n_experts, max_rows, ff, act, clamp,
                out.ptr, ff, T::DTYPE,
            )
        })
    }

    fn rope_checks<T: Elem>(&self, c: &RopeCall<'_>, q: &DeviceBuffer<T>, k: &DeviceBuffer<T>) -> Result<()> {
        let d = c.head_dim as i64;
        q.need("q", (c.rows * c.nq as i64 * d) as usize)?;
        k.need("k", (c.rows * c.nk as i64 * d) as usize)?;
        c.positions.need("positions", c.rows as usize)?;
        let half = (c.n_dims / 2) as usize;
        if half == 0 || c.cos.len() % half != 0 || c.sin.len() != c.cos.len() {
            return Err(arg_error("rope tables are not [rows, n_dims / 2]".into()));
        }
        let qn = if c.qk_norm_full { (c.nq as i64 * d) as usize } else { d as usize };
        let kn = if c.qk_norm_full { (c.nk as i64 * d) as usize } else { d as usize };
        if let Some(w) = c.q_norm {
            w.need("q_norm", qn)?;
        }
        if let Some(w) = c.k_norm {
            w.need("k_norm", kn)?;
        }
        Ok(())
    }

    /// apply_rope on Q [rows, nq, d] and K [rows, nk, d] in place, with the
    /// QK-norm in front (cpu.rs:2837-2871, 3040-3055; gpu.rs:5922-5964).
    pub fn rope<T: Elem>(&self, c: &RopeCall<'_>, q: &mut DeviceBuffer<T>, k: &mut DeviceBuffer<T>) -> Result<()> {
        self.rope_checks(c, q, k)?;
        let d = c.head_dim as i64;
        let table_rows = (c.cos.len() / (c.n_dims / 2) as usize) as i64;
        let f = if c.qk_norm_full { cuca_hip_rope_full } else { cuca_hip_rope };
        // SAFETY: rope_checks checked every buffer against the call's shape.
        self.check(unsafe {
            f(
                self.raw,
                q.ptr,
                c.nq as i64 * d,
                k.ptr,
                c.nk as i64 * d,
                c.rows,
                c.nq,
                c.nk,
                c.head_dim,
                c.n_dims,
                c.kind,
                c.cos.as_ptr().cast(),
                c.sin.as_ptr().cast(),
                table_rows,
                c.positions.as_ptr().cast(),
                c.q_norm.map_or(ptr::null(), |b| b.as_ptr().cast()),
                c.k_norm.map_or(ptr::null(), |b| b.as_ptr().cast()),
                c.eps,
                T::DTYPE,
            )
        })
    }

    /// store_kv (cpu.rs:3028-3097): Q rotated in place, K rotated and V
    /// (weightless norm when `v_norm`) written into the paged pools
    /// [n_blocks, nk, 16, d] at `slots` (cuca_hip_kv_slots).
    #[allow(clippy::too_many_arguments)]
    pub fn rope_store_kv<T: Elem>(
        &self,
        c: &RopeCall<'_>,
        q: &mut DeviceBuffer<T>,
        k: &DeviceBuffer<T>,
        v: &DeviceBuffer<T>,
        v_norm: bool,
        pool_k: &mut DeviceBuffer<T>,
        pool_v: &mut DeviceBuffer<T>,
        n_blocks: i64,
        slots: &DeviceBuffer<i32>,
    ) -> Result<()> {
        self.rope_checks(c, q, k)?;
        let d = c.head_dim as i64;
        v.need("v", (c.rows * c.nk as i64 * d) as usize)?;
        let pool = (n_blocks * c.nk as i64 * CUCA_KV_BLOCK * d) as usize;
        pool_k.need("pool_k", pool)?;
        pool_v.need("pool_v", pool)?;
        slots.need("slots", c.rows as usize)?;
        let table_rows = (c.cos.len() / (c.n_dims / 2) as usize) as i64;
        let f = if c.qk_norm_full { cuca_hip_rope_store_kv_full } else { cuca_hip_rope_store_kv };
        // SAFETY: every buffer was checked against the call's shape; slots
        // outside the pool are skipped and reported by the device.
        self.check(unsafe {
            f(
                self.raw,
                q.ptr,
                c.nq as i64 * d,
                k.ptr,
                c.nk as i64 * d,
                v.ptr,
                c.nk as i64 * d,
                c.rows,
                c.nq,
                c.nk,
                c.head_dim,
                c.n_dims,
                c.kind,
                c.cos.as_ptr().cast(),
                c.sin.as_ptr().cast(),
                table_rows,
                c.positions.as_ptr().cast(),
                c.q_norm.map_or(ptr::null(), |b| b.as_ptr().cast()),
                c.k_norm.map_or(ptr::null(), |b| b.as_ptr().cast()),
                v_norm as i32,
                c.eps,
                pool_k.ptr,
                pool_v.ptr,
                n_blocks,
                slots.as_ptr().cast(),
                T::DTYPE,
            )
        })
    }

    /// Paged decode attention over the pools (paged_kernel.rs:92-282): q
    /// [rows, n_head, d], tables u32 [rows, max_blocks], ranges i32 [rows, 2],
    /// out [rows, n_head, d]; the partials use the library's per-GPU scratch
    /// (cuca_hip_paged_decode_noalloc), so the call allocates nothing.
    #[allow(clippy::too_many_arguments)]
    pub fn paged_decode<T: Elem>(
        &self,
        q: &DeviceBuffer<T>,
        pool_k: &DeviceBuffer<T>,
        pool_v: &DeviceBuffer<T>,
        n_blocks: i64,
        tables: &DeviceBuffer<u32>,
        ranges: &DeviceBuffer<i32>,
        n_head: i32,
        n_kv: i32,
        head_dim: i32,
        scale: f32,
        out: &mut DeviceBuffer<T>,
    ) -> Result<()> {
        let rows = ranges.len() as i64 / 2;
        if rows == 0 || tables.len() as i64 % rows != 0 {
            return Err(arg_error("attention: tables are not [rows, max_blocks]".into()));
        }
        let max_blocks = tables.len() as i64 / rows;
        let row = (n_head as i64 * head_dim as i64) as usize;
        q.need("q", rows as usize * row)?;
        out.need("out", rows as usize * row)?;
        let pool = (n_blocks * n_kv as i64 * CUCA_KV_BLOCK * head_dim as i64) as usize;
        pool_k.need("pool_k", pool)?;
        pool_v.need("pool_v", pool)?;
        // SAFETY: every buffer was checked against the shape; block ids and
        // ranges are checked on the device.
        self.check(unsafe {
            cuca_hip_paged_decode_noalloc(
                self.raw,
                q.ptr,
                row as i64,
                pool_k.ptr,
                pool_v.ptr,
                n_blocks,
                tables.as_ptr().cast(),
                max_blocks,
                ranges.as_ptr().cast(),
                rows,
                n_head,
                n_kv,
                head_dim,
                scale,
                out.ptr,
                T::DTYPE,
            )
        })
    }

    /// Capture every op `f` issues into a graph (a decode step's layers).
    pub fn capture(&self, f: impl FnOnce(&Self) -> Result<()>) -> Result<Graph> {
        // SAFETY: live context.
        self.check(unsafe { cuca_hip_graph_begin(self.raw) })?;
        let body = f(self);
        let mut g = ptr::null_mut();
        // SAFETY: out-pointer to a local; ends the capture begun above.
        let end = self.check(unsafe { cuca_hip_graph_end(self.raw, &mut g) });
        body?;
        end?;
        Ok(Graph { raw: g, ctx: Rc::clone(&self.inner) })
    }
}

/// RopeSpec::tables (rope.rs:118-151) on the host: (cos, sin), each
/// [positions, n_dims / 2], the reference's f32 bits.
pub fn rope_tables(spec: &cuca_rope_spec, factors: Option<&[f32]>, positions: i64) -> Result<(Vec<f32>, Vec<f32>)> {
    let half = (spec.n_dims.max(0) / 2) as usize;
    if let Some(f) = factors {
        if f.len() != half {
            return Err(arg_error(format!("{} rope factors for {half} pairs", f.len())));
        }
    }
    let n = positions.max(0) as usize * half;
    let (mut cos, mut sin) = (vec![0f32; n], vec![0f32; n]);
    // SAFETY: both outputs hold positions x n_dims / 2 values.
    let st = unsafe {
        cuca_hip_rope_tables(spec, factors.map_or(ptr::null(), |f| f.as_ptr()), positions, cos.as_mut_ptr(), sin.as_mut_ptr())
    };
    if st != CUCA_OK {
        return Err(HipError { status: st, message: message(ptr::null()) });
    }
    Ok((cos, sin))
}

/// The pool rows of cache indices start..start+t of a sequence with block
/// table `table` (paged.rs:9-16): block * 16 + position % 16.
pub fn kv_slots(table: &[u32], start: i64, t: i64, n_blocks: i64) -> Result<Vec<i32>> {
    let mut out = vec![0i32; t.max(0) as usize];
    // SAFETY: out holds t values; the table is read within its length.
    let st = unsafe { cuca_hip_kv_slots(table.as_ptr(), table.len() as i64, start, t, n_blocks, out.as_mut_ptr()) };
    if st != CUCA_OK {
        return Err(HipError { status: st, message: message(ptr::null()) });
    }
    Ok(out)
}
