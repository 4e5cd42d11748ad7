"""The reference's per-layer op surface, over the C ABI.

Names, argument meaning and errors follow provider-local's op sites (paths
under src/provider/local/model/ of nassor/cuca 0.10.0), so that a caller
(and the parity tests) read like the reference:

    TokenEmbedding(dtype, data, rows, row_len).rows(tokens, scale)  quant.rs:352-411
    rms(x, weight, eps)                                              cpu.rs:3652
    add_rms(x, branch, weight, eps, ...)  (x + branch, rms of it)    cpu.rs:2650-2711
    Glu(act, clamp).apply(gate, up)                                  cpu.rs:342-371
    apply_rope(x, cos, sin, kind, n_dims, positions)                 cpu.rs:3672-3688
    RopeSpec.plain(kind, n_dims, base).tables(factors, positions)    rope.rs:62-151
    QmmWeight.from_raw(dtype, data, n, k).forward_rows(x, m, rows)    qmm.rs:1744-1838
    QmmWeight.glu(gate, up, x, glu)  (act(gate x) * up x, fused)     cpu.rs:342-371, 3554-3566
    ExpertBank.from_raw(...).expert_sum(x, per_expert, glu)           cpu.rs:373-419, 3599-3642

Tensors are DeviceArrays (device memory through the C ABI); every op runs on
the gfx950 kernels of libcuca_hip.so.  There is no host fallback.
"""

import numpy as np

from . import hip
from .hip import CucaError, DeviceArray

_GGML_NAME = {hip.GGML_Q4_0: "Q4_0", hip.GGML_Q8_0: "Q8_0"}
_BLOCK_BYTES = {hip.GGML_Q4_0: 18, hip.GGML_Q8_0: 34}


def byte_len(ggml_type, n):
    """GgufType::byte_len for Q4_0 / Q8_0 (gguf/dtype.rs:195-250): bytes of n
    values, or None when n is not a whole number of 32-value blocks."""
    if ggml_type not in _BLOCK_BYTES or n % 32 != 0:
        return None
    return n // 32 * _BLOCK_BYTES[ggml_type]


class TokenEmbedding:
    """The token-embedding table held in the file's type (quant.rs:352-411),
    resident in HBM; a lookup dequantizes only the rows it reads, on the GPU."""

    def __init__(self, ctx, dtype, data, rows, row_len):
        if dtype not in _BLOCK_BYTES:
            raise CucaError(hip.UNSUPPORTED, f"ggml type {dtype}: only Q4_0 and Q8_0 are supported")
        name = _GGML_NAME[dtype]
        row_bytes = byte_len(dtype, row_len)
        if row_bytes is None:  # quant.rs:362-367
            raise CucaError(hip.INVALID_ARG, f"token embedding: row length {row_len} is not a "
                            f"whole number of {name} blocks")
        data = np.ascontiguousarray(np.frombuffer(data, np.uint8) if isinstance(data, bytes)
                                    else data, dtype=np.uint8).reshape(-1)
        if rows * row_bytes != data.size:  # quant.rs:368-374
            raise CucaError(hip.INVALID_ARG, f"token embedding: {data.size} bytes do not hold "
                            f"{rows} rows of {row_len} {name} values")
        self.ctx = ctx
        self.dtype = dtype
        self.rows_n = rows
        self.row_len = row_len
        self.row_bytes = row_bytes
        self.table = ctx.array(data)

    def rows(self, tokens, scale, out_dtype=np.float32, norm_eps=None):
        """Embedding rows of `tokens`, concatenated and multiplied by `scale`
        (quant.rs:391-411): a DeviceArray [len(tokens), row_len].  With
        norm_eps (the archs with embd_norm), each row then gets
        norm_embeddings' scale-less norm (params.rs:374-379) in the same
        pass."""
        ids = np.asarray(tokens, dtype=np.int64).reshape(-1)
        for i in ids:  # quant.rs:395-400, before anything runs
            if i < 0 or i >= self.rows_n:
                raise CucaError(hip.OUT_OF_RANGE, f"token id {int(i)} outside the embedding table "
                                f"of {self.rows_n} rows")
        dev_ids = self.ctx.array(ids.astype(np.uint32))
        out = self.ctx.empty((ids.size, self.row_len), out_dtype)
        self.rows_device(dev_ids, scale, out, norm_eps)
        return out

    def rows_rms(self, tokens, scale, weight, eps, out_dtype=np.float32):
        """The gather fused with the first block's attention norm: returns
        (x, h), x the embedding rows of `tokens` times `scale` (as rows()),
        h = rms(x, weight, eps) (Transformer::block, cpu.rs:2670-2673).
        weight None is the weightless norm."""
        ids = np.asarray(tokens, dtype=np.int64).reshape(-1)
        for i in ids:  # quant.rs:395-400, before anything runs
            if i < 0 or i >= self.rows_n:
                raise CucaError(hip.OUT_OF_RANGE, f"token id {int(i)} outside the embedding table "
                                f"of {self.rows_n} rows")
        dev_ids = self.ctx.array(ids.astype(np.uint32))
        x = self.ctx.empty((ids.size, self.row_len), out_dtype)
        h = self.ctx.empty((ids.size, self.row_len), out_dtype)
        w = _w(self.ctx, weight)
        self.ctx.embed_gguf_rms(self.table.ptr, self.dtype, self.rows_n, self.row_len, dev_ids.ptr,
                                ids.size, scale, None if w is None else w.ptr, eps, x.ptr, h.ptr,
                                hip.dtype_code(out_dtype))
        return x, h

    def rows_device(self, ids, scale, out, norm_eps=None):
        """The gather for ids already on the device (u32 DeviceArray); bad ids
        are reported by ctx.check_device()."""
        if norm_eps is None:
            self.ctx.embed_gguf(self.table.ptr, self.dtype, self.rows_n, self.row_len, ids.ptr,
                                ids.size, scale, out.ptr, hip.dtype_code(out.dtype))
        else:
            self.ctx.embed_gguf_norm(self.table.ptr, self.dtype, self.rows_n, self.row_len, ids.ptr,
                                     ids.size, scale, norm_eps, out.ptr, hip.dtype_code(out.dtype))
        return out


def _w(ctx, w):
    if w is None or isinstance(w, DeviceArray):
        return w
    return ctx.array(np.asarray(w, dtype=np.float32))


def add_rms(x, branch, weight, eps, w_post=None, post_eps=None, residual_scale=1.0,
            write_x=True, x_out=None, h_out=None):
    """The fused residual add + RMSNorm of Transformer::block
    (cpu.rs:2650-2711): returns (x', h) with x' = x + rs * [rms(branch,
    w_post, post_eps)] and h = rms(x', weight, eps).  x_out may be x."""
    ctx = x.ctx
    rows, hidden = x.shape[0], int(np.prod(x.shape[1:]))
    w = _w(ctx, weight)
    wp = _w(ctx, w_post)
    if write_x and x_out is None:
        x_out = ctx.empty(x.shape, x.dtype)
    if h_out is None:
        h_out = ctx.empty(x.shape, x.dtype)
    ctx.add_rmsnorm(x.ptr, None if branch is None else branch.ptr, None if w is None else w.ptr,
                    None if wp is None else wp.ptr, eps, eps if post_eps is None else post_eps,
                    residual_scale, rows, hidden, None if x_out is None else x_out.ptr,
                    h_out.ptr, hip.dtype_code(x.dtype))
    return (x_out if write_x else None), h_out


def rms(x, weight, eps):
    """RMSNorm with a learned weight, no `1 + w` (cpu.rs:3652); weight None
    is the weightless norm (gpu.rs:5895).  The last dim is normalized."""
    hidden = x.shape[-1]
    rows = x.size // hidden
    ctx = x.ctx
    w = _w(ctx, weight)
    out = ctx.empty(x.shape, x.dtype)
    ctx.add_rmsnorm(x.ptr, None, None if w is None else w.ptr, None, eps, eps, 1.0, rows, hidden,
                    None, out.ptr, hip.dtype_code(x.dtype))
    return out


class Glu:
    """The gated activation `act(gate) * up` with the optional clamp
    (cpu.rs:342-371)."""

    def __init__(self, act, clamp=None):
        self.act = act
        self.clamp = clamp if (clamp is not None and clamp > 0.0) else None

    @classmethod
    def clamped(cls, act, limit):
        return cls(act, limit if limit > 0.0 else None)

    def apply(self, gate, up, out=None, rows=None, ff=None, gate_ld=None, up_ld=None):
        ctx = gate.ctx
        ff = gate.shape[-1] if ff is None else ff
        rows = gate.size // gate.shape[-1] if rows is None else rows
        if out is None:
            out = ctx.empty((rows, ff), gate.dtype)
        ctx.glu(gate.ptr, gate_ld or ff, up.ptr, up_ld or ff, rows, ff, self.act,
                self.clamp or 0.0, out.ptr, ff, hip.dtype_code(gate.dtype))
        return out

    def apply_fused(self, y, ff):
        """GateUp::Fused: y [rows, 2*ff] = [gate | up] (cpu.rs:3559-3562)."""
        rows = y.shape[0]
        return self.apply(y, y.view(ff, y.shape), rows=rows, ff=ff, gate_ld=2 * ff, up_ld=2 * ff)

    def apply_ragged(self, gate, up, expert_offsets, n_experts, out=None):
        """Rows grouped by expert (moe.rs:39-94); expert_offsets is a device
        int32 [n_experts + 1] prefix sum read on the device."""
        ctx = gate.ctx
        rows, ff = gate.shape
        if out is None:
            out = ctx.empty((rows, ff), gate.dtype)
        ctx.glu_ragged(gate.ptr, ff, up.ptr, ff, expert_offsets.ptr, n_experts, rows, ff,
                       self.act, self.clamp or 0.0, out.ptr, ff, hip.dtype_code(gate.dtype))
        return out


def apply_rope(x, cos, sin, kind, n_dims, positions, norm_w=None, eps=1e-6):
    """Rotate the first n_dims values of every head of x [rows, heads, d] in
    place (apply_rope, cpu.rs:3672-3688); cos/sin are device [table_rows,
    n_dims/2] tables and positions a device int32 [rows].  norm_w fuses the
    per-head QK-norm in front (cpu.rs:2840-2864)."""
    rows, heads, d = x.shape
    ctx = x.ctx
    nw = _w(ctx, norm_w)
    ctx.rope(x.ptr, heads * d, None, 0, rows, heads, 0, d, n_dims, kind, cos.ptr, sin.ptr,
             cos.shape[0], positions.ptr, None if nw is None else nw.ptr, None, eps,
             hip.dtype_code(x.dtype))
    return x


def rope_qk(q, k, cos, sin, kind, n_dims, positions, q_norm_w=None, k_norm_w=None, eps=1e-6,
            qk_norm_full=False):
    """Q and K of one attention call in one launch, with the optional QK-norm:
    per head (weights [head_dim]), or with qk_norm_full over each row's whole
    Q and K projection (weights [nq * head_dim], [nk * head_dim]; the OLMo 2
    path, cpu.rs:2838-2843, 3042-3045)."""
    rows, nq, d = q.shape
    nk = 0 if k is None else k.shape[1]
    ctx = q.ctx
    qw, kw = _w(ctx, q_norm_w), _w(ctx, k_norm_w)
    call = ctx.rope_full if qk_norm_full else ctx.rope
    call(q.ptr, nq * d, None if k is None else k.ptr, nk * d, rows, nq, nk, d, n_dims, kind,
         cos.ptr, sin.ptr, cos.shape[0], positions.ptr, None if qw is None else qw.ptr,
         None if kw is None else kw.ptr, eps, hip.dtype_code(q.dtype))
    return q, k


class KvPool:
    """One K/V-owning layer's paged cache on the device (KvPool, gpu.rs:1774-1781;
    KvLayer, cpu.rs:689-714): keys and values [n_blocks, n_kv_head, 16,
    head_dim] of the activation dtype, zero-filled.  Position p of a sequence
    lives in block table[p // 16], row p % 16 (paged.rs:9-16)."""

    def __init__(self, ctx, n_blocks, n_kv_head, head_dim, dtype=np.float32):
        self.ctx = ctx
        self.n_blocks, self.n_kv_head, self.head_dim = n_blocks, n_kv_head, head_dim
        shape = (n_blocks, n_kv_head, hip.KV_BLOCK, head_dim)
        self.k = ctx.array(np.zeros(shape, dtype))
        self.v = ctx.array(np.zeros(shape, dtype))

    def slots(self, table, start, t):
        """Pool rows of cache indices start..start+t (host, int32[t])."""
        return hip.kv_slots(table, start, t, self.n_blocks)

    def store_kv(self, q, k, v, cos, sin, kind, n_dims, positions, slots, q_norm_w=None,
                 k_norm_w=None, v_norm=False, eps=1e-6, qk_norm_full=False):
        """Normalise and rotate q [rows, nq, d] in place, and k [rows, nk, d]
        into the pool, with v (normalised without a weight when v_norm) beside
        it (store_kv, cpu.rs:3028-3097), in one launch.  slots: device int32
        [rows] from `slots`.  qk_norm_full: the Q/K norms span each row's whole
        projection (weights [nq * d], [nk * d])."""
        rows, nq, d = q.shape
        nk = k.shape[1]
        if k.shape != (rows, nk, d) or v.shape != (rows, nk, d) or nk != self.n_kv_head \
                or d != self.head_dim:
            raise CucaError(hip.INVALID_ARG, "store_kv: row shape mismatch")
        ctx = q.ctx
        qw, kw = _w(ctx, q_norm_w), _w(ctx, k_norm_w)
        call = ctx.rope_store_kv_full if qk_norm_full else ctx.rope_store_kv
        call(q.ptr, nq * d, k.ptr, nk * d, v.ptr, nk * d, rows, nq, nk, d, n_dims, kind,
             cos.ptr, sin.ptr, cos.shape[0], positions.ptr,
             None if qw is None else qw.ptr, None if kw is None else kw.ptr, v_norm,
             eps, self.k.ptr, self.v.ptr, self.n_blocks, slots.ptr,
             hip.dtype_code(q.dtype))
        return q

    def attend_rows(self, q, table, ranges, n_head, scale):
        """Attention of q [rows, n_head, d], rows of ONE sequence, over this
        pool (attend_paged_rows, cpu/paged_attn.rs:177-213): table device u32
        [max_blocks], ranges device int32 [rows, 2] (lo, hi).  Returns a
        DeviceArray [rows, n_head, d]."""
        rows, nh, d = q.shape
        if nh != n_head or d != self.head_dim:
            raise CucaError(hip.INVALID_ARG, "attention: query shape mismatch")
        out = self.ctx.empty((rows, n_head, d), q.dtype)
        self.ctx.attend_rows(q.ptr, n_head * d, self.k.ptr, self.v.ptr, self.n_blocks, table.ptr,
                             table.shape[0], ranges.ptr, rows, n_head, self.n_kv_head, d, scale, out.ptr,
                             n_head * d, hip.dtype_code(q.dtype))
        return out

    def decode(self, q, tables, ranges, n_head, scale, workspace=None):
        """Paged decode attention of q [rows, n_head, d] (one query row per
        sequence) over this pool (paged_kernel.rs decode, gpu.rs:6002-6011):
        tables device u32 [rows, max_blocks], ranges device int32 [rows, 2]
        (lo, hi).  Returns a DeviceArray [rows, n_head, d].  `workspace`: a
        DeviceArray of at least paged_decode_workspace bytes, or one is made."""
        rows, nh, d = q.shape
        if nh != n_head or d != self.head_dim:
            raise CucaError(hip.INVALID_ARG, "attention: query shape mismatch")
        max_blocks = tables.shape[1]
        need = hip.paged_decode_workspace(rows, n_head, d, max_blocks)
        if workspace is None:
            workspace = self.ctx.empty((max(need, 16),), np.uint8)
        out = self.ctx.empty((rows, n_head, d), q.dtype)
        self.ctx.paged_decode(q.ptr, self.k.ptr, self.v.ptr, self.n_blocks, tables.ptr, max_blocks,
                              ranges.ptr, rows, n_head, self.n_kv_head, d, scale, workspace.ptr,
                              workspace.nbytes, out.ptr, hip.dtype_code(q.dtype))
        return out

    def decode_noalloc(self, q, tables, ranges, n_head, scale, out=None):
        """`decode` through cuca_hip_paged_decode_noalloc: no workspace, the
        call allocates nothing on the device (`out`, a DeviceArray [rows,
        n_head, d], may be passed in; else one is made here, outside the
        call)."""
        rows, nh, d = q.shape
        if nh != n_head or d != self.head_dim:
            raise CucaError(hip.INVALID_ARG, "attention: query shape mismatch")
        if out is None:
            out = self.ctx.empty((rows, n_head, d), q.dtype)
        self.ctx.paged_decode_noalloc(q.ptr, self.k.ptr, self.v.ptr, self.n_blocks, tables.ptr,
                                      tables.shape[1], ranges.ptr, rows, n_head, self.n_kv_head, d,
                                      scale, out.ptr, hip.dtype_code(q.dtype))
        return out

    def read(self, slots):
        """The rows `slots` name, the inverse of the store (KvPool::read,
        gpu.rs:1808-1830): host (k, v) [len(slots), n_kv_head, head_dim]."""
        slots = np.asarray(slots, np.int64)
        b, r = slots // hip.KV_BLOCK, slots % hip.KV_BLOCK
        kp, vp = self.k.numpy(), self.v.numpy()
        return kp[b, :, r, :], vp[b, :, r, :]


class RopeSpec:
    """One rotary embedding (rope.rs:62-79)."""

    def __init__(self, kind, n_dims, base, freq_scale=1.0, yarn=None, attn_factor=1.0):
        self.kind = kind
        self.n_dims = n_dims
        self.base = base
        self.freq_scale = freq_scale
        self.yarn = yarn
        self.attn_factor = attn_factor

    @classmethod
    def plain(cls, kind, n_dims, base):
        return cls(kind, n_dims, base)

    def tables(self, factors, positions):
        """Host (cos, sin) f32 [positions, n_dims/2] (rope.rs:136-151)."""
        return hip.rope_tables(self.kind, self.n_dims, self.base, positions, self.freq_scale,
                               self.yarn, self.attn_factor, factors)

    def device_tables(self, ctx, factors, positions):
        cos, sin = self.tables(factors, positions)
        return ctx.array(cos), ctx.array(sin)


class QmmWeight:
    """A quantized [n, k] weight (y = x w^T) on the row-batched kernel
    (QmmWeight, qmm.rs:1744-1838), Q4_0 or Q8_0, resident in HBM in the
    kernels' packed layout (the file's bytes, reordered once on the device).
    Products are the reference CPU engine's bits, row by row."""

    def __init__(self, ctx, dtype, packed, n, k):
        self.ctx, self.dtype, self.packed, self.n_, self.k_ = ctx, dtype, packed, n, k

    @classmethod
    def from_raw(cls, ctx, dtype, data, n, k):
        """The weight of GGUF type `dtype` over its file bytes, or None for a
        type the kernel does not serve, a row that is not whole blocks or a
        wrong byte count (qmm.rs:1763-1783)."""
        row = byte_len(dtype, k)
        data = np.ascontiguousarray(np.frombuffer(data, np.uint8) if isinstance(data, bytes)
                                    else data, dtype=np.uint8).reshape(-1)
        if row is None or n <= 0 or row * n != data.size:
            return None
        raw = ctx.array(data)
        packed = ctx.empty((hip.qweight_bytes(dtype, n, k),), np.uint8)
        ctx.qweight_pack(raw.ptr, dtype, n, k, packed.ptr)
        ctx.sync()
        raw.free()
        return cls(ctx, dtype, packed, n, k)

    def n(self):
        """Output width (weight rows)."""
        return self.n_

    def k(self):
        """Input width (weight columns)."""
        return self.k_

    def forward(self, x, out=None):
        return self.forward_rows(x, self.n_, out=out)

    def forward_rows(self, x, rows, out=None):
        """x [m, k] (DeviceArray, f32 or f16) times the first `rows` weight
        rows: [m, rows] in x's dtype.  Row j depends on x[j] only, bit for bit."""
        m, width = x.shape
        if width != self.k_:  # qmm.rs:1815-1821
            raise CucaError(hip.INVALID_ARG, f"qmm: activations hold {x.size} floats, expected "
                            f"{m} rows of {self.k_}")
        if out is None:
            out = self.ctx.empty((m, rows), x.dtype)
        self.ctx.qmm(self.packed.ptr, self.dtype, self.n_, self.k_, x.ptr, self.k_, m, rows,
                     out.ptr, out.shape[1], hip.dtype_code(x.dtype))
        return out

    @staticmethod
    def glu(gate, up, x, glu, out=None):
        """act(gate x) * up x (FfnWeights::forward, GateUp::Split, with
        Glu::apply, cpu.rs:3554-3566, 342-371) in one launch."""
        ctx = gate.ctx
        m, width = x.shape
        if gate.dtype != up.dtype or gate.n_ != up.n_ or gate.k_ != up.k_ or width != gate.k_:
            raise CucaError(hip.INVALID_ARG, "qmm glu: gate and up differ in type or shape")
        if out is None:
            out = ctx.empty((m, gate.n_), x.dtype)
        ctx.qmm_glu(gate.packed.ptr, up.packed.ptr, gate.dtype, gate.n_, gate.k_, x.ptr, gate.k_, m,
                    glu.act, glu.clamp if glu.clamp is not None else 0.0, out.ptr, out.shape[1],
                    hip.dtype_code(x.dtype))
        return out


class ExpertBank:
    """The routed experts of one MoE layer, resident in HBM: per expert the
    gate, up and down matrices (GGUF Q4_0 / Q8_0) packed into three pools, one
    expert every `stride` bytes (the reference GPU engine's expert slots,
    moe_kernel.rs)."""

    def __init__(self, ctx, dtype, n_embd, ff, n_experts, pools, stride_gu, stride_d):
        self.ctx, self.dtype, self.n_embd, self.ff, self.n_experts = ctx, dtype, n_embd, ff, n_experts
        self.gate, self.up, self.down = pools
        self.stride_gu, self.stride_d = stride_gu, stride_d

    @classmethod
    def from_raw(cls, ctx, dtype, experts, n_embd, ff):
        """experts[e] = (gate, up, down) GGUF bytes of [ff, n_embd],
        [ff, n_embd], [n_embd, ff]."""
        def pool(mats, n, k):
            one = hip.qweight_bytes(dtype, n, k)
            stride = (one + 15) // 16 * 16
            dst = ctx.empty((stride * len(mats),), np.uint8)
            for e, raw in enumerate(mats):
                src = ctx.array(np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1))
                ctx.qweight_pack(src.ptr, dtype, n, k, dst.ptr + e * stride)
                ctx.sync()
                src.free()
            return dst, stride
        g, sgu = pool([m[0] for m in experts], ff, n_embd)
        u, _ = pool([m[1] for m in experts], ff, n_embd)
        d, sd = pool([m[2] for m in experts], n_embd, ff)
        return cls(ctx, dtype, n_embd, ff, len(experts), (g, u, d), sgu, sd)

    @staticmethod
    def grouped(per_expert, n_tokens, n_used):
        """Routing (moe.rs:15-21) as device-ready arrays: offsets
        [n_experts + 1], pair_token and pair_weight in expert order, and per
        token its pairs in ascending expert order ([n_tokens, n_used], -1
        where a token has fewer)."""
        offsets = np.zeros(len(per_expert) + 1, np.int32)
        tok, wt = [], []
        token_pairs = np.full((n_tokens, n_used), -1, np.int32)
        fill = np.zeros(n_tokens, np.int64)
        for e, picks in enumerate(per_expert):
            for t, w in picks:
                token_pairs[t, fill[t]] = len(tok)
                fill[t] += 1
                tok.append(t)
                wt.append(w)
            offsets[e + 1] = len(tok)
        return (offsets, np.asarray(tok, np.int32), np.asarray(wt, np.float32), token_pairs)

    def expert_sum(self, x, per_expert, glu, n_used, mm="qmm"):
        """The routed experts' output over the rows x ([t, n_embd] DeviceArray)
        for `per_expert` = [(token, weight)] per expert: moe_up, moe_down,
        moe_sum.  The per-pair hidden activations are held in x's dtype (f32
        keeps the reference CPU engine's values).  mm="qgemm" runs the up and
        down projections as grouped GEMMs on the matrix cores (the GPU
        engine's arithmetic class, for prefill-sized pair counts).  Returns
        (out [t, n_embd] in x's dtype, hidden, scratch)."""
        hidden_dtype = x.dtype
        ctx = self.ctx
        t = x.shape[0]
        offsets, tok, wt, token_pairs = self.grouped(per_expert, t, n_used)
        pairs = max(len(tok), 1)
        d_off, d_tok = ctx.array(offsets), ctx.array(tok if len(tok) else np.zeros(1, np.int32))
        d_wt = ctx.array(wt if len(wt) else np.zeros(1, np.float32))
        d_tp = ctx.array(token_pairs)
        hidden = ctx.empty((pairs, self.ff), hidden_dtype)
        scratch = ctx.empty((pairs, self.n_embd), np.float32)
        out = ctx.empty((t, self.n_embd), x.dtype)
        keep = ()
        if mm == "qgemm":
            wsb = max(hip.moe_qgemm_workspace(self.dtype, self.n_embd, self.n_experts, len(tok)),
                      hip.moe_qgemm_workspace(self.dtype, self.ff, self.n_experts, len(tok)), 16)
            ws = ctx.empty((wsb,), np.uint8)
            keep = (ws,)
            ctx.moe_up_qgemm(self.gate.ptr, self.up.ptr, self.stride_gu, self.dtype, self.ff, self.n_embd,
                             self.n_experts, x.ptr, self.n_embd, t, d_off.ptr, d_tok.ptr, len(tok), glu.act,
                             glu.clamp or 0.0, ws.ptr, wsb, hidden.ptr, self.ff, hip.dtype_code(hidden_dtype))
            ctx.moe_down_qgemm(self.down.ptr, self.stride_d, self.dtype, self.n_embd, self.ff, self.n_experts,
                               hidden.ptr, self.ff, d_off.ptr, d_wt.ptr, len(tok), ws.ptr, wsb, scratch.ptr,
                               self.n_embd, hip.dtype_code(hidden_dtype))
        else:
            ctx.moe_up(self.gate.ptr, self.up.ptr, self.stride_gu, self.dtype, self.ff, self.n_embd,
                       self.n_experts, x.ptr, self.n_embd, t, d_off.ptr, d_tok.ptr, len(tok), glu.act,
                       glu.clamp or 0.0, hidden.ptr, self.ff, hip.dtype_code(hidden_dtype))
            ctx.moe_down(self.down.ptr, self.stride_d, self.dtype, self.n_embd, self.ff, self.n_experts,
                         hidden.ptr, self.ff, d_off.ptr, d_wt.ptr, len(tok), scratch.ptr, self.n_embd,
                         hip.dtype_code(hidden_dtype))
        ctx.moe_sum(scratch.ptr, self.n_embd, len(tok), d_tp.ptr, n_used, t, self.n_embd, out.ptr,
                    self.n_embd, hip.dtype_code(x.dtype))
        # the routing arrays live as long as the output the queued kernels write
        out.keep = (d_off, d_tok, d_wt, d_tp) + keep
        return out, hidden, scratch
