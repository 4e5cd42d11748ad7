"""numpy front end of the CPU oracle (liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker.  The product (cuca_amd) never
imports it.

Arrays are numpy: float32 for f32 activations, float16 for f16 ones (their
bits are passed through unchanged), uint8 for quantized tables.
"""

import ctypes
import os

import numpy as np

from . import build as _build

_LIB = None

F32, F16 = 0, 1
Q4_0, Q8_0 = 2, 8
SILU, GELU_TANH = 0, 1
ROPE_NORM, ROPE_NEOX = 0, 2

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_f64 = ctypes.c_double
_int = ctypes.c_int


def lib():
    """Load liboracle.so, building it first when it is missing."""
    global _LIB
    if _LIB is None:
        path = _build.LIB
        if not os.path.exists(path):
            _build.build()
        L = ctypes.CDLL(path)
        L.oracle_f16_to_f32.restype = _f32
        L.oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.oracle_f32_to_f16.restype = ctypes.c_uint16
        L.oracle_f32_to_f16.argtypes = [_f32]
        L.oracle_f16_to_f32_n.argtypes = [_p, _p, _i64]
        L.oracle_f32_to_f16_n.argtypes = [_p, _p, _i64]
        L.oracle_f16_to_f32_soft_n.argtypes = [_p, _p, _i64]
        L.oracle_f32_to_f16_soft_n.argtypes = [_p, _p, _i64]
        L.oracle_has_f16c.restype = _int
        L.oracle_row_bytes.restype = _i64
        L.oracle_row_bytes.argtypes = [ctypes.c_uint32, _i64]
        L.oracle_dequant_row.restype = _int
        L.oracle_dequant_row.argtypes = [ctypes.c_uint32, _p, _i64, _f32, _p, _i64]
        L.oracle_embed.restype = _int
        L.oracle_embed.argtypes = [_p, ctypes.c_uint32, _i64, _i64, _p, _i64, _f32,
                                   _p, _int, _int, ctypes.POINTER(_i64)]
        L.oracle_embed_norm.restype = _int
        L.oracle_embed_norm.argtypes = [_p, ctypes.c_uint32, _i64, _i64, _p, _i64, _f32, _int,
                                        _f32, _p, _int, _int, ctypes.POINTER(_i64)]
        L.oracle_rms_norm_rows.argtypes = [_p, _i64, _i64, _f32]
        L.oracle_add_rmsnorm.argtypes = [_p, _p, _p, _p, _f32, _f32, _f32, _i64, _i64,
                                         _p, _p, _int, _int]
        L.oracle_glu.argtypes = [_p, _i64, _p, _i64, _i64, _i64, _int, _f32, _p, _i64,
                                 _int, _int]
        L.oracle_rope_tables.argtypes = [_int, _f64, _f64, _f64, _f64, _f64, _i64, _f64,
                                         _p, _i64, _p, _p]
        L.oracle_rope.argtypes = [_p, _i64, _i64, _int, _int, _int, _int, _p, _p, _p, _p,
                                  _f32, _int, _int]
        L.oracle_rope_full.argtypes = L.oracle_rope.argtypes
        L.oracle_store_rows.restype = _int
        L.oracle_store_rows.argtypes = [_p, _i64, _i64, _i64, _p, _p, _i64, _int, _int, _int]
        L.oracle_paged_attention.restype = _int
        L.oracle_paged_attention.argtypes = [_p, _i64, _int, _int, _int, _p, _i64, _p, _p, _p,
                                             _i64, _f32, _p, _int, _int]
        L.oracle_gather.restype = _int
        L.oracle_gather.argtypes = [_p, _i64, _i64, _i64, _p, _p, _i64, _int, _int, _int]
        L.oracle_q8_acts.argtypes = [_p, _i64, _i64, _i64, _int, _p, _p]
        L.oracle_cap_logits.argtypes = [_p, _i64, _f32, _f32, _f32]
        L.oracle_greedy.restype = ctypes.c_uint32
        L.oracle_greedy.argtypes = [_p, _i64]
        L.oracle_splitmix64.restype = ctypes.c_uint64
        L.oracle_splitmix64.argtypes = [ctypes.POINTER(ctypes.c_uint64)]
        L.oracle_next_f32.restype = _f32
        L.oracle_next_f32.argtypes = [ctypes.POINTER(ctypes.c_uint64)]
        L.oracle_select_top_k.restype = _i64
        L.oracle_select_top_k.argtypes = [_p, _i64, _f32, _i64, _p, _p]
        L.oracle_sample.restype = ctypes.c_uint32
        L.oracle_sample.argtypes = [_p, _i64, _f32, _i64, _f32, ctypes.POINTER(ctypes.c_uint64)]
        L.oracle_qmm.restype = _int
        L.oracle_qmm.argtypes = [_p, ctypes.c_uint32, _i64, _i64, _p, _i64, _i64, _i64, _p,
                                 _int, _int]
        _LIB = L
    return _LIB


def _ptr(a):
    return None if a is None else a.ctypes.data


def _dtype_code(a):
    if a.dtype == np.float32:
        return F32
    if a.dtype == np.float16:
        return F16
    raise TypeError(f"activations must be float32 or float16, not {a.dtype}")


def f16_to_f32(h):
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().oracle_f16_to_f32_n(_ptr(h), _ptr(out), h.size)
    return out


def f32_to_f16(f):
    f = np.ascontiguousarray(f, dtype=np.float32)
    out = np.empty(f.shape, np.uint16)
    lib().oracle_f32_to_f16_n(_ptr(f), _ptr(out), f.size)
    return out


def row_bytes(ggml_type, hidden):
    return int(lib().oracle_row_bytes(ggml_type, hidden))


def dequant_row(ggml_type, data, scale, n):
    data = np.ascontiguousarray(data, dtype=np.uint8)
    out = np.empty(n, np.float32)
    rc = lib().oracle_dequant_row(ggml_type, _ptr(data), data.size, scale, _ptr(out), n)
    if rc != 0:
        raise ValueError(f"row of {data.size} bytes does not hold {n} elements")
    return out


class OracleError(ValueError):
    pass


def rms_norm_rows(rows, eps):
    """rms_norm_rows (quant.rs:324-339) on a copy of f32 rows [n, row_len]."""
    r = np.array(rows, dtype=np.float32, copy=True, order="C")
    lib().oracle_rms_norm_rows(_ptr(r), r.shape[0], r.shape[1], eps)
    return r


def embed(table, ggml_type, vocab, hidden, ids, scale, out_dtype=np.float32, threads=1,
          norm_eps=None):
    """TokenEmbedding::rows; norm_eps given: then norm_embeddings'
    rms_norm_rows with that eps (the embd_norm archs)."""
    table = np.ascontiguousarray(table, dtype=np.uint8)
    ids = np.ascontiguousarray(ids, dtype=np.uint32)
    out = np.empty((ids.size, hidden), out_dtype)
    bad = _i64(-1)
    norm = norm_eps is not None
    rc = lib().oracle_embed_norm(_ptr(table), ggml_type, vocab, hidden, _ptr(ids), ids.size,
                                 scale, 1 if norm else 0, norm_eps if norm else 0.0, _ptr(out),
                                 _dtype_code(out), threads, ctypes.byref(bad))
    if rc == -1:
        raise OracleError(f"row length {hidden} is not a whole number of blocks")
    if rc == -2:
        raise OracleError(f"token id {int(ids[bad.value])} outside the embedding table "
                          f"of {vocab} rows")
    return out


def add_rmsnorm(x, branch, w, eps, w_post=None, post_eps=None, residual_scale=1.0,
                threads=1, write_x=True):
    """Returns (x_out or None, h)."""
    x = np.ascontiguousarray(x)
    rows, hidden = x.shape
    if branch is not None:
        branch = np.ascontiguousarray(branch, dtype=x.dtype)
    w = None if w is None else np.ascontiguousarray(w, dtype=np.float32)
    w_post = None if w_post is None else np.ascontiguousarray(w_post, dtype=np.float32)
    x_out = np.empty_like(x) if write_x else None
    h = np.empty_like(x)
    lib().oracle_add_rmsnorm(_ptr(x), _ptr(branch), _ptr(w), _ptr(w_post), eps,
                             eps if post_eps is None else post_eps, residual_scale,
                             rows, hidden, _ptr(x_out), _ptr(h), _dtype_code(x), threads)
    return x_out, h


def glu(gate, up, act, clamp=0.0, threads=1):
    """act(gate) * up over [rows, ff] views (row strides taken from the arrays)."""
    assert gate.shape == up.shape and gate.dtype == up.dtype
    rows, ff = gate.shape
    for a in (gate, up):
        assert a.strides[1] == a.itemsize, "rows must be contiguous"
    out = np.empty((rows, ff), gate.dtype)
    lib().oracle_glu(_ptr(gate), gate.strides[0] // gate.itemsize, _ptr(up),
                     up.strides[0] // up.itemsize, rows, ff, act, clamp, _ptr(out), ff,
                     _dtype_code(gate), threads)
    return out


def rope_tables(n_dims, base, positions, freq_scale=1.0, yarn=None, attn_factor=1.0,
                factors=None):
    """yarn: None or (ext_factor, beta_fast, beta_slow, n_ctx_orig)."""
    half = n_dims // 2
    cos = np.empty((positions, half), np.float32)
    sin = np.empty((positions, half), np.float32)
    ext, bf, bs, nco = yarn if yarn is not None else (0.0, 32.0, 1.0, 0)
    f = None if factors is None else np.ascontiguousarray(factors, dtype=np.float32)
    lib().oracle_rope_tables(n_dims, base, freq_scale, ext, bf, bs, nco, attn_factor,
                             _ptr(f), positions, _ptr(cos), _ptr(sin))
    return cos, sin


def rope(x, cos, sin, positions, kind, n_dims=None, norm_w=None, eps=1e-6, threads=1,
         full=False):
    """Rotate a copy of x [rows, heads, d] (returned); optional fused QK-norm,
    per head (norm_w [d]) or, with full, over the row's whole projection
    (norm_w [heads * d], the qk_norm_full archs)."""
    x = np.array(x, copy=True, order="C")
    rows, heads, d = x.shape
    n_dims = d if n_dims is None else n_dims
    cos = np.ascontiguousarray(cos, dtype=np.float32)
    sin = np.ascontiguousarray(sin, dtype=np.float32)
    pos = np.ascontiguousarray(positions, dtype=np.int32)
    nw = None if norm_w is None else np.ascontiguousarray(norm_w, dtype=np.float32)
    fn = lib().oracle_rope_full if full else lib().oracle_rope
    fn(_ptr(x), heads * d, rows, heads, d, n_dims, kind, _ptr(cos), _ptr(sin), _ptr(pos),
       _ptr(nw), eps, _dtype_code(x), threads)
    return x


KV_BLOCK = 16
NO_BLOCK = 0xFFFFFFFF


class KvError(ValueError):
    """A position without a K/V block (check_range, cpu/paged_attn.rs:42-65)."""


def store_rows(table, start, src, pool):
    """store_rows (cpu/paged_attn.rs:370-400): src [n_kv, rows, d] into the
    positions start.. of `pool` [n_blocks, n_kv, 16, d] (modified in place)."""
    n_blocks, n_kv, bs, d = pool.shape
    assert bs == KV_BLOCK and pool.flags.c_contiguous and src.dtype == pool.dtype
    src = np.ascontiguousarray(src)
    assert src.shape[0] == n_kv and src.shape[2] == d
    tab = np.ascontiguousarray(table, dtype=np.uint32)
    rc = lib().oracle_store_rows(_ptr(tab), tab.size, start, src.shape[1], _ptr(src), _ptr(pool),
                                 n_blocks, n_kv, d, _dtype_code(pool))
    if rc != 0:
        raise KvError(f"position range {start}..{start + src.shape[1]} has no K/V block")
    return pool


def gather(table, lo, hi, pool):
    """gather (cpu/paged_attn.rs:340-362): positions lo..hi of `pool` as
    [n_kv, hi - lo, d]."""
    n_blocks, n_kv, bs, d = pool.shape
    pool = np.ascontiguousarray(pool)
    tab = np.ascontiguousarray(table, dtype=np.uint32)
    out = np.empty((n_kv, hi - lo, d), pool.dtype)
    rc = lib().oracle_gather(_ptr(tab), tab.size, lo, hi, _ptr(pool), _ptr(out), n_blocks, n_kv,
                             d, _dtype_code(pool))
    if rc != 0:
        raise KvError(f"position range {lo}..{hi} has no K/V block")
    return out


def store_kv(q, k, v, cos, sin, kind, n_dims, calls, pool_k, pool_v, q_norm_w=None,
             k_norm_w=None, v_norm=False, eps=1e-6, threads=1, full=False):
    """store_kv (cpu.rs:3028-3097) for the rows of several calls: q, k, v
    [rows, heads, d]; calls = [(offset, start, rope_start, t, table)], the
    call's rows offset.. at cache indices start.. and RoPE positions
    rope_start.. (AttnCall, cpu.rs:1314-1325).  Q and K are normalised
    (per head) and rotated, V normalised without a weight when v_norm
    (gpu.rs:5277), K and V stored into the pools (modified in place).
    With full, the Q and K norms span each row's whole projection
    (qk_norm_full, cpu.rs:2838-2843, 3042-3045).  Returns the rotated Q."""
    rows, nk, d = k.shape
    pos = np.zeros(rows, np.int32)
    for off, start, rope_start, t, table in calls:
        pos[off:off + t] = np.arange(rope_start, rope_start + t)
    qr = rope(q, cos, sin, pos, kind, n_dims, norm_w=q_norm_w, eps=eps, threads=threads, full=full)
    kr = rope(k, cos, sin, pos, kind, n_dims, norm_w=k_norm_w, eps=eps, threads=threads, full=full)
    vv = np.ascontiguousarray(v)
    if v_norm:
        _, h = add_rmsnorm(vv.reshape(rows * nk, d), None, None, eps, threads=threads, write_x=False)
        vv = h.reshape(rows, nk, d)
    for off, start, rope_start, t, table in calls:
        store_rows(table, start, kr[off:off + t].transpose(1, 0, 2), pool_k)
        store_rows(table, start, vv[off:off + t].transpose(1, 0, 2), pool_v)
    return qr


def paged_attention(q, tables, ranges, pool_k, pool_v, scale, threads=1):
    """attend_paged_rows per row: q [rows, n_head, d]; tables u32 [rows,
    max_blocks]; ranges int32 [rows, 2]; pools [n_blocks, n_kv, 16, d] of q's
    dtype.  Returns [rows, n_head, d]; raises KvError for a bad range."""
    q = np.ascontiguousarray(q)
    rows, n_head, d = q.shape
    n_blocks, n_kv, bs, d2 = pool_k.shape
    assert bs == KV_BLOCK and d2 == d and pool_v.shape == pool_k.shape
    assert pool_k.dtype == q.dtype == pool_v.dtype
    tab = np.ascontiguousarray(tables, dtype=np.uint32).reshape(rows, -1)
    rng = np.ascontiguousarray(ranges, dtype=np.int32).reshape(rows, 2)
    pk, pv = np.ascontiguousarray(pool_k), np.ascontiguousarray(pool_v)
    out = np.empty_like(q)
    rc = lib().oracle_paged_attention(_ptr(q), rows, n_head, n_kv, d, _ptr(tab), tab.shape[1],
                                      _ptr(rng), _ptr(pk), _ptr(pv), n_blocks, scale, _ptr(out),
                                      _dtype_code(q), threads)
    if rc != 0:
        raise KvError("attention over an empty key range or a position without a K/V block")
    return out


def q8_acts(x):
    """Acts::new (qmm.rs:1272-1343) for a format without minima: x [m, k]
    (float32, or float16 widened) -> (quants int8 [m, k], scales f32 [m, k/32])."""
    x = np.ascontiguousarray(x)
    m, k = x.shape
    q = np.empty((m, k), np.int8)
    s = np.empty((m, k // 32), np.float32)
    lib().oracle_q8_acts(_ptr(x), k, m, k, _dtype_code(x), _ptr(q), _ptr(s))
    return q, s


def qmm(w, ggml_type, n, k, x, rows=None, threads=1):
    """QmmWeight::forward_rows (qmm.rs:1810-1838) for Q4_0 / Q8_0: w the GGUF
    bytes of an [n, k] weight, x [m, k] (float32 or float16); returns the
    f32 [m, rows] product with the first `rows` weight rows (default n)."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x)
    if x.ndim == 1:
        x = x.reshape(1, -1)
    m = x.shape[0]
    rows = n if rows is None else rows
    if x.shape[1] != k:
        raise OracleError(f"qmm: activations hold {x.size} floats, expected {m} rows of {k}")
    if w.size != n * row_bytes(ggml_type, k):
        raise OracleError(f"qmm: weight holds {w.size} bytes, expected {n} rows")
    out = np.empty((m, rows), np.float32)
    rc = lib().oracle_qmm(_ptr(w), ggml_type, n, k, _ptr(x), k, m, rows, _ptr(out),
                          _dtype_code(x), threads)
    if rc != 0:
        raise OracleError(f"qmm: {rows} weight rows of {n}")
    return out


def expert_sum(x, experts, qtype, per_expert, act, clamp=0.0, threads=1):
    """expert_sum (cpu.rs:3599-3642) with CpuExpert::forward / add_picks
    (cpu.rs:373-419): x [t, n_embd] (f32 or f16, widened); experts[e] =
    (gate, up, down) GGUF bytes of [ff, n_embd], [ff, n_embd], [n_embd, ff];
    per_expert[e] = [(token, weight)] in token order.  Every non-empty expert
    runs once over its picked rows, in ascending expert order, and
    out[token] += y * weight (f32, each product and sum rounded) from zeros.
    Returns (out f32 [t, n_embd], hidden {(e, i): f32 [ff]}) -- hidden is the
    activation each pick's down projection read."""
    x = np.ascontiguousarray(x)
    t, n_embd = x.shape
    out = np.zeros((t, n_embd), np.float32)
    hidden = {}
    for e, picks in enumerate(per_expert):
        if not picks:
            continue
        gate, up, down = experts[e]
        ff = gate.size // row_bytes(qtype, n_embd)
        rows = x[[tok for tok, _ in picks]].astype(np.float32)
        g = qmm(gate, qtype, ff, n_embd, rows, threads=threads)
        u = qmm(up, qtype, ff, n_embd, rows, threads=threads)
        h = glu(g, u, act, clamp=clamp, threads=threads)
        y = qmm(down, qtype, n_embd, ff, h, threads=threads)
        for i, (tok, w) in enumerate(picks):
            hidden[(e, i)] = h[i]
            out[tok] = (out[tok] + (y[i] * np.float32(w)).astype(np.float32)).astype(np.float32)
    return out, hidden


def cap_logits(v, logit_scale=1.0, logit_mult=1.0, softcap=0.0):
    """cap_logits (cpu.rs:2603-2617) on a copy of f32 logits."""
    v = np.array(v, dtype=np.float32, copy=True, order="C")
    lib().oracle_cap_logits(_ptr(v), v.size, logit_scale, logit_mult, softcap)
    return v


def greedy(logits):
    """greedy (sampler.rs:44-56): the first maximum."""
    v = np.ascontiguousarray(logits, dtype=np.float32)
    return int(lib().oracle_greedy(_ptr(v), v.size))


class SplitMix64:
    """SplitMix64 (sampler.rs:18-35) over the oracle's C implementation."""

    def __init__(self, seed):
        self.state = ctypes.c_uint64(seed)

    def next_u64(self):
        return int(lib().oracle_splitmix64(ctypes.byref(self.state)))

    def next_f32(self):
        return float(lib().oracle_next_f32(ctypes.byref(self.state)))


def select_top_k(logits, temperature, k):
    """select_top_k (sampler.rs:254-286): ((logit / temperature) f32[c], ids u32[c])."""
    v = np.ascontiguousarray(logits, dtype=np.float32)
    out_l = np.empty(max(k, 1), np.float32)
    out_i = np.empty(max(k, 1), np.uint32)
    c = lib().oracle_select_top_k(_ptr(v), v.size, temperature, k, _ptr(out_l), _ptr(out_i))
    return out_l[:c], out_i[:c]


def sample(logits, temperature, top_k, top_p, rng):
    """sample (sampler.rs:308-334) on a copy of the logits with a SplitMix64."""
    v = np.array(logits, dtype=np.float32, copy=True, order="C")
    return int(lib().oracle_sample(_ptr(v), v.size, temperature, top_k, top_p, ctypes.byref(rng.state)))
