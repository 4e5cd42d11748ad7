"""ctypes binding of the C ABI in include/cuca_hip.h (libcuca_hip.so).

The library is loaded from this package's directory only (the in-tree build
of cuca_amd/build.py).  There is no fallback: when the library is missing,
importing the bindings raises, so no caller can silently run anything else.
"""

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libcuca_hip.so")

OK, INVALID_ARG, OUT_OF_RANGE, HIP_ERROR, NOT_GFX950, UNSUPPORTED = range(6)
F32, F16 = 0, 1
GGML_Q4_0, GGML_Q8_0 = 2, 8
ACT_SILU, ACT_GELU_TANH = 0, 1
ROPE_NORM, ROPE_NEOX = 0, 2

# Every entry point of include/cuca_hip.h: (restype, argtypes).
_p = ctypes.c_void_p
_pp = ctypes.POINTER(ctypes.c_void_p)
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_u32 = ctypes.c_uint32
_f32 = ctypes.c_float
_sz = ctypes.c_size_t
_st = ctypes.c_int


class RopeSpecC(ctypes.Structure):
    """cuca_rope_spec."""
    _fields_ = [("kind", _i32), ("n_dims", _i32), ("base", ctypes.c_double),
                ("freq_scale", ctypes.c_double), ("yarn_ext_factor", ctypes.c_double),
                ("yarn_beta_fast", ctypes.c_double), ("yarn_beta_slow", ctypes.c_double),
                ("yarn_n_ctx_orig", _i64), ("attn_factor", ctypes.c_double)]


class KernelTime(ctypes.Structure):
    """cuca_hip_kernel_time."""
    _fields_ = [("kernel", ctypes.c_char_p), ("ms", _f32)]


SIGNATURES = {
    "cuca_hip_ctx_create": (_st, [ctypes.c_int, _pp]),
    "cuca_hip_ctx_destroy": (None, [_p]),
    "cuca_hip_last_error": (ctypes.c_char_p, [_p]),
    "cuca_hip_set_stream": (_st, [_p, _p]),
    "cuca_hip_get_stream": (_p, [_p]),
    "cuca_hip_device": (ctypes.c_int, [_p]),
    "cuca_hip_malloc": (_st, [_p, _sz, _pp]),
    "cuca_hip_free": (_st, [_p, _p]),
    "cuca_hip_memcpy_h2d_async": (_st, [_p, _p, _p, _sz]),
    "cuca_hip_memcpy_d2h_async": (_st, [_p, _p, _p, _sz]),
    "cuca_hip_memcpy_d2d_async": (_st, [_p, _p, _p, _sz]),
    "cuca_hip_stream_sync": (_st, [_p]),
    "cuca_hip_check_device": (_st, [_p]),
    "cuca_hip_selftest_group_sum": (_st, [_p, _p, _i64, _p]),
    "cuca_hip_embed_gguf": (_st, [_p, _p, _u32, _i64, _i64, _p, _i64, _f32, _p, _st]),
    "cuca_hip_embed_gguf_norm": (_st, [_p, _p, _u32, _i64, _i64, _p, _i64, _f32, _f32, _p, _st]),
    "cuca_hip_embed_gguf_rms": (_st, [_p, _p, _u32, _i64, _i64, _p, _i64, _f32, _p, _f32, _p, _p, _st]),
    "cuca_hip_add_rmsnorm": (_st, [_p, _p, _p, _p, _p, _f32, _f32, _f32, _i64, _i64, _p, _p, _st]),
    "cuca_hip_glu": (_st, [_p, _p, _i64, _p, _i64, _i64, _i64, _st, _f32, _p, _i64, _st]),
    "cuca_hip_glu_ragged": (_st, [_p, _p, _i64, _p, _i64, _p, _i32, _i64, _i64, _st, _f32, _p,
                                  _i64, _st]),
    "cuca_hip_rope": (_st, [_p, _p, _i64, _p, _i64, _i64, _i32, _i32, _i32, _i32, _st, _p, _p,
                            _i64, _p, _p, _p, _f32, _st]),
    "cuca_hip_rope_store_kv": (_st, [_p, _p, _i64, _p, _i64, _p, _i64, _i64, _i32, _i32, _i32, _i32,
                                     _st, _p, _p, _i64, _p, _p, _p, _i32, _f32, _p, _p, _i64, _p,
                                     _st]),
    "cuca_hip_rope_full": (_st, [_p, _p, _i64, _p, _i64, _i64, _i32, _i32, _i32, _i32, _st, _p, _p,
                                 _i64, _p, _p, _p, _f32, _st]),
    "cuca_hip_rope_store_kv_full": (_st, [_p, _p, _i64, _p, _i64, _p, _i64, _i64, _i32, _i32, _i32,
                                          _i32, _st, _p, _p, _i64, _p, _p, _p, _i32, _f32, _p, _p,
                                          _i64, _p, _st]),
    "cuca_hip_kv_slots": (_st, [_p, _i64, _i64, _i64, _i64, _p]),
    "cuca_hip_paged_decode_workspace": (_st, [_i64, _i32, _i32, _i64, ctypes.POINTER(_sz)]),
    "cuca_hip_paged_decode": (_st, [_p, _p, _i64, _p, _p, _i64, _p, _i64, _p, _i64, _i32, _i32,
                                    _i32, _f32, _p, _sz, _p, _st]),
    "cuca_hip_paged_decode_noalloc": (_st, [_p, _p, _i64, _p, _p, _i64, _p, _i64, _p, _i64, _i32,
                                            _i32, _i32, _f32, _p, _st]),
    "cuca_hip_attend_rows": (_st, [_p, _p, _i64, _p, _p, _i64, _p, _i64, _p, _i64, _i32, _i32, _i32,
                                   _f32, _p, _i64, _st]),
    "cuca_hip_attend_latent_rows": (_st, [_p, _p, _i64, _p, _i64, _p, _i64, _p, _i64, _i32, _i32,
                                          _i32, _f32, _p, _i64, _st]),
    "cuca_hip_rope_tables": (_st, [ctypes.POINTER(RopeSpecC), _p, _i64, _p, _p]),
    "cuca_hip_qweight_bytes": (_st, [_u32, _i64, _i64, ctypes.POINTER(_sz)]),
    "cuca_hip_qweight_pack": (_st, [_p, _p, _u32, _i64, _i64, _p]),
    "cuca_hip_qmm": (_st, [_p, _p, _u32, _i64, _i64, _p, _i64, _i64, _i64, _p, _i64, _st]),
    "cuca_hip_qmm_rope_store_kv": (_st, [_p, _p, _u32, _i64, _p, _i64, _i64, _i32, _i32, _i32, _i32,
                                         _st, _p, _p, _i64, _p, _p, _i64, _p, _p, _i64, _p, _st]),
    "cuca_hip_qmm_glu": (_st, [_p, _p, _p, _u32, _i64, _i64, _p, _i64, _i64, _st, _f32, _p, _i64,
                               _st]),
    "cuca_hip_add_rmsnorm_qmm": (_st, [_p, _p, _p, _p, _f32, _f32, _p, _p, _p, _u32, _i64, _i64, _i64,
                                       _i64, _p, _i64, _st]),
    "cuca_hip_add_rmsnorm_qmm_glu": (_st, [_p, _p, _p, _p, _f32, _f32, _p, _p, _p, _p, _u32, _i64, _i64,
                                           _i64, _st, _f32, _p, _i64, _st]),
    "cuca_hip_add_rmsnorm_qmm_rope_store_kv": (_st, [_p, _p, _p, _p, _f32, _f32, _p, _p, _p, _u32, _i64,
                                                     _i64, _i32, _i32, _i32, _i32, _st, _p, _p, _i64, _p,
                                                     _p, _i64, _p, _p, _i64, _p, _st]),
    "cuca_hip_qgemm_workspace": (_st, [_u32, _i64, _i64, _i64, _i32, ctypes.POINTER(ctypes.c_size_t)]),
    "cuca_hip_qweight_dequant": (_st, [_p, _p, _u32, _i64, _i64, _p]),
    "cuca_hip_gemm_w16_workspace": (_st, [_i64, _i64, _i64, _i32, _st, ctypes.POINTER(ctypes.c_size_t)]),
    "cuca_hip_gemm_w16": (_st, [_p, _p, _i64, _i64, _p, _i64, _i64, _i64, _p, _sz, _p, _i64, _st]),
    "cuca_hip_gemm_w16_glu": (_st, [_p, _p, _i64, _i64, _p, _i64, _i64, _st, _f32, _p, _sz, _p, _i64,
                                    _st]),
    "cuca_hip_qgemm": (_st, [_p, _p, _u32, _i64, _i64, _p, _i64, _i64, _i64, _p, _sz, _p, _i64, _st]),
    "cuca_hip_qgemm_glu": (_st, [_p, _p, _p, _u32, _i64, _i64, _p, _i64, _i64, _st, _f32, _p, _sz, _p,
                                 _i64, _st]),
    "cuca_hip_moe_up": (_st, [_p, _p, _p, _i64, _u32, _i64, _i64, _i32, _p, _i64, _i64, _p, _p, _i64,
                              _st, _f32, _p, _i64, _st]),
    "cuca_hip_moe_down": (_st, [_p, _p, _i64, _u32, _i64, _i64, _i32, _p, _i64, _p, _p, _i64, _p,
                                _i64, _st]),
    "cuca_hip_moe_qgemm_workspace": (_st, [_u32, _i64, _i32, _i64, _p]),
    "cuca_hip_moe_up_qgemm": (_st, [_p, _p, _p, _i64, _u32, _i64, _i64, _i32, _p, _i64, _i64, _p, _p, _i64,
                                    _st, _f32, _p, _sz, _p, _i64, _st]),
    "cuca_hip_moe_down_qgemm": (_st, [_p, _p, _i64, _u32, _i64, _i64, _i32, _p, _i64, _p, _p, _i64, _p, _sz,
                                      _p, _i64, _st]),
    "cuca_hip_moe_sum": (_st, [_p, _p, _i64, _i64, _p, _i32, _i64, _i64, _p, _i64, _st]),
    "cuca_hip_q8_acts": (_st, [_p, _p, _i64, _i64, _i64, _st, _p, _p]),
    "cuca_hip_qmv": (_st, [_p, _p, _u32, _i64, _i64, _p, _p, _i64, _i64, _p, _i64, _st]),
    "cuca_hip_qmv_glu": (_st, [_p, _p, _p, _u32, _i64, _i64, _p, _p, _i64, _st, _f32, _p, _i64, _st]),
    "cuca_hip_lm_head": (_st, [_p, _p, _u32, _i64, _i64, _p, _i64, _i64, _i64, _f32, _f32, _f32, _p,
                               _i64, _st]),
    "cuca_hip_lm_head_indexed_workspace": (_st, [_u32, _i64, _i64, ctypes.POINTER(_sz)]),
    "cuca_hip_lm_head_indexed": (_st, [_p, _p, _u32, _i64, _i64, _p, _i64, _i64, _p, _i64, _f32, _f32,
                                       _f32, _p, _sz, _p, _i64, _st]),
    "cuca_hip_argmax": (_st, [_p, _p, _i64, _i64, _i64, _st, _p]),
    "cuca_hip_top_k": (_st, [_p, _p, _i64, _i64, _i64, _st, _i32, _f32, _p, _p, _p]),
    "cuca_hip_sample_candidates": (_st, [_p, _p, _i32, _f32, _u32, ctypes.POINTER(ctypes.c_uint64),
                                         ctypes.POINTER(_u32)]),
    "cuca_hip_graph_begin": (_st, [_p]),
    "cuca_hip_graph_end": (_st, [_p, _pp]),
    "cuca_hip_graph_launch": (_st, [_p, _p]),
    "cuca_hip_graph_destroy": (None, [_p]),
    "cuca_hip_timer_start": (_st, [_p]),
    "cuca_hip_timer_stop": (_st, [_p, ctypes.POINTER(_f32)]),
    "cuca_hip_profile_start": (_st, [_p, _i32]),
    "cuca_hip_profile_stop": (_st, [_p, ctypes.POINTER(KernelTime), _i32,
                                    ctypes.POINTER(_i32)]),
}

_LIB = None


class CucaError(RuntimeError):
    """A non-OK cuca_status, with the library's message (the reference maps
    the same failures to CucaError::Provider(Local, msg), model/mod.rs:222-228)."""

    def __init__(self, status, message):
        super().__init__(f"{message} (status {status})")
        self.status = status
        self.message = message


def lib():
    """The loaded libcuca_hip.so (raises when it has not been built)."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: build it with `python -m cuca_amd.build` "
                              "(there is no other implementation of these ops)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = L
    return _LIB


def _check(st, ctx_ptr=None):
    if st != OK:
        msg = lib().cuca_hip_last_error(ctx_ptr).decode(errors="replace")
        raise CucaError(st, msg)


_NP = {F32: np.float32, F16: np.float16}


def dtype_code(dt):
    dt = np.dtype(dt)
    if dt == np.float32:
        return F32
    if dt == np.float16:
        return F16
    raise TypeError(f"activations are float32 or float16, not {dt}")


class DeviceArray:
    """A device buffer with a numpy shape and dtype, owned by a Context."""

    def __init__(self, ctx, shape, dtype, ptr=None, owner=True):
        self.ctx = ctx
        self.shape = tuple(int(s) for s in shape)
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        self.owner = owner and ptr is None
        if ptr is None:
            ptr = ctx.malloc(self.nbytes)
        self.ptr = ptr

    @property
    def size(self):
        return int(np.prod(self.shape, dtype=np.int64))

    def numpy(self):
        out = np.empty(self.shape, self.dtype)
        self.ctx.d2h(out, self)
        self.ctx.sync()
        return out

    def upload(self, arr):
        arr = np.ascontiguousarray(arr, dtype=self.dtype)
        assert arr.nbytes == self.nbytes, (arr.shape, self.shape)
        self.ctx.h2d(self, arr)
        self.ctx.sync()
        return self

    def view(self, offset_elems, shape):
        """A non-owning view starting offset_elems elements in."""
        return DeviceArray(self.ctx, shape, self.dtype,
                           ptr=(self.ptr or 0) + offset_elems * self.dtype.itemsize, owner=False)

    def free(self):
        if self.owner and self.ptr:
            self.ctx.free(self.ptr)
        self.ptr = None

    def __del__(self):
        try:
            if self.owner and self.ptr and self.ctx.ptr:
                self.ctx.free(self.ptr)
        except Exception:
            pass


class Context:
    """One cuca_hip_ctx: a gfx950 device, its stream and the loaded kernels."""

    def __init__(self, device=0):
        L = lib()
        p = ctypes.c_void_p()
        _check(L.cuca_hip_ctx_create(device, ctypes.byref(p)), None)
        self.ptr = p.value
        self.L = L

    def close(self):
        if self.ptr:
            self.L.cuca_hip_ctx_destroy(self.ptr)
            self.ptr = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def check(self, st):
        _check(st, self.ptr)

    # memory and stream ------------------------------------------------
    def malloc(self, nbytes):
        p = ctypes.c_void_p()
        self.check(self.L.cuca_hip_malloc(self.ptr, nbytes, ctypes.byref(p)))
        return p.value

    def free(self, ptr):
        self.check(self.L.cuca_hip_free(self.ptr, ptr))

    def h2d(self, dst, arr):
        self.check(self.L.cuca_hip_memcpy_h2d_async(self.ptr, dst.ptr, arr.ctypes.data, arr.nbytes))

    def d2h(self, arr, src):
        self.check(self.L.cuca_hip_memcpy_d2h_async(self.ptr, arr.ctypes.data, src.ptr, arr.nbytes))

    def sync(self):
        self.check(self.L.cuca_hip_stream_sync(self.ptr))

    def check_device(self):
        self.check(self.L.cuca_hip_check_device(self.ptr))

    def selftest_group_sum(self, inp, n, out):
        self.check(self.L.cuca_hip_selftest_group_sum(self.ptr, inp, n, out))

    def array(self, arr, dtype=None):
        """Upload a numpy array."""
        arr = np.ascontiguousarray(arr, dtype=dtype)
        return DeviceArray(self, arr.shape, arr.dtype).upload(arr)

    def empty(self, shape, dtype):
        return DeviceArray(self, shape, dtype)

    def set_stream(self, stream_ptr):
        self.check(self.L.cuca_hip_set_stream(self.ptr, stream_ptr))

    @property
    def stream(self):
        return self.L.cuca_hip_get_stream(self.ptr)

    # timing and graphs ------------------------------------------------
    def timer_start(self):
        self.check(self.L.cuca_hip_timer_start(self.ptr))

    def timer_stop(self):
        ms = ctypes.c_float()
        self.check(self.L.cuca_hip_timer_stop(self.ptr, ctypes.byref(ms)))
        return ms.value

    def profile_start(self, max_launches):
        self.check(self.L.cuca_hip_profile_start(self.ptr, max_launches))
        self._prof_max = max_launches

    def profile_stop(self):
        """[(kernel name, ms)] of the launches since profile_start, in order."""
        n = max(getattr(self, "_prof_max", 0), 1)
        buf = (KernelTime * n)()
        count = _i32()
        self.check(self.L.cuca_hip_profile_stop(self.ptr, buf, n, ctypes.byref(count)))
        return [(buf[i].kernel.decode(), buf[i].ms) for i in range(count.value)]

    def graph_begin(self):
        self.check(self.L.cuca_hip_graph_begin(self.ptr))

    def graph_end(self):
        g = ctypes.c_void_p()
        self.check(self.L.cuca_hip_graph_end(self.ptr, ctypes.byref(g)))
        return Graph(self, g.value)

    # raw ops (device pointers) ----------------------------------------
    def embed_gguf(self, table, ggml_type, vocab, hidden, ids, n, scale, out, out_dtype):
        self.check(self.L.cuca_hip_embed_gguf(self.ptr, table, ggml_type, vocab, hidden, ids, n,
                                              scale, out, out_dtype))

    def embed_gguf_norm(self, table, ggml_type, vocab, hidden, ids, n, scale, norm_eps, out,
                        out_dtype):
        self.check(self.L.cuca_hip_embed_gguf_norm(self.ptr, table, ggml_type, vocab, hidden, ids,
                                                   n, scale, norm_eps, out, out_dtype))

    def embed_gguf_rms(self, table, ggml_type, vocab, hidden, ids, n, scale, w, eps, x_out, h_out,
                       out_dtype):
        self.check(self.L.cuca_hip_embed_gguf_rms(self.ptr, table, ggml_type, vocab, hidden, ids, n,
                                                  scale, w, eps, x_out, h_out, out_dtype))

    def add_rmsnorm(self, x, branch, w, w_post, eps, post_eps, residual_scale, rows, hidden,
                    x_out, h_out, dtype):
        self.check(self.L.cuca_hip_add_rmsnorm(self.ptr, x, branch, w, w_post, eps, post_eps,
                                               residual_scale, rows, hidden, x_out, h_out, dtype))

    def glu(self, gate, gate_ld, up, up_ld, rows, ff, act, clamp, out, out_ld, dtype):
        self.check(self.L.cuca_hip_glu(self.ptr, gate, gate_ld, up, up_ld, rows, ff, act, clamp,
                                       out, out_ld, dtype))

    def glu_ragged(self, gate, gate_ld, up, up_ld, offsets, n_experts, max_rows, ff, act, clamp,
                   out, out_ld, dtype):
        self.check(self.L.cuca_hip_glu_ragged(self.ptr, gate, gate_ld, up, up_ld, offsets,
                                              n_experts, max_rows, ff, act, clamp, out, out_ld,
                                              dtype))

    def rope(self, q, q_ld, k, k_ld, rows, nq, nk, head_dim, n_dims, kind, cos, sin, table_rows,
             positions, q_norm_w, k_norm_w, eps, dtype):
        self.check(self.L.cuca_hip_rope(self.ptr, q, q_ld, k, k_ld, rows, nq, nk, head_dim, n_dims,
                                        kind, cos, sin, table_rows, positions, q_norm_w, k_norm_w,
                                        eps, dtype))

    def rope_full(self, q, q_ld, k, k_ld, rows, nq, nk, head_dim, n_dims, kind, cos, sin, table_rows,
                  positions, q_norm_w, k_norm_w, eps, dtype):
        self.check(self.L.cuca_hip_rope_full(self.ptr, q, q_ld, k, k_ld, rows, nq, nk, head_dim, n_dims,
                                             kind, cos, sin, table_rows, positions, q_norm_w, k_norm_w,
                                             eps, dtype))

    def rope_store_kv_full(self, q, q_ld, k, k_ld, v, v_ld, rows, nq, nk, head_dim, n_dims, kind, cos,
                           sin, table_rows, positions, q_norm_w, k_norm_w, v_norm, eps, pool_k, pool_v,
                           n_blocks, slots, dtype):
        self.check(self.L.cuca_hip_rope_store_kv_full(self.ptr, q, q_ld, k, k_ld, v, v_ld, rows, nq, nk,
                                                      head_dim, n_dims, kind, cos, sin, table_rows,
                                                      positions, q_norm_w, k_norm_w, int(v_norm), eps,
                                                      pool_k, pool_v, n_blocks, slots, dtype))

    def paged_decode(self, q, pool_k, pool_v, n_blocks, tables, max_blocks, ranges, rows, n_head,
                     n_kv, head_dim, scale, workspace, workspace_bytes, out, dtype, q_ld=None):
        """q_ld: the row stride of q in elements (default: packed rows of
        n_head * head_dim)."""
        if q_ld is None:
            q_ld = n_head * head_dim
        self.check(self.L.cuca_hip_paged_decode(self.ptr, q, q_ld, pool_k, pool_v, n_blocks, tables,
                                                max_blocks, ranges, rows, n_head, n_kv, head_dim,
                                                scale, workspace, workspace_bytes, out, dtype))

    def paged_decode_noalloc(self, q, pool_k, pool_v, n_blocks, tables, max_blocks, ranges, rows,
                             n_head, n_kv, head_dim, scale, out, dtype, q_ld=None):
        """cuca_hip_paged_decode without a workspace: the partials go to the
        library's per-device scratch array (no allocation in the call)."""
        if q_ld is None:
            q_ld = n_head * head_dim
        self.check(self.L.cuca_hip_paged_decode_noalloc(self.ptr, q, q_ld, pool_k, pool_v, n_blocks,
                                                        tables, max_blocks, ranges, rows, n_head, n_kv,
                                                        head_dim, scale, out, dtype))

    def attend_rows(self, q, q_ld, pool_k, pool_v, n_blocks, table, max_blocks, ranges, rows, n_head,
                    n_kv, head_dim, scale, out, out_ld, dtype):
        self.check(self.L.cuca_hip_attend_rows(self.ptr, q, q_ld, pool_k, pool_v, n_blocks, table,
                                               max_blocks, ranges, rows, n_head, n_kv, head_dim, scale,
                                               out, out_ld, dtype))

    def attend_latent_rows(self, q, q_ld, pool, n_blocks, table, max_blocks, ranges, rows, n_head,
                           head_dim, v_width, scale, out, out_ld, dtype):
        self.check(self.L.cuca_hip_attend_latent_rows(self.ptr, q, q_ld, pool, n_blocks, table,
                                                      max_blocks, ranges, rows, n_head, head_dim,
                                                      v_width, scale, out, out_ld, dtype))

    def rope_store_kv(self, q, q_ld, k, k_ld, v, v_ld, rows, nq, nk, head_dim, n_dims, kind, cos,
                      sin, table_rows, positions, q_norm_w, k_norm_w, v_norm, eps, pool_k, pool_v,
                      n_blocks, slots, dtype):
        self.check(self.L.cuca_hip_rope_store_kv(self.ptr, q, q_ld, k, k_ld, v, v_ld, rows, nq, nk,
                                                 head_dim, n_dims, kind, cos, sin, table_rows,
                                                 positions, q_norm_w, k_norm_w, int(v_norm), eps,
                                                 pool_k, pool_v, n_blocks, slots, dtype))


    def qweight_pack(self, gguf, ggml_type, n, k, packed):
        self.check(self.L.cuca_hip_qweight_pack(self.ptr, gguf, ggml_type, n, k, packed))

    def qmm(self, w, ggml_type, n, k, x, ldx, m, rows, out, out_ld, dtype):
        self.check(self.L.cuca_hip_qmm(self.ptr, w, ggml_type, n, k, x, ldx, m, rows, out, out_ld,
                                       dtype))

    def qgemm(self, w, ggml_type, n, k, x, ldx, m, rows, ws, ws_bytes, out, out_ld, dtype):
        self.check(self.L.cuca_hip_qgemm(self.ptr, w, ggml_type, n, k, x, ldx, m, rows, ws, ws_bytes,
                                         out, out_ld, dtype))

    def qgemm_glu(self, gate, up, ggml_type, ff, k, x, ldx, m, act, clamp, ws, ws_bytes, out, out_ld,
                  dtype):
        self.check(self.L.cuca_hip_qgemm_glu(self.ptr, gate, up, ggml_type, ff, k, x, ldx, m, act,
                                             clamp, ws, ws_bytes, out, out_ld, dtype))

    def qweight_dequant(self, packed, ggml_type, n, k, w16):
        self.check(self.L.cuca_hip_qweight_dequant(self.ptr, packed, ggml_type, n, k, w16))

    def gemm_w16(self, w16, n, k, x, ldx, m, rows, ws, ws_bytes, out, out_ld, dtype):
        self.check(self.L.cuca_hip_gemm_w16(self.ptr, w16, n, k, x, ldx, m, rows, ws, ws_bytes, out,
                                            out_ld, dtype))

    def gemm_w16_glu(self, w16, ff, k, x, ldx, m, act, clamp, ws, ws_bytes, out, out_ld, dtype):
        self.check(self.L.cuca_hip_gemm_w16_glu(self.ptr, w16, ff, k, x, ldx, m, act, clamp, ws,
                                                ws_bytes, out, out_ld, dtype))

    def qmm_rope_store_kv(self, w, ggml_type, k, x, ldx, m, nq, nk, head_dim, n_dims, kind, cos, sin,
                          table_rows, positions, q_out, q_ld, pool_k, pool_v, n_blocks, slots, dtype):
        self.check(self.L.cuca_hip_qmm_rope_store_kv(self.ptr, w, ggml_type, k, x, ldx, m, nq, nk, head_dim,
                                                     n_dims, kind, cos, sin, table_rows, positions, q_out,
                                                     q_ld, pool_k, pool_v, n_blocks, slots, dtype))

    def qmm_glu(self, gate, up, ggml_type, ff, k, x, ldx, m, act, clamp, out, out_ld, dtype):
        self.check(self.L.cuca_hip_qmm_glu(self.ptr, gate, up, ggml_type, ff, k, x, ldx, m, act,
                                           clamp, out, out_ld, dtype))

    # the residual add + RMSNorm fused into the projection that reads it
    def add_rmsnorm_qmm(self, x, branch, norm_w, eps, residual_scale, x_out, h_out, w, ggml_type, n, k, m,
                        rows, out, out_ld, dtype):
        self.check(self.L.cuca_hip_add_rmsnorm_qmm(self.ptr, x, branch, norm_w, eps, residual_scale, x_out,
                                                   h_out, w, ggml_type, n, k, m, rows, out, out_ld, dtype))

    def add_rmsnorm_qmm_glu(self, x, branch, norm_w, eps, residual_scale, x_out, h_out, gate, up, ggml_type,
                            ff, k, m, act, clamp, out, out_ld, dtype):
        self.check(self.L.cuca_hip_add_rmsnorm_qmm_glu(self.ptr, x, branch, norm_w, eps, residual_scale, x_out,
                                                       h_out, gate, up, ggml_type, ff, k, m, act, clamp, out,
                                                       out_ld, dtype))

    def add_rmsnorm_qmm_rope_store_kv(self, x, branch, norm_w, eps, residual_scale, x_out, h_out, w, ggml_type,
                                      k, m, nq, nk, head_dim, n_dims, kind, cos, sin, table_rows, positions,
                                      q_out, q_ld, pool_k, pool_v, n_blocks, slots, dtype):
        self.check(self.L.cuca_hip_add_rmsnorm_qmm_rope_store_kv(
            self.ptr, x, branch, norm_w, eps, residual_scale, x_out, h_out, w, ggml_type, k, m, nq, nk, head_dim,
            n_dims, kind, cos, sin, table_rows, positions, q_out, q_ld, pool_k, pool_v, n_blocks, slots, dtype))


    def moe_up(self, gate, up, estride, ggml_type, ff, n_embd, n_experts, x, ldx, n_tokens, offsets,
               pair_token, max_pairs, act, clamp, hidden, hidden_ld, dtype):
        self.check(self.L.cuca_hip_moe_up(self.ptr, gate, up, estride, ggml_type, ff, n_embd, n_experts,
                                          x, ldx, n_tokens, offsets, pair_token, max_pairs, act, clamp,
                                          hidden, hidden_ld, dtype))

    def moe_down(self, down, estride, ggml_type, n_embd, ff, n_experts, hidden, hidden_ld, offsets,
                 pair_weight, max_pairs, scratch, scratch_ld, dtype):
        self.check(self.L.cuca_hip_moe_down(self.ptr, down, estride, ggml_type, n_embd, ff, n_experts,
                                            hidden, hidden_ld, offsets, pair_weight, max_pairs, scratch,
                                            scratch_ld, dtype))

    def moe_up_qgemm(self, gate, up, estride, ggml_type, ff, n_embd, n_experts, x, ldx, n_tokens, offsets,
                     pair_token, max_pairs, act, clamp, ws, ws_bytes, hidden, hidden_ld, dtype):
        self.check(self.L.cuca_hip_moe_up_qgemm(self.ptr, gate, up, estride, ggml_type, ff, n_embd, n_experts,
                                                x, ldx, n_tokens, offsets, pair_token, max_pairs, act, clamp,
                                                ws, ws_bytes, hidden, hidden_ld, dtype))

    def moe_down_qgemm(self, down, estride, ggml_type, n_embd, ff, n_experts, hidden, hidden_ld, offsets,
                       pair_weight, max_pairs, ws, ws_bytes, scratch, scratch_ld, dtype):
        self.check(self.L.cuca_hip_moe_down_qgemm(self.ptr, down, estride, ggml_type, n_embd, ff, n_experts,
                                                  hidden, hidden_ld, offsets, pair_weight, max_pairs, ws,
                                                  ws_bytes, scratch, scratch_ld, dtype))

    def moe_sum(self, scratch, scratch_ld, max_pairs, token_pairs, n_used, n_tokens, n_embd, out,
                out_ld, dtype):
        self.check(self.L.cuca_hip_moe_sum(self.ptr, scratch, scratch_ld, max_pairs, token_pairs,
                                           n_used, n_tokens, n_embd, out, out_ld, dtype))


    def q8_acts(self, x, ldx, m, k, dtype, quants, scales):
        self.check(self.L.cuca_hip_q8_acts(self.ptr, x, ldx, m, k, dtype, quants, scales))

    def qmv(self, w, ggml_type, n, k, quants, scales, m, rows, out, out_ld, dtype):
        self.check(self.L.cuca_hip_qmv(self.ptr, w, ggml_type, n, k, quants, scales, m, rows, out, out_ld,
                                       dtype))

    def qmv_glu(self, gate, up, ggml_type, ff, k, quants, scales, m, act, clamp, out, out_ld, dtype):
        self.check(self.L.cuca_hip_qmv_glu(self.ptr, gate, up, ggml_type, ff, k, quants, scales, m, act,
                                           clamp, out, out_ld, dtype))

    def lm_head(self, w, ggml_type, vocab, n_embd, x, ldx, m, rows, logit_scale, logit_mult, softcap,
                logits, logits_ld, dtype):
        self.check(self.L.cuca_hip_lm_head(self.ptr, w, ggml_type, vocab, n_embd, x, ldx, m, rows,
                                           logit_scale, logit_mult, softcap, logits, logits_ld, dtype))

    def lm_head_indexed(self, w, ggml_type, vocab, n_embd, x, ldx, m, ids, n_ids, logit_scale, logit_mult,
                        softcap, ws, ws_bytes, logits, logits_ld, dtype):
        self.check(self.L.cuca_hip_lm_head_indexed(self.ptr, w, ggml_type, vocab, n_embd, x, ldx, m, ids,
                                                   n_ids, logit_scale, logit_mult, softcap, ws, ws_bytes,
                                                   logits, logits_ld, dtype))

    def argmax(self, logits, ld, rows, vocab, dtype, ids):
        self.check(self.L.cuca_hip_argmax(self.ptr, logits, ld, rows, vocab, dtype, ids))

    def top_k(self, logits, ld, rows, vocab, dtype, k, temperature, out_logits, out_ids, out_count):
        self.check(self.L.cuca_hip_top_k(self.ptr, logits, ld, rows, vocab, dtype, k, temperature,
                                         out_logits, out_ids, out_count))


class Graph:
    def __init__(self, ctx, ptr):
        self.ctx = ctx
        self.ptr = ptr

    def launch(self):
        self.ctx.check(self.ctx.L.cuca_hip_graph_launch(self.ctx.ptr, self.ptr))

    def destroy(self):
        if self.ptr:
            self.ctx.L.cuca_hip_graph_destroy(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


KV_BLOCK = 16          # positions per paged K/V block (paged.rs:45)
NO_BLOCK = 0xFFFFFFFF  # a released block's table entry (paged.rs:49)
NOALLOC_SCRATCH_BYTES = 64 << 20  # CUCA_NOALLOC_SCRATCH_BYTES


def qgemm_workspace(ggml_type, n, k, m, glu=False):
    """Bytes of workspace cuca_hip_qgemm / _qgemm_glu need (host)."""
    out = _sz(0)
    _check(lib().cuca_hip_qgemm_workspace(ggml_type, n, k, m, 1 if glu else 0, ctypes.byref(out)), None)
    return out.value


def moe_qgemm_workspace(ggml_type, k, n_experts, max_pairs):
    """Bytes of workspace cuca_hip_moe_up_qgemm / _down_qgemm need (host):
    k = n_embd for up, ff for down."""
    out = _sz(0)
    _check(lib().cuca_hip_moe_qgemm_workspace(ggml_type, k, n_experts, max_pairs, ctypes.byref(out)), None)
    return out.value


def gemm_w16_workspace(n, k, m, glu, dtype):
    """Bytes of workspace cuca_hip_gemm_w16 / _gemm_w16_glu need (host); n is
    the output width (rows, or ff for the GLU)."""
    out = _sz(0)
    _check(lib().cuca_hip_gemm_w16_workspace(n, k, m, 1 if glu else 0, dtype, ctypes.byref(out)), None)
    return out.value


def paged_decode_workspace(rows, n_head, head_dim, max_blocks):
    """Bytes of workspace cuca_hip_paged_decode needs (host)."""
    out = _sz(0)
    _check(lib().cuca_hip_paged_decode_workspace(rows, n_head, head_dim, max_blocks,
                                                 ctypes.byref(out)), None)
    return out.value


def lm_head_indexed_workspace(ggml_type, n_embd, n_ids):
    """Bytes of workspace cuca_hip_lm_head_indexed needs (host)."""
    b = _sz(0)
    _check(lib().cuca_hip_lm_head_indexed_workspace(ggml_type, n_embd, n_ids, ctypes.byref(b)))
    return b.value


def qweight_bytes(ggml_type, n, k):
    """Bytes of the packed layout of an [n, k] Q4_0 / Q8_0 weight (host)."""
    out = _sz(0)
    _check(lib().cuca_hip_qweight_bytes(ggml_type, n, k, ctypes.byref(out)), None)
    return out.value


def sample_candidates(logits, ids, top_p, fallback, rng_state):
    """cuca_hip_sample_candidates (host): one row's top-k candidates (best
    first) -> the drawn id; rng_state (a ctypes.c_uint64) advances."""
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    ii = np.ascontiguousarray(ids, dtype=np.uint32)
    out = _u32(0)
    _check(lib().cuca_hip_sample_candidates(lg.ctypes.data if lg.size else None,
                                            ii.ctypes.data if ii.size else None, lg.size, top_p,
                                            fallback, ctypes.byref(rng_state), ctypes.byref(out)), None)
    return out.value


def kv_slots(table, start, t, n_blocks):
    """Pool rows of cache indices start..start+t of a sequence with block
    table `table` (cuca_hip_kv_slots, host): int32[t], block * 16 + p % 16."""
    tab = np.ascontiguousarray(table, dtype=np.uint32)
    out = np.empty(t, np.int32)
    _check(lib().cuca_hip_kv_slots(tab.ctypes.data if tab.size else None, tab.size, start, t,
                                   n_blocks, out.ctypes.data), None)
    return out


def rope_tables(kind, n_dims, base, positions, freq_scale=1.0, yarn=None, attn_factor=1.0,
                factors=None):
    """RopeSpec::tables through cuca_hip_rope_tables (host): (cos, sin) f32
    [positions, n_dims/2].  yarn: None or (ext_factor, beta_fast, beta_slow,
    n_ctx_orig)."""
    ext, bf, bs, nco = yarn if yarn is not None else (0.0, 32.0, 1.0, 0)
    spec = RopeSpecC(kind, n_dims, base, freq_scale, ext, bf, bs, nco, attn_factor)
    half = n_dims // 2
    cos = np.empty((positions, half), np.float32)
    sin = np.empty((positions, half), np.float32)
    f = None if factors is None else np.ascontiguousarray(factors, dtype=np.float32)
    _check(lib().cuca_hip_rope_tables(ctypes.byref(spec), None if f is None else f.ctypes.data,
                                      positions, cos.ctypes.data, sin.ctypes.data), None)
    return cos, sin
