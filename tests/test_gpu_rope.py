"""RoPE (and the fused QK-norm) on the GPU against the oracle.

Bars: without a norm, bit-exact with the oracle's f32 rotation (the
reference's a*c - b*s with separately rounded products), in f32 and f16.
With the QK-norm: within 1e-5 of the rotated pair's magnitude (f32) or
2 f16 ulps plus that, since a*c - b*s cancels.  Covers configs A-E (NEOX and
NORM, head_dim 128 and 256, Q/K head counts, random and prefix positions),
partial rotary dims, Q and K inside a fused QKV row, the generic kernel
(head_dim 80, n_dims 6 of 8 = the cpu.rs:4336 case), bad positions and the
full config C size on sampled rows.  In-place RoPE of whole heads (two a
lane) runs the _h2w kernels, which must give the bits of the per-head _h2
kernels: pinned on calls that reach both.
"""
import numpy as np
import pytest

from cuca_amd import hip, ops
from cuca_amd import workloads as W
from helpers import assert_bits_equal, assert_close
from oracle import oracle as O

pytestmark = pytest.mark.gpu

NP = {"f32": np.float32, "f16": np.float16}
KIND = {"neox": hip.ROPE_NEOX, "norm": hip.ROPE_NORM}


def pair_floor(want, kind, n_dims):
    """1e-5 x the magnitude of each rotated pair, broadcast to its two values."""
    w = want.astype(np.float64)
    half = n_dims // 2
    a = np.arange(half) if kind == hip.ROPE_NEOX else 2 * np.arange(half)
    b = a + half if kind == hip.ROPE_NEOX else a + 1
    mag = np.zeros_like(w)
    m = np.hypot(w[..., a], w[..., b])
    mag[..., a], mag[..., b] = m, m
    return 1e-5 * mag


def run(ctx, q, k, cos, sin, pos, kind, n_dims, qw=None, kw=None, eps=1e-6):
    dq, dk = ctx.array(q), None if k is None else ctx.array(k)
    ops.rope_qk(dq, dk, ctx.array(cos), ctx.array(sin), kind, n_dims, ctx.array(pos),
                q_norm_w=qw, k_norm_w=kw, eps=eps)
    return dq.numpy(), None if k is None else dk.numpy()


@pytest.mark.parametrize("cfg_name,n,dtype", [("A", 128, "f32"), ("B", 1, "f32"), ("B", 32, "f32"),
                                              ("C", 300, "f16"), ("D", 8, "f32"), ("D", 64, "f16"),
                                              ("E", 64, "f32"), ("E", 40, "f16")])
def test_configs(ctx, cfg_name, n, dtype):
    cfg = W.CONFIGS[cfg_name]
    rng = np.random.default_rng(cfg["seed"] + n)
    d, kind = cfg["head_dim"], KIND[cfg["rope"]]
    q = rng.standard_normal((n, cfg["nq"], d)).astype(NP[dtype])
    k = rng.standard_normal((n, cfg["nk"], d)).astype(NP[dtype])
    pos = W.positions(cfg, n, rng)
    cos, sin = hip.rope_tables(kind, d, cfg["theta"], W.table_rows_needed(cfg, n))
    if cfg.get("qk_norm"):
        qw = (1 + 0.02 * rng.standard_normal(d)).astype(np.float32)
        kw = (1 + 0.02 * rng.standard_normal(d)).astype(np.float32)
        gq, gk = run(ctx, q, k, cos, sin, pos, kind, d, qw, kw, cfg["eps"])
        wq = O.rope(q, cos, sin, pos, kind, norm_w=qw, eps=cfg["eps"])
        wk = O.rope(k, cos, sin, pos, kind, norm_w=kw, eps=cfg["eps"])
        assert_close(gq, wq, floor=pair_floor(wq, kind, d), what="q")
        assert_close(gk, wk, floor=pair_floor(wk, kind, d), what="k")
    else:
        gq, gk = run(ctx, q, k, cos, sin, pos, kind, d)
        assert_bits_equal(gq, O.rope(q, cos, sin, pos, kind), "q")
        assert_bits_equal(gk, O.rope(k, cos, sin, pos, kind), "k")


@pytest.mark.parametrize("kind", [hip.ROPE_NEOX, hip.ROPE_NORM])
@pytest.mark.parametrize("dtype,d,n_dims", [("f32", 128, 64), ("f16", 128, 96), ("f32", 256, 128),
                                            ("f32", 80, 80), ("f16", 80, 40), ("f32", 128, 20),
                                            ("f32", 8, 6), ("f16", 64, 64)])
def test_partial_and_generic(ctx, kind, dtype, d, n_dims):
    rng = np.random.default_rng(d + n_dims)
    q = rng.standard_normal((13, 5, d)).astype(NP[dtype])
    k = rng.standard_normal((13, 2, d)).astype(NP[dtype])
    pos = rng.integers(0, 100, 13).astype(np.int32)
    cos, sin = hip.rope_tables(kind, n_dims, 1e4, 100)
    gq, gk = run(ctx, q, k, cos, sin, pos, kind, n_dims)
    assert_bits_equal(gq, O.rope(q, cos, sin, pos, kind, n_dims), "q")
    assert_bits_equal(gk, O.rope(k, cos, sin, pos, kind, n_dims), "k")
    qw = (1 + 0.02 * rng.standard_normal(d)).astype(np.float32)
    gq, _ = run(ctx, q, None, cos, sin, pos, kind, n_dims, qw=qw)
    wq = O.rope(q, cos, sin, pos, kind, n_dims, norm_w=qw)
    assert_close(gq, wq, floor=pair_floor(wq, kind, n_dims), what="normed q")


def test_reference_case_cpu_rs_4336(ctx):
    # heads 2, t 3, d 8, n_dims 6, values ((i*7)%13)-6, cos/sin(i*0.37)
    heads, t, d, n_dims = 2, 3, 8, 6
    values = np.array([((i * 7 % 13) - 6.0) for i in range(heads * t * d)], np.float32)
    x = values.reshape(heads, t, d).transpose(1, 0, 2).copy()
    half = n_dims // 2
    cos = np.cos(np.arange(t * half, dtype=np.float32) * np.float32(0.37)).reshape(t, half)
    sin = np.sin(np.arange(t * half, dtype=np.float32) * np.float32(0.37)).reshape(t, half)
    for kind in (hip.ROPE_NORM, hip.ROPE_NEOX):
        got, _ = run(ctx, x, None, cos.astype(np.float32), sin.astype(np.float32),
                     np.arange(t, dtype=np.int32), kind, n_dims)
        assert_bits_equal(got, O.rope(x, cos, sin, np.arange(t), kind, n_dims))


def test_q_and_k_inside_a_fused_qkv_row(ctx):
    rng = np.random.default_rng(9)
    n, nq, nk, d = 21, 32, 8, 128
    qkv = rng.standard_normal((n, (nq + 2 * nk) * d)).astype(np.float32)
    pos = np.arange(n, dtype=np.int32) + 5
    cos, sin = hip.rope_tables(hip.ROPE_NEOX, d, 1e6, 64)
    buf = ctx.array(qkv)
    ld = (nq + 2 * nk) * d
    dcos, dsin, dpos = ctx.array(cos), ctx.array(sin), ctx.array(pos)
    ctx.rope(buf.ptr, ld, buf.ptr + nq * d * 4, ld, n, nq, nk, d, d, hip.ROPE_NEOX, dcos.ptr,
             dsin.ptr, 64, dpos.ptr, None, None, 1e-6, hip.F32)
    got = buf.numpy()
    wq = O.rope(qkv[:, :nq * d].reshape(n, nq, d), cos, sin, pos, hip.ROPE_NEOX)
    wk = O.rope(qkv[:, nq * d:(nq + nk) * d].reshape(n, nk, d), cos, sin, pos, hip.ROPE_NEOX)
    assert_bits_equal(got[:, :nq * d].reshape(n, nq, d), wq)
    assert_bits_equal(got[:, nq * d:(nq + nk) * d].reshape(n, nk, d), wk)
    assert_bits_equal(got[:, (nq + nk) * d:], qkv[:, (nq + nk) * d:])   # V untouched


def test_bad_positions_are_reported_and_skipped(ctx):
    rng = np.random.default_rng(10)
    q = rng.standard_normal((4, 2, 128)).astype(np.float32)
    cos, sin = hip.rope_tables(hip.ROPE_NORM, 128, 1e4, 16)
    pos = np.array([3, 16, -1, 15], np.int32)
    dq = ctx.array(q)
    ops.apply_rope(dq, ctx.array(cos), ctx.array(sin), hip.ROPE_NORM, 128, ctx.array(pos))
    with pytest.raises(hip.CucaError, match="position 16 outside the rope table of 16 rows"):
        ctx.check_device()
    got = dq.numpy()
    assert_bits_equal(got[[1, 2]], q[[1, 2]])
    good = np.array([0, 3])
    assert_bits_equal(got[good], O.rope(q[good], cos, sin, pos[good], hip.ROPE_NORM))


def test_full_size_config_c_sampled_rows(ctx):
    torch = pytest.importorskip("torch")
    cfg = W.CONFIGS["C"]
    n, nq, nk, d = 16384, cfg["nq"], cfg["nk"], cfg["head_dim"]
    gen = torch.Generator(device="cuda").manual_seed(2)
    q = torch.randn((n, nq, d), device="cuda", generator=gen).to(torch.float16)
    k = torch.randn((n, nk, d), device="cuda", generator=gen).to(torch.float16)
    q0, k0 = q.clone(), k.clone()
    cos, sin = hip.rope_tables(hip.ROPE_NORM, d, cfg["theta"], n)
    dcos, dsin = torch.from_numpy(cos).cuda(), torch.from_numpy(sin).cuda()
    pos = torch.arange(n, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    ctx.rope(q.data_ptr(), nq * d, k.data_ptr(), nk * d, n, nq, nk, d, d, hip.ROPE_NORM,
             dcos.data_ptr(), dsin.data_ptr(), n, pos.data_ptr(), None, None, 1e-5, hip.F16)
    ctx.sync()
    ctx.check_device()
    s = np.unique(np.concatenate([[0, n - 1], np.random.default_rng(3).integers(0, n, 62)]))
    st = torch.from_numpy(s).cuda()
    wq = O.rope(q0[st].cpu().numpy(), cos, sin, s.astype(np.int32), hip.ROPE_NORM)
    wk = O.rope(k0[st].cpu().numpy(), cos, sin, s.astype(np.int32), hip.ROPE_NORM)
    assert_bits_equal(q[st].cpu().numpy(), wq)
    assert_bits_equal(k[st].cpu().numpy(), wk)


# ---------------------------------------------------------------------------
# full-width QK-norm (qk_norm_full: OLMo 2 / OLMoE, cpu.rs:2838-2843, 3042-3045)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("nq,nk,d,kind,n_dims,rows", [
    (32, 32, 128, hip.ROPE_NEOX, 128, 33),     # OLMo-2-7B
    (16, 16, 128, hip.ROPE_NEOX, 128, 200),    # OLMoE-1B-7B
    (32, 8, 128, hip.ROPE_NORM, 128, 5),       # GQA, interleaved
    (8, 2, 64, hip.ROPE_NEOX, 32, 17),         # partial rotary
    (40, 8, 128, hip.ROPE_NEOX, 128, 1)])      # decode row
def test_full_width_qk_norm(ctx, dtype, nq, nk, d, kind, n_dims, rows):
    rng = np.random.default_rng(nq + nk + d + rows)
    q = (rng.standard_normal((rows, nq, d)) * rng.uniform(0.5, 3, (1, nq, 1))).astype(NP[dtype])
    k = rng.standard_normal((rows, nk, d)).astype(NP[dtype])
    qw = (1 + 0.02 * rng.standard_normal(nq * d)).astype(np.float32)
    kw = (1 + 0.02 * rng.standard_normal(nk * d)).astype(np.float32)
    cos, sin = hip.rope_tables(kind, n_dims, 5e5, 4096)
    pos = rng.integers(0, 4096, rows).astype(np.int32)
    dq, dk = ctx.array(q), ctx.array(k)
    ops.rope_qk(dq, dk, ctx.array(cos), ctx.array(sin), kind, n_dims, ctx.array(pos), q_norm_w=qw,
                k_norm_w=kw, eps=1e-6, qk_norm_full=True)
    ctx.check_device()
    wq = O.rope(q, cos, sin, pos, kind, n_dims, norm_w=qw, eps=1e-6, full=True)
    wk = O.rope(k, cos, sin, pos, kind, n_dims, norm_w=kw, eps=1e-6, full=True)
    assert_close(dq.numpy(), wq, floor=pair_floor(wq, kind, n_dims), what="full-norm q")
    assert_close(dk.numpy(), wk, floor=pair_floor(wk, kind, n_dims), what="full-norm k")
    # only Q normalised (no K weights): K is rotated, not normalised
    dq, dk = ctx.array(q), ctx.array(k)
    ops.rope_qk(dq, dk, ctx.array(cos), ctx.array(sin), kind, n_dims, ctx.array(pos), q_norm_w=qw,
                eps=1e-6, qk_norm_full=True)
    assert_bits_equal(dk.numpy(), O.rope(k, cos, sin, pos, kind, n_dims), "unnormed k")


def test_full_width_qk_norm_inside_a_fused_qkv_row_and_bad_shapes(ctx):
    rng = np.random.default_rng(40)
    n, nq, nk, d = 9, 16, 16, 128
    qkv = rng.standard_normal((n, (nq + 2 * nk) * d)).astype(np.float32)
    qw = (1 + 0.02 * rng.standard_normal(nq * d)).astype(np.float32)
    kw = (1 + 0.02 * rng.standard_normal(nk * d)).astype(np.float32)
    pos = np.arange(n, dtype=np.int32)
    cos, sin = hip.rope_tables(hip.ROPE_NEOX, d, 1e4, 16)
    buf, dcos, dsin, dpos = ctx.array(qkv), ctx.array(cos), ctx.array(sin), ctx.array(pos)
    dqw, dkw = ctx.array(qw), ctx.array(kw)
    ld = (nq + 2 * nk) * d
    ctx.rope_full(buf.ptr, ld, buf.ptr + nq * d * 4, ld, n, nq, nk, d, d, hip.ROPE_NEOX, dcos.ptr, dsin.ptr,
                  16, dpos.ptr, dqw.ptr, dkw.ptr, 1e-6, hip.F32)
    got = buf.numpy()
    wq = O.rope(qkv[:, :nq * d].reshape(n, nq, d), cos, sin, pos, hip.ROPE_NEOX, norm_w=qw, full=True)
    wk = O.rope(qkv[:, nq * d:(nq + nk) * d].reshape(n, nk, d), cos, sin, pos, hip.ROPE_NEOX, norm_w=kw,
                full=True)
    assert_close(got[:, :nq * d].reshape(n, nq, d), wq, floor=pair_floor(wq, hip.ROPE_NEOX, d))
    assert_close(got[:, nq * d:(nq + nk) * d].reshape(n, nk, d), wk, floor=pair_floor(wk, hip.ROPE_NEOX, d))
    assert_bits_equal(got[:, (nq + nk) * d:], qkv[:, (nq + nk) * d:])   # V untouched
    with pytest.raises(hip.CucaError, match="full-width QK-norm needs"):
        q80 = ctx.array(np.zeros((2, 2, 80), np.float32))
        c80, s80 = hip.rope_tables(hip.ROPE_NEOX, 80, 1e4, 4)
        ops.rope_qk(q80, None, ctx.array(c80), ctx.array(s80), hip.ROPE_NEOX, 80,
                    ctx.array(np.zeros(2, np.int32)), q_norm_w=np.ones(160, np.float32),
                    qk_norm_full=True)


@pytest.mark.parametrize("dtype,kind,d,rows", [("f16", hip.ROPE_NEOX, 128, 200), ("f32", hip.ROPE_NEOX, 128, 96),
                                               ("f16", hip.ROPE_NORM, 128, 200), ("f32", hip.ROPE_NORM, 64, 96),
                                               ("f16", hip.ROPE_NEOX, 32, 64), ("f16", hip.ROPE_NEOX, 128, 8192),
                                               ("f32", hip.ROPE_NORM, 128, 4096)])
def test_whole_head_kernels_give_the_per_head_bits(ctx, dtype, kind, d, rows):
    """A Q-only QK-norm call (32 heads, nk 0) with a K norm weight given runs
    the whole-head kernel (_h2w: no per-value selects, one norm factor per
    lane pair); the same call without it runs the per-head kernel (_h2).
    Both normalise Q with the same weights, so the bits must agree, and both
    stay within the QK-norm bar of the oracle.  At 64 MiB of heads the calls
    take the nontemporal-load kernels (_nt_h2w / _nt_h2); head_dim 32 f16
    NEOX has two lanes a head, the smallest the whole-head form takes."""
    nq = 32
    rng = np.random.default_rng(rows + d)
    q = rng.standard_normal((rows, nq, d)).astype(NP[dtype])
    qw = (1 + 0.02 * rng.standard_normal(d)).astype(np.float32)
    kw = (1 + 0.02 * rng.standard_normal(d)).astype(np.float32)
    pos = rng.integers(0, 4 * rows, rows).astype(np.int32)
    cos, sin = hip.rope_tables(kind, d, 10000.0, 4 * rows)
    dcos, dsin, dpos, dqw, dkw = (ctx.array(a) for a in (cos, sin, pos, qw, kw))
    big = rows * nq * d * q.itemsize >= 48 << 20
    stem = f"cuca_rope_{dtype}_{'neox' if kind == hip.ROPE_NEOX else 'norm'}_qkn_{'nt_' if big else ''}h2"
    got = {}
    for kname, kptr in ((stem + "w", dkw.ptr), (stem, 0)):
        dq = ctx.array(q)
        ctx.profile_start(4)
        ctx.rope(dq.ptr, nq * d, 0, 0, rows, nq, 0, d, d, kind, dcos.ptr, dsin.ptr, 4 * rows, dpos.ptr, dqw.ptr,
                 kptr, 1e-6, hip.dtype_code(NP[dtype]))
        names = [k for k, _ in ctx.profile_stop()]
        assert names == [kname], names
        got[kname] = dq.numpy()
    assert_bits_equal(got[stem + "w"], got[stem], "whole-head q")
    sel = np.arange(0, rows, max(1, rows // 64))
    want = O.rope(q[sel], cos, sin, pos[sel], kind, norm_w=qw, eps=1e-6)
    assert_close(got[stem + "w"][sel], want, floor=pair_floor(want, kind, d), what="q")
