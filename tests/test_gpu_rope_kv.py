"""QK-norm + RoPE fused with the paged K/V store, on the GPU, against the
oracle's store_kv (cpu.rs:3028-3097 restated: rope, norm, store_rows into
[n_blocks, n_kv, 16, d] pools).

Bars: Q, and the pools' K and V rows, bit-exact with the oracle without a
norm (f32 and f16); with the QK-norm within 1e-5 of the rotated pair's
magnitude (2 f16 ulps plus that); V's weightless norm within 1e-5 relative
(2 f16 ulps).  Pool rows no call names stay as they were.  Several calls
(sequences) per launch, with scrambled block tables, runs that start and
end inside a block, configs A-E, the generic kernel (head_dim 80, partial
rotary), a bad slot and a bad position (reported, row left untouched) and
the full config C size on sampled rows.
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
    w = want.astype(np.float64)
    half = n_dims // 2
    a = np.arange(half) if kind == hip.ROPE_NEOX else 2 * np.arange(half)
    b = a + half if kind == hip.ROPE_NEOX else a + 1
    mag = np.zeros_like(w)
    m = np.hypot(w[..., a], w[..., b])
    mag[..., a], mag[..., b] = m, m
    return 1e-5 * mag


def make_calls(rng, lengths, n_blocks):
    """Sequences of the given row counts at random cache offsets, each with a
    scrambled block table over a shared pool: [(offset, start, rope_start, t,
    table)], the rows' slots and positions."""
    perm = rng.permutation(n_blocks)
    used = 0
    calls, slots, pos = [], [], []
    off = 0
    for t in lengths:
        start = int(rng.integers(0, 40))
        nb = (start + t + 15) // 16
        table = [int(b) for b in perm[used:used + nb]]
        used += nb
        rope_start = start + int(rng.integers(0, 3))
        calls.append((off, start, rope_start, t, table))
        slots.append(hip.kv_slots(table, start, t, n_blocks))
        pos.append(np.arange(rope_start, rope_start + t, dtype=np.int32))
        off += t
    assert used <= n_blocks
    return calls, np.concatenate(slots), np.concatenate(pos)


def run(ctx, q, k, v, cos, sin, kind, n_dims, pos, slots, n_blocks, qw=None, kw=None,
        v_norm=False, eps=1e-6, pool_init=None):
    rows, nk, d = k.shape
    pool = ops.KvPool(ctx, n_blocks, nk, d, q.dtype)
    if pool_init is not None:
        pool.k.upload(pool_init[0])
        pool.v.upload(pool_init[1])
    dq, dk, dv = ctx.array(q), ctx.array(k), ctx.array(v)
    pool.store_kv(dq, dk, dv, ctx.array(cos), ctx.array(sin), kind, n_dims, ctx.array(pos),
                  ctx.array(slots), q_norm_w=qw, k_norm_w=kw, v_norm=v_norm, eps=eps)
    # the k and v inputs are read, not written
    assert_bits_equal(dk.numpy(), k, "k input")
    assert_bits_equal(dv.numpy(), v, "v input")
    return dq.numpy(), pool.k.numpy(), pool.v.numpy()


@pytest.mark.parametrize("cfg_name,lengths,dtype", [
    ("A", [128], "f32"), ("B", [1, 1, 1, 1], "f32"), ("B", [32, 5], "f32"),
    ("C", [200, 17, 64], "f16"), ("D", [8], "f32"), ("D", [33, 31], "f16"),
    ("E", [64], "f32"), ("E", [40, 3], "f16")])
def test_configs(ctx, cfg_name, lengths, dtype):
    cfg = W.CONFIGS[cfg_name]
    rng = np.random.default_rng(cfg["seed"] + sum(lengths))
    d, kind, nq, nk = cfg["head_dim"], KIND[cfg["rope"]], cfg["nq"], cfg["nk"]
    n_blocks = 64
    calls, slots, pos = make_calls(rng, lengths, n_blocks)
    n = sum(lengths)
    q = rng.standard_normal((n, nq, d)).astype(NP[dtype])
    k = rng.standard_normal((n, nk, d)).astype(NP[dtype])
    v = rng.standard_normal((n, nk, d)).astype(NP[dtype])
    cos, sin = hip.rope_tables(kind, d, cfg["theta"], int(pos.max()) + 1)
    pk = np.zeros((n_blocks, nk, 16, d), NP[dtype])
    pv = np.zeros_like(pk)
    qn = cfg.get("qk_norm")
    qw = (1 + 0.02 * rng.standard_normal(d)).astype(np.float32) if qn else None
    kw = (1 + 0.02 * rng.standard_normal(d)).astype(np.float32) if qn else None
    gq, gk, gv = run(ctx, q, k, v, cos, sin, kind, d, pos, slots, n_blocks, qw, kw,
                     v_norm=bool(qn), eps=cfg["eps"])
    wq = O.store_kv(q, k, v, cos, sin, kind, d, calls, pk, pv, q_norm_w=qw, k_norm_w=kw,
                    v_norm=bool(qn), eps=cfg["eps"])
    if qn:
        assert_close(gq, wq, floor=pair_floor(wq, kind, d), what="q")
        assert_close(gk, pk, floor=pair_floor(pk, kind, d), what="pool k")
        assert_close(gv, pv, what="pool v")
    else:
        assert_bits_equal(gq, wq, "q")
        assert_bits_equal(gk, pk, "pool k")
        assert_bits_equal(gv, pv, "pool v")


@pytest.mark.parametrize("kind", [hip.ROPE_NEOX, hip.ROPE_NORM])
@pytest.mark.parametrize("dtype,d,n_dims", [("f32", 128, 64), ("f16", 128, 96), ("f32", 80, 80),
                                            ("f16", 80, 40), ("f32", 8, 6)])
def test_partial_rotary_and_generic_kernel(ctx, kind, dtype, d, n_dims):
    rng = np.random.default_rng(d + n_dims + kind)
    n_blocks = 16
    calls, slots, pos = make_calls(rng, [9, 20], n_blocks)
    q = rng.standard_normal((29, 3, d)).astype(NP[dtype])
    k = rng.standard_normal((29, 2, d)).astype(NP[dtype])
    v = rng.standard_normal((29, 2, d)).astype(NP[dtype])
    cos, sin = hip.rope_tables(kind, n_dims, 1e4, 80)
    pk = np.zeros((n_blocks, 2, 16, d), NP[dtype])
    pv = np.zeros_like(pk)
    gq, gk, gv = run(ctx, q, k, v, cos, sin, kind, n_dims, pos, slots, n_blocks)
    wq = O.store_kv(q, k, v, cos, sin, kind, n_dims, calls, pk, pv)
    assert_bits_equal(gq, wq, "q")
    assert_bits_equal(gk, pk, "pool k")
    assert_bits_equal(gv, pv, "pool v")
    # K norm only, V norm only
    kw = (1 + 0.02 * rng.standard_normal(d)).astype(np.float32)
    pk[:] = 0
    pv[:] = 0
    gq, gk, gv = run(ctx, q, k, v, cos, sin, kind, n_dims, pos, slots, n_blocks, kw=kw, v_norm=True)
    wq = O.store_kv(q, k, v, cos, sin, kind, n_dims, calls, pk, pv, k_norm_w=kw, v_norm=True)
    assert_bits_equal(gq, wq, "q (no norm)")
    assert_close(gk, pk, floor=pair_floor(pk, kind, n_dims), what="normed pool k")
    assert_close(gv, pv, what="normed pool v")


def test_rows_no_call_names_keep_their_contents(ctx):
    rng = np.random.default_rng(11)
    n_blocks, nk, d = 12, 2, 64
    calls, slots, pos = make_calls(rng, [5, 7], n_blocks)
    q = rng.standard_normal((12, 4, d)).astype(np.float32)
    k = rng.standard_normal((12, nk, d)).astype(np.float32)
    v = rng.standard_normal((12, nk, d)).astype(np.float32)
    cos, sin = hip.rope_tables(hip.ROPE_NEOX, d, 1e4, 64)
    pk = rng.standard_normal((n_blocks, nk, 16, d)).astype(np.float32)
    pv = rng.standard_normal((n_blocks, nk, 16, d)).astype(np.float32)
    init = (pk.copy(), pv.copy())
    gq, gk, gv = run(ctx, q, k, v, cos, sin, hip.ROPE_NEOX, d, pos, slots, n_blocks,
                     pool_init=init)
    O.store_kv(q, k, v, cos, sin, hip.ROPE_NEOX, d, calls, pk, pv)
    assert_bits_equal(gk, pk, "pool k")
    assert_bits_equal(gv, pv, "pool v")


def test_bad_slot_and_bad_position_are_reported_and_skipped(ctx):
    rng = np.random.default_rng(12)
    n_blocks, nk, d = 4, 1, 128
    q = rng.standard_normal((4, 2, d)).astype(np.float32)
    k = rng.standard_normal((4, nk, d)).astype(np.float32)
    v = rng.standard_normal((4, nk, d)).astype(np.float32)
    cos, sin = hip.rope_tables(hip.ROPE_NORM, d, 1e4, 16)
    pos = np.array([3, 4, 5, 6], np.int32)
    slots = np.array([0, 64, 2, -1], np.int32)   # 64 = 4 blocks * 16: outside
    pool = ops.KvPool(ctx, n_blocks, nk, d, np.float32)
    dq = ctx.array(q)
    pool.store_kv(dq, ctx.array(k), ctx.array(v), ctx.array(cos), ctx.array(sin), hip.ROPE_NORM,
                  d, ctx.array(pos), ctx.array(slots))
    with pytest.raises(hip.CucaError, match="K/V slot 64 outside the pool of 4 blocks"):
        ctx.check_device()
    got_q, pk, pv = dq.numpy(), pool.k.numpy(), pool.v.numpy()
    assert_bits_equal(got_q[[1, 3]], q[[1, 3]], "skipped rows")
    good = np.array([0, 2])
    assert_bits_equal(got_q[good], O.rope(q[good], cos, sin, pos[good], hip.ROPE_NORM))
    wk = O.rope(k[good], cos, sin, pos[good], hip.ROPE_NORM)
    # pk[0, :, [0, 2]] is [rows, nk, d] (separated advanced indices come first)
    assert_bits_equal(pk[0, :, [0, 2]], wk)
    assert_bits_equal(pv[0, :, [0, 2]], v[good])
    pk[0, :, [0, 2]] = 0
    pv[0, :, [0, 2]] = 0
    assert not pk.any() and not pv.any()
    # a bad position
    pool2 = ops.KvPool(ctx, n_blocks, nk, d, np.float32)
    pool2.store_kv(ctx.array(q), ctx.array(k), ctx.array(v), ctx.array(cos), ctx.array(sin),
                   hip.ROPE_NORM, d, ctx.array(np.array([3, 16, 5, 6], np.int32)),
                   ctx.array(np.array([0, 1, 2, 3], np.int32)))
    with pytest.raises(hip.CucaError, match="position 16 outside the rope table of 16 rows"):
        ctx.check_device()
    assert not pool2.k.numpy()[0, :, 1].any()


def test_host_rejects_bad_arguments(ctx):
    pool = ops.KvPool(ctx, 2, 1, 16, np.float32)
    q = ctx.array(np.zeros((2, 1, 16), np.float32))
    kv = ctx.array(np.zeros((2, 1, 16), np.float32))
    cos, sin = (ctx.array(t) for t in hip.rope_tables(hip.ROPE_NEOX, 16, 1e4, 4))
    pos = ctx.array(np.zeros(2, np.int32))
    slots = ctx.array(np.zeros(2, np.int32))
    with pytest.raises(hip.CucaError, match="v row stride"):
        ctx.rope_store_kv(q.ptr, 16, kv.ptr, 16, kv.ptr, 8, 2, 1, 1, 16, 16, hip.ROPE_NEOX, cos.ptr,
                          sin.ptr, 4, pos.ptr, None, None, 0, 1e-6, pool.k.ptr, pool.v.ptr, 2,
                          slots.ptr, hip.F32)
    with pytest.raises(hip.CucaError, match="bad pool size"):
        ctx.rope_store_kv(q.ptr, 16, kv.ptr, 16, kv.ptr, 16, 2, 1, 1, 16, 16, hip.ROPE_NEOX,
                          cos.ptr, sin.ptr, 4, pos.ptr, None, None, 0, 1e-6, pool.k.ptr,
                          pool.v.ptr, 0, slots.ptr, hip.F32)
    with pytest.raises(hip.CucaError, match="null slots"):
        ctx.rope_store_kv(q.ptr, 16, kv.ptr, 16, kv.ptr, 16, 2, 1, 1, 16, 16, hip.ROPE_NEOX,
                          cos.ptr, sin.ptr, 4, pos.ptr, None, None, 0, 1e-6, pool.k.ptr,
                          pool.v.ptr, 2, None, hip.F32)
    with pytest.raises(hip.CucaError, match="row shape mismatch"):
        pool.store_kv(q, ctx.array(np.zeros((2, 2, 16), np.float32)), kv, cos, sin,
                      hip.ROPE_NEOX, 16, pos, slots)


def test_full_size_config_c_sampled_rows(ctx):
    torch = pytest.importorskip("torch")
    cfg = W.CONFIGS["C"]
    n, nq, nk, d = 16384, cfg["nq"], cfg["nk"], cfg["head_dim"]
    n_blocks = n // 16 + 8
    gen = torch.Generator(device="cuda").manual_seed(4)
    q = torch.randn((n, nq, d), device="cuda", generator=gen).to(torch.float16)
    k = torch.randn((n, nk, d), device="cuda", generator=gen).to(torch.float16)
    v = torch.randn((n, nk, d), device="cuda", generator=gen).to(torch.float16)
    q0 = q.clone()
    pk = torch.zeros((n_blocks, nk, 16, d), dtype=torch.float16, device="cuda")
    pv = torch.zeros_like(pk)
    table = np.random.default_rng(4).permutation(n_blocks)[: n // 16].astype(np.uint32)
    slots = hip.kv_slots(table, 0, n, n_blocks)
    cos, sin = hip.rope_tables(hip.ROPE_NORM, d, cfg["theta"], n)
    dcos, dsin = torch.from_numpy(cos).cuda(), torch.from_numpy(sin).cuda()
    pos = torch.arange(n, dtype=torch.int32, device="cuda")
    dslots = torch.from_numpy(slots).cuda()
    torch.cuda.synchronize()
    ctx.rope_store_kv(q.data_ptr(), nq * d, k.data_ptr(), nk * d, v.data_ptr(), nk * d, n, nq, nk,
                      d, d, hip.ROPE_NORM, dcos.data_ptr(), dsin.data_ptr(), n, pos.data_ptr(),
                      None, None, 0, 1e-5, pk.data_ptr(), pv.data_ptr(), n_blocks,
                      dslots.data_ptr(), hip.F16)
    ctx.sync()
    ctx.check_device()
    s = np.unique(np.concatenate([[0, 15, 16, n - 1], np.random.default_rng(5).integers(0, n, 60)]))
    st = torch.from_numpy(s).cuda()
    wq = O.rope(q0[st].cpu().numpy(), cos, sin, s.astype(np.int32), hip.ROPE_NORM)
    wk = O.rope(k[st].cpu().numpy(), cos, sin, s.astype(np.int32), hip.ROPE_NORM)
    assert_bits_equal(q[st].cpu().numpy(), wq, "q")
    b, r = torch.from_numpy(slots[s] // 16).cuda(), torch.from_numpy(slots[s] % 16).cuda()
    assert_bits_equal(pk[b, :, r].cpu().numpy(), wk, "pool k")
    assert_bits_equal(pv[b, :, r].cpu().numpy(), v[st].cpu().numpy(), "pool v")


@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("nq,nk,d,lengths", [(32, 32, 128, [17, 40]), (16, 16, 128, [1, 1, 1]),
                                             (32, 8, 128, [64])])
def test_full_width_qk_norm_store(ctx, dtype, nq, nk, d, lengths):
    """The K/V store with the full-width QK-norm (OLMo 2 / OLMoE, qk_norm_full,
    cpu.rs:2838-2843, 3042-3045): Q and the pool's K within the normed-RoPE
    bar of the oracle's store_kv(full=True); V's weightless per-head norm
    within 1e-5 / 2 f16 ulps."""
    rng = np.random.default_rng(nq + nk + sum(lengths))
    n_blocks = 32
    calls, slots, pos = make_calls(rng, lengths, n_blocks)
    n = sum(lengths)
    q = rng.standard_normal((n, nq, d)).astype(NP[dtype])
    k = (rng.standard_normal((n, nk, d)) * rng.uniform(0.5, 2, (1, nk, 1))).astype(NP[dtype])
    v = rng.standard_normal((n, nk, d)).astype(NP[dtype])
    qw = (1 + 0.02 * rng.standard_normal(nq * d)).astype(np.float32)
    kw = (1 + 0.02 * rng.standard_normal(nk * d)).astype(np.float32)
    cos, sin = hip.rope_tables(hip.ROPE_NEOX, d, 5e5, int(pos.max()) + 1)
    pool = ops.KvPool(ctx, n_blocks, nk, d, NP[dtype])
    dq, dk, dv = ctx.array(q), ctx.array(k), ctx.array(v)
    pool.store_kv(dq, dk, dv, ctx.array(cos), ctx.array(sin), hip.ROPE_NEOX, d, ctx.array(pos),
                  ctx.array(slots), q_norm_w=qw, k_norm_w=kw, v_norm=True, eps=1e-6, qk_norm_full=True)
    ctx.check_device()
    pk = np.zeros((n_blocks, nk, 16, d), NP[dtype])
    pv = np.zeros_like(pk)
    wq = O.store_kv(q, k, v, cos, sin, hip.ROPE_NEOX, d, calls, pk, pv, q_norm_w=qw, k_norm_w=kw,
                    v_norm=True, eps=1e-6, full=True)
    assert_close(dq.numpy(), wq, floor=pair_floor(wq, hip.ROPE_NEOX, d), what="full-norm q")
    assert_close(pool.k.numpy(), pk, floor=pair_floor(pk, hip.ROPE_NEOX, d), what="full-norm pool k")
    assert_close(pool.v.numpy(), pv, what="pool v")
