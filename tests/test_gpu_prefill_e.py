"""Config E prefill (Qwen3-30B-A3B layer, 8192 f16 tokens) at full size on
the GPU, against the oracle on sampled rows.

At this size the calls cross the streaming threshold (48 MiB of input), so
they run the nontemporal kernels that the smaller tests never reach.  Each
test names the kernel it means to cover and checks, from the C ABI's
per-kernel profile, that the call launched exactly that kernel:
  add_rmsnorm, H 2048: 2 x 8192 x 2048 f16 in = 64 MiB -> cuca_norm_f16_t256_nts
    (the streamlined prefill form: a branch, weights, x' written, rs 1)
  QK-norm RoPE, Q 32 + K 4 heads x 128: 72 MiB  -> cuca_rope_f16_neox_qkn_nt_h2w (two whole heads
    per lane)
  the same + the paged K/V store (V 4 heads): 80 MiB -> cuca_rope_f16_neox_qkn_kv_nt_h2
  the SwiGLU over the 65536 expert-grouped rows of width 768 (Zipf(1.1)
  routing, 8 of 128 experts per token) -> cuca_glu_f16_silu_ragged
Bars as everywhere (cpu.rs:2840-2864 for Q, 3040-3055 for K, 3652 for the
norm): x' bit-exact; h, V and the activation within 2 f16 ulps of the
oracle's f16; the QK-normed rotation within 2 f16 ulps plus 1e-5 of the
rotated pair's magnitude.  The raw errors are in the session summary.
"""
import numpy as np
import pytest

from cuca_amd import hip
from cuca_amd import workloads as W
from helpers import assert_bits_equal, assert_close, pair_floor
from oracle import oracle as O

pytestmark = pytest.mark.gpu

CFG = W.CONFIGS["E"]
N = 8192


@pytest.fixture(scope="module")
def torch():
    return pytest.importorskip("torch")


def launched(ctx, call):
    """The kernels `call` launches, by name."""
    ctx.profile_start(16)
    call()
    return [k for k, _ in ctx.profile_stop()]


def sample(n, seed, extra=()):
    return np.unique(np.concatenate([[0, n - 1], np.array(extra, np.int64),
                                     np.random.default_rng(seed).integers(0, n, 60)])).astype(np.int64)


def test_norm_streaming_kernel_at_8192_tokens(ctx, torch):
    H, eps = CFG["hidden"], CFG["eps"]
    gen = torch.Generator(device="cuda").manual_seed(40)
    x = torch.randn((N, H), device="cuda", generator=gen).to(torch.float16)
    b = torch.randn((N, H), device="cuda", generator=gen).to(torch.float16)
    w = (1 + 0.02 * torch.randn(H, device="cuda", generator=gen)).float()
    xo, h = torch.empty_like(x), torch.empty_like(x)
    torch.cuda.synchronize()
    names = launched(ctx, lambda: ctx.add_rmsnorm(x.data_ptr(), b.data_ptr(), w.data_ptr(), None, eps,
                                                  eps, 1.0, N, H, xo.data_ptr(), h.data_ptr(), hip.F16))
    assert names == ["cuca_norm_f16_t256_nts"], names
    ctx.check_device()
    st = torch.from_numpy(sample(N, 41)).cuda()
    wx, wh = O.add_rmsnorm(x[st].cpu().numpy(), b[st].cpu().numpy(), w.cpu().numpy(), eps)
    assert_bits_equal(xo[st].cpu().numpy(), wx, "x'")
    assert_close(h[st].cpu().numpy(), wh, what="h")


def test_qk_norm_rope_streaming_kernel_at_8192_tokens(ctx, torch):
    nq, nk, d = CFG["nq"], CFG["nk"], CFG["head_dim"]
    gen = torch.Generator(device="cuda").manual_seed(42)
    q = torch.randn((N, nq, d), device="cuda", generator=gen).to(torch.float16)
    k = torch.randn((N, nk, d), device="cuda", generator=gen).to(torch.float16)
    qw = (1 + 0.02 * torch.randn(d, device="cuda", generator=gen)).float()
    kw = (1 + 0.02 * torch.randn(d, device="cuda", generator=gen)).float()
    q0, k0 = q.clone(), k.clone()
    cos, sin = hip.rope_tables(hip.ROPE_NEOX, d, CFG["theta"], N)
    dcos, dsin = torch.from_numpy(cos).cuda(), torch.from_numpy(sin).cuda()
    pos = torch.arange(N, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    names = launched(ctx, lambda: ctx.rope(q.data_ptr(), nq * d, k.data_ptr(), nk * d, N, nq, nk, d, d,
                                           hip.ROPE_NEOX, dcos.data_ptr(), dsin.data_ptr(), N,
                                           pos.data_ptr(), qw.data_ptr(), kw.data_ptr(), CFG["eps"],
                                           hip.F16))
    assert names == ["cuca_rope_f16_neox_qkn_nt_h2w"], names
    ctx.check_device()
    s = sample(N, 43)
    st = torch.from_numpy(s).cuda()
    for got, src, nw, what in ((q, q0, qw, "q"), (k, k0, kw, "k")):
        want = O.rope(src[st].cpu().numpy(), cos, sin, s.astype(np.int32), hip.ROPE_NEOX,
                      norm_w=nw.cpu().numpy(), eps=CFG["eps"])
        assert_close(got[st].cpu().numpy(), want, floor=pair_floor(want, True, d), what=what)


def test_qk_norm_rope_kv_store_streaming_kernel_at_8192_tokens(ctx, torch):
    nq, nk, d, eps = CFG["nq"], CFG["nk"], CFG["head_dim"], CFG["eps"]
    n_blocks = N // 16 + 8
    gen = torch.Generator(device="cuda").manual_seed(44)
    q = torch.randn((N, nq, d), device="cuda", generator=gen).to(torch.float16)
    k = torch.randn((N, nk, d), device="cuda", generator=gen).to(torch.float16)
    v = torch.randn((N, nk, d), device="cuda", generator=gen).to(torch.float16)
    qw = (1 + 0.02 * torch.randn(d, device="cuda", generator=gen)).float()
    kw = (1 + 0.02 * torch.randn(d, device="cuda", generator=gen)).float()
    q0 = q.clone()
    pk = torch.zeros((n_blocks, nk, 16, d), dtype=torch.float16, device="cuda")
    pv = torch.zeros_like(pk)
    table = np.random.default_rng(45).permutation(n_blocks)[: N // 16].astype(np.uint32)
    slots = hip.kv_slots(table, 0, N, n_blocks)
    cos, sin = hip.rope_tables(hip.ROPE_NEOX, d, CFG["theta"], N)
    dcos, dsin = torch.from_numpy(cos).cuda(), torch.from_numpy(sin).cuda()
    pos = torch.arange(N, dtype=torch.int32, device="cuda")
    dslots = torch.from_numpy(slots).cuda()
    torch.cuda.synchronize()
    names = launched(ctx, lambda: ctx.rope_store_kv(
        q.data_ptr(), nq * d, k.data_ptr(), nk * d, v.data_ptr(), nk * d, N, nq, nk, d, d,
        hip.ROPE_NEOX, dcos.data_ptr(), dsin.data_ptr(), N, pos.data_ptr(), qw.data_ptr(),
        kw.data_ptr(), 1, eps, pk.data_ptr(), pv.data_ptr(), n_blocks, dslots.data_ptr(), hip.F16))
    assert names == ["cuca_rope_f16_neox_qkn_kv_nt_h2"], names
    ctx.check_device()
    s = sample(N, 46, extra=(15, 16))
    st = torch.from_numpy(s).cuda()
    p = s.astype(np.int32)
    wq = O.rope(q0[st].cpu().numpy(), cos, sin, p, hip.ROPE_NEOX, norm_w=qw.cpu().numpy(), eps=eps)
    wk = O.rope(k[st].cpu().numpy(), cos, sin, p, hip.ROPE_NEOX, norm_w=kw.cpu().numpy(), eps=eps)
    _, wv = O.add_rmsnorm(v[st].cpu().numpy().reshape(-1, d), None, None, eps, write_x=False)
    assert_close(q[st].cpu().numpy(), wq, floor=pair_floor(wq, True, d), what="q")
    b, r = torch.from_numpy(slots[s] // 16).cuda(), torch.from_numpy(slots[s] % 16).cuda()
    gk = pk[b, :, r].cpu().numpy()
    assert_close(gk, wk, floor=pair_floor(wk, True, d), what="pool k")
    assert_close(pv[b, :, r].cpu().numpy(), wv.reshape(-1, nk, d), what="pool v")


def test_ragged_swiglu_at_8192_tokens(ctx, torch):
    F = CFG["ff"]
    n_exp, top = CFG["moe"]
    offsets, _ = W.zipf_expert_rows(np.random.default_rng(CFG["seed"]), N, n_exp, top)
    rows = int(offsets[-1])
    assert rows == N * top
    gen = torch.Generator(device="cuda").manual_seed(47)
    g = torch.randn((rows, F), device="cuda", generator=gen).to(torch.float16)
    u = torch.randn((rows, F), device="cuda", generator=gen).to(torch.float16)
    out = torch.full((rows + 5, F), float("nan"), device="cuda", dtype=torch.float16)
    doff = torch.from_numpy(offsets).cuda()
    torch.cuda.synchronize()
    names = launched(ctx, lambda: ctx.glu_ragged(g.data_ptr(), F, u.data_ptr(), F, doff.data_ptr(), n_exp,
                                                 rows + 5, F, hip.ACT_SILU, 0.0, out.data_ptr(), F,
                                                 hip.F16))
    assert names == ["cuca_glu_f16_silu_ragged"], names
    ctx.check_device()
    # the first and last row of every fifth expert, and random rows
    ends = np.concatenate([offsets[:-1][::5], offsets[1:][::5] - 1])
    s = np.unique(np.concatenate([sample(rows, 48), ends[(ends >= 0) & (ends < rows)]]))
    st = torch.from_numpy(s).cuda()
    want = O.glu(g[st].cpu().numpy(), u[st].cpu().numpy(), O.SILU)
    assert_close(out[st].cpu().numpy(), want, what="swiglu")
    # rows past the routed count are left alone
    assert torch.isnan(out[rows:]).all()
