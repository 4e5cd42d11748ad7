"""Fused residual add + RMSNorm on the GPU against the oracle.

Bars: x' (the residual sum) bit-exact; h within 1e-5 relative (f32) or
2 f16 ulps of the oracle's f16 output.  With the Gemma sandwich, x' = x +
rms(branch) cancels where x ~ -rms(branch), so x' carries a floor of 1e-5 of
the normalized branch term and h that floor divided by its row's rms.  Covers the hidden sizes of configs
A-E (1024, 4096, 3584, 2048), the QK-norm row width 128, short rows
(several rows per wave), the Gemma sandwich, the residual scale, the
weightless norm, in-place x' = x, empty and ragged row counts, the generic
kernel (hidden not a multiple of the chunk, rows wider than the register
kernel, misaligned buffers), the full config C size on sampled rows and
the streamlined prefill kernels (calls of 48 MiB or more in the plain form).
"""
import numpy as np
import pytest

from cuca_amd import hip, ops
from helpers import assert_bits_equal, assert_close
from oracle import oracle as O

pytestmark = pytest.mark.gpu

NP = {"f32": np.float32, "f16": np.float16}


def run(ctx, x, b, w, eps, wp=None, post_eps=None, rs=1.0, in_place=False):
    dx = ctx.array(x)
    db = None if b is None else ctx.array(b)
    xo = dx if in_place else None
    x_out, h = ops.add_rms(dx, db, w, eps, w_post=wp, post_eps=post_eps, residual_scale=rs,
                           x_out=xo)
    return x_out.numpy(), h.numpy()


def sandwich_floors(xo_want, b, wp, w, post_eps, eps):
    """x' = x + rms(b, wp) cancels where x ~ -rms(b, wp): allow 1e-5 of the
    normalized branch term in x', and that error carried through h = x'/m*w."""
    b64 = b.astype(np.float64)
    bp = np.abs(b64 / np.sqrt((b64 ** 2).mean(-1, keepdims=True) + post_eps) * wp)
    fx = 1e-5 * bp
    x64 = xo_want.astype(np.float64)
    m = np.sqrt((x64 ** 2).mean(-1, keepdims=True) + eps)
    fh = fx / m * (1.0 if w is None else np.abs(w.astype(np.float64)))
    return fx, fh


def data(rows, hidden, dtype, seed, std=1.0):
    rng = np.random.default_rng(seed)
    x = (std * rng.standard_normal((rows, hidden))).astype(NP[dtype])
    b = (std * rng.standard_normal((rows, hidden))).astype(NP[dtype])
    w = (1 + 0.02 * rng.standard_normal(hidden)).astype(np.float32)
    return x, b, w


@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("hidden,eps,rows", [(1024, 1e-6, 128), (4096, 1e-5, 32), (4096, 1e-5, 1),
                                             (3584, 1e-6, 9), (2048, 1e-6, 64), (128, 1e-6, 77),
                                             (64, 1e-5, 5), (8192, 1e-5, 3), (32, 1e-5, 33)])
def test_add_rmsnorm_matches_oracle(ctx, dtype, hidden, eps, rows):
    x, b, w = data(rows, hidden, dtype, hidden + rows)
    xo, h = run(ctx, x, b, w, eps)
    wx, wh = O.add_rmsnorm(x, b, w, eps)
    assert_bits_equal(xo, wx, "x'")
    assert_close(h, wh, what="h")


@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_gemma_sandwich_residual_scale_and_weightless(ctx, dtype):
    x, b, w = data(8, 3584, dtype, 3, std=2.0)
    wp = (1 + 0.02 * np.random.default_rng(4).standard_normal(3584)).astype(np.float32)
    xo, h = run(ctx, x, b, w, 1e-6, wp=wp, post_eps=1e-5)
    wx, wh = O.add_rmsnorm(x, b, w, 1e-6, w_post=wp, post_eps=1e-5)
    # the branch's own norm sums in another order: x' is within tolerance, not exact
    fx, fh = sandwich_floors(wx, b, wp, w, 1e-5, 1e-6)
    assert_close(xo, wx, floor=fx, what="sandwich x'")
    assert_close(h, wh, floor=fh, what="sandwich h")
    xo, h = run(ctx, x, b, None, 1e-6, rs=0.22)
    wx, wh = O.add_rmsnorm(x, b, None, 1e-6, residual_scale=0.22)
    assert_bits_equal(xo, wx, "scaled x'")
    assert_close(h, wh, what="weightless h")


@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_plain_rms_and_in_place(ctx, dtype):
    x, b, w = data(17, 2048, dtype, 5)
    got = ops.rms(ctx.array(x), w, 1e-6).numpy()
    _, want = O.add_rmsnorm(x, None, w, 1e-6, write_x=False)
    assert_close(got, want, what="rms")
    xo, h = run(ctx, x, b, w, 1e-6, in_place=True)
    wx, wh = O.add_rmsnorm(x, b, w, 1e-6)
    assert_bits_equal(xo, wx, "in-place x'")
    assert_close(h, wh, what="in-place h")


def test_zero_rows_is_a_no_op(ctx):
    x = ctx.empty((0, 1024), np.float32)
    ops.add_rms(x, x, None, 1e-6)


@pytest.mark.parametrize("dtype,hidden", [("f32", 1001), ("f16", 1004), ("f16", 20000),
                                          ("f32", 9000), ("f32", 3)])
def test_generic_kernel(ctx, dtype, hidden):
    x, b, w = data(6, hidden, dtype, hidden)
    wp = np.linspace(0.5, 1.5, hidden).astype(np.float32)
    xo, h = run(ctx, x, b, w, 1e-5, wp=wp, post_eps=1e-6)
    wx, wh = O.add_rmsnorm(x, b, w, 1e-5, w_post=wp, post_eps=1e-6)
    fx, fh = sandwich_floors(wx, b, wp, w, 1e-6, 1e-5)
    assert_close(xo, wx, floor=fx, what="generic x'")
    assert_close(h, wh, floor=fh, what="generic h")


def test_misaligned_buffers_take_the_generic_kernel(ctx):
    x, b, w = data(5, 1024, "f32", 11)
    buf = ctx.array(np.concatenate([np.zeros(1, np.float32), x.reshape(-1)]))
    dx = buf.view(1, x.shape)   # 4 bytes past a 16-byte boundary
    xo, h = ops.add_rms(dx, ctx.array(b), w, 1e-6)
    wx, wh = O.add_rmsnorm(x, b, w, 1e-6)
    assert_bits_equal(xo.numpy(), wx)
    assert_close(h.numpy(), wh)


def test_full_size_config_c_sampled_rows(ctx):
    torch = pytest.importorskip("torch")
    n, hidden = 16384, 4096
    gen = torch.Generator(device="cuda").manual_seed(2)
    x = torch.randn((n, hidden), device="cuda", generator=gen).to(torch.float16)
    b = torch.randn((n, hidden), device="cuda", generator=gen).to(torch.float16)
    w = (1 + 0.02 * torch.randn(hidden, device="cuda", generator=gen)).float()
    xo = torch.empty_like(x)
    h = torch.empty_like(x)
    torch.cuda.synchronize()
    ctx.add_rmsnorm(x.data_ptr(), b.data_ptr(), w.data_ptr(), None, 1e-5, 1e-5, 1.0, n, hidden,
                    xo.data_ptr(), h.data_ptr(), 1)
    ctx.sync()
    sample = torch.from_numpy(np.unique(np.concatenate(
        [[0, n - 1], np.random.default_rng(1).integers(0, n, 126)]))).cuda()
    xs, bs = x[sample].cpu().numpy(), b[sample].cpu().numpy()
    wx, wh = O.add_rmsnorm(xs, bs, w.cpu().numpy(), 1e-5)
    assert_bits_equal(xo[sample].cpu().numpy(), wx)
    assert_close(h[sample].cpu().numpy(), wh)


def test_group_sum_matches_shfl_butterfly(ctx):
    """The kernels' wave reductions (DPP, ds_swizzle and permlane partners)
    give the bits of the __shfl_xor butterfly (partner i ^ off, off = g/2
    down to 1) for every group size, and both equal that butterfly in numpy
    f32: values spread over 2^-40..2^40 so the order of the additions shows,
    with denormals, signed zeros and overflow to infinity."""
    rng = np.random.default_rng(3)
    n = 1 << 16
    x = (rng.standard_normal(n) * np.exp2(rng.integers(-40, 40, n))).astype(np.float32)
    x[0:4] = [0.0, -0.0, 1e-45, -1e-45]
    x[64:66] = [3.4e38, 3.4e38]           # a group that overflows to +inf
    x[128] = -np.inf
    dx = ctx.array(x)
    out = ctx.empty((12, n), np.float32)
    ctx.selftest_group_sum(dx.ptr, n, out.ptr)
    o = out.numpy()
    with np.errstate(over="ignore"):
        for gi, g in enumerate((2, 4, 8, 16, 32, 64)):
            want = x.copy()
            off = g // 2
            while off >= 1:
                want = (want + want[np.arange(n) ^ off]).astype(np.float32)
                off //= 2
            assert_bits_equal(o[2 * gi + 1], want, f"shfl butterfly, groups of {g}")
            assert_bits_equal(o[2 * gi], want, f"group_sum, groups of {g}")
    with pytest.raises(hip.CucaError, match="multiple of 256"):
        ctx.selftest_group_sum(dx.ptr, 100, out.ptr)


def launched(ctx, call):
    ctx.profile_start(16)
    call()
    return [k for k, _ in ctx.profile_stop()]


@pytest.mark.parametrize("dtype,hidden,rows,kernel", [
    ("f16", 2048, 6145, "cuca_norm_f16_t256_nts"), ("f32", 1024, 6145, "cuca_norm_f32_t256_nts"),
    ("f16", 4096, 3073, "cuca_norm_f16_t512_nts"), ("f32", 2048, 3073, "cuca_norm_f32_t512_nts"),
    ("f16", 8192, 1537, "cuca_norm_f16_t1024_nts"), ("f32", 4096, 1537, "cuca_norm_f32_t1024_nts")])
def test_streamlined_prefill_kernels(ctx, dtype, hidden, rows, kernel):
    """Calls of 48 MiB or more in the plain residual form (a branch, weights,
    x' written, rs 1) take the streamlined kernels: the kernel named, x'
    bit-exact, h against the oracle and bit-identical to the small-call
    kernel's h on the same rows; an odd row count leaves the last block of
    two 256-thread rows half empty.  Another residual scale stays on the
    general streaming kernel."""
    torch = pytest.importorskip("torch")
    tdt = torch.float16 if dtype == "f16" else torch.float32
    code = hip.F16 if dtype == "f16" else hip.F32
    gen = torch.Generator(device="cuda").manual_seed(hidden + rows)
    x = torch.randn((rows, hidden), device="cuda", generator=gen).to(tdt)
    b = torch.randn((rows, hidden), device="cuda", generator=gen).to(tdt)
    w = (1 + 0.02 * torch.randn(hidden, device="cuda", generator=gen)).float()
    xo, h = torch.empty_like(x), torch.empty_like(x)
    torch.cuda.synchronize()
    names = launched(ctx, lambda: ctx.add_rmsnorm(x.data_ptr(), b.data_ptr(), w.data_ptr(), None, 1e-5,
                                                  1e-5, 1.0, rows, hidden, xo.data_ptr(), h.data_ptr(), code))
    assert names == [kernel], names
    ctx.check_device()
    # the small-call kernel on the first and last 33 rows
    for lo in (0, rows - 33):
        so, sh = torch.empty((33, hidden), dtype=tdt, device="cuda"), torch.empty((33, hidden), dtype=tdt,
                                                                                  device="cuda")
        ctx.add_rmsnorm(x[lo].data_ptr(), b[lo].data_ptr(), w.data_ptr(), None, 1e-5, 1e-5, 1.0, 33, hidden,
                        so.data_ptr(), sh.data_ptr(), code)
        ctx.sync()
        assert_bits_equal(xo[lo:lo + 33].cpu().numpy(), so.cpu().numpy(), "x' vs small call")
        assert_bits_equal(h[lo:lo + 33].cpu().numpy(), sh.cpu().numpy(), "h vs small call")
    sample = torch.from_numpy(np.unique(np.concatenate(
        [[0, 1, rows - 2, rows - 1], np.random.default_rng(rows).integers(0, rows, 60)]))).cuda()
    wx, wh = O.add_rmsnorm(x[sample].cpu().numpy(), b[sample].cpu().numpy(), w.cpu().numpy(), 1e-5)
    assert_bits_equal(xo[sample].cpu().numpy(), wx, "x'")
    assert_close(h[sample].cpu().numpy(), wh, what="h")
    names = launched(ctx, lambda: ctx.add_rmsnorm(x.data_ptr(), b.data_ptr(), w.data_ptr(), None, 1e-5,
                                                  1e-5, 0.5, rows, hidden, xo.data_ptr(), h.data_ptr(), code))
    assert names == [kernel[:-1]], names
    ctx.check_device()
    wx, wh = O.add_rmsnorm(x[sample].cpu().numpy(), b[sample].cpu().numpy(), w.cpu().numpy(), 1e-5,
                           residual_scale=0.5)
    assert_bits_equal(xo[sample].cpu().numpy(), wx, "scaled x'")
    assert_close(h[sample].cpu().numpy(), wh, what="scaled h")
