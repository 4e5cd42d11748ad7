"""The streaming (nontemporal-load) GLU kernels at the sizes that select them.

Dense gate/up inputs of at least 192 MiB are read with nontemporal loads
(runtime.cpp, kGluStreamBytes); each case here crosses that threshold,
checks from the C ABI's per-kernel profile that the call launched exactly
the streaming kernel it names, and compares sampled rows (the first, the
last and 60 random ones) with the oracle (Glu::apply, cpu.rs:342-371):
  GeGLU-tanh f16, Gemma-2-9B shape (F 14336), 4096 tokens, fused gate|up
    layout: 2 x 4096 x 14336 x 2 B = 224 MiB -> cuca_glu_f16_gelu_nt
  SwiGLU f16, the same                        -> cuca_glu_f16_silu_nt
  GeGLU-tanh / SwiGLU f32, 2048 tokens: 224 MiB -> cuca_glu_f32_{gelu,silu}_nt
  and a clamped SwiGLU (the clamp reaches the streaming kernels too);
  SwiGLU f16 at Llama-2-7B's F 11008 (1376 chunks a row, not a multiple of
    the 64-lane workgroup: the last workgroup of each row is half idle),
    4608 tokens: 194 MiB -> cuca_glu_f16_silu_nt.
Bars (cuca_hip_glu): 1e-5 relative in f32, 2 f16 ulps of the oracle's f16,
plus for GELU-tanh the floor 2^-22 |0.5 g u| (the rounding of candle's
1 + tanh(z), which cancels for z << 0).
"""
import numpy as np
import pytest

from cuca_amd import hip
from cuca_amd import workloads as W
from helpers import assert_close
from oracle import oracle as O

pytestmark = pytest.mark.gpu

F = W.CONFIGS["D"]["ff"]


@pytest.fixture(scope="module")
def torch():
    return pytest.importorskip("torch")


@pytest.mark.parametrize("dtype,act,n,clamp,kernel,F", [
    ("f16", hip.ACT_GELU_TANH, 4096, 0.0, "cuca_glu_f16_gelu_nt", F),
    ("f16", hip.ACT_SILU, 4096, 0.0, "cuca_glu_f16_silu_nt", F),
    ("f32", hip.ACT_GELU_TANH, 2048, 0.0, "cuca_glu_f32_gelu_nt", F),
    ("f32", hip.ACT_SILU, 2048, 0.0, "cuca_glu_f32_silu_nt", F),
    ("f16", hip.ACT_SILU, 4096, 1.5, "cuca_glu_f16_silu_nt", F),
    ("f16", hip.ACT_SILU, 4608, 0.0, "cuca_glu_f16_silu_nt", 11008),
])
def test_streaming_glu(ctx, torch, dtype, act, n, clamp, kernel, F):
    tdt = torch.float16 if dtype == "f16" else torch.float32
    es = 2 if dtype == "f16" else 4
    assert 2 * n * F * es >= 192 << 20
    gen = torch.Generator(device="cuda").manual_seed(n + act + int(clamp * 10) + F)
    gu = (2.0 * torch.randn((n, 2 * F), device="cuda", generator=gen)).to(tdt)  # Gemma acts ~N(0,2)
    out = torch.full((n, F), float("nan"), device="cuda", dtype=tdt)
    torch.cuda.synchronize()
    ctx.profile_start(4)
    ctx.glu(gu.data_ptr(), 2 * F, gu.data_ptr() + es * F, 2 * F, n, F, act, clamp, out.data_ptr(), F,
            hip.F16 if dtype == "f16" else hip.F32)
    names = [k for k, _ in ctx.profile_stop()]
    assert names == [kernel], names
    ctx.check_device()
    s = np.unique(np.concatenate([[0, n - 1], np.random.default_rng(n).integers(0, n, 60)]))
    st = torch.from_numpy(s).cuda()
    rows = gu[st].cpu().numpy()
    g, u = rows[:, :F], rows[:, F:]
    want = O.glu(np.ascontiguousarray(g), np.ascontiguousarray(u), act, clamp=clamp)
    floor = None
    if act == hip.ACT_GELU_TANH:
        floor = 2.0 ** -22 * np.abs(0.5 * g.astype(np.float64) * u.astype(np.float64))
    assert_close(out[st].cpu().numpy(), want.astype(rows.dtype), floor=floor,
                 what=f"{kernel} clamp {clamp}")
