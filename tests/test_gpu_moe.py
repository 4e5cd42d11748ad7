"""Routed experts (MoE) on the GPU against the oracle's expert_sum, through
the C ABI (cuca_hip_moe_up / moe_down / moe_sum).

Bars:
- moe_up: the gate and up products are cuca_hip_qmm's bits; the activation
  is held to cuca_hip_glu's bar (1e-5 relative in f32, 2 f16 ulps, plus for
  GELU-tanh the floor 2^-22 |0.5 g u|);
- moe_down: bit-exact, (down . h) * w, on the oracle's hidden rows (f32)
  and on the device's own f16 hidden rows (f16 activations);
- moe_sum: bit-exact, the f32 sum from 0 in the token's pair order (the
  ascending expert order of expert_sum), pinned by a case whose answer
  depends on that order;
- the whole layer, f32: within 1e-4 of the largest |output| of the token
  (the reference's own qmm bar, qmm/tests.rs:477-556), since the
  activation's last-bit differences can move a Q8_0 quant of the hidden row;
  f16 activations round the hidden rows to f16 (the reference is f32
  throughout), checked to 1e-2 as a sanity bound only.
Covers Q4_0 / Q8_0, f32 / f16, SiLU / GELU-tanh, both kernels (the decode
GEMV, and the one-pass kernel for rows too long for its LDS: hidden 8192),
experts with no pairs,
Zipf(1.1) routing over 128 experts at the Qwen3-30B-A3B shapes (decode
batch 64, top 8), and a pair token outside the rows (reported, skipped).
"""
import numpy as np
import pytest

from cuca_amd import hip, ops
from cuca_amd import workloads as W
from helpers import assert_bits_equal, assert_close
from oracle import oracle as O

pytestmark = pytest.mark.gpu

QT = {"q4_0": hip.GGML_Q4_0, "q8_0": hip.GGML_Q8_0}


def routing(rng, t, n_experts, n_used, zipf=None):
    """per_expert[e] = [(token, weight)] in token order; each token picks
    n_used distinct experts (uniform, or Zipf(zipf) ranks)."""
    per = [[] for _ in range(n_experts)]
    for tok in range(t):
        if zipf:
            p = 1.0 / np.arange(1, n_experts + 1) ** zipf
            es = rng.choice(n_experts, n_used, replace=False, p=p / p.sum())
        else:
            es = rng.choice(n_experts, n_used, replace=False)
        w = rng.uniform(0.05, 1.0, n_used).astype(np.float32)
        for e, wi in zip(sorted(es), w):
            per[e].append((tok, float(wi)))
    return per


def bank(ctx, rng, qtype, n_experts, n_embd, ff):
    experts = [(W.quant_table(rng, ff, n_embd, qtype, (0.01, 0.05)),
                W.quant_table(rng, ff, n_embd, qtype, (0.01, 0.05)),
                W.quant_table(rng, n_embd, ff, qtype, (0.004, 0.02))) for _ in range(n_experts)]
    return experts, ops.ExpertBank.from_raw(ctx, QT[qtype], experts, n_embd, ff)


def glu_floor(g, u, act):
    if act != hip.ACT_GELU_TANH:
        return None
    return 2.0 ** -22 * np.abs(0.5 * g.astype(np.float64) * u.astype(np.float64))


@pytest.mark.parametrize("qtype", ["q4_0", "q8_0"])
@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("act", [hip.ACT_SILU, hip.ACT_GELU_TANH])
@pytest.mark.parametrize("t,n_experts,n_used,n_embd,ff", [(10, 8, 3, 128, 96), (3, 16, 2, 256, 64),
                                                         (40, 6, 2, 64, 160), (40, 6, 2, 8192, 96),
                                                         (1, 64, 2, 128, 96)])
def test_moe_layer(ctx, qtype, dtype, act, t, n_experts, n_used, n_embd, ff):
    rng = np.random.default_rng(t * 100 + n_experts + ff + act)
    experts, eb = bank(ctx, rng, qtype, n_experts, n_embd, ff)
    per = routing(rng, t, n_experts, n_used)
    npd = np.float16 if dtype == "f16" else np.float32
    # activations shrink with the row length, so that the hidden rows (gate
    # and up sums over n_embd values) stay within f16's range
    x = (rng.standard_normal((t, n_embd)) * min(1.0, np.sqrt(256.0 / n_embd))).astype(npd)
    glu = ops.Glu(act)
    out, hidden, scratch = eb.expert_sum(ctx.array(x), per, glu, n_used)
    want, want_hidden = O.expert_sum(x, experts, QT[qtype], per, act)
    offsets, tok, wt, token_pairs = ops.ExpertBank.grouped(per, t, n_used)
    # moe_up: pair p of expert e is pick i of that expert
    got_h = hidden.numpy()
    for e in range(n_experts):
        for i in range(offsets[e + 1] - offsets[e]):
            p = offsets[e] + i
            gate, up, _ = experts[e]
            xr = x[tok[p]:tok[p] + 1]
            g = O.qmm(gate, QT[qtype], ff, n_embd, xr)
            u = O.qmm(up, QT[qtype], ff, n_embd, xr)
            wh = O.glu(g, u, act)
            if dtype == "f16":
                assert_close(got_h[p:p + 1], wh.astype(np.float16), floor=glu_floor(g, u, act),
                             what=f"moe_up pair {p}")
            else:
                assert_close(got_h[p:p + 1], wh, floor=glu_floor(g, u, act), what=f"moe_up pair {p}")
    # moe_down: bit-exact on the hidden rows it reads -- the oracle's (f32),
    # and the device's own (f16 rows, widened as the kernel widens them)
    rows_h = np.stack([want_hidden[(e, i)] for e in range(n_experts)
                       for i in range(offsets[e + 1] - offsets[e])]).astype(np.float32)
    if dtype == "f16":
        rows_h = got_h.astype(np.float32)
    dh = ctx.array(rows_h.astype(npd))
    d_off, d_wt = ctx.array(offsets), ctx.array(wt)
    scr = ctx.empty((len(tok), n_embd), np.float32)
    ctx.moe_down(eb.down.ptr, eb.stride_d, QT[qtype], n_embd, ff, n_experts, dh.ptr, ff,
                 d_off.ptr, d_wt.ptr, len(tok), scr.ptr, n_embd, hip.dtype_code(npd))
    got_s = scr.numpy()
    want_s = np.empty_like(got_s)
    for e in range(n_experts):
        lo, hi = offsets[e], offsets[e + 1]
        if hi > lo:
            y = O.qmm(experts[e][2], QT[qtype], n_embd, ff, rows_h[lo:hi])
            want_s[lo:hi] = (y * wt[lo:hi, None]).astype(np.float32)
    assert_bits_equal(got_s, want_s, "moe_down")
    # moe_sum: bit-exact against the sequential sum of the device scratch
    s = scratch.numpy()
    ref = np.zeros((t, n_embd), np.float32)
    for tt in range(t):
        for p in token_pairs[tt]:
            if p >= 0:
                ref[tt] = (ref[tt] + s[p]).astype(np.float32)
    got = out.numpy()
    assert_bits_equal(got, ref.astype(npd), "moe_sum")
    # the whole layer: f32 holds the reference's values; f16 rounds the hidden
    # rows (2^-11 relative) before the down projection, a sanity bound only
    scale = np.max(np.abs(want), axis=1, keepdims=True)
    assert np.all(np.abs(got.astype(np.float64) - want) <= (1e-4 if dtype == "f32" else 1e-2) * scale)


def test_moe_sum_adds_in_the_given_order(ctx):
    """2^30, 1, -2^30 summed in order from 0 is 0 (2^30 + 1 rounds to 2^30);
    the order 2^30, -2^30, 1 gives 1, and -2^30, (none), 1 gives -2^30."""
    s = np.zeros((3, 8), np.float32)
    s[0, :] = 2.0 ** 30
    s[1, :] = 1.0
    s[2, :] = -2.0 ** 30
    pairs = np.array([[0, 1, 2], [0, 2, 1], [2, -1, 1]], np.int32)
    out = ctx.empty((3, 8), np.float32)
    ds, dp = ctx.array(s), ctx.array(pairs)
    ctx.moe_sum(ds.ptr, 8, 3, dp.ptr, 3, 3, 8, out.ptr, 8, hip.F32)
    got = out.numpy()
    assert np.all(got[0] == 0.0) and np.all(got[1] == 1.0) and np.all(got[2] == -2.0 ** 30)


def test_qwen3_30b_a3b_shapes_zipf_routing(ctx):
    """Config E: 128 experts, hidden 2048, expert FFN 768, top 8 of 128 with
    Zipf(1.1) expert ids, decode batch 64, Q4_0, f32."""
    rng = np.random.default_rng(4)
    n_experts, n_embd, ff, t, n_used = 128, 2048, 768, 64, 8
    experts, eb = bank(ctx, rng, "q4_0", n_experts, n_embd, ff)
    per = routing(rng, t, n_experts, n_used, zipf=1.1)
    assert any(len(p) == 0 for p in per) and max(len(p) for p in per) > 16
    x = rng.standard_normal((t, n_embd)).astype(np.float32)
    out, hidden, scratch = eb.expert_sum(ctx.array(x), per, ops.Glu(hip.ACT_SILU), n_used)
    want, _ = O.expert_sum(x, experts, hip.GGML_Q4_0, per, hip.ACT_SILU, threads=8)
    got = out.numpy()
    scale = np.max(np.abs(want), axis=1, keepdims=True)
    assert np.all(np.abs(got.astype(np.float64) - want) <= 1e-4 * scale)


@pytest.mark.parametrize("n_experts", [4, 128])
def test_a_pair_token_outside_the_rows_is_reported(ctx, n_experts):
    """On both kernels: the decode GEMV (4 pairs over 4 experts) and the
    one-pass kernel (4 pairs over 128 experts)."""
    rng = np.random.default_rng(9)
    experts, eb = bank(ctx, rng, "q8_0", n_experts, 64, 32)
    x = ctx.array(rng.standard_normal((5, 64)).astype(np.float32))
    offsets = ctx.array(np.array([0, 2, 2, 3] + [4] * (n_experts - 3), np.int32))  # n_experts + 1
    tok = ctx.array(np.array([0, 7, 1, 4], np.int32))
    hidden = ctx.empty((4, 32), np.float32)
    ctx.moe_up(eb.gate.ptr, eb.up.ptr, eb.stride_gu, hip.GGML_Q8_0, 32, 64, n_experts, x.ptr, 64, 5,
               offsets.ptr, tok.ptr, 4, hip.ACT_SILU, 0.0, hidden.ptr, 32, hip.F32)
    with pytest.raises(hip.CucaError, match=r"routed token \(7\) outside the 5 rows"):
        ctx.check_device()
    ctx.check_device()  # cleared
