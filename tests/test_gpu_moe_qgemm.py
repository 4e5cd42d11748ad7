"""Routed experts at prefill on the matrix cores (cuca_hip_moe_up_qgemm,
cuca_hip_moe_down_qgemm, cuca_hip_moe_qgemm_workspace) through the C ABI.

The arithmetic is cuca_hip_qgemm's class (the reference GPU engine's MoE
kernels, moe_kernel.rs:1163-1300: f32 sums of products of f16(d * q)
weights and f16 activations), not the CPU engine's bits.  Bars, per pair
p of expert e, against the f64 products of the oracle's dequantised
weights (dequant_row) and the activations:
- up: g = gate_e . x[tok[p]], u = up_e . x[tok[p]] each within
  (2^-10 + k 2^-24) sum |w x|, carried through act(g) * u as
  test_gpu_qgemm.py carries them (|act'| <= 1.2), + 2^-11 |want| in f16;
- down: (down_e . h[p]) * w[p] on the device's own hidden rows, within
  the same bound times w[p];
- the whole layer (moe_sum of the scratch rows) against its f64 value over
  the dequantised weights and the exact activations (the oracle's
  expert_sum carries the CPU engine's Q8_0 rounding of the activations,
  which this class does not have): 1e-2 of the token's largest |output|,
  a sanity bound only.
Covers Q4_0 / Q8_0, f32 / f16, SiLU / GELU-tanh, tiles of 64 and 128
pairs, experts without pairs, Zipf routing over 128 experts at config E's
expert shapes (n_embd 2048, ff 768, top 8) at a prefill size (sampled
pairs), a pair token outside the rows (reported, skipped), offsets that
are not non-decreasing (clamped) and the host's checks.
"""
import numpy as np
import pytest

from cuca_amd import hip, ops
from cuca_amd import workloads as W
from oracle import oracle as O
from test_gpu_moe import QT, bank, routing

pytestmark = pytest.mark.gpu


def dense(raw, qtype, n, k, rows=None):
    rb = W.row_bytes(qtype, k)
    rows = range(n) if rows is None else rows
    return np.stack([O.dequant_row(QT[qtype], raw[i * rb:(i + 1) * rb], 1.0, k) for i in rows]).astype(np.float64)


def bound(x, w, k):
    return (2.0 ** -10 + k * 2.0 ** -24) * (np.abs(x) @ np.abs(w).T)


def act_f(g, act):
    if act == hip.ACT_SILU:
        return g / (1.0 + np.exp(-g))
    return 0.5 * g * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (g + 0.044715 * g ** 3)))


def layer_f64(x, experts, qtype, per, act, n_embd, ff):
    """The routed experts' output in f64: per token, the routing-weighted
    down projections of act(gate . x) * (up . x), added in ascending expert
    order."""
    out = np.zeros((x.shape[0], n_embd))
    for e, picks in enumerate(per):
        if not picks:
            continue
        wg, wu = dense(experts[e][0], qtype, ff, n_embd), dense(experts[e][1], qtype, ff, n_embd)
        wd = dense(experts[e][2], qtype, n_embd, ff)
        toks = np.array([t for t, _ in picks])
        w = np.array([wi for _, wi in picks])
        xr = x[toks].astype(np.float64)
        h = act_f(xr @ wg.T, act) * (xr @ wu.T)
        out[toks] += (h @ wd.T) * w[:, None]
    return out


def check_up(got_h, x, experts, qtype, offsets, tok, act, n_embd, ff, dtype, sample=None):
    for e in range(len(experts)):
        lo, hi = int(offsets[e]), int(offsets[e + 1])
        ps = [p for p in range(lo, hi) if sample is None or p in sample]
        if not ps:
            continue
        wg = dense(experts[e][0], qtype, ff, n_embd)
        wu = dense(experts[e][1], qtype, ff, n_embd)
        xr = x[tok[ps]].astype(np.float64)
        g, u = xr @ wg.T, xr @ wu.T
        bg, bu = bound(xr, wg, n_embd), bound(xr, wu, n_embd)
        a = act_f(g, act)
        want = a * u
        tol = 1.2 * bg * (np.abs(u) + bu) + np.abs(a) * bu + 1e-5 * np.abs(want) + 1e-30
        if dtype == "f16":
            tol = tol + 2.0 ** -11 * np.abs(want)
        err = np.abs(got_h[ps].astype(np.float64) - want)
        assert np.all(err <= tol), (e, float(np.max(err / tol)))


def check_down(got_s, h, experts, qtype, offsets, wt, n_embd, ff, sample=None):
    for e in range(len(experts)):
        lo, hi = int(offsets[e]), int(offsets[e + 1])
        ps = [p for p in range(lo, hi) if sample is None or p in sample]
        if not ps:
            continue
        wd = dense(experts[e][2], qtype, n_embd, ff)
        hr = h[ps].astype(np.float64)
        want = (hr @ wd.T) * wt[ps, None]
        tol = bound(hr, wd, ff) * wt[ps, None] + 1e-30
        err = np.abs(got_s[ps].astype(np.float64) - want)
        assert np.all(err <= tol), (e, float(np.max(err / tol)))


@pytest.mark.parametrize("qtype", ["q4_0", "q8_0"])
@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("act", [hip.ACT_SILU, hip.ACT_GELU_TANH])
@pytest.mark.parametrize("t,n_experts,n_used,n_embd,ff", [(60, 8, 3, 128, 96), (40, 16, 2, 256, 160),
                                                         (300, 4, 2, 512, 64), (5, 64, 2, 128, 96)])
def test_moe_qgemm_layer(ctx, qtype, dtype, act, t, n_experts, n_used, n_embd, ff):
    rng = np.random.default_rng(t * 31 + n_experts + ff + act)
    experts, eb = bank(ctx, rng, qtype, n_experts, n_embd, ff)
    per = routing(rng, t, n_experts, n_used)
    npd = np.float16 if dtype == "f16" else np.float32
    x = (rng.standard_normal((t, n_embd)) * min(1.0, np.sqrt(256.0 / n_embd))).astype(npd)
    out, hidden, scratch = eb.expert_sum(ctx.array(x), per, ops.Glu(act), n_used, mm="qgemm")
    ctx.check_device()
    offsets, tok, wt, _ = ops.ExpertBank.grouped(per, t, n_used)
    got_h = hidden.numpy()
    check_up(got_h, x, experts, qtype, offsets, tok, act, n_embd, ff, dtype)
    check_down(scratch.numpy(), got_h, experts, qtype, offsets, wt, n_embd, ff)
    want = layer_f64(x, experts, qtype, per, act, n_embd, ff)
    scale = np.max(np.abs(want), axis=1, keepdims=True)
    assert np.all(np.abs(out.numpy().astype(np.float64) - want) <= 1e-2 * scale + 1e-30)


def test_config_e_prefill_shapes_zipf_sampled(ctx):
    """128 experts, top 8, n_embd 2048, ff 768 (Qwen3-30B-A3B's experts) at
    1024 tokens (8192 pairs, tiles of 128 pairs), Zipf(1.1) routing; the
    pairs of a few experts checked, the most and least loaded among them."""
    rng = np.random.default_rng(77)
    t, n_experts, n_used, n_embd, ff = 1024, 128, 8, 2048, 768
    experts, eb = bank(ctx, rng, "q4_0", n_experts, n_embd, ff)
    per = routing(rng, t, n_experts, n_used, zipf=1.1)
    x = (rng.standard_normal((t, n_embd)) * 0.35).astype(np.float16)
    out, hidden, scratch = eb.expert_sum(ctx.array(x), per, ops.Glu(hip.ACT_SILU), n_used, mm="qgemm")
    ctx.check_device()
    offsets, tok, wt, _ = ops.ExpertBank.grouped(per, t, n_used)
    counts = np.diff(offsets)
    assert int(offsets[-1]) == t * n_used and counts.max() > 128
    picks = [int(np.argmax(counts)), int(np.argmin(counts + (counts == 0) * 10 ** 9)), 5, 77]
    sample = set()
    for e in picks:
        lo, hi = int(offsets[e]), int(offsets[e + 1])
        sample.update(range(lo, min(hi, lo + 40)))
        sample.update(range(max(lo, hi - 3), hi))
    got_h = hidden.numpy()
    for e in picks:
        lo, hi = int(offsets[e]), int(offsets[e + 1])
        ps = sorted(p for p in sample if lo <= p < hi)
        one = np.array([0, len(ps)])
        check_up(got_h[ps], x, [experts[e]], "q4_0", one, tok[ps], hip.ACT_SILU, n_embd, ff, "f16")
        check_down(scratch.numpy()[ps], got_h[ps], [experts[e]], "q4_0", one, wt[ps], n_embd, ff)


def test_a_pair_token_outside_the_rows_is_reported(ctx):
    rng = np.random.default_rng(8)
    n_experts, n_embd, ff, t = 4, 128, 96, 6
    experts, eb = bank(ctx, rng, "q8_0", n_experts, n_embd, ff)
    offsets = np.array([0, 3, 3, 5, 6], np.int32)
    tok = np.array([0, 1, 9, 2, 3, 5], np.int32)  # pair 2 names token 9 of 6
    x = rng.standard_normal((t, n_embd)).astype(np.float32)
    dx, d_off, d_tok = ctx.array(x), ctx.array(offsets), ctx.array(tok)
    wsb = hip.moe_qgemm_workspace(hip.GGML_Q8_0, n_embd, n_experts, 6)
    ws = ctx.empty((wsb,), np.uint8)
    hidden = ctx.empty((6, ff), np.float32)
    ctx.moe_up_qgemm(eb.gate.ptr, eb.up.ptr, eb.stride_gu, hip.GGML_Q8_0, ff, n_embd, n_experts, dx.ptr, n_embd, t,
                     d_off.ptr, d_tok.ptr, 6, hip.ACT_SILU, 0.0, ws.ptr, wsb, hidden.ptr, ff, hip.F32)
    with pytest.raises(hip.CucaError):
        ctx.check_device()
    got = hidden.numpy()
    # the bad pair's activation row is zero: act(0) * 0 = 0
    assert np.all(got[2] == 0)
    ok = [0, 1, 3, 4, 5]
    check_up(got, x, experts, "q8_0", offsets, np.where(tok < t, tok, 0), hip.ACT_SILU, n_embd, ff, "f32",
             sample=set(ok))


def test_offsets_are_clamped_and_host_checks(ctx):
    rng = np.random.default_rng(9)
    n_experts, n_embd, ff, t = 3, 128, 96, 4
    experts, eb = bank(ctx, rng, "q4_0", n_experts, n_embd, ff)
    x = rng.standard_normal((t, n_embd)).astype(np.float32)
    dx = ctx.array(x)
    tok = ctx.array(np.array([0, 1, 2, 3], np.int32))
    hidden = ctx.empty((4, ff), np.float32)
    wsb = hip.moe_qgemm_workspace(hip.GGML_Q4_0, n_embd, n_experts, 4)
    ws = ctx.empty((wsb,), np.uint8)
    # decreasing and too large offsets: expert 0 gets [0, 3), expert 1 nothing, expert 2 [3, 4)
    bad_off = ctx.array(np.array([0, 3, 1, 99], np.int32))
    ctx.moe_up_qgemm(eb.gate.ptr, eb.up.ptr, eb.stride_gu, hip.GGML_Q4_0, ff, n_embd, n_experts, dx.ptr, n_embd, t,
                     bad_off.ptr, tok.ptr, 4, hip.ACT_SILU, 0.0, ws.ptr, wsb, hidden.ptr, ff, hip.F32)
    ctx.check_device()
    check_up(hidden.numpy(), x, experts, "q4_0", np.array([0, 3, 3, 4]), np.arange(4), hip.ACT_SILU, n_embd, ff,
             "f32")
    with pytest.raises(hip.CucaError, match="workspace"):
        ctx.moe_up_qgemm(eb.gate.ptr, eb.up.ptr, eb.stride_gu, hip.GGML_Q4_0, ff, n_embd, n_experts, dx.ptr,
                         n_embd, t, bad_off.ptr, tok.ptr, 4, hip.ACT_SILU, 0.0, ws.ptr, wsb - 16, hidden.ptr, ff,
                         hip.F32)
    with pytest.raises(hip.CucaError, match="expert stride"):
        ctx.moe_up_qgemm(eb.gate.ptr, eb.up.ptr, 16, hip.GGML_Q4_0, ff, n_embd, n_experts, dx.ptr, n_embd, t,
                         bad_off.ptr, tok.ptr, 4, hip.ACT_SILU, 0.0, ws.ptr, wsb, hidden.ptr, ff, hip.F32)
    with pytest.raises(hip.CucaError, match="experts"):
        ctx.moe_up_qgemm(eb.gate.ptr, eb.up.ptr, eb.stride_gu, hip.GGML_Q4_0, ff, n_embd, 5000, dx.ptr, n_embd, t,
                         bad_off.ptr, tok.ptr, 4, hip.ACT_SILU, 0.0, ws.ptr, wsb, hidden.ptr, ff, hip.F32)
