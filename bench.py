#!/usr/bin/env python3
"""Benchmark of the fused per-layer ops on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

Metric: fused layer-op HBM GB/s and % of the 8 TB/s peak;
per-layer non-matmul microseconds at decode.

Workload (config.workload): the Llama-3-8B layer ops.  One step is one pass
of the hot path over one batch of 16384 prefill tokens with f16 activations
(configs[2] at its larger size, the largest single-GPU configuration; the
4096-token step is measured beside it): the Q8_0 embedding gather of the batch
fused with the first block's attention RMSNorm (x and h in one pass), a
block's attention-side residual add + RMSNorm, RoPE on Q 32x128 / K 8x128,
the SwiGLU over F 14336, and the FFN-side residual add + RMSNorm.  `value` is
the algorithmic bytes of a step divided by its time (K steps between two HIP
events, synchronized on both sides), with every input resident in HBM
(synthetic data generated on the device).  The decode figure
is the same layer's non-matmul sequence (two fused norms, RoPE, SwiGLU) at
batch 1 and 32 in f32, 32 layers captured in one hipGraph and
replayed, in microseconds per layer.

Algorithmic bytes per unit (s = bytes per activation, H 4096, F 14336):
  embed_rms   34 H/32 + 4 + 2 s H      per token (block bytes, id, x and h out)
  add_rmsnorm 4 s H                    per row   (x, branch in; x', h out)
  rope        2 s (nq + nk) D + 4 D    per row   (Q, K in and out; cos+sin)
  glu         3 s F                    per row   (gate, up in; out)
Per-call constants (gamma, norm weights) are counted once.

`configs` repeats the step for the other workload configs (A Qwen3-0.6B,
B Llama-3-8B decode batch, D Gemma-2-9B with the sandwich norms, GeGLU and
interleaved RoPE, E Qwen3-30B-A3B with QK-norm RoPE and the ragged
expert-grouped SwiGLU), each op's kernel GB/s from its timestamps.
`prefill_bar` (near the end of the line) gathers every op's fraction of
the HBM peak at the sizes of the 70 % bar (config C at 4096 and 16384
tokens, config E at 8192), `decode_bar` the batch-1 decode figures.

roofline: the dominant kernel (SwiGLU) -- its algorithmic bytes per launch
divided by its average launch duration over the timed steps, from the start
and stop events the C ABI's profile attaches to every kernel
(hipExtModuleLaunchKernel on the ops' stream; the same durations rocprofv3
reports), against the 8 TB/s HBM peak.

cpu_baseline: the oracle's C restatement of the reference's candle CPU path
(oracle/) over the same 16384-token step, on the step's own inputs, with the
CPUs this process is given (the CPU model and counts are recorded); each op
timed alone, per-op GB/s beside the GPU's.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


STEP_OPS = ("embed_rms", "add_rmsnorm_attn", "rope", "glu", "add_rmsnorm_ffn")


class LayerStep:
    """Device buffers of one pass of the hot path for a workload config
    (cuca_amd.workloads.CONFIGS) at n tokens in `dtype`, and its launches:
    the embedding gather of the batch, the attention-side residual add +
    RMSNorm (Gemma: with the post-norm sandwich), RoPE on Q and K (Qwen3-MoE:
    with the QK-norm), the gated activation (SwiGLU / GeGLU-tanh; Qwen3-MoE:
    over the expert-grouped rows of top-k routing), and the FFN-side
    residual add + RMSNorm.  Inputs are generated on the device."""

    def __init__(self, ctx, torch, name, n, dtype):
        from cuca_amd import hip
        from cuca_amd import workloads as W
        import numpy as np
        cfg = W.CONFIGS[name]
        self.hip, self.ctx, self.torch, self.name, self.n, self.cfg = hip, ctx, torch, name, n, cfg
        self.dt = hip.F16 if dtype == "f16" else hip.F32
        tdt = torch.float16 if dtype == "f16" else torch.float32
        s = 2 if dtype == "f16" else 4
        H, F, d, nq, nk = cfg["hidden"], cfg["ff"], cfg["head_dim"], cfg["nq"], cfg["nk"]
        dev = "cuda"
        gen = torch.Generator(device=dev).manual_seed(cfg["seed"] * 1000 + n)
        std = cfg["std"]

        def act(*shape):
            return (std * torch.randn(shape, device=dev, generator=gen)).to(tdt)

        def gamma(k):
            return (1 + 0.02 * torch.randn(k, device=dev, generator=gen)).float()
        self.qtype = W.GGML_ID[cfg["qtype"]]
        self.table = W.quant_table_torch(gen, cfg["vocab"], H, cfg["qtype"], cfg["d_range"])
        self.ids = torch.randint(0, cfg["vocab"], (n,), device=dev, generator=gen, dtype=torch.int32)
        self.emb = torch.empty((n, H), device=dev, dtype=tdt)
        self.norm = []
        for _ in range(2):
            self.norm.append(dict(x=act(n, H), b=act(n, H), xo=torch.empty((n, H), device=dev, dtype=tdt),
                                  h=torch.empty((n, H), device=dev, dtype=tdt), w=gamma(H),
                                  wp=gamma(H) if cfg.get("sandwich") else None))
        self.q, self.k = act(n, nq, d), act(n, nk, d)
        self.q0, self.k0 = self.q.clone(), self.k.clone()
        self.kind = hip.ROPE_NEOX if cfg["rope"] == "neox" else hip.ROPE_NORM
        trows = W.table_rows_needed(cfg, n)
        cos, sin = hip.rope_tables(self.kind, d, cfg["theta"], trows)
        self.trows = trows
        self.cos, self.sin = torch.from_numpy(cos).to(dev), torch.from_numpy(sin).to(dev)
        pos = W.positions(cfg, n, np.random.default_rng(cfg["seed"]))
        self.pos = torch.from_numpy(pos).to(dev)
        self.qn = gamma(d) if cfg.get("qk_norm") else None
        self.kn = gamma(d) if cfg.get("qk_norm") else None
        self.act = hip.ACT_GELU_TANH if cfg["act"] == "gelu" else hip.ACT_SILU
        if cfg.get("moe"):
            n_exp, k = cfg["moe"]
            offsets, _ = W.zipf_expert_rows(np.random.default_rng(cfg["seed"]), n, n_exp, k)
            self.n_exp, self.rows_glu = n_exp, int(offsets[-1])
            self.offsets = torch.from_numpy(offsets).to(dev)
            self.gate, self.up = act(self.rows_glu, F), act(self.rows_glu, F)
        else:
            self.offsets = None
            self.rows_glu = n
            self.gu = act(n, 2 * F)
        self.out = torch.empty((self.rows_glu, F), device=dev, dtype=tdt)
        # the first block's attention norm, fused with the gather
        self.emb_h = torch.empty((n, H), device=dev, dtype=tdt)
        self.emb_w = gamma(H)
        bb = 18 if cfg["qtype"] == "q4_0" else 34
        nw = 2 if cfg.get("sandwich") else 1
        self.bytes = {
            "embed_rms": n * (bb * H // 32 + 4 + 2 * s * H) + 4 * H,
            "add_rmsnorm_attn": n * 4 * s * H + nw * 4 * H,
            "rope": n * (2 * s * (nq + nk) * d + 4 * d) + (8 * d if cfg.get("qk_norm") else 0),
            "glu": self.rows_glu * 3 * s * F,
            "add_rmsnorm_ffn": n * 4 * s * H + nw * 4 * H,
        }

    def launch(self, name):
        c, hip, cfg, n, dt = self.ctx, self.hip, self.cfg, self.n, self.dt
        H, F, d, nq, nk = cfg["hidden"], cfg["ff"], cfg["head_dim"], cfg["nq"], cfg["nk"]
        es = 2 if dt == hip.F16 else 4
        if name == "embed_rms":
            c.embed_gguf_rms(self.table.data_ptr(), self.qtype, cfg["vocab"], H, self.ids.data_ptr(), n,
                             cfg["embd_scale"], self.emb_w.data_ptr(), cfg["eps"], self.emb.data_ptr(),
                             self.emb_h.data_ptr(), dt)
        elif name.startswith("add_rmsnorm"):
            b = self.norm[0 if name.endswith("attn") else 1]
            c.add_rmsnorm(b["x"].data_ptr(), b["b"].data_ptr(), b["w"].data_ptr(),
                          None if b["wp"] is None else b["wp"].data_ptr(), cfg["eps"], cfg["eps"], 1.0,
                          n, H, b["xo"].data_ptr(), b["h"].data_ptr(), dt)
        elif name == "rope":
            c.rope(self.q.data_ptr(), nq * d, self.k.data_ptr(), nk * d, n, nq, nk, d, d, self.kind,
                   self.cos.data_ptr(), self.sin.data_ptr(), self.trows, self.pos.data_ptr(),
                   None if self.qn is None else self.qn.data_ptr(),
                   None if self.kn is None else self.kn.data_ptr(), cfg["eps"], dt)
        elif name == "glu":
            if self.offsets is not None:
                c.glu_ragged(self.gate.data_ptr(), F, self.up.data_ptr(), F, self.offsets.data_ptr(),
                             self.n_exp, self.rows_glu, F, self.act, 0.0, self.out.data_ptr(), F, dt)
            else:
                c.glu(self.gu.data_ptr(), 2 * F, self.gu.data_ptr() + es * F, 2 * F, n, F, self.act,
                      0.0, self.out.data_ptr(), F, dt)

    def step(self):
        for name in STEP_OPS:
            self.launch(name)

    def verify(self, rows=16):
        """Run the step once from fresh Q/K and compare sampled rows of every
        output with the oracle (the timed kernels did the work they claim):
        the gather and plain RoPE bit for bit, the rest to 1e-5 relative (f32)
        or 2 f16 ulps, with the floors of the parity tests for the GELU
        cancellation, the sandwich sum and the QK-normed rotation."""
        import numpy as np
        from oracle import oracle as O
        torch, cfg, n = self.torch, self.cfg, self.n
        H, F, d = cfg["hidden"], cfg["ff"], cfg["head_dim"]
        self.q.copy_(self.q0)
        self.k.copy_(self.k0)
        self.step()
        torch.cuda.synchronize()
        self.ctx.check_device()
        f16 = self.dt == self.hip.F16
        npdt = np.float16 if f16 else np.float32
        rng = np.random.default_rng(7)
        s = np.unique(np.concatenate([[0, n - 1], rng.integers(0, n, rows)]))
        st = torch.from_numpy(s).cuda()

        def host(t, idx=st):
            return t[idx].cpu().numpy()

        raw = {}

        def close(got, want, what, floor=0.0):
            # the bar, and the raw error before the floor: max relative error
            # (f32) or f16 ulps, and the values inside the bar only by the floor
            # (an expected NaN needs a NaN, an expected inf the same inf, an
            # expected finite value a finite one: no tolerance sees those)
            g, w = got.astype(np.float64), want.astype(np.float64)
            nonfinite = np.where(np.isnan(w), ~np.isnan(g),
                                 np.where(np.isinf(w), g != w, ~np.isfinite(g)))
            assert not nonfinite.any(), \
                f"{self.name} n={n} {what}: {nonfinite.sum()} values with a different NaN/inf pattern"
            fin = np.isfinite(w)
            g, w = g[fin], w[fin]
            ulp = np.spacing(np.abs(w).astype(np.float16)).astype(np.float64) if f16 else None
            if np.ndim(floor):
                floor = np.broadcast_to(floor, fin.shape)[fin]
            plain = (2 * ulp if f16 else 1e-5 * np.abs(w)) + 1e-37
            d = np.abs(g - w)
            bad = d > plain + floor
            assert not bad.any(), f"{self.name} n={n} {what}: {bad.sum()} values outside tolerance"
            err = d / np.where(ulp > 0, ulp, 1.0) if f16 else d / np.maximum(np.abs(w), 1e-30)
            r = raw.setdefault(what, {"max_ulp" if f16 else "max_rel": 0.0, "floored": 0, "n": 0})
            k = "max_ulp" if f16 else "max_rel"
            r[k] = max(r[k], float(err.max()) if err.size else 0.0)
            r["floored"] += int(np.count_nonzero(d > plain))
            r["n"] += int(d.size)

        rb = (18 if cfg["qtype"] == "q4_0" else 34) * H // 32
        sub = self.table.view(cfg["vocab"], rb)[self.ids[st].long()].cpu().numpy().reshape(-1)
        want = O.embed(sub, self.qtype, s.size, H, np.arange(s.size, dtype=np.uint32),
                       cfg["embd_scale"], out_dtype=npdt)
        assert np.array_equal(host(self.emb).view(np.uint8), want.view(np.uint8)), "embed"
        _, wh = O.add_rmsnorm(want, None, self.emb_w.cpu().numpy(), cfg["eps"], write_x=False)
        close(host(self.emb_h), wh, "embed h")
        for b in self.norm:
            x, br = host(b["x"]), host(b["b"])
            wp = None if b["wp"] is None else b["wp"].cpu().numpy()
            wx, wh = O.add_rmsnorm(x, br, b["w"].cpu().numpy(), cfg["eps"], w_post=wp)
            if wp is None:
                assert np.array_equal(host(b["xo"]).view(np.uint8), wx.view(np.uint8)), "x'"
                close(host(b["h"]), wh, "h")
            else:
                b64 = br.astype(np.float64)
                fx = 1e-5 * np.abs(b64 / np.sqrt((b64 ** 2).mean(-1, keepdims=True) + cfg["eps"]) * wp)
                m = np.sqrt((wx.astype(np.float64) ** 2).mean(-1, keepdims=True) + cfg["eps"])
                close(host(b["xo"]), wx, "sandwich x'", fx)
                close(host(b["h"]), wh, "sandwich h", fx / m * np.abs(b["w"].cpu().numpy()))
        cos, sin = self.cos.cpu().numpy(), self.sin.cpu().numpy()
        pos = self.pos[st].cpu().numpy()
        for t, t0, nw in ((self.q, self.q0, self.qn), (self.k, self.k0, self.kn)):
            if nw is None:
                w = O.rope(host(t0), cos, sin, pos, self.kind)
                assert np.array_equal(host(t).view(np.uint8), w.view(np.uint8)), "rope"
            else:
                w = O.rope(host(t0), cos, sin, pos, self.kind, norm_w=nw.cpu().numpy(), eps=cfg["eps"])
                # 1e-5 of each rotated pair's magnitude (a*c - b*s cancels)
                w64 = w.astype(np.float64)
                ia = np.arange(d // 2) if self.kind == self.hip.ROPE_NEOX else 2 * np.arange(d // 2)
                ib = ia + d // 2 if self.kind == self.hip.ROPE_NEOX else ia + 1
                mag = np.zeros_like(w64)
                mag[..., ia] = mag[..., ib] = np.hypot(w64[..., ia], w64[..., ib])
                close(host(t), w, "normed rope", 1e-5 * mag)
        gs = np.unique(np.concatenate([[0, self.rows_glu - 1],
                                       rng.integers(0, self.rows_glu, rows)]))
        gst = torch.from_numpy(gs).cuda()
        if self.offsets is not None:
            g, u = host(self.gate, gst), host(self.up, gst)
        else:
            gu = host(self.gu, gst)
            g, u = gu[:, :F], gu[:, F:]
        wa = O.glu(np.ascontiguousarray(g), np.ascontiguousarray(u),
                   O.GELU_TANH if self.act == self.hip.ACT_GELU_TANH else O.SILU)
        fl = 2.0 ** -22 * np.abs(0.5 * g.astype(np.float64) * u.astype(np.float64))
        close(host(self.out, gst), wa, "glu", fl if self.act == self.hip.ACT_GELU_TANH else 0.0)
        for r in raw.values():
            for k in ("max_rel", "max_ulp"):
                if k in r:
                    r[k] = float(f"{r[k]:.3g}")
        return int(s.size + gs.size), raw


def time_steps(torch, fn, steps, warmup):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(steps):
        fn()
    t1.record()
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) / steps


def profiled_steps(torch, ctx, step, steps, warmup):
    """Time `steps` steps between two HIP events on the ops' stream, with
    every kernel also carrying start/stop events of its own (the C ABI's
    profile, hipExtModuleLaunchKernel): returns (ms per step, {op: (kernel,
    average kernel ms)})."""
    for _ in range(warmup):
        step.step()
    torch.cuda.synchronize()
    ctx.profile_start(len(STEP_OPS) * steps)
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(steps):
        step.step()
    t1.record()
    recs = ctx.profile_stop()
    torch.cuda.synchronize()
    assert len(recs) == len(STEP_OPS) * steps, len(recs)
    per = {}
    for i, (kernel, kms) in enumerate(recs):
        name = STEP_OPS[i % len(STEP_OPS)]
        k, tot = per.get(name, (kernel, 0.0))
        per[name] = (kernel, tot + kms)
    return t0.elapsed_time(t1) / steps, {n: (k, t / steps) for n, (k, t) in per.items()}


def profiled_windows(torch, ctx, step, steps, warmup, windows=5):
    """profiled_steps over `windows` windows of `steps` steps each: the
    median per op of the windows' average kernel times (and of the step
    times).  The kernels of freshly allocated buffers run slower for the
    first tens of steps on MI355X (config E's steps of 8192 tokens: the
    gather 13.96 us in the first window of 20 steps after 25 unprofiled
    ones, 12.8-13.1 in the next three), and from window to window an op
    varies by about 2 % with what the kernels before it left in the caches;
    the median of five windows reports the steady state."""
    import numpy as np
    runs = [profiled_steps(torch, ctx, step, steps, warmup) for _ in range(windows)]
    ms = float(np.median([r[0] for r in runs]))
    per = {}
    for name in runs[0][1]:
        per[name] = (runs[0][1][name][0], float(np.median([r[1][name][1] for r in runs])))
    return ms, per


def kv_store_bench(ctx, torch, name, n, dtype, steps=20, warmup=5):
    """QK-norm + RoPE + paged K/V store (cuca_hip_rope_store_kv) at n tokens of
    config `name`: the fused kernel's time and GB/s over its algorithmic bytes
    (Q in and out, K and V in, K and V into the pool, the cos/sin rows), next
    to the unfused sequence it replaces -- this library's RoPE on Q and K in
    place, then K and V scattered into the pool by torch (index_put) -- and
    sampled rows checked against the oracle."""
    import numpy as np
    from cuca_amd import hip
    from cuca_amd import workloads as W
    from oracle import oracle as O
    cfg = W.CONFIGS[name]
    d, nq, nk, eps = cfg["head_dim"], cfg["nq"], cfg["nk"], cfg["eps"]
    dt = hip.F16 if dtype == "f16" else hip.F32
    tdt = torch.float16 if dtype == "f16" else torch.float32
    s = 2 if dtype == "f16" else 4
    kind = hip.ROPE_NEOX if cfg["rope"] == "neox" else hip.ROPE_NORM
    gen = torch.Generator(device="cuda").manual_seed(cfg["seed"] * 7 + n)
    q = (cfg["std"] * torch.randn((n, nq, d), device="cuda", generator=gen)).to(tdt)
    k = (cfg["std"] * torch.randn((n, nk, d), device="cuda", generator=gen)).to(tdt)
    v = (cfg["std"] * torch.randn((n, nk, d), device="cuda", generator=gen)).to(tdt)
    q0 = q.clone()
    n_blocks = n // hip.KV_BLOCK + 64
    pk = torch.zeros((n_blocks, nk, hip.KV_BLOCK, d), device="cuda", dtype=tdt)
    pv = torch.zeros_like(pk)
    table = np.random.default_rng(cfg["seed"]).permutation(n_blocks)[:(n + 15) // 16]
    slots = hip.kv_slots(table.astype(np.uint32), 0, n, n_blocks)
    dslots = torch.from_numpy(slots).cuda()
    sb, sr = dslots.long() // hip.KV_BLOCK, dslots.long() % hip.KV_BLOCK
    cos, sin = hip.rope_tables(kind, d, cfg["theta"], n)
    dcos, dsin = torch.from_numpy(cos).cuda(), torch.from_numpy(sin).cuda()
    pos = torch.arange(n, dtype=torch.int32, device="cuda")
    qn = kn = None
    if cfg.get("qk_norm"):
        qn = (1 + 0.02 * torch.randn(d, device="cuda", generator=gen)).float()
        kn = (1 + 0.02 * torch.randn(d, device="cuda", generator=gen)).float()
    ptr = (lambda t: None if t is None else t.data_ptr())
    v_norm = 1 if cfg.get("qk_norm") else 0

    def fused():
        ctx.rope_store_kv(q.data_ptr(), nq * d, k.data_ptr(), nk * d, v.data_ptr(), nk * d, n, nq,
                          nk, d, d, kind, dcos.data_ptr(), dsin.data_ptr(), n, pos.data_ptr(),
                          ptr(qn), ptr(kn), v_norm, eps, pk.data_ptr(), pv.data_ptr(), n_blocks,
                          dslots.data_ptr(), dt)

    kw = k.clone()

    def unfused():
        ctx.rope(q.data_ptr(), nq * d, kw.data_ptr(), nk * d, n, nq, nk, d, d, kind,
                 dcos.data_ptr(), dsin.data_ptr(), n, pos.data_ptr(), ptr(qn), ptr(kn), eps, dt)
        pk[sb, :, sr] = kw
        pv[sb, :, sr] = v

    for _ in range(warmup):
        fused()
    torch.cuda.synchronize()
    ctx.profile_start(steps)
    for _ in range(steps):
        fused()
    recs = ctx.profile_stop()
    kernel = recs[0][0]
    k_ms = sum(t for _, t in recs) / len(recs)
    un_ms = time_steps(torch, unfused, steps, warmup)
    # one clean pass for the check (q is rotated in place)
    q.copy_(q0)
    pk.zero_()
    pv.zero_()
    fused()
    torch.cuda.synchronize()
    ctx.check_device()
    sm = np.unique(np.concatenate([[0, 15, 16, n - 1], np.random.default_rng(5).integers(0, n, 28)]))
    st = torch.from_numpy(sm).cuda()
    hq, hk, hv = (t[st].cpu().numpy() for t in (q0, k, v))
    p32 = sm.astype(np.int32)
    hqn, hkn = (None if t is None else t.cpu().numpy() for t in (qn, kn))
    wq = O.rope(hq, cos, sin, p32, kind, norm_w=hqn, eps=eps)
    wk = O.rope(hk, cos, sin, p32, kind, norm_w=hkn, eps=eps)
    wv = hv
    if v_norm:
        _, h = O.add_rmsnorm(hv.reshape(-1, d), None, None, eps, write_x=False)
        wv = h.reshape(hv.shape)
    got = (q[st].cpu().numpy(), pk[sb[st], :, sr[st]].cpu().numpy(),
           pv[sb[st], :, sr[st]].cpu().numpy())
    for g, w, what in zip(got, (wq, wk, wv), ("q", "pool k", "pool v")):
        if qn is None:
            assert np.array_equal(g.view(np.uint16 if dtype == "f16" else np.uint32),
                                  w.view(np.uint16 if dtype == "f16" else np.uint32)), what
        else:
            assert np.all(np.isfinite(w)) and np.all(np.isfinite(g)), (what, "non-finite")
            err = np.abs(g.astype(np.float64) - w) / (np.abs(w.astype(np.float64)).max(-1, keepdims=True))
            assert err.max() <= (4e-3 if dtype == "f16" else 1e-5), (what, err.max())
    b = n * (2 * s * (nq + 2 * nk) * d + 4 * d) + (8 * d if qn is not None else 0)
    return dict(kernel=kernel, us=round(k_ms * 1000, 2), bytes=b,
                gbs=round(b / (k_ms / 1e3) / 1e9, 1), frac=round(b / (k_ms / 1e3) / 1e9 / HBM_PEAK_GBS, 4),
                unfused_us=round(un_ms * 1000, 2), verified_rows=int(sm.size))


def attn_bench(ctx, torch, name, rows, ctx_len, dtype, steps=20, warmup=5):
    """Paged decode attention (cuca_hip_paged_decode): `rows` sequences of
    config `name`, each with one query row over ctx_len keys in scrambled
    blocks of a shared pool.  Algorithmic bytes: the keys and values of the
    ranges (2 ctx_len n_kv d s per row) plus q and out.  Reports the split
    and merge kernels and the total, and checks two rows against the oracle."""
    import numpy as np
    from cuca_amd import hip
    from cuca_amd import workloads as W
    from oracle import oracle as O
    cfg = W.CONFIGS[name]
    d, nq, nk = cfg["head_dim"], cfg["nq"], cfg["nk"]
    dt = hip.F16 if dtype == "f16" else hip.F32
    tdt = torch.float16 if dtype == "f16" else torch.float32
    s = 2 if dtype == "f16" else 4
    nb_row = ctx_len // hip.KV_BLOCK
    n_blocks = rows * nb_row + 16
    gen = torch.Generator(device="cuda").manual_seed(cfg["seed"] * 11 + rows)
    pk = torch.randn((n_blocks, nk, hip.KV_BLOCK, d), device="cuda", generator=gen).to(tdt)
    pv = torch.randn((n_blocks, nk, hip.KV_BLOCK, d), device="cuda", generator=gen).to(tdt)
    q = torch.randn((rows, nq, d), device="cuda", generator=gen).to(tdt)
    out = torch.empty_like(q)
    tables = np.random.default_rng(rows).permutation(n_blocks)[:rows * nb_row].reshape(rows, nb_row)
    dtab = torch.from_numpy(tables.astype(np.int32)).cuda()
    ranges = np.tile(np.array([0, ctx_len], np.int32), (rows, 1))
    drng = torch.from_numpy(ranges).cuda()
    wsb = hip.paged_decode_workspace(rows, nq, d, nb_row)
    ws = torch.empty(max(wsb, 16), dtype=torch.uint8, device="cuda")
    scale = 1.0 / float(np.sqrt(d))

    def call():
        ctx.paged_decode(q.data_ptr(), pk.data_ptr(), pv.data_ptr(), n_blocks, dtab.data_ptr(),
                         nb_row, drng.data_ptr(), rows, nq, nk, d, scale, ws.data_ptr(), wsb,
                         out.data_ptr(), dt)
    for _ in range(warmup):
        call()
    torch.cuda.synchronize()
    ctx.profile_start(2 * steps)
    for _ in range(steps):
        call()
    recs = ctx.profile_stop()
    ctx.check_device()
    split_ms = sum(t for k, t in recs[0::2]) / steps
    merge_ms = sum(t for k, t in recs[1::2]) / steps
    total_ms = time_steps(torch, call, steps, warmup)
    call()
    torch.cuda.synchronize()
    chk = [0, rows - 1]
    got = out[chk].cpu().numpy()
    want = O.paged_attention(q[chk].cpu().numpy(), tables[chk].astype(np.uint32), ranges[chk],
                             pk.cpu().numpy(), pv.cpu().numpy(), scale, threads=8)
    err = np.max(np.abs(got.astype(np.float64) - want) / (1e-5 + np.abs(want.astype(np.float64))))
    vmax = float(pv.abs().max().item())
    assert np.max(np.abs(got.astype(np.float64) - want)) <= (
        2 * np.spacing(np.abs(want).astype(np.float16)).astype(np.float64).max() if dtype == "f16" else 0
    ) + 1e-5 * (np.abs(want).max() + vmax), err
    b = rows * (2 * ctx_len * nk * d * s + 2 * nq * d * s)
    return dict(kernels=[recs[0][0], recs[1][0]], split_us=round(split_ms * 1000, 2),
                merge_us=round(merge_ms * 1000, 2), us=round(total_ms * 1000, 2), bytes=b,
                gbs=round(b / (total_ms / 1e3) / 1e9, 1),
                frac=round(b / (total_ms / 1e3) / 1e9 / HBM_PEAK_GBS, 4),
                split_frac=round(b / (split_ms / 1e3) / 1e9 / HBM_PEAK_GBS, 4))


class DecodeLayers:
    """32 layers of the decode step's non-matmul ops (config B, f32)."""

    def __init__(self, ctx, torch, n, layers=32, seed=1):
        from cuca_amd import hip
        from cuca_amd import workloads as W
        cfg = W.CONFIGS["B"]
        self.hip, self.ctx, self.n, self.cfg, self.layers = hip, ctx, n, cfg, layers
        H, F, d, nq, nk = cfg["hidden"], cfg["ff"], cfg["head_dim"], cfg["nq"], cfg["nk"]
        gen = torch.Generator(device="cuda").manual_seed(seed)

        def r(*shape):
            return torch.randn(shape, device="cuda", generator=gen)
        self.x, self.h = r(n, H), r(n, H)
        self.L = []
        for _ in range(layers):
            self.L.append(dict(attn=r(n, H), ffn=r(n, H), w1=1 + 0.02 * r(H), w2=1 + 0.02 * r(H),
                               q=r(n, nq, d), k=r(n, nk, d), gu=r(n, 2 * F),
                               act=torch.empty((n, F), device="cuda")))
        cos, sin = hip.rope_tables(hip.ROPE_NORM, d, cfg["theta"], 8192)
        self.cos, self.sin = torch.from_numpy(cos).cuda(), torch.from_numpy(sin).cuda()
        self.pos = torch.randint(0, 8192, (n,), device="cuda", generator=gen, dtype=torch.int32)

    def issue(self):
        c, hip, cfg, n = self.ctx, self.hip, self.cfg, self.n
        H, F, d, nq, nk, eps = cfg["hidden"], cfg["ff"], cfg["head_dim"], cfg["nq"], cfg["nk"], cfg["eps"]
        for l in self.L:
            # (QKV matmul) -> RoPE on Q, K
            c.rope(l["q"].data_ptr(), nq * d, l["k"].data_ptr(), nk * d, n, nq, nk, d, d,
                   hip.ROPE_NORM, self.cos.data_ptr(), self.sin.data_ptr(), 8192,
                   self.pos.data_ptr(), None, None, eps, hip.F32)
            # (attention, O matmul) -> x += attn; h = ffn_norm(x)
            c.add_rmsnorm(self.x.data_ptr(), l["attn"].data_ptr(), l["w1"].data_ptr(), None, eps,
                          eps, 1.0, n, H, self.x.data_ptr(), self.h.data_ptr(), hip.F32)
            # (gate/up matmul) -> SwiGLU
            c.glu(l["gu"].data_ptr(), 2 * F, l["gu"].data_ptr() + 4 * F, 2 * F, n, F,
                  hip.ACT_SILU, 0.0, l["act"].data_ptr(), F, hip.F32)
            # (down matmul) -> x += ffn; h = next layer's attn_norm(x)
            c.add_rmsnorm(self.x.data_ptr(), l["ffn"].data_ptr(), l["w2"].data_ptr(), None, eps,
                          eps, 1.0, n, H, self.x.data_ptr(), self.h.data_ptr(), hip.F32)


class DecodeLayersAttn(DecodeLayers):
    """DecodeLayers with the attention-side ops a K/V-owning layer adds: the
    fused QK-norm-less RoPE + paged K/V store of the new token (its K and V
    into the layer's pool) and the paged decode attention over ctx_len keys
    (the new one included), per layer, config B, f32."""

    def __init__(self, ctx, torch, n, ctx_len, layers=32, seed=1):
        super().__init__(ctx, torch, n, layers, seed)
        import numpy as np
        hip, cfg = self.hip, self.cfg
        d, nq, nk = cfg["head_dim"], cfg["nq"], cfg["nk"]
        nbr = (ctx_len + 15) // 16
        self.n_blocks = n * nbr
        gen = torch.Generator(device="cuda").manual_seed(seed + 1)
        for l in self.L:
            l["v"] = torch.randn((n, nk, d), device="cuda", generator=gen)
            l["pk"] = torch.randn((self.n_blocks, nk, 16, d), device="cuda", generator=gen)
            l["pv"] = torch.randn((self.n_blocks, nk, 16, d), device="cuda", generator=gen)
            l["o"] = torch.empty((n, nq, d), device="cuda")
        tables = np.arange(self.n_blocks, dtype=np.int32).reshape(n, nbr)
        self.tables = torch.from_numpy(tables).cuda()
        self.max_blocks = nbr
        pos = np.full(n, ctx_len - 1, np.int32)   # the new token's position
        self.pos = torch.from_numpy(pos).cuda()
        slots = np.concatenate([hip.kv_slots(tables[r].astype(np.uint32), ctx_len - 1, 1, self.n_blocks)
                                for r in range(n)])
        self.slots = torch.from_numpy(slots).cuda()
        self.ranges = torch.from_numpy(np.tile(np.array([0, ctx_len], np.int32), (n, 1))).cuda()
        self.ws_bytes = hip.paged_decode_workspace(n, nq, d, nbr)
        self.ws = torch.empty(max(self.ws_bytes, 16), dtype=torch.uint8, device="cuda")
        self.scale = 1.0 / float(np.sqrt(d))

    def issue(self):
        c, hip, cfg, n = self.ctx, self.hip, self.cfg, self.n
        H, F, d, nq, nk, eps = cfg["hidden"], cfg["ff"], cfg["head_dim"], cfg["nq"], cfg["nk"], cfg["eps"]
        for l in self.L:
            # (QKV matmul) -> RoPE on Q, K; K and V of the new token into the pool
            c.rope_store_kv(l["q"].data_ptr(), nq * d, l["k"].data_ptr(), nk * d, l["v"].data_ptr(),
                            nk * d, n, nq, nk, d, d, hip.ROPE_NORM, self.cos.data_ptr(),
                            self.sin.data_ptr(), 8192, self.pos.data_ptr(), None, None, 0, eps,
                            l["pk"].data_ptr(), l["pv"].data_ptr(), self.n_blocks,
                            self.slots.data_ptr(), hip.F32)
            # paged attention over the context
            c.paged_decode(l["q"].data_ptr(), l["pk"].data_ptr(), l["pv"].data_ptr(), self.n_blocks,
                           self.tables.data_ptr(), self.max_blocks, self.ranges.data_ptr(), n, nq,
                           nk, d, self.scale, self.ws.data_ptr(), self.ws_bytes, l["o"].data_ptr(),
                           hip.F32)
            # (O matmul) -> x += attn; h = ffn_norm(x)
            c.add_rmsnorm(self.x.data_ptr(), l["attn"].data_ptr(), l["w1"].data_ptr(), None, eps,
                          eps, 1.0, n, H, self.x.data_ptr(), self.h.data_ptr(), hip.F32)
            c.glu(l["gu"].data_ptr(), 2 * F, l["gu"].data_ptr() + 4 * F, 2 * F, n, F,
                  hip.ACT_SILU, 0.0, l["act"].data_ptr(), F, hip.F32)
            c.add_rmsnorm(self.x.data_ptr(), l["ffn"].data_ptr(), l["w2"].data_ptr(), None, eps,
                          eps, 1.0, n, H, self.x.data_ptr(), self.h.data_ptr(), hip.F32)


class DecodeStep:
    """A whole decode step of the 8B model at batch n (config B shapes:
    hidden 4096, 32 query / 8 K/V heads of 128, FFN 14336, vocab 128256),
    f32 activations, every op a kernel of this library:
      embed (Q8_0 table) ->
      32 layers of [residual + attention RMSNorm, the fused Q|K|V
        projection (qmm), RoPE + paged K/V store of the new token, paged
        decode attention over ctx_len keys, o projection, residual + FFN
        RMSNorm, gate/up projections with SwiGLU (qmm_glu), down projection]
      -> residual + final RMSNorm -> LM head (Q8_0) -> argmax.
    The projections run on qmm (the CPU engine's bits) or, with
    mm="qgemm", on the matrix cores (the GPU engine's arithmetic class).
    Layer weights are Q4_0 (or `qtype`), 32 distinct layers (3.9 GB Q4_0),
    generated as GGUF bytes on the device and packed once; the K/V pools
    hold ctx_len keys per sequence in consecutive blocks."""

    def __init__(self, ctx, torch, n, ctx_len, qtype="q4_0", layers=32, seed=3, mm="qmm", fuse_rope=False,
                 fuse_norm=False):
        import numpy as np
        from cuca_amd import hip
        from cuca_amd import workloads as W
        cfg = W.CONFIGS["B"]
        self.hip, self.ctx, self.torch, self.n, self.cfg, self.layers = hip, ctx, torch, n, cfg, layers
        H, F, d, nq, nk = cfg["hidden"], cfg["ff"], cfg["head_dim"], cfg["nq"], cfg["nk"]
        self.vocab = cfg["vocab"]
        dev = "cuda"
        gen = torch.Generator(device=dev).manual_seed(seed)
        T = W.GGML_ID[qtype]
        self.T = T

        def packed(rows, cols, qt, d_range):
            raw = W.quant_table_torch(gen, rows, cols, qt, d_range)
            out = torch.empty(hip.qweight_bytes(W.GGML_ID[qt], rows, cols), dtype=torch.uint8, device=dev)
            ctx.qweight_pack(raw.data_ptr(), W.GGML_ID[qt], rows, cols, out.data_ptr())
            torch.cuda.synchronize()
            del raw
            return out

        def r(*shape):
            return torch.randn(shape, device=dev, generator=gen)
        self.table = W.quant_table_torch(gen, self.vocab, H, "q8_0", cfg["d_range"])
        self.head = packed(self.vocab, H, "q8_0", (0.001, 0.02))
        nb_row = (ctx_len + 15) // 16
        self.n_blocks = n * nb_row
        self.L = []
        for _ in range(layers):
            self.L.append(dict(
                wqkv=packed((nq + 2 * nk) * d, H, qtype, (0.001, 0.01)),
                wo=packed(H, nq * d, qtype, (0.001, 0.01)), wg=packed(F, H, qtype, (0.001, 0.01)),
                wu=packed(F, H, qtype, (0.001, 0.01)), wd=packed(H, F, qtype, (0.0005, 0.005)),
                n1=1 + 0.02 * r(H), n2=1 + 0.02 * r(H),
                pk=r(self.n_blocks, nk, 16, d), pv=r(self.n_blocks, nk, 16, d)))
        self.nout = 1 + 0.02 * r(H)
        self.ids = torch.randint(0, self.vocab, (n,), device=dev, generator=gen, dtype=torch.int32)
        self.x, self.h, self.ffn = r(n, H), r(n, H), r(n, H)
        self.qkv, self.o, self.attn = r(n, (nq + 2 * nk) * d), r(n, nq * d), r(n, H)
        self.act = r(n, F)
        self.logits = torch.empty((n, self.vocab), device=dev)
        self.out_ids = torch.empty((n,), device=dev, dtype=torch.int32)
        cos, sin = hip.rope_tables(hip.ROPE_NORM, d, cfg["theta"], 8192)
        self.cos, self.sin = torch.from_numpy(cos).to(dev), torch.from_numpy(sin).to(dev)
        tables = np.arange(self.n_blocks, dtype=np.int32).reshape(n, nb_row)
        self.tables = torch.from_numpy(tables).to(dev)
        self.max_blocks = nb_row
        self.pos = torch.from_numpy(np.full(n, ctx_len - 1, np.int32)).to(dev)
        slots = np.concatenate([hip.kv_slots(tables[i].astype(np.uint32), ctx_len - 1, 1, self.n_blocks)
                                for i in range(n)])
        self.slots = torch.from_numpy(slots).to(dev)
        self.ranges = torch.from_numpy(np.tile(np.array([0, ctx_len], np.int32), (n, 1))).to(dev)
        self.ws_bytes = hip.paged_decode_workspace(n, nq, d, nb_row)
        self.ws = torch.empty(max(self.ws_bytes, 16), dtype=torch.uint8, device=dev)
        self.scale = 1.0 / float(np.sqrt(d))
        # the projections: the CPU engine's bits (qmm), or the matrix cores
        # (qgemm, the GPU engine's arithmetic class) with one workspace
        self.mm = mm
        # the Q|K|V projection carries RoPE and the K/V store in its epilogue
        # (cuca_hip_qmm_rope_store_kv) instead of a launch of its own
        self.fuse_rope = fuse_rope and mm == "qmm"
        # the two residual + RMSNorm launches ride in the prologue of the
        # matmul that reads them (cuca_hip_add_rmsnorm_qmm_rope_store_kv,
        # _qmm_glu); the layer's mid residual then goes to x_mid (the fused
        # call's outputs may not overlap its inputs)
        self.fuse_norm = fuse_norm and self.fuse_rope
        self.x_mid = r(n, H)
        if mm == "qgemm":
            self.qg_bytes = max([hip.qgemm_workspace(T, rows, cols, n, glu) for rows, cols, glu in (
                ((nq + 2 * nk) * d, H, False), (H, nq * d, False), (F, H, True), (H, F, False))]
                + [hip.qgemm_workspace(hip.GGML_Q8_0, self.vocab, H, n, False)])
            self.qg_ws = torch.empty(self.qg_bytes, dtype=torch.uint8, device=dev)
        self.weight_bytes = sum(t.numel() for l in self.L for t in (l["wqkv"], l["wo"], l["wg"], l["wu"],
                                                                      l["wd"]))

    def mat(self, w, rows, cols, x, out):
        if self.mm == "qgemm":
            self.ctx.qgemm(w.data_ptr(), self.T, rows, cols, x.data_ptr(), cols, self.n, rows,
                           self.qg_ws.data_ptr(), self.qg_bytes, out.data_ptr(), rows, self.hip.F32)
        else:
            self.ctx.qmm(w.data_ptr(), self.T, rows, cols, x.data_ptr(), cols, self.n, rows, out.data_ptr(),
                         rows, self.hip.F32)

    def issue_layers(self):
        c, hip, cfg, n, T = self.ctx, self.hip, self.cfg, self.n, self.T
        H, F, d, nq, nk, eps = cfg["hidden"], cfg["ff"], cfg["head_dim"], cfg["nq"], cfg["nk"], cfg["eps"]
        f32 = hip.F32
        for l in self.L:
            # one Q|K|V projection; RoPE, the K/V store and the attention
            # read their heads in place from its rows
            qkv_ld = (nq + 2 * nk) * d
            q_ptr = self.qkv.data_ptr()
            if self.fuse_norm:
                c.add_rmsnorm_qmm_rope_store_kv(self.x.data_ptr(), self.ffn.data_ptr(), l["n1"].data_ptr(), eps,
                                                1.0, self.x_mid.data_ptr(), self.h.data_ptr(), l["wqkv"].data_ptr(),
                                                T, H, n, nq, nk, d, d, hip.ROPE_NORM, self.cos.data_ptr(),
                                                self.sin.data_ptr(), 8192, self.pos.data_ptr(), q_ptr, qkv_ld,
                                                l["pk"].data_ptr(), l["pv"].data_ptr(), self.n_blocks,
                                                self.slots.data_ptr(), f32)
            else:
                c.add_rmsnorm(self.x.data_ptr(), self.ffn.data_ptr(), l["n1"].data_ptr(), None, eps, eps, 1.0,
                              n, H, self.x.data_ptr(), self.h.data_ptr(), f32)
                if self.fuse_rope:
                    c.qmm_rope_store_kv(l["wqkv"].data_ptr(), T, H, self.h.data_ptr(), H, n, nq, nk, d, d,
                                        hip.ROPE_NORM, self.cos.data_ptr(), self.sin.data_ptr(), 8192,
                                        self.pos.data_ptr(), q_ptr, qkv_ld, l["pk"].data_ptr(), l["pv"].data_ptr(),
                                        self.n_blocks, self.slots.data_ptr(), f32)
                else:
                    self.mat(l["wqkv"], qkv_ld, H, self.h, self.qkv)
                    c.rope_store_kv(q_ptr, qkv_ld, q_ptr + 4 * nq * d, qkv_ld, q_ptr + 4 * (nq + nk) * d, qkv_ld,
                                    n, nq, nk, d, d, hip.ROPE_NORM, self.cos.data_ptr(), self.sin.data_ptr(), 8192,
                                    self.pos.data_ptr(), None, None, 0, eps, l["pk"].data_ptr(),
                                    l["pv"].data_ptr(), self.n_blocks, self.slots.data_ptr(), f32)
            c.paged_decode(q_ptr, l["pk"].data_ptr(), l["pv"].data_ptr(), self.n_blocks,
                           self.tables.data_ptr(), self.max_blocks, self.ranges.data_ptr(), n, nq, nk, d,
                           self.scale, self.ws.data_ptr(), self.ws_bytes, self.o.data_ptr(), f32,
                           q_ld=qkv_ld)
            self.mat(l["wo"], H, nq * d, self.o, self.attn)
            if self.fuse_norm:
                c.add_rmsnorm_qmm_glu(self.x_mid.data_ptr(), self.attn.data_ptr(), l["n2"].data_ptr(), eps, 1.0,
                                      self.x.data_ptr(), self.h.data_ptr(), l["wg"].data_ptr(), l["wu"].data_ptr(),
                                      T, F, H, n, hip.ACT_SILU, 0.0, self.act.data_ptr(), F, f32)
            else:
                c.add_rmsnorm(self.x.data_ptr(), self.attn.data_ptr(), l["n2"].data_ptr(), None, eps, eps, 1.0,
                              n, H, self.x.data_ptr(), self.h.data_ptr(), f32)
                if self.mm == "qgemm":
                    c.qgemm_glu(l["wg"].data_ptr(), l["wu"].data_ptr(), T, F, H, self.h.data_ptr(), H, n,
                                hip.ACT_SILU, 0.0, self.qg_ws.data_ptr(), self.qg_bytes, self.act.data_ptr(), F,
                                f32)
                else:
                    c.qmm_glu(l["wg"].data_ptr(), l["wu"].data_ptr(), T, F, H, self.h.data_ptr(), H, n,
                              hip.ACT_SILU, 0.0, self.act.data_ptr(), F, f32)
            self.mat(l["wd"], H, F, self.act, self.ffn)

    def issue_step(self):
        c, hip, cfg, n = self.ctx, self.hip, self.cfg, self.n
        H, eps = cfg["hidden"], cfg["eps"]
        c.embed_gguf(self.table.data_ptr(), hip.GGML_Q8_0, self.vocab, H, self.out_ids.data_ptr(), n, 1.0,
                     self.x.data_ptr(), hip.F32)
        self.issue_layers()
        if self.fuse_norm:  # the final norm in the LM head's prologue (no logit scale or soft-cap here)
            c.add_rmsnorm_qmm(self.x.data_ptr(), self.ffn.data_ptr(), self.nout.data_ptr(), eps, 1.0, None,
                              self.h.data_ptr(), self.head.data_ptr(), hip.GGML_Q8_0, self.vocab, H, n, self.vocab,
                              self.logits.data_ptr(), self.vocab, hip.F32)
            c.argmax(self.logits.data_ptr(), self.vocab, n, self.vocab, hip.F32, self.out_ids.data_ptr())
            return
        c.add_rmsnorm(self.x.data_ptr(), self.ffn.data_ptr(), self.nout.data_ptr(), None, eps, eps, 1.0, n,
                      H, self.x.data_ptr(), self.h.data_ptr(), hip.F32)
        if self.mm == "qgemm":  # no logit scale or soft-cap in this model: the plain matmul
            c.qgemm(self.head.data_ptr(), hip.GGML_Q8_0, self.vocab, H, self.h.data_ptr(), H, n, self.vocab,
                    self.qg_ws.data_ptr(), self.qg_bytes, self.logits.data_ptr(), self.vocab, hip.F32)
        else:
            c.lm_head(self.head.data_ptr(), hip.GGML_Q8_0, self.vocab, H, self.h.data_ptr(), H, n, self.vocab,
                      1.0, 1.0, 0.0, self.logits.data_ptr(), self.vocab, hip.F32)
        c.argmax(self.logits.data_ptr(), self.vocab, n, self.vocab, hip.F32, self.out_ids.data_ptr())


# The kernels of a decode layer by role, from their symbol names.
def kernel_role(name):
    if name.startswith(("cuca_qmm_rope_kv", "cuca_qmd_rope_kv")):
        return "qkv_rope_kv"
    if name.startswith(("cuca_qmm", "cuca_qmd", "cuca_qgemm", "cuca_qmv", "cuca_q8_acts")):
        return "matmul"
    if name.startswith("cuca_attn"):
        return "attention"
    if name.startswith(("cuca_norm", "cuca_rope", "cuca_glu")):
        return "non_matmul"
    return "other"


def decode_step_bench(ctx, torch, n, ctx_len, replays=10, mm="qmm", fuse_rope=False, fuse_norm=False):
    """DecodeStep's 32 layers and its whole step, each captured in one
    hipGraph and replayed: microseconds per layer, per step, and tokens/s
    (n tokens per step).  The step's own kernels, timed on the device
    (kernel timestamps of one eager step), give the per-layer split: the
    non-matmul sequence (residual + RMSNorm twice, RoPE + K/V store when it
    is a launch of its own, a separate activation), the matmuls, the fused
    Q|K|V + RoPE + K/V-store launch, attention.  Checked: the step's ids are
    the argmax of its own logits, and the logits are finite."""
    import numpy as np
    ds = DecodeStep(ctx, torch, n, ctx_len, mm=mm, fuse_rope=fuse_rope, fuse_norm=fuse_norm)
    ds.out_ids.copy_(ds.ids)
    torch.cuda.synchronize()
    ds.issue_step()  # eager, once
    torch.cuda.synchronize()
    ctx.check_device()
    ctx.profile_start(16 * ds.layers + 16)
    ds.issue_layers()
    recs = ctx.profile_stop()
    roles = {}
    for k, ms in recs:
        r = kernel_role(k)
        roles[r] = roles.get(r, 0.0) + ms
    split = {r + "_us_per_layer": round(t * 1000 / ds.layers, 2) for r, t in roles.items()}
    # with every non-matmul op fused into a matmul there is no launch of that role
    split.setdefault("non_matmul_us_per_layer", 0.0)
    ctx.graph_begin()
    ds.issue_layers()
    gl = ctx.graph_end()
    layers_ms = time_steps(torch, gl.launch, replays, 2)
    gl.destroy()
    ctx.graph_begin()
    ds.issue_step()
    gs = ctx.graph_end()
    step_ms = time_steps(torch, gs.launch, replays, 2)
    gs.launch()
    torch.cuda.synchronize()
    gs.destroy()
    lg = ds.logits.cpu().numpy()
    got = ds.out_ids.cpu().numpy()
    assert np.all(np.isfinite(lg)), "decode step: non-finite logits"
    assert got.tolist() == [int(np.argmax(lg[i])) for i in range(n)], "decode step: ids"
    wb = ds.weight_bytes
    del ds
    torch.cuda.empty_cache()
    return dict(batch=n, ctx_len=ctx_len, layer_weights="q4_0", head="q8_0", matmul=mm,
                rope_in_qkv_epilogue=bool(fuse_rope and mm == "qmm"),
                norm_in_matmul_prologue=bool(fuse_norm and fuse_rope and mm == "qmm"),
                non_matmul_ops_fused_into=("the Q|K|V, gate/up and LM head prologues (residual + RMSNorm), the Q|K|V "
                                           "epilogue (RoPE + K/V store)" if fuse_norm and fuse_rope and mm == "qmm"
                                           else "the Q|K|V epilogue (RoPE + K/V store)" if fuse_rope and mm == "qmm"
                                           else None),
                us_per_layer=round(layers_ms * 1000 / 32, 2), us_per_step=round(step_ms * 1000, 1),
                tokens_per_s=round(n / (step_ms / 1e3), 1),
                layer_weight_gbs=round(wb / (layers_ms / 1e3) / 1e9, 1), **split)


def decode_us_per_layer(ctx, torch, n, replays=50, ctx_len=None):
    dl = DecodeLayers(ctx, torch, n) if ctx_len is None else DecodeLayersAttn(ctx, torch, n, ctx_len)
    torch.cuda.synchronize()
    eager_ms = time_steps(torch, dl.issue, 10, 3)
    ctx.graph_begin()
    dl.issue()
    g = ctx.graph_end()
    graph_ms = time_steps(torch, g.launch, replays, 5)
    g.destroy()
    return graph_ms * 1000.0 / dl.layers, eager_ms * 1000.0 / dl.layers


def kernel_calls(ctx, call, reps, warmup=5, per_call=8):
    """Run call(i) `reps` times with per-kernel timestamps: returns (median
    of the per-call kernel-time sums in ms, [(kernel, median ms)] of one
    call's launches).  per_call: the most launches one call makes."""
    import numpy as np
    for i in range(warmup):
        call(i)
    ctx.sync()
    ctx.profile_start(per_call * reps)
    for i in range(reps):
        call(i)
    recs = ctx.profile_stop()
    ctx.check_device()
    per = len(recs) // reps
    calls = [recs[i * per:(i + 1) * per] for i in range(reps)]
    parts = [(k, float(np.median([c[j][1] for c in calls]))) for j, (k, _) in enumerate(calls[0])]
    return float(np.median([sum(t for _, t in c) for c in calls])), parts


# Llama-3-8B's decode matmuls (n rows of weights, k inputs): the fused
# gate/up GLU, down, q/o, k/v; then the LM head.
QMM_SHAPES = (("gate_up", 14336, 4096, True), ("down", 4096, 14336, False),
              ("q_o", 4096, 4096, False), ("k_v", 1024, 4096, False))


def qmm_bench(ctx, torch, reps=30):
    """The quantized matmul (cuca_hip_qmm, cuca_hip_qmm_glu) at the 8B
    decode shapes, Q4_0 and Q8_0, f32 activations, 1 and 4 rows.  Weights
    are rotated over copies totalling > 256 MiB so that no call finds its
    weights in the last-level cache.  Algorithmic bytes per call: the weight
    blocks (18 or 34 bytes per 32 values; both matrices for the GLU), the
    activations in and the outputs, f32.  Each shape's first 64 output
    columns are checked bit for bit against the oracle (the GLU's
    activation to 1e-5 relative)."""
    import numpy as np
    from cuca_amd import hip, ops
    from cuca_amd import workloads as W
    from oracle import oracle as O
    res = {}
    for qtype in ("q4_0", "q8_0"):
        gid = W.GGML_ID[qtype]
        for name, n, k, glu in QMM_SHAPES:
            rng = np.random.default_rng(n + k)
            raws = [W.quant_table(rng, n, k, qtype, (0.001, 0.02)) for _ in range(2 if glu else 1)]
            wbytes = sum(r.size for r in raws)
            copies = max(2, int(np.ceil(320e6 / wbytes)))
            ws = [[ops.QmmWeight.from_raw(ctx, gid, r, n, k) for r in raws] for _ in range(copies)]
            for m in (1, 4):
                x = rng.standard_normal((m, k)).astype(np.float32)
                dx = ctx.array(x)
                out = ctx.empty((m, n), np.float32)

                def call(i, dx=dx, out=out):
                    w = ws[i % copies]
                    if glu:
                        ops.QmmWeight.glu(w[0], w[1], dx, ops.Glu(hip.ACT_SILU), out=out)
                    else:
                        w[0].forward(dx, out=out)
                ms, parts = kernel_calls(ctx, call, reps)
                call(0)
                got = out.numpy()[:, :64]
                want = [O.qmm(r, gid, n, k, x, rows=64, threads=8) for r in raws]
                if glu:
                    want = O.glu(want[0], want[1], hip.ACT_SILU)
                    assert np.all(np.abs(got - want) <= 1e-5 * np.abs(want) + 1e-30), f"qmm {name} {qtype}"
                else:
                    assert np.array_equal(got.view(np.uint32), want[0].view(np.uint32)), f"qmm {name} {qtype}"
                b = wbytes + m * k * 4 + m * n * 4
                res[f"{name}_{qtype}_m{m}"] = dict(
                    kernels=[p for p, _ in parts], us=round(ms * 1000, 2), bytes=b,
                    gbs=round(b / (ms / 1e3) / 1e9, 1), frac=round(b / (ms / 1e3) / 1e9 / HBM_PEAK_GBS, 4))
                dx.free()
                out.free()
            for w in ws:
                for q in w:
                    q.packed.free()
    return res


def qgemm_bench(ctx, torch, reps=10):
    """The matrix-core quantized matmul (cuca_hip_qgemm / _qgemm_glu) at the
    8B layer shapes, Q4_0, f32 activations, 32, 512 and 4096 rows (a decode
    batch, a chunk of prefill, a prefill): kernel time of the call (the
    activation prep, the matmul, the split reduce when there is one), its
    f16 TFLOP/s against the 2.5 PFLOP/s dense peak.  Weights are generated
    as GGUF bytes on the device; every output of sampled rows is checked
    against the f64 product of the dequantised weights within the kernel's
    bound (2^-10 + k 2^-24) sum |w x|."""
    import numpy as np
    from cuca_amd import hip
    from cuca_amd import workloads as W
    from oracle import oracle as O
    gen = torch.Generator(device="cuda").manual_seed(7)
    T = hip.GGML_Q4_0
    res = {}
    for name, n, k, glu in (("gate_up", 14336, 4096, True), ("down", 4096, 14336, False), ("q_o", 4096, 4096, False)):
        raws = [W.quant_table_torch(gen, n, k, "q4_0", (0.001, 0.02)) for _ in range(2 if glu else 1)]
        ws = []
        for r in raws:
            p = torch.empty(hip.qweight_bytes(T, n, k), dtype=torch.uint8, device="cuda")
            ctx.qweight_pack(r.data_ptr(), T, n, k, p.data_ptr())
            ws.append(p)
        torch.cuda.synchronize()
        for m in (32, 512, 4096):
            x = torch.randn(m, k, device="cuda", generator=gen)
            out = torch.empty(m, n, device="cuda")
            wsb = hip.qgemm_workspace(T, n, k, m, glu)
            wsp = torch.empty(wsb, dtype=torch.uint8, device="cuda")

            def call(i, x=x, out=out, wsp=wsp, wsb=wsb, m=m):
                if glu:
                    ctx.qgemm_glu(ws[0].data_ptr(), ws[1].data_ptr(), T, n, k, x.data_ptr(), k, m,
                                  hip.ACT_SILU, 0.0, wsp.data_ptr(), wsb, out.data_ptr(), n, hip.F32)
                else:
                    ctx.qgemm(ws[0].data_ptr(), T, n, k, x.data_ptr(), k, m, n, wsp.data_ptr(), wsb,
                              out.data_ptr(), n, hip.F32)
            ms, parts = kernel_calls(ctx, call, reps, 2)
            call(0)
            torch.cuda.synchronize()
            # check 3 token rows x 256 weight rows against the f64 product
            toks = [0, m // 2, m - 1]
            xs = x[toks].cpu().numpy().astype(np.float64)
            rb = W.row_bytes("q4_0", k)
            cols = np.arange(0, n, max(1, n // 256))[:256]
            sel = torch.from_numpy(cols).to("cuda")
            dq = []
            for r in raws:
                rows_b = r.view(n, rb).index_select(0, sel).cpu().numpy()
                dq.append(np.stack([O.dequant_row(T, rows_b[i], 1.0, k) for i in range(cols.size)]).astype(np.float64))
            got = out[toks][:, cols].cpu().numpy().astype(np.float64)
            g = xs @ dq[0].T
            bg = (2.0 ** -10 + k * 2.0 ** -24) * (np.abs(xs) @ np.abs(dq[0]).T)
            if glu:
                u = xs @ dq[1].T
                bu = (2.0 ** -10 + k * 2.0 ** -24) * (np.abs(xs) @ np.abs(dq[1]).T)
                a = g / (1.0 + np.exp(-g))
                want, tol = a * u, 1.2 * bg * (np.abs(u) + bu) + np.abs(a) * bu + 1e-5 * np.abs(a * u)
            else:
                want, tol = g, bg
            assert np.all(np.abs(got - want) <= tol + 1e-30), f"qgemm {name} m={m}"
            flops = 2.0 * m * n * k * (2 if glu else 1)
            res[f"{name}_q4_0_m{m}"] = dict(
                kernels=[p for p, _ in parts], us=round(ms * 1000, 2), parts_us=[round(t * 1000, 2) for _, t in parts],
                tflops=round(flops / (ms / 1e3) / 1e12, 1), mfma_frac=round(flops / (ms / 1e3) / 2.5e15, 4))
        del ws, raws
        torch.cuda.empty_cache()
    return res


def prefill_layer_bench(ctx, torch, name="C", n=4096, reps=5, dense=False):
    """A whole prefill layer of config `name` at n f16 tokens on this
    library, end to end: the fused gather + first-block norm, the Q|K|V
    projection (cuca_hip_qgemm, Q4_0), RoPE + paged K/V store, the causal
    attention of the n rows over the cache they were just stored in
    (cuca_hip_attend_rows), the output projection, residual + norm, the
    gate/up projection with the SwiGLU in its epilogue (cuca_hip_qgemm_glu),
    down, residual + norm.  dense: the four projections on the dense f16
    path instead (the Q4_0 weights dequantised once, untimed, then
    cuca_hip_gemm_w16 / _gemm_w16_glu: the reference GPU engine's prefill
    form).  Per op: kernel time (per-kernel timestamps, median of `reps`
    layers); the attention also as TFLOP/s of its causal products (4 d heads
    per (row, key) pair).  Checked: sampled attention rows against the
    oracle's attend_paged_rows, finite outputs."""
    import numpy as np
    from cuca_amd import hip
    from cuca_amd import workloads as W
    from oracle import oracle as O
    cfg = W.CONFIGS[name]
    H, F, nq, nk, d, eps = cfg["hidden"], cfg["ff"], cfg["nq"], cfg["nk"], cfg["head_dim"], cfg["eps"]
    T, f16 = hip.GGML_Q4_0, hip.F16
    dev, hf = "cuda", torch.float16
    gen = torch.Generator(device=dev).manual_seed(cfg["seed"] * 31 + n)
    nqkv = (nq + 2 * nk) * d

    def weight(rows, k):
        raw = W.quant_table_torch(gen, rows, k, "q4_0", (0.001, 0.02))
        p = torch.empty(hip.qweight_bytes(T, rows, k), dtype=torch.uint8, device=dev)
        ctx.qweight_pack(raw.data_ptr(), T, rows, k, p.data_ptr())
        return p
    wqkv, wo, wg, wu, wd = weight(nqkv, H), weight(H, nq * d), weight(F, H), weight(F, H), weight(H, F)
    table_e = W.quant_table_torch(gen, cfg["vocab"], H, cfg["qtype"], cfg["d_range"])
    ids = torch.randint(0, cfg["vocab"], (n,), device=dev, generator=gen, dtype=torch.int32)
    wn = [(1 + 0.02 * torch.randn(H, device=dev, generator=gen)).float() for _ in range(3)]
    x, h = torch.empty((n, H), device=dev, dtype=hf), torch.empty((n, H), device=dev, dtype=hf)
    qkv = torch.empty((n, nqkv), device=dev, dtype=hf)
    attn = torch.empty((n, nq * d), device=dev, dtype=hf)
    br = torch.empty((n, H), device=dev, dtype=hf)
    act = torch.empty((n, F), device=dev, dtype=hf)
    n_blocks = n // 16 + 8
    pk = torch.zeros((n_blocks, nk, 16, d), device=dev, dtype=hf)
    pv = torch.zeros_like(pk)
    rng = np.random.default_rng(cfg["seed"] + n)
    table = rng.permutation(n_blocks)[: (n + 15) // 16].astype(np.uint32)
    slots = torch.from_numpy(hip.kv_slots(table, 0, n, n_blocks)).to(dev)
    dtab = torch.from_numpy(table.view(np.int32)).to(dev)
    ranges_np = np.stack([np.zeros(n), np.arange(n) + 1], 1).astype(np.int32)
    ranges = torch.from_numpy(ranges_np).to(dev)
    pos = torch.arange(n, dtype=torch.int32, device=dev)
    kind = hip.ROPE_NEOX if cfg["rope"] == "neox" else hip.ROPE_NORM
    cos, sin = hip.rope_tables(kind, d, cfg["theta"], n)
    dcos, dsin = torch.from_numpy(cos).to(dev), torch.from_numpy(sin).to(dev)
    qn = kn = None
    if cfg.get("qk_norm"):
        qn = (1 + 0.02 * torch.randn(d, device=dev, generator=gen)).float()
        kn = (1 + 0.02 * torch.randn(d, device=dev, generator=gen)).float()
    wsb = max(hip.qgemm_workspace(T, nqkv, H, n), hip.qgemm_workspace(T, H, nq * d, n),
              hip.qgemm_workspace(T, F, H, n, True), hip.qgemm_workspace(T, H, F, n))
    dq_us = 0.0
    if dense:  # resident f16 copies (gate rows, then up rows, for the GLU)
        def w16_of(ps, rows, k):
            w = torch.empty((len(ps) * rows, k), dtype=hf, device=dev)
            for i, p in enumerate(ps):
                ctx.qweight_dequant(p.data_ptr(), T, rows, k, w.data_ptr() + i * rows * k * 2)
            return w
        t0 = time.perf_counter()
        wqkv, wo, wgu, wd = w16_of([wqkv], nqkv, H), w16_of([wo], H, nq * d), w16_of([wg, wu], F, H), w16_of([wd], H, F)
        torch.cuda.synchronize()
        dq_us = (time.perf_counter() - t0) * 1e6
        wg = wu = None
        wsb = max(hip.gemm_w16_workspace(nqkv, H, n, False, f16), hip.gemm_w16_workspace(H, nq * d, n, False, f16),
                  hip.gemm_w16_workspace(F, H, n, True, f16), hip.gemm_w16_workspace(H, F, n, False, f16), 16)
    wsp = torch.empty(wsb, dtype=torch.uint8, device=dev)

    def matmul(w, rows, k, xin, out):
        if dense:
            return ctx.gemm_w16(w.data_ptr(), rows, k, xin.data_ptr(), k, n, rows, wsp.data_ptr(), wsb,
                                out.data_ptr(), rows, f16)
        return ctx.qgemm(w.data_ptr(), T, rows, k, xin.data_ptr(), k, n, rows, wsp.data_ptr(), wsb, out.data_ptr(),
                         rows, f16)
    scale = 1.0 / float(np.sqrt(d))
    ops = []

    def op(label, fn):
        ops.append((label, fn))
    op("embed_rms", lambda: ctx.embed_gguf_rms(table_e.data_ptr(), W.GGML_ID[cfg["qtype"]], cfg["vocab"], H,
                                               ids.data_ptr(), n, cfg["embd_scale"], wn[0].data_ptr(), eps,
                                               x.data_ptr(), h.data_ptr(), f16))
    op("qkv_matmul", lambda: matmul(wqkv, nqkv, H, h, qkv))
    op("rope_store_kv", lambda: ctx.rope_store_kv(
        qkv.data_ptr(), nqkv, qkv.data_ptr() + 2 * nq * d, nqkv, qkv.data_ptr() + 2 * (nq + nk) * d, nqkv, n, nq,
        nk, d, d, kind, dcos.data_ptr(), dsin.data_ptr(), n, pos.data_ptr(),
        None if qn is None else qn.data_ptr(), None if kn is None else kn.data_ptr(), bool(cfg.get("qk_norm")),
        eps, pk.data_ptr(), pv.data_ptr(), n_blocks, slots.data_ptr(), f16))
    op("attention", lambda: ctx.attend_rows(qkv.data_ptr(), nqkv, pk.data_ptr(), pv.data_ptr(), n_blocks,
                                            dtab.data_ptr(), len(table), ranges.data_ptr(), n, nq, nk, d, scale,
                                            attn.data_ptr(), nq * d, f16))
    op("o_matmul", lambda: matmul(wo, H, nq * d, attn, br))
    op("add_rmsnorm_attn", lambda: ctx.add_rmsnorm(x.data_ptr(), br.data_ptr(), wn[1].data_ptr(), None, eps, eps,
                                                   1.0, n, H, x.data_ptr(), h.data_ptr(), f16))
    if dense:
        op("gate_up_glu_matmul", lambda: ctx.gemm_w16_glu(wgu.data_ptr(), F, H, h.data_ptr(), H, n, hip.ACT_SILU, 0.0,
                                                          wsp.data_ptr(), wsb, act.data_ptr(), F, f16))
    else:
        op("gate_up_glu_matmul", lambda: ctx.qgemm_glu(wg.data_ptr(), wu.data_ptr(), T, F, H, h.data_ptr(), H, n,
                                                       hip.ACT_SILU, 0.0, wsp.data_ptr(), wsb, act.data_ptr(), F,
                                                       f16))
    op("down_matmul", lambda: matmul(wd, H, F, act, br))
    op("add_rmsnorm_ffn", lambda: ctx.add_rmsnorm(x.data_ptr(), br.data_ptr(), wn[2].data_ptr(), None, eps, eps,
                                                  1.0, n, H, x.data_ptr(), h.data_ptr(), f16))
    torch.cuda.synchronize()
    # one layer, then check the attention of sampled rows against the oracle
    for _, fn in ops[:4]:
        fn()
    torch.cuda.synchronize()
    ctx.check_device()
    rows = np.array([0, 1, 15, 16, 777, n // 2, n - 1])
    q_rows = qkv[torch.from_numpy(rows).to(dev), : nq * d].cpu().numpy().reshape(len(rows), nq, d)
    want = O.paged_attention(q_rows, np.repeat(table[None], len(rows), 0), ranges_np[rows], pk.cpu().numpy(),
                             pv.cpu().numpy(), scale, threads=8)
    got = attn[torch.from_numpy(rows).to(dev)].cpu().numpy().reshape(len(rows), nq, d)
    vmax = np.abs(pv.cpu().numpy().astype(np.float64)).max()
    ulp = np.spacing(np.abs(want).astype(np.float16)).astype(np.float64)
    assert np.all(np.abs(got.astype(np.float64) - want) <= 2 * ulp + 1e-5 * vmax), "prefill layer attention"
    # timed layers (the K/V store and attention rewrite the same pool rows)
    counts = []
    for _, fn in ops:
        ctx.profile_start(64)
        fn()
        counts.append(len(ctx.profile_stop()))

    def layer(i):
        for _, fn in ops:
            fn()
    ms, parts = kernel_calls(ctx, layer, reps, 2, per_call=sum(counts))
    assert len(parts) == sum(counts), (len(parts), counts)
    assert torch.isfinite(h.float()).all(), "prefill layer: non-finite h"
    per, j = {}, 0
    for (label, _), c in zip(ops, counts):
        per[label] = dict(kernels=[k for k, _ in parts[j:j + c]], us=round(sum(t for _, t in parts[j:j + c]) * 1000, 2))
        j += c
    att_flops = 4.0 * d * nq * (n * (n + 1) / 2)
    per["attention"]["tflops"] = round(att_flops / (per["attention"]["us"] / 1e6) / 1e12, 1)
    per["attention"]["mfma_frac"] = round(att_flops / (per["attention"]["us"] / 1e6) / 2.5e15, 4)
    mm = sum(per[k]["us"] for k in ("qkv_matmul", "o_matmul", "gate_up_glu_matmul", "down_matmul"))
    del wqkv, wo, wg, wu, wd, table_e
    if dense:
        del wgu
    torch.cuda.empty_cache()
    res = dict(config=name, tokens=n, dtype="f16", weights="q4_0 dequantised to f16 once" if dense else "q4_0",
               us_per_layer=round(ms * 1000, 1), tokens_per_s_per_layer=round(n / (ms / 1e3), 0),
               matmul_us=round(mm, 1), attention_us=per["attention"]["us"], checked_attention_rows=int(rows.size),
               ops=per)
    if dense:
        res["dequant_once_us"] = round(dq_us, 1)
    return res


def gemm_w16_bench(ctx, torch, reps=10):
    """The dense f16 path for many rows (cuca_hip_qweight_dequant once, then
    cuca_hip_gemm_w16 / _gemm_w16_glu per call: the library's f16 GEMM on
    the matrix cores, f32 accumulation, the GLU in registers) at the 8B
    layer shapes, 512 and 4096 rows of f32 activations and 4096 of f16: time
    of the whole call on the stream (the f16 rounding of f32 activations
    and the GEMM), its f16 TFLOP/s against
    the 2.5 PFLOP/s dense peak, and the one-time dequantisation.  Sampled
    outputs are checked against the f64 product within the qgemm bound."""
    import numpy as np
    from cuca_amd import hip
    from cuca_amd import workloads as W
    from oracle import oracle as O
    gen = torch.Generator(device="cuda").manual_seed(9)
    T = hip.GGML_Q4_0
    res = {}
    for name, n, k, glu in (("gate_up", 14336, 4096, True), ("down", 4096, 14336, False), ("q_o", 4096, 4096, False)):
        raws = [W.quant_table_torch(gen, n, k, "q4_0", (0.001, 0.02)) for _ in range(2 if glu else 1)]
        w16 = torch.empty((len(raws) * n, k), dtype=torch.float16, device="cuda")
        packed = torch.empty(hip.qweight_bytes(T, n, k), dtype=torch.uint8, device="cuda")
        dq_ms = 0.0
        for i, r in enumerate(raws):
            ctx.qweight_pack(r.data_ptr(), T, n, k, packed.data_ptr())
            dq_ms += time_steps(torch, lambda i=i: ctx.qweight_dequant(packed.data_ptr(), T, n, k,
                                                                       w16.data_ptr() + i * n * k * 2), 3, 1)
        del packed
        torch.cuda.synchronize()
        for m, dt in ((512, "f32"), (4096, "f32"), (4096, "f16")):
            tdt, code = (torch.float16, hip.F16) if dt == "f16" else (torch.float32, hip.F32)
            x = torch.randn(m, k, device="cuda", generator=gen).to(tdt)
            out = torch.empty(m, n, device="cuda", dtype=tdt)
            wsb = hip.gemm_w16_workspace(n, k, m, glu, code)
            wsp = torch.empty(wsb, dtype=torch.uint8, device="cuda")

            def call(x=x, out=out, wsp=wsp, wsb=wsb, m=m, code=code):
                if glu:
                    ctx.gemm_w16_glu(w16.data_ptr(), n, k, x.data_ptr(), k, m, hip.ACT_SILU, 0.0, wsp.data_ptr(),
                                     wsb, out.data_ptr(), n, code)
                else:
                    ctx.gemm_w16(w16.data_ptr(), n, k, x.data_ptr(), k, m, n, wsp.data_ptr(), wsb, out.data_ptr(),
                                 n, code)
            ms = time_steps(torch, call, reps, 3)
            call()
            torch.cuda.synchronize()
            toks = [0, m // 2, m - 1]
            xs = x[toks].float().cpu().numpy().astype(np.float64)
            rb = W.row_bytes("q4_0", k)
            cols = np.arange(0, n, max(1, n // 256))[:256]
            sel = torch.from_numpy(cols).to("cuda")
            dq = []
            for r in raws:
                rows_b = r.view(n, rb).index_select(0, sel).cpu().numpy()
                dq.append(np.stack([O.dequant_row(T, rows_b[i], 1.0, k) for i in range(cols.size)]).astype(np.float64))
            got = out[toks][:, cols].float().cpu().numpy().astype(np.float64)
            g = xs @ dq[0].T
            bg = (2.0 ** -10 + k * 2.0 ** -24) * (np.abs(xs) @ np.abs(dq[0]).T)
            if glu:
                u = xs @ dq[1].T
                bu = (2.0 ** -10 + k * 2.0 ** -24) * (np.abs(xs) @ np.abs(dq[1]).T)
                a = g / (1.0 + np.exp(-g))
                want, tol = a * u, 1.2 * bg * (np.abs(u) + bu) + np.abs(a) * bu + 1e-5 * np.abs(a * u)
            else:
                want, tol = g, bg
            if dt == "f16":
                tol = tol + 2.0 ** -11 * np.abs(want)
            assert np.all(np.abs(got - want) <= tol + 1e-30), f"gemm_w16 {name} m={m} {dt}"
            flops = 2.0 * m * n * k * (2 if glu else 1)
            res[f"{name}_q4_0_m{m}_{dt}"] = dict(
                us=round(ms * 1000, 2), tflops=round(flops / (ms / 1e3) / 1e12, 1),
                mfma_frac=round(flops / (ms / 1e3) / 2.5e15, 4), dequant_once_us=round(dq_ms * 1000, 1),
                w16_bytes=int(w16.numel() * 2))
        del w16, raws
        torch.cuda.empty_cache()
    return res


def moe_bench(ctx, torch, reps=30):
    """Routed experts at config E (Qwen3-30B-A3B: 128 experts of ff 768 over
    hidden 2048, Q4_0, top 8): moe_up (gate/up + SwiGLU), moe_down (times the
    routing weight), moe_sum, f32, at decode batches of 1 and 32 tokens with
    uniform routing; and at an 8192-token prefill (below).  Algorithmic bytes: the weights of the experts the
    batch touches, the tokens' rows in, the hidden rows out and back in, the
    output rows.  Checked against the oracle's expert_sum to 1e-4 of each
    token's largest |output| (the bar of the layer test)."""
    import numpy as np
    from cuca_amd import hip, ops
    from cuca_amd import workloads as W
    from oracle import oracle as O
    cfg = W.CONFIGS["E"]
    H, F = cfg["hidden"], cfg["ff"]
    n_exp, n_used = cfg["moe"]
    qtype = cfg["qtype"]
    rng = np.random.default_rng(5)
    # eight distinct expert triples, each packed into every sixteenth slot:
    # 128 separate experts in memory (340 MB), no two slots sharing bytes
    base = [(W.quant_table(rng, F, H, qtype, (0.01, 0.05)), W.quant_table(rng, F, H, qtype, (0.01, 0.05)),
             W.quant_table(rng, H, F, qtype, (0.004, 0.02))) for _ in range(8)]
    experts = [base[e % 8] for e in range(n_exp)]
    bank = ops.ExpertBank.from_raw(ctx, W.GGML_ID[qtype], experts, H, F)
    per_matrix = [m.size for m in base[0]]
    res = {}
    for t in (1, 32):
        x = rng.standard_normal((t, H)).astype(np.float32)
        dx = ctx.array(x)
        per = [[] for _ in range(n_exp)]
        for tok in range(t):
            for e, w in zip(sorted(rng.choice(n_exp, n_used, replace=False)),
                            rng.uniform(0.05, 1.0, n_used).astype(np.float32)):
                per[e].append((tok, float(w)))
        touched = sum(1 for p in per if p)
        keep = []

        def call(i):
            keep.append(bank.expert_sum(dx, per, ops.Glu(hip.ACT_SILU), n_used))
            if len(keep) > 4:
                keep.pop(0)
        ms, parts = kernel_calls(ctx, call, reps)
        out = keep[-1][0].numpy()
        want, _ = O.expert_sum(x, experts, W.GGML_ID[qtype], per, hip.ACT_SILU, threads=8)
        assert np.all(np.abs(out - want) <= 1e-4 * np.abs(want).max(-1, keepdims=True)), "moe"
        pairs = t * n_used
        b = touched * sum(per_matrix) + t * H * 4 + 2 * pairs * F * 4 + t * H * 4
        res[f"E_decode_t{t}"] = dict(kernels=[p for p, _ in parts], us=round(ms * 1000, 2),
                                     parts_us=[round(v * 1000, 2) for _, v in parts],
                                     experts_touched=touched, bytes=b, gbs=round(b / (ms / 1e3) / 1e9, 1),
                                     frac=round(b / (ms / 1e3) / 1e9 / HBM_PEAK_GBS, 4))
        keep.clear()
        dx.free()
    # prefill: 8192 tokens of f16 activations, Zipf(1.1) routing (65536
    # pairs, a few hot experts), the up and down projections as grouped GEMMs
    # on the matrix cores (cuca_hip_moe_up_qgemm / _down_qgemm) against the
    # decode GEMV path at the same size.  FLOPs: 2 pairs (2 ff H + H ff).
    # Checked: four tokens' outputs against their f64 value over the
    # dequantised weights (1e-2 of the token's largest |output|).
    t = 8192
    p = 1.0 / np.arange(1, n_exp + 1) ** 1.1
    p = p / p.sum()
    per = [[] for _ in range(n_exp)]
    for tok in range(t):
        for e, w in zip(sorted(rng.choice(n_exp, n_used, replace=False, p=p)),
                        rng.uniform(0.05, 1.0, n_used).astype(np.float32)):
            per[e].append((tok, float(w)))
    x = (rng.standard_normal((t, H)) * 0.35).astype(np.float16)
    dx = ctx.array(x)
    pairs = t * n_used
    flops = 2.0 * pairs * (2 * F * H + H * F)
    for mm, reps_mm in (("qgemm", 10), ("qmm", 2)):
        keep = []

        def call(i, mm=mm):
            keep.append(bank.expert_sum(dx, per, ops.Glu(hip.ACT_SILU), n_used, mm=mm))
            if len(keep) > 2:
                keep.pop(0)
        ms, parts = kernel_calls(ctx, call, reps_mm, 1)
        entry = dict(kernels=[k for k, _ in parts], us=round(ms * 1000, 2),
                     parts_us=[round(v * 1000, 2) for _, v in parts], pairs=pairs,
                     max_pairs_per_expert=max(len(q) for q in per),
                     tflops=round(flops / (ms / 1e3) / 1e12, 1), mfma_frac=round(flops / (ms / 1e3) / 2.5e15, 4))
        if mm == "qgemm":
            out = keep[-1][0].numpy()
            deq = [tuple(np.stack([O.dequant_row(W.GGML_ID[qtype], m[i * W.row_bytes(qtype, k):(i + 1) *
                                                                     W.row_bytes(qtype, k)], 1.0, k)
                                   for i in range(n)]).astype(np.float64)
                         for m, n, k in ((b[0], F, H), (b[1], F, H), (b[2], H, F))) for b in base]
            for tok in (0, 1, t // 2, t - 1):
                want = np.zeros(H)
                for e, picks in enumerate(per):
                    for tt, w in picks:
                        if tt == tok:
                            wg, wu, wd = deq[e % 8]
                            xr = x[tok].astype(np.float64)
                            g, u = wg @ xr, wu @ xr
                            want += (wd @ (g / (1.0 + np.exp(-g)) * u)) * w
                assert np.all(np.abs(out[tok] - want) <= 1e-2 * np.abs(want).max()), "moe qgemm"
        res[f"E_prefill_t{t}_{mm}"] = entry
        keep.clear()
    dx.free()
    for p in (bank.gate, bank.up, bank.down):
        p.free()
    return res


def head_bench(ctx, torch, reps=30):
    """The end of a decode step for the 8B model at batch 1, f32: the LM head
    (cuca_hip_lm_head, Q8_0 and Q4_0 128256 x 4096; the decode GEMV after the
    activation quantisation) with the logits written once, then greedy
    (cuca_hip_argmax) or top-k 40 at temperature 0.8 (cuca_hip_top_k).
    Algorithmic bytes of the head: the weight blocks, the row in, the logits
    out.  Checked: the first 64 logits bit for bit, the argmax and the top-k
    against the oracle on the device's own logits."""
    import numpy as np
    from cuca_amd import hip, ops
    from cuca_amd import workloads as W
    from oracle import oracle as O
    vocab, H = 128256, 4096
    res = {}
    for qtype in ("q8_0", "q4_0"):
        gid = W.GGML_ID[qtype]
        rng = np.random.default_rng(9)
        raw = W.quant_table(rng, vocab, H, qtype, (0.001, 0.02))
        ws = [ops.QmmWeight.from_raw(ctx, gid, raw, vocab, H) for _ in range(2)]
        x = rng.standard_normal((1, H)).astype(np.float32)
        dx = ctx.array(x)
        logits = ctx.empty((1, vocab), np.float32)
        ids = ctx.empty((1,), np.uint32)
        tl, ti, tc = ctx.empty((1, 40), np.float32), ctx.empty((1, 40), np.uint32), ctx.empty((1,), np.int32)

        def head(i):
            w = ws[i % 2]
            ctx.lm_head(w.packed.ptr, gid, vocab, H, dx.ptr, H, 1, vocab, 1.0, 1.0, 0.0, logits.ptr,
                        vocab, hip.F32)
        ms, parts = kernel_calls(ctx, head, reps)
        b = raw.size + H * 4 + vocab * 4
        r = dict(kernels=[p for p, _ in parts], us=round(ms * 1000, 2), bytes=b,
                 gbs=round(b / (ms / 1e3) / 1e9, 1), frac=round(b / (ms / 1e3) / 1e9 / HBM_PEAK_GBS, 4))
        if qtype == "q8_0":
            g_ms, _ = kernel_calls(ctx, lambda i: ctx.argmax(logits.ptr, vocab, 1, vocab, hip.F32, ids.ptr),
                                   reps)
            k_ms, _ = kernel_calls(ctx, lambda i: ctx.top_k(logits.ptr, vocab, 1, vocab, hip.F32, 40, 0.8,
                                                              tl.ptr, ti.ptr, tc.ptr), reps)
            r.update(argmax_us=round(g_ms * 1000, 2), top_k40_us=round(k_ms * 1000, 2))
        head(0)
        ctx.argmax(logits.ptr, vocab, 1, vocab, hip.F32, ids.ptr)
        ctx.top_k(logits.ptr, vocab, 1, vocab, hip.F32, 40, 0.8, tl.ptr, ti.ptr, tc.ptr)
        lg = logits.numpy()
        want = O.qmm(raw, gid, vocab, H, x, rows=64, threads=8)
        assert np.array_equal(lg[:, :64].view(np.uint32), want.view(np.uint32)), "lm head"
        assert int(ids.numpy()[0]) == O.greedy(lg[0]), "argmax"
        wl, wi = O.select_top_k(lg[0], 0.8, 40)
        assert ti.numpy()[0, :tc.numpy()[0]].tolist() == wi.tolist(), "top-k"
        res[f"lm_head_{qtype}_b1"] = r
        for a in (dx, logits, ids, tl, ti, tc):
            a.free()
        for w in ws:
            w.packed.free()
    return res


def host_cpu():
    """(CPU model, logical CPUs of the host, CPUs this process may run on,
    threads the baseline uses).  The threads are the CPUs this process is
    given -- a GPU box grants one GPU's job a share of its host (the
    OMP_NUM_THREADS it exports), not the whole machine."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    total = os.cpu_count() or 1
    avail = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else total
    try:
        share = int(os.environ.get("OMP_NUM_THREADS", "") or avail)
    except ValueError:
        share = avail
    return model, total, avail, max(1, min(avail, share))


def cpu_baseline(st, seconds=12.0):
    """The oracle -- the candle-equivalent C restatement of the reference's
    CPU path -- over the same step as the GPU line: config C at st.n tokens,
    on the very inputs the GPU step read (copied from the device), with
    preallocated outputs and the oracle's persistent thread pool.  Each op is
    repeated for about seconds / 5 and its median call time taken; per-op
    GB/s use the GPU ops' algorithmic bytes, and the step time is the sum of
    the ops' medians."""
    import ctypes
    import numpy as np
    from oracle import oracle as O
    L = O.lib()
    model, total, avail, threads = host_cpu()
    cfg, n = st.cfg, st.n
    H, F, d, nq, nk = cfg["hidden"], cfg["ff"], cfg["head_dim"], cfg["nq"], cfg["nk"]
    f16 = st.dt == st.hip.F16
    dt = O.F16 if f16 else O.F32
    npdt = np.float16 if f16 else np.float32

    def host(t):
        return np.ascontiguousarray(t.cpu().numpy())

    def ptr(a):
        return a.ctypes.data

    table, ids = host(st.table), host(st.ids).astype(np.uint32)
    emb = np.empty((n, H), npdt)
    emb_h = np.empty((n, H), npdt)
    emb_w = host(st.emb_w)
    bad = ctypes.c_int64(-1)
    norm = [dict(x=host(b["x"]), b=host(b["b"]), w=host(b["w"]), xo=np.empty((n, H), npdt),
                 h=np.empty((n, H), npdt)) for b in st.norm]
    q, k = host(st.q0), host(st.k0)
    cos, sin, pos = host(st.cos), host(st.sin), host(st.pos).astype(np.int32)
    gu = host(st.gu)
    out = np.empty((n, F), npdt)
    kind = O.ROPE_NEOX if st.kind == st.hip.ROPE_NEOX else O.ROPE_NORM
    act = O.GELU_TANH if st.act == st.hip.ACT_GELU_TANH else O.SILU
    es = 2 if f16 else 4

    def embed_rms():
        L.oracle_embed(ptr(table), st.qtype, cfg["vocab"], H, ptr(ids), n, cfg["embd_scale"], ptr(emb), dt,
                       threads, ctypes.byref(bad))
        L.oracle_add_rmsnorm(ptr(emb), None, ptr(emb_w), None, cfg["eps"], cfg["eps"], 1.0, n, H, None,
                             ptr(emb_h), dt, threads)

    def add_rmsnorm(b):
        return lambda: L.oracle_add_rmsnorm(ptr(b["x"]), ptr(b["b"]), ptr(b["w"]), None, cfg["eps"],
                                            cfg["eps"], 1.0, n, H, ptr(b["xo"]), ptr(b["h"]), dt, threads)

    def rope():
        L.oracle_rope(ptr(q), nq * d, n, nq, d, d, kind, ptr(cos), ptr(sin), ptr(pos), None, cfg["eps"], dt,
                      threads)
        L.oracle_rope(ptr(k), nk * d, n, nk, d, d, kind, ptr(cos), ptr(sin), ptr(pos), None, cfg["eps"], dt,
                      threads)

    def glu():
        L.oracle_glu(ptr(gu), 2 * F, gu.ctypes.data + F * es, 2 * F, n, F, act, 0.0, ptr(out), F, dt, threads)

    fns = {"embed_rms": embed_rms, "add_rmsnorm_attn": add_rmsnorm(norm[0]), "rope": rope, "glu": glu,
           "add_rmsnorm_ffn": add_rmsnorm(norm[1])}
    ops, total_s, calls = {}, 0.0, 0
    for name, fn in fns.items():
        fn()  # first touch of the outputs
        times, t_end = [], time.perf_counter() + seconds / len(fns)
        while len(times) < 3 or time.perf_counter() < t_end:
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
        med = float(np.median(times))
        total_s += sum(times)
        calls += len(times)
        ops[name] = dict(ms=round(med * 1e3, 3), gbs=round(st.bytes[name] / med / 1e9, 2), calls=len(times))
    step_s = sum(o["ms"] for o in ops.values()) / 1e3
    step_bytes = sum(st.bytes.values())
    return dict(value=round(step_bytes / step_s / 1e9, 3), unit="GB/s", cores=threads, kind="port",
                cpu_model=model, host_cpus=total, cpus_available=avail, ms_per_step=round(step_s * 1e3, 2),
                ops=ops,
                sample=f"config C step at {n} tokens ({cfg['qtype']} table of {cfg['vocab']} rows, "
                       f"{'f16' if f16 else 'f32'} activations), the GPU step's own inputs; each op "
                       f"timed alone, median of {calls} calls in {total_s:.1f} s; oracle/ C "
                       f"restatement of the candle CPU path on {threads} threads (persistent pool) of "
                       f"{avail} available, {model}")


def traffic_from_profiles(kernel, algorithmic_bytes):
    """HBM bytes per launch of the roofline kernel measured by rocprofv3
    --pmc (FETCH_SIZE, WRITE_SIZE, scaled by a copy kernel's reading), from
    the committed summary -- but only while the kernel's machine code is the
    code that was measured (the summary records its SHA-256): (bytes or
    None, why None)."""
    from cuca_amd import build
    p = os.path.join(ROOT, "profiles", "swiglu_traffic.json")
    if not os.path.exists(p):
        return None, "no traffic summary"
    with open(p) as f:
        rec = json.load(f)
    if rec.get("kernel") != kernel:
        return None, f"the summary measured {rec.get('kernel')}, the roofline kernel is {kernel}"
    if rec.get("algorithmic_bytes_per_launch") != algorithmic_bytes:
        return None, (f"the summary measured launches of {rec.get('algorithmic_bytes_per_launch')} "
                      f"algorithmic bytes, this run's are {algorithmic_bytes}")
    now = build.kernel_code_sha256(kernel)
    if now is None or now != rec.get("code_sha256"):
        return None, "the kernel's code changed since the counters were read"
    return rec.get("hbm_bytes_per_launch"), None


def prefill_bar(ops, tokens, big, configs):
    """Every fused op's fraction of the HBM peak at the prefill sizes the
    north star's 70 % bar covers (>= 4096 tokens: config C at both sizes,
    config E at 8192), and the smallest of them."""
    bar = {}

    def take(key, o):
        if o:
            bar[key] = {name: r["frac"] for name, r in o.items()}
    take(f"C_{tokens}", ops)
    if big:
        take(f"C_{big['tokens']}", big["ops"])
    if configs and "E_8192_f16" in configs:
        take("E_8192", configs["E_8192_f16"]["ops"])
    fr = [f for o in bar.values() for f in o.values()]
    bar["min"] = min(fr) if fr else None
    bar["all_at_least_0.70"] = bool(fr) and min(fr) >= 0.70
    return bar


def decode_bar(decode, attn):
    """The batch-1 decode figures in brief: the fully fused step's tokens/s,
    its per-layer attention and non-matmul time (the norms' in-kernel cost
    when they ride in the matmul prologues), and the non-matmul sequence of
    a layer as its own launches in a graph."""
    if not decode:
        return None
    out = {}
    f = decode.get("step_batch1_ctx4096_qmm_norm_rope_in_qkv")
    if f:
        out["step_batch1_fused_tokens_per_s"] = f["tokens_per_s"]
        out["step_batch1_fused_attention_us_per_layer"] = f.get("attention_us_per_layer")
        out["step_batch1_fused_non_matmul_us_per_layer"] = f.get("non_matmul_us_per_layer")
        out["step_batch1_fused_us_per_layer"] = f["us_per_layer"]
    b1 = decode.get("batch1")
    if b1:
        out["non_matmul_sequence_batch1_graph_us_per_layer"] = b1["graph_us_per_layer"]
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--tokens", type=int, default=16384)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-large", action="store_true",
                    help="skip the second config C size (4096 tokens beside the 16384-token headline)")
    ap.add_argument("--no-configs", action="store_true", help="skip the A/B/D/E config steps")
    ap.add_argument("--no-kv", action="store_true", help="skip the fused RoPE + paged K/V store")
    ap.add_argument("--no-attn", action="store_true", help="skip the paged decode attention")
    ap.add_argument("--no-qmm", action="store_true",
                    help="skip the quantized matmuls, routed experts and LM head")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: these ops run on one GPU's share of the work and "
              f"no collective is part of the path (asked for --gpus {args.gpus})", file=sys.stderr)
        sys.exit(2)

    import torch
    from cuca_amd import hip
    if not os.path.exists(hip.LIB_PATH):
        from cuca_amd import build
        build.build()
    log("context")
    # one explicit stream (default priority) carries torch's data generation,
    # the HIP events and every cuca launch
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    ctx = hip.Context(0)
    ctx.set_stream(stream.cuda_stream)

    # A plain streaming kernel of known size, for context and as the
    # reference reading of the HBM counters (FETCH_SIZE / WRITE_SIZE): torch's
    # elementwise negation of 256 MiB of f16 reads 256 MiB and writes 256 MiB.
    cal_n = (256 << 20) // 2
    cal_src = torch.ones(cal_n, device="cuda", dtype=torch.float16)
    cal_dst = torch.empty_like(cal_src)
    cal_ms = time_steps(torch, lambda: torch.neg(cal_src, out=cal_dst), 10, 3)
    copy_gbs = 2 * cal_n * 2 / (cal_ms / 1e3) / 1e9
    del cal_src, cal_dst

    parity_raw = {}

    def run_size(n, steps, warmup, name="C", dtype="f16", cpu_hook=None):
        log(f"config {name}: step buffers, {n} tokens, {dtype}")
        st = LayerStep(ctx, torch, name, n, dtype)
        torch.cuda.synchronize()
        log("timed steps (unprofiled)")
        ms_plain = time_steps(torch, st.step, steps, warmup)
        log("timed steps (kernel timestamps, median of five windows)")
        ms, per = profiled_windows(torch, ctx, st, steps, warmup)
        ctx.check_device()
        log(f"{ms * 1000:.1f} us per step ({ms_plain * 1000:.1f} unprofiled)")
        ops = {name: dict(kernel=k, us=round(t * 1000, 2), bytes=st.bytes[name],
                          gbs=round(st.bytes[name] / (t / 1e3) / 1e9, 1),
                          frac=round(st.bytes[name] / (t / 1e3) / 1e9 / HBM_PEAK_GBS, 4))
               for name, (k, t) in per.items()}
        log("verify sampled rows against the oracle")
        rows, raw = st.verify()
        parity_raw[f"{name}_{n}_{dtype}"] = raw
        step_bytes = sum(st.bytes.values())
        if cpu_hook is not None:
            cpu_hook(st)
        del st
        torch.cuda.empty_cache()
        return ms, step_bytes, ops, rows, ms_plain

    cpu = None
    cpu_box = {}

    def cpu_leg(st):
        if not args.no_cpu:
            log("cpu baseline (the same step on the host's cores)")
            cpu_box["cpu"] = cpu_baseline(st, args.cpu_seconds)

    ms_prof, step_bytes, ops, checked_rows, ms = run_size(args.tokens, args.steps, args.warmup,
                                                          cpu_hook=cpu_leg)
    cpu = cpu_box.get("cpu")
    value = step_bytes / (ms / 1e3) / 1e9
    glu = ops["glu"]
    big, other = None, (4096 if args.tokens != 4096 else 16384)
    if not args.no_large:
        _, bytes_l, ops_l, rows_l, ms_l = run_size(other, args.steps, args.warmup)
        checked_rows += rows_l
        big = dict(tokens=other, us_per_step=round(ms_l * 1000, 1),
                   gbs=round(bytes_l / (ms_l / 1e3) / 1e9, 1),
                   frac=round(bytes_l / (ms_l / 1e3) / 1e9 / HBM_PEAK_GBS, 4), ops=ops_l)

    configs = None
    if not args.no_configs:
        # every workload config's own step (per-op kernel GB/s); configs[1]
        # and [2] are Llama-3-8B (B at batch 32 here, C above)
        configs = {}
        for name, n, dtype in (("A", 128, "f32"), ("B", 32, "f32"), ("D", 8, "f32"),
                               ("D", 2048, "f16"), ("E", 64, "f32"), ("E", 8192, "f16")):
            _, b_c, ops_c, rows_c, ms_c = run_size(n, 20, 5, name, dtype)
            checked_rows += rows_c
            configs[f"{name}_{n}_{dtype}"] = dict(
                us_per_step=round(ms_c * 1000, 2), gbs=round(b_c / (ms_c / 1e3) / 1e9, 1),
                frac=round(b_c / (ms_c / 1e3) / 1e9 / HBM_PEAK_GBS, 4), ops=ops_c)

    kv = None
    if not args.no_kv:
        log("rope + paged K/V store")
        kv = {}
        for name, n, dtype in (("C", 4096, "f16"), ("C", 16384, "f16"), ("E", 8192, "f16"),
                               ("B", 32, "f32")):
            r = kv_store_bench(ctx, torch, name, n, dtype)
            checked_rows += r.pop("verified_rows")
            kv[f"{name}_{n}_{dtype}"] = r
        torch.cuda.empty_cache()

    attn = None
    if not args.no_attn:
        log("paged decode attention")
        attn = {}
        for name, rows, clen, dtype in (("B", 1, 8192, "f16"), ("B", 32, 8192, "f16"),
                                        ("B", 64, 8192, "f16"), ("B", 32, 8192, "f32"),
                                        ("B", 8, 32768, "f16"), ("E", 32, 8192, "f16")):
            attn[f"{name}_b{rows}_{clen}_{dtype}"] = attn_bench(ctx, torch, name, rows, clen, dtype)
            checked_rows += 2
        torch.cuda.empty_cache()

    qmm = moe = head = qgemm = gemm16 = player = player_dense = None
    if not args.no_qmm and not args.no_attn:
        log("a whole prefill layer (config C, 4096 tokens, f16): matmuls, RoPE + K/V store, attention")
        player = prefill_layer_bench(ctx, torch, "C", 4096)
        log("the same layer with the projections on the dense f16 path")
        player_dense = prefill_layer_bench(ctx, torch, "C", 4096, dense=True)
    if not args.no_qmm:
        log("quantized matmuls (8B decode shapes)")
        qmm = qmm_bench(ctx, torch)
        log("matrix-core quantized matmul (8B shapes, 32 / 512 / 4096 rows)")
        qgemm = qgemm_bench(ctx, torch)
        log("dense f16 path: dequantised weights + f16 GEMM (8B shapes, 512 / 4096 rows)")
        gemm16 = gemm_w16_bench(ctx, torch)
        log("routed experts (config E decode)")
        moe = moe_bench(ctx, torch)
        log("LM head + greedy / top-k")
        head = head_bench(ctx, torch)
        torch.cuda.empty_cache()

    decode = None
    if not args.no_decode:
        log("decode graphs")
        decode = {}
        for n in (1, 32):
            g_us, e_us = decode_us_per_layer(ctx, torch, n)
            decode[f"batch{n}"] = dict(graph_us_per_layer=round(g_us, 2),
                                       eager_us_per_layer=round(e_us, 2))
        # with the K/V store and the paged attention of a K/V-owning layer
        for n, clen in ((1, 8192), (32, 1024)):
            g_us, e_us = decode_us_per_layer(ctx, torch, n, ctx_len=clen)
            decode[f"batch{n}_with_attention_ctx{clen}"] = dict(graph_us_per_layer=round(g_us, 2),
                                                                eager_us_per_layer=round(e_us, 2))
            torch.cuda.empty_cache()
        torch.cuda.empty_cache()
        if not args.no_qmm:
            log("whole decode steps (32 layers + head, hipGraph)")
            # fuse: "" none; "rope": RoPE + K/V store in the Q|K|V epilogue;
            # "norm": that and both residual + RMSNorm launches in the
            # prologues of the Q|K|V and gate/up matmuls
            for n, clen, mm, fuse in ((1, 4096, "qmm", ""), (1, 4096, "qmm", "rope"), (1, 4096, "qmm", "norm"),
                                      (32, 1024, "qmm", "rope"), (32, 1024, "qgemm", "")):
                key = f"step_batch{n}_ctx{clen}_{mm}" + {"": "", "rope": "_rope_in_qkv",
                                                         "norm": "_norm_rope_in_qkv"}[fuse]
                decode[key] = decode_step_bench(ctx, torch, n, clen, mm=mm, fuse_rope=fuse != "",
                                                fuse_norm=fuse == "norm")
            torch.cuda.empty_cache()
            # With both norms in the matmul prologues no launch is a non-matmul
            # op, but the norms still cost time inside those matmuls: their
            # cost is the fused step's matmul time (Q|K|V + RoPE/K/V-store,
            # the others) minus the same launches without the prologue.
            fused = decode.get("step_batch1_ctx4096_qmm_norm_rope_in_qkv")
            plain = decode.get("step_batch1_ctx4096_qmm_rope_in_qkv")
            if fused is not None and plain is not None:
                def mm_us(r):
                    return r.get("matmul_us_per_layer", 0.0) + r.get("qkv_rope_kv_us_per_layer", 0.0)
                fused["non_matmul_launch_us_per_layer"] = fused.pop("non_matmul_us_per_layer", 0.0)
                fused["norm_prologue_us_per_layer"] = round(mm_us(fused) - mm_us(plain), 2)
                fused["non_matmul_us_per_layer"] = round(fused["non_matmul_launch_us_per_layer"]
                                                         + fused["norm_prologue_us_per_layer"], 2)

    traffic, why = traffic_from_profiles(glu["kernel"], glu["bytes"])
    traffic_src = ("profiles/swiglu_traffic.json (rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE; same kernel code)"
                   if traffic is not None else why)
    out = {
        "metric": "fused layer-op HBM GB/s & % of 8 TB/s peak; per-layer non-matmul us at decode",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "ms_per_step_profiled": round(ms_prof, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (device-generated, seeded)",
        "config": {"workload": "llama3-8b layer ops: prefill step (embed Q8_0 + first-block rmsnorm, "
                               "add_rmsnorm x2, rope, swiglu) + decode graph",
                   "tokens": args.tokens, "hidden": 4096, "ff": 14336, "heads": "32q/8k x 128",
                   "activations": "f16 (decode: f32)", "bytes_per_step": step_bytes},
        "hbm_frac": round(value / HBM_PEAK_GBS, 4),
        "copy_gbs": round(copy_gbs, 1),
        "verified_rows": checked_rows,
        "parity_raw": parity_raw,
        "ops": ops,
        f"prefill_{other}": big,
        "configs": configs,
        "rope_store_kv": kv,
        "paged_decode": attn,
        "qmm_decode": qmm,
        "qgemm": qgemm,
        "gemm_w16": gemm16,
        "moe_decode": moe,
        "end_of_step": head,
        "decode_us_per_layer": decode,
        "prefill_layer": player,
        "prefill_layer_dense": player_dense,
        "prefill_bar": prefill_bar(ops, args.tokens, big, configs),
        "decode_bar": decode_bar(decode, attn),
        "roofline": {"kernel": glu["kernel"], "bound": "hbm",
                     "achieved": glu["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": glu["frac"], "traffic": traffic,
                     "traffic_source": traffic_src,
                     "algorithmic_bytes_per_launch": glu["bytes"], "avg_launch_us": glu["us"]},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
