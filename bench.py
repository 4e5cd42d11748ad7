#!/usr/bin/env python3
"""Benchmark of the fused per-layer ops on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

Metric: fused layer-op HBM GB/s and % of the 8 TB/s peak;
per-layer non-matmul microseconds at decode.

Workload (config.workload): the Llama-3-8B layer ops.  One step is one pass
of the hot path over one batch of 4096 prefill tokens with f16 activations
(configs[2] at its smaller size): the Q8_0 embedding gather of the batch,
the attention-side residual add + RMSNorm, RoPE on Q 32x128 / K 8x128, the
SwiGLU over F 14336, and the FFN-side residual add + RMSNorm.  `value` is
the algorithmic bytes of a step divided by its time (K steps between two HIP
events, synchronized on both sides), with every input resident in HBM
(synthetic data generated on the device).  The decode figure
is the same layer's non-matmul sequence (two fused norms, RoPE, SwiGLU) at
batch 1 and 32 in f32, 32 layers captured in one hipGraph and
replayed, in microseconds per layer.

Algorithmic bytes per unit (s = bytes per activation, H 4096, F 14336):
  embed       34 H/32 + 4 + s H        per token (block bytes, id, output)
  add_rmsnorm 4 s H                    per row   (x, branch in; x', h out)
  rope        2 s (nq + nk) D + 4 D    per row   (Q, K in and out; cos+sin)
  swiglu      3 s F                    per row   (gate, up in; out)
Per-call constants (gamma, norm weights) are counted once.

roofline: the dominant kernel (SwiGLU) -- its algorithmic bytes per launch
divided by its average launch duration over the timed steps, from the start
and stop events the C ABI's profile attaches to every kernel
(hipExtModuleLaunchKernel on the ops' stream; the same durations rocprofv3
reports), against the 8 TB/s HBM peak.

cpu_baseline: the oracle's C restatement of the reference's candle CPU path
(oracle/), on the host's cores, over a bounded sample of the same step.
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


def op_bytes(op, n, s, H=4096, F=14336, nq=32, nk=8, D=128, qbytes=34):
    if op == "embed":
        return n * (qbytes * H // 32 + 4 + s * H)
    if op == "add_rmsnorm":
        return n * 4 * s * H + 4 * H
    if op == "rope":
        return n * (2 * s * (nq + nk) * D + 4 * D)
    if op == "swiglu":
        return n * 3 * s * F
    raise KeyError(op)


STEP_OPS = ("embed", "add_rmsnorm_attn", "rope", "swiglu", "add_rmsnorm_ffn")


def op_kind(name):
    return "add_rmsnorm" if name.startswith("add_rmsnorm") else name


class PrefillStep:
    """Device buffers of one prefill step (config C shapes) and its launches."""

    def __init__(self, ctx, torch, n, seed=2):
        from cuca_amd import hip
        from cuca_amd import workloads as W
        cfg = W.CONFIGS["C"]
        self.hip, self.ctx, self.n, self.cfg = hip, ctx, n, cfg
        H, F, d, nq, nk = cfg["hidden"], cfg["ff"], cfg["head_dim"], cfg["nq"], cfg["nk"]
        dev = "cuda"
        gen = torch.Generator(device=dev).manual_seed(seed)
        f16 = torch.float16
        self.table = W.quant_table_torch(gen, cfg["vocab"], H, cfg["qtype"], cfg["d_range"])
        self.ids = torch.randint(0, cfg["vocab"], (n,), device=dev, generator=gen, dtype=torch.int32)
        self.emb = torch.empty((n, H), device=dev, dtype=f16)

        def act(*shape):
            return torch.randn(shape, device=dev, generator=gen).to(f16)
        self.x1, self.b1, self.xo1, self.h1 = act(n, H), act(n, H), act(n, H), act(n, H)
        self.x2, self.b2, self.xo2, self.h2 = act(n, H), act(n, H), act(n, H), act(n, H)
        self.w1 = (1 + 0.02 * torch.randn(H, device=dev, generator=gen)).float()
        self.w2 = (1 + 0.02 * torch.randn(H, device=dev, generator=gen)).float()
        self.q, self.k = act(n, nq, d), act(n, nk, d)
        self.q0, self.k0 = self.q.clone(), self.k.clone()
        cos, sin = hip.rope_tables(hip.ROPE_NORM, d, cfg["theta"], n)
        self.cos, self.sin = torch.from_numpy(cos).to(dev), torch.from_numpy(sin).to(dev)
        self.pos = torch.arange(n, device=dev, dtype=torch.int32)
        self.gu = act(n, 2 * F)
        self.out = torch.empty((n, F), device=dev, dtype=f16)
        self.bytes = {name: op_bytes(op_kind(name), n, 2) for name in STEP_OPS}

    def launch(self, name):
        c, hip, cfg, n = self.ctx, self.hip, self.cfg, self.n
        H, F, d, nq, nk = cfg["hidden"], cfg["ff"], cfg["head_dim"], cfg["nq"], cfg["nk"]
        if name == "embed":
            c.embed_gguf(self.table.data_ptr(), hip.GGML_Q8_0, cfg["vocab"], H, self.ids.data_ptr(),
                         n, 1.0, self.emb.data_ptr(), hip.F16)
        elif name == "add_rmsnorm_attn":
            c.add_rmsnorm(self.x1.data_ptr(), self.b1.data_ptr(), self.w1.data_ptr(), None,
                          cfg["eps"], cfg["eps"], 1.0, n, H, self.xo1.data_ptr(),
                          self.h1.data_ptr(), hip.F16)
        elif name == "rope":
            c.rope(self.q.data_ptr(), nq * d, self.k.data_ptr(), nk * d, n, nq, nk, d, d,
                   hip.ROPE_NORM, self.cos.data_ptr(), self.sin.data_ptr(), n, self.pos.data_ptr(),
                   None, None, cfg["eps"], hip.F16)
        elif name == "swiglu":
            c.glu(self.gu.data_ptr(), 2 * F, self.gu.data_ptr() + 2 * F, 2 * F, n, F,
                  hip.ACT_SILU, 0.0, self.out.data_ptr(), F, hip.F16)
        elif name == "add_rmsnorm_ffn":
            c.add_rmsnorm(self.x2.data_ptr(), self.b2.data_ptr(), self.w2.data_ptr(), None,
                          cfg["eps"], cfg["eps"], 1.0, n, H, self.xo2.data_ptr(),
                          self.h2.data_ptr(), hip.F16)

    def step(self):
        for name in STEP_OPS:
            self.launch(name)

    def verify(self, torch, rows=24):
        """Run the step once from fresh Q/K and compare sampled rows of every
        output with the oracle (the timed kernels did the work they claim)."""
        import numpy as np
        from oracle import oracle as O
        from cuca_amd import workloads as W
        cfg, n = self.cfg, self.n
        H, F, d = cfg["hidden"], cfg["ff"], cfg["head_dim"]
        self.q.copy_(self.q0)
        self.k.copy_(self.k0)
        self.step()
        torch.cuda.synchronize()
        self.ctx.check_device()
        s = np.unique(np.concatenate([[0, n - 1], np.random.default_rng(7).integers(0, n, rows)]))
        st = torch.from_numpy(s).cuda()
        host = lambda t: t[st].cpu().numpy()
        rb = W.row_bytes(cfg["qtype"], H)
        sub = self.table.view(cfg["vocab"], rb)[self.ids[st].long()].cpu().numpy().reshape(-1)
        want = O.embed(sub, O.Q8_0, s.size, H, np.arange(s.size, dtype=np.uint32), 1.0,
                       out_dtype=np.float16)
        assert np.array_equal(host(self.emb).view(np.uint16), want.view(np.uint16)), "embed"
        for x, b, w, xo, h in ((self.x1, self.b1, self.w1, self.xo1, self.h1),
                               (self.x2, self.b2, self.w2, self.xo2, self.h2)):
            wx, wh = O.add_rmsnorm(host(x), host(b), w.cpu().numpy(), cfg["eps"])
            assert np.array_equal(host(xo).view(np.uint16), wx.view(np.uint16)), "x'"
            g = host(h).astype(np.float64)
            ulp = np.spacing(np.abs(wh).astype(np.float16)).astype(np.float64)
            assert np.all(np.abs(g - wh.astype(np.float64)) <= 2 * ulp), "add_rmsnorm"
        cos, sin = self.cos.cpu().numpy(), self.sin.cpu().numpy()
        for t, t0 in ((self.q, self.q0), (self.k, self.k0)):
            w = O.rope(host(t0), cos, sin, s.astype(np.int32), O.ROPE_NORM)
            assert np.array_equal(host(t).view(np.uint16), w.view(np.uint16)), "rope"
        gu = host(self.gu)
        wa = O.glu(gu[:, :F], gu[:, F:], O.SILU)
        g = host(self.out).astype(np.float64)
        ulp = np.spacing(np.abs(wa).astype(np.float16)).astype(np.float64)
        assert np.all(np.abs(g - wa.astype(np.float64)) <= 2 * ulp + 1e-37), "swiglu"
        return int(s.size)


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


def decode_us_per_layer(ctx, torch, n, replays=50):
    dl = DecodeLayers(ctx, torch, n)
    torch.cuda.synchronize()
    eager_ms = time_steps(torch, dl.issue, 10, 3)
    ctx.graph_begin()
    dl.issue()
    g = ctx.graph_end()
    graph_ms = time_steps(torch, g.launch, replays, 5)
    g.destroy()
    return graph_ms * 1000.0 / dl.layers, eager_ms * 1000.0 / dl.layers


def cpu_baseline(seconds=10.0, n=64):
    """The oracle (candle-equivalent C restatement) over the same step's ops
    on n tokens, repeated for about `seconds`, on the host's cores."""
    import numpy as np
    from cuca_amd import workloads as W
    from oracle import oracle as O
    cfg = W.CONFIGS["C"]
    H, F, d, nq, nk = cfg["hidden"], cfg["ff"], cfg["head_dim"], cfg["nq"], cfg["nk"]
    threads = max(1, min(16, os.cpu_count() or 1))
    rng = np.random.default_rng(2)
    vocab = 4096  # the gather touches n rows; a smaller table holds them
    table = W.quant_table(rng, vocab, H, cfg["qtype"], cfg["d_range"])
    ids = rng.integers(0, vocab, n).astype(np.uint32)
    f16 = np.float16
    x, b = rng.standard_normal((n, H)).astype(f16), rng.standard_normal((n, H)).astype(f16)
    w = (1 + 0.02 * rng.standard_normal(H)).astype(np.float32)
    q, k = rng.standard_normal((n, nq, d)).astype(f16), rng.standard_normal((n, nk, d)).astype(f16)
    cos, sin = O.rope_tables(d, cfg["theta"], n)
    pos = np.arange(n, dtype=np.int32)
    gu = rng.standard_normal((n, 2 * F)).astype(f16)
    step_bytes = sum(op_bytes(op_kind(name), n, 2) for name in STEP_OPS)

    def step():
        O.embed(table, O.Q8_0, vocab, H, ids, 1.0, out_dtype=f16, threads=threads)
        O.add_rmsnorm(x, b, w, cfg["eps"], threads=threads)
        O.rope(q, cos, sin, pos, O.ROPE_NORM, threads=threads)
        O.rope(k, cos, sin, pos, O.ROPE_NORM, threads=threads)
        O.glu(gu[:, :F], gu[:, F:], O.SILU, threads=threads)
        O.add_rmsnorm(x, b, w, cfg["eps"], threads=threads)

    step()
    iters, t0 = 0, time.perf_counter()
    while True:
        step()
        iters += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    return dict(value=round(step_bytes * iters / el / 1e9, 3), unit="GB/s", cores=threads,
                kind="port",
                sample=f"{iters} repetitions of the step on {n} tokens (config C shapes, f16 "
                       f"activations, Q8_0 table of {vocab} rows), {el:.1f} s, oracle/ C "
                       f"restatement of the candle CPU path, {threads} threads")


def traffic_from_profiles():
    """HBM bytes per SwiGLU launch measured by rocprofv3 --pmc (FETCH_SIZE,
    WRITE_SIZE, scaled by a copy kernel's reading), when that summary exists."""
    p = os.path.join(ROOT, "profiles", "swiglu_traffic.json")
    if not os.path.exists(p):
        return None
    with open(p) as f:
        return json.load(f).get("hbm_bytes_per_launch")


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--tokens", type=int, default=4096)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-large", action="store_true", help="skip the 16384-token step")
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

    def run_size(n, steps, warmup):
        log(f"prefill step buffers, {n} tokens")
        st = PrefillStep(ctx, torch, n)
        torch.cuda.synchronize()
        log("timed steps (unprofiled)")
        ms_plain = time_steps(torch, st.step, steps, warmup)
        log("timed steps (kernel timestamps)")
        ms, per = profiled_steps(torch, ctx, st, steps, warmup)
        ctx.check_device()
        log(f"{ms * 1000:.1f} us per step ({ms_plain * 1000:.1f} unprofiled)")
        ops = {name: dict(kernel=k, us=round(t * 1000, 2), bytes=st.bytes[name],
                          gbs=round(st.bytes[name] / (t / 1e3) / 1e9, 1),
                          frac=round(st.bytes[name] / (t / 1e3) / 1e9 / HBM_PEAK_GBS, 4))
               for name, (k, t) in per.items()}
        log("verify sampled rows against the oracle")
        rows = st.verify(torch)
        step_bytes = sum(st.bytes.values())
        del st
        torch.cuda.empty_cache()
        return ms, step_bytes, ops, rows, ms_plain

    ms_prof, step_bytes, ops, checked_rows, ms = run_size(args.tokens, args.steps, args.warmup)
    value = step_bytes / (ms / 1e3) / 1e9
    glu = ops["swiglu"]
    big = None
    if args.tokens != 16384 and not args.no_large:
        _, bytes_l, ops_l, rows_l, ms_l = run_size(16384, max(5, args.steps // 4), 3)
        checked_rows += rows_l
        big = dict(tokens=16384, us_per_step=round(ms_l * 1000, 1),
                   gbs=round(bytes_l / (ms_l / 1e3) / 1e9, 1),
                   frac=round(bytes_l / (ms_l / 1e3) / 1e9 / HBM_PEAK_GBS, 4), ops=ops_l)

    decode = None
    if not args.no_decode:
        log("decode graphs")
        decode = {}
        for n in (1, 32):
            g_us, e_us = decode_us_per_layer(ctx, torch, n)
            decode[f"batch{n}"] = dict(graph_us_per_layer=round(g_us, 2),
                                       eager_us_per_layer=round(e_us, 2))
        torch.cuda.empty_cache()

    cpu = None
    if not args.no_cpu:
        log("cpu baseline")
        cpu = cpu_baseline(args.cpu_seconds)

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
        "config": {"workload": "llama3-8b layer ops: prefill step (embed Q8_0, add_rmsnorm x2, "
                               "rope, swiglu) + decode graph",
                   "tokens": args.tokens, "hidden": 4096, "ff": 14336, "heads": "32q/8k x 128",
                   "activations": "f16 (decode: f32)", "bytes_per_step": step_bytes},
        "hbm_frac": round(value / HBM_PEAK_GBS, 4),
        "verified_rows": checked_rows,
        "ops": ops,
        "prefill_16384": big,
        "decode_us_per_layer": decode,
        "roofline": {"kernel": glu["kernel"], "bound": "hbm",
                     "achieved": glu["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": glu["frac"], "traffic": traffic_from_profiles(),
                     "algorithmic_bytes_per_launch": glu["bytes"], "avg_launch_us": glu["us"]},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
