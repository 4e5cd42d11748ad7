"""The decode-step graph: the per-layer non-matmul launches of config B
(batch 1 and 32) captured once and replayed.  Every replay is compared with
the eager result, with eager work and synchronizations between replays."""
import numpy as np
import pytest

from cuca_amd import hip
from cuca_amd import workloads as W
from helpers import assert_bits_equal

pytestmark = pytest.mark.gpu


class Layer:
    """Buffers of one decode layer: residual x, branch, h, q, k, gate/up, out."""

    def __init__(self, ctx, rng, n, cfg):
        H, F, d = cfg["hidden"], cfg["ff"], cfg["head_dim"]
        self.ctx = ctx
        self.n = n
        self.x = ctx.array(rng.standard_normal((n, H)).astype(np.float32))
        self.attn = ctx.array(rng.standard_normal((n, H)).astype(np.float32))
        self.ffn = ctx.array(rng.standard_normal((n, H)).astype(np.float32))
        self.w1 = ctx.array((1 + 0.02 * rng.standard_normal(H)).astype(np.float32))
        self.w2 = ctx.array((1 + 0.02 * rng.standard_normal(H)).astype(np.float32))
        self.h = ctx.empty((n, H), np.float32)
        self.q0 = rng.standard_normal((n, cfg["nq"], d)).astype(np.float32)
        self.k0 = rng.standard_normal((n, cfg["nk"], d)).astype(np.float32)
        self.q = ctx.array(self.q0)
        self.k = ctx.array(self.k0)
        self.gu = ctx.array(rng.standard_normal((n, 2 * F)).astype(np.float32))
        self.act = ctx.empty((n, F), np.float32)
        cos, sin = hip.rope_tables(hip.ROPE_NORM, d, cfg["theta"], 8192)
        self.cos, self.sin = ctx.array(cos), ctx.array(sin)
        self.pos = ctx.array(rng.integers(0, 8192, n).astype(np.int32))
        self.cfg = cfg

    def issue(self):
        """attn residual + ffn norm, rope, glu, ffn residual + next attn norm."""
        c, cfg, n = self.ctx, self.cfg, self.n
        H, F, d = cfg["hidden"], cfg["ff"], cfg["head_dim"]
        c.add_rmsnorm(self.x.ptr, self.attn.ptr, self.w1.ptr, None, cfg["eps"], cfg["eps"], 1.0, n,
                      H, self.x.ptr, self.h.ptr, hip.F32)
        c.rope(self.q.ptr, cfg["nq"] * d, self.k.ptr, cfg["nk"] * d, n, cfg["nq"], cfg["nk"], d, d,
               hip.ROPE_NORM, self.cos.ptr, self.sin.ptr, 8192, self.pos.ptr, None, None, 1e-6,
               hip.F32)
        c.glu(self.gu.ptr, 2 * F, self.gu.ptr + 4 * F, 2 * F, n, F, hip.ACT_SILU, 0.0, self.act.ptr,
              F, hip.F32)
        c.add_rmsnorm(self.x.ptr, self.ffn.ptr, self.w2.ptr, None, cfg["eps"], cfg["eps"], 1.0, n,
                      H, self.x.ptr, self.h.ptr, hip.F32)

    def snapshot(self):
        return [a.numpy() for a in (self.x, self.h, self.q, self.k, self.act)]

    def reset(self, x0):
        self.x.upload(x0)
        self.q.upload(self.q0)
        self.k.upload(self.k0)


@pytest.mark.parametrize("n", [1, 32])
def test_graph_replays_match_eager(ctx, n):
    cfg = W.CONFIGS["B"]
    rng = np.random.default_rng(n)
    layer = Layer(ctx, rng, n, cfg)
    x0 = layer.x.numpy()
    layer.issue()
    eager = layer.snapshot()
    layer.reset(x0)
    ctx.graph_begin()
    layer.issue()
    graph = ctx.graph_end()
    for rep in range(4):
        layer.reset(x0)
        graph.launch()
        ctx.sync()
        got = layer.snapshot()
        for g, e in zip(got, eager):
            assert_bits_equal(g, e, f"replay {rep}")
        # eager work between replays
        layer.issue()
        ctx.sync()
    graph.destroy()


def test_profile_records_every_launch_in_order(ctx):
    cfg = W.CONFIGS["B"]
    rng = np.random.default_rng(3)
    layer = Layer(ctx, rng, 4, cfg)
    ctx.profile_start(8)
    layer.issue()
    recs = ctx.profile_stop()
    names = [k for k, _ in recs]
    assert len(recs) == 4
    assert names[0].startswith("cuca_norm_f32") and names[1].startswith("cuca_rope_f32")
    assert names[2].startswith("cuca_glu_f32") and names[3].startswith("cuca_norm_f32")
    assert all(0.0 < ms < 100.0 for _, ms in recs)
    # past the limit, launches still run, unrecorded
    ctx.profile_start(2)
    layer.issue()
    assert len(ctx.profile_stop()) == 2
    with pytest.raises(hip.CucaError, match="not started"):
        ctx.profile_stop()
