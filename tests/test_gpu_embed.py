"""Embedding dequant-gather on the GPU against the oracle: bit-exact.

Covers the reference's golden blocks, the table shapes of configs A/B/D/E
(at a reduced vocab so the oracle runs in seconds), f32 and f16 output, the
2-byte-aligned staging path, the scale fold, the host-side errors of
TokenEmbedding::rows and the device-side guard for ids the host never saw.
The full-size table (config C, 532 MiB Q8_0, 16384 ids) is checked on
sampled rows.
"""
import os

import numpy as np
import pytest

from cuca_amd import hip, ops
from cuca_amd import workloads as W
from helpers import assert_bits_equal
from oracle import oracle as O

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "quants_legacy.npz")


@pytest.mark.parametrize("name,ty", [("q4_0", hip.GGML_Q4_0), ("q8_0", hip.GGML_Q8_0)])
@pytest.mark.parametrize("hidden", [1024, 32])
def test_golden_blocks(ctx, name, ty, hidden):
    g = np.load(GOLDEN)
    blocks, expected = g[name + "_blocks"], g[name + "_expected"]
    rows = 1024 // hidden   # one row of 32 blocks, or 32 rows of one block (2-byte aligned rows)
    emb = ops.TokenEmbedding(ctx, ty, blocks, rows, hidden)
    ids = np.arange(rows)[::-1].copy()
    got = emb.rows(ids, 1.0).numpy()
    assert_bits_equal(got, expected.reshape(rows, hidden)[ids], f"{name} golden")
    got16 = emb.rows(ids, 1.0, out_dtype=np.float16).numpy()
    assert_bits_equal(got16, expected.reshape(rows, hidden)[ids].astype(np.float16))


@pytest.mark.parametrize("cfg_name", ["A", "B", "D", "E"])
@pytest.mark.parametrize("out", [np.float32, np.float16])
def test_config_tables_bit_exact(ctx, cfg_name, out):
    cfg = W.CONFIGS[cfg_name]
    rng = np.random.default_rng(cfg["seed"])
    vocab, hidden = 2048, cfg["hidden"]
    table = W.quant_table(rng, vocab, hidden, cfg["qtype"], cfg["d_range"])
    ty = W.GGML_ID[cfg["qtype"]]
    ids = rng.integers(0, vocab, 96).astype(np.uint32)
    ids[:3] = [0, vocab - 1, 0]
    emb = ops.TokenEmbedding(ctx, ty, table, vocab, hidden)
    got = emb.rows(ids, cfg["embd_scale"], out_dtype=out).numpy()
    want = O.embed(table, ty, vocab, hidden, ids, cfg["embd_scale"], out_dtype=out, threads=8)
    assert_bits_equal(got, want, f"config {cfg_name}")


# Row lengths whose rows start on a 2-byte (not 4-byte) boundary, that leave
# the last round of units part-filled, or that take several rounds (more than
# 8 units of 8 values per lane: hidden > 4096).
@pytest.mark.parametrize("hidden", [96, 160, 3584 + 32, 8192 + 96])
def test_odd_row_lengths_and_multi_round_rows(ctx, hidden):
    rng = np.random.default_rng(hidden)
    for qtype in ("q4_0", "q8_0"):
        table = W.quant_table(rng, 64, hidden, qtype, (0.001, 0.05))
        ty = W.GGML_ID[qtype]
        ids = rng.integers(0, 64, 41).astype(np.uint32)
        emb = ops.TokenEmbedding(ctx, ty, table, 64, hidden)
        got = emb.rows(ids, 1.37).numpy()
        assert_bits_equal(got, O.embed(table, ty, 64, hidden, ids, 1.37), qtype)
        got16 = emb.rows(ids, 1.37, out_dtype=np.float16).numpy()
        want16 = O.embed(table, ty, 64, hidden, ids, 1.37, out_dtype=np.float16)
        assert_bits_equal(got16, want16, qtype + " f16")


def test_empty_and_single_token(ctx):
    rng = np.random.default_rng(1)
    table = W.quant_table(rng, 8, 64, "q4_0", (0.001, 0.05))
    emb = ops.TokenEmbedding(ctx, hip.GGML_Q4_0, table, 8, 64)
    assert emb.rows([], 1.0).shape == (0, 64)
    got = emb.rows([7], 2.0).numpy()
    assert_bits_equal(got, O.embed(table, O.Q4_0, 8, 64, np.array([7], np.uint32), 2.0))


def test_host_rejects_bad_ids_like_the_reference(ctx):
    table = np.zeros(4 * 18, np.uint8)
    emb = ops.TokenEmbedding(ctx, hip.GGML_Q4_0, table, 4, 32)
    with pytest.raises(hip.CucaError, match="token id 4 outside the embedding table of 4 rows"):
        emb.rows([1, 4], 1.0)


def test_device_guard_reports_bad_ids_and_writes_zero_rows(ctx):
    rng = np.random.default_rng(2)
    table = W.quant_table(rng, 16, 128, "q8_0", (0.001, 0.02))
    emb = ops.TokenEmbedding(ctx, hip.GGML_Q8_0, table, 16, 128)
    ids = ctx.array(np.array([3, 16, 5, 99999], np.uint32))
    out = ctx.empty((4, 128), np.float32)
    emb.rows_device(ids, 1.0, out)
    with pytest.raises(hip.CucaError, match="token id 16 outside the embedding table of 16 rows"):
        ctx.check_device()
    got = out.numpy()
    assert np.all(got[1] == 0) and np.all(got[3] == 0)
    want = O.embed(table, O.Q8_0, 16, 128, np.array([3, 5], np.uint32), 1.0)
    assert_bits_equal(got[[0, 2]], want)
    ctx.check_device()   # the status was cleared


def test_full_size_config_c_sampled_rows(ctx):
    torch = pytest.importorskip("torch")
    cfg = W.CONFIGS["C"]
    gen = torch.Generator(device="cuda").manual_seed(cfg["seed"])
    vocab, hidden, n = cfg["vocab"], cfg["hidden"], 16384
    table = W.quant_table_torch(gen, vocab, hidden, cfg["qtype"], cfg["d_range"])
    ids = torch.randint(0, vocab, (n,), device="cuda", generator=gen, dtype=torch.int32)
    out = torch.empty((n, hidden), dtype=torch.float16, device="cuda")
    torch.cuda.synchronize()
    ctx.embed_gguf(table.data_ptr(), hip.GGML_Q8_0, vocab, hidden, ids.data_ptr(), n, 1.0,
                   out.data_ptr(), hip.F16)
    ctx.sync()
    ctx.check_device()
    rb = W.row_bytes(cfg["qtype"], hidden)
    sample = np.unique(np.concatenate([[0, n - 1], np.random.default_rng(0).integers(0, n, 254)]))
    ids_h = ids.cpu().numpy().astype(np.uint32)
    got = out[torch.from_numpy(sample).cuda()].cpu().numpy()
    rows = table.view(vocab, rb)[torch.from_numpy(ids_h[sample].astype(np.int64)).cuda()]
    sub_table = rows.cpu().numpy().reshape(-1)
    want = O.embed(sub_table, O.Q8_0, sample.size, hidden, np.arange(sample.size, dtype=np.uint32),
                   1.0, out_dtype=np.float16)
    assert_bits_equal(got, want, "config C full-size sample")


# ---------------------------------------------------------------------------
# the gather fused with norm_embeddings' rms_norm_rows (params.rs:374-379,
# quant.rs:324-339): bit-exact with the oracle's sequential f64 sum
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("qname", ["q4_0", "q8_0"])
@pytest.mark.parametrize("out", [np.float32, np.float16])
@pytest.mark.parametrize("hidden,eps,scale", [
    (1024, 1e-6, 1.0), (2048, 1e-6, 1.0), (3584, 1e-6, float(np.float32(np.sqrt(3584.0)))),
    (4096, 1e-5, 1.0), (5120, 1e-5, 1.0), (8192, 1e-6, 0.5), (32, 1e-5, 1.0), (96, 0.0, 2.0)])
def test_embed_norm_bit_exact(ctx, qname, out, hidden, eps, scale):
    rng = np.random.default_rng(hidden + (qname == "q8_0"))
    vocab = 512
    table = W.quant_table(rng, vocab, hidden, qname, (0.001, 0.05))
    ty = W.GGML_ID[qname]
    ids = rng.integers(0, vocab, 67).astype(np.uint32)
    emb = ops.TokenEmbedding(ctx, ty, table, vocab, hidden)
    got = emb.rows(ids, scale, out_dtype=out, norm_eps=eps).numpy()
    ctx.check_device()
    want = O.embed(table, ty, vocab, hidden, ids, scale, out_dtype=out, norm_eps=eps)
    assert_bits_equal(got, want, f"embed+norm {qname} {hidden}")


def test_embed_norm_fallback_row_bit_exact(ctx):
    """A row built so that the device's error bound cannot decide the f32
    scale (tests/test_oracle_embed_norm.py checks that on the CPU): the
    kernel re-sums it in index order and must still give the oracle's bits,
    alone and among ordinary rows."""
    from test_oracle_embed_norm import fallback_case
    row, eps = fallback_case()
    rng = np.random.default_rng(3)
    others = W.quant_table(rng, 7, 4096, "q8_0", (0.001, 0.02))
    table = np.concatenate([others, row])
    emb = ops.TokenEmbedding(ctx, hip.GGML_Q8_0, table, 8, 4096)
    ids = np.array([7, 0, 7, 3, 6, 7], np.uint32)
    for out in (np.float32, np.float16):
        got = emb.rows(ids, 1.0, out_dtype=out, norm_eps=eps).numpy()
        ctx.check_device()
        want = O.embed(table, O.Q8_0, 8, 4096, ids, 1.0, out_dtype=out, norm_eps=eps)
        assert_bits_equal(got, want, "fallback row")


def test_embed_norm_bad_id_zero_row(ctx):
    rng = np.random.default_rng(4)
    table = W.quant_table(rng, 16, 256, "q4_0", (0.001, 0.05))
    emb = ops.TokenEmbedding(ctx, hip.GGML_Q4_0, table, 16, 256)
    ids = ctx.array(np.array([3, 16, 5], np.uint32))
    out = ctx.empty((3, 256), np.float32)
    emb.rows_device(ids, 1.0, out, norm_eps=1e-6)
    with pytest.raises(hip.CucaError, match="token id 16 outside the embedding table of 16 rows"):
        ctx.check_device()
    got = out.numpy()
    assert np.all(got[1] == 0)
    want = O.embed(table, O.Q4_0, 16, 256, np.array([3, 5], np.uint32), 1.0, norm_eps=1e-6)
    assert_bits_equal(got[[0, 2]], want)
    with pytest.raises(hip.CucaError, match="eps"):
        emb.rows_device(ids, 1.0, out, norm_eps=-1.0)


def test_embed_norm_full_table_sampled_rows(ctx):
    """A 151936 x 2048 Q4_0 table (config E's shape) and 8192 ids gathered
    with the norm, checked on sampled rows."""
    torch = pytest.importorskip("torch")
    cfg = W.CONFIGS["E"]
    gen = torch.Generator(device="cuda").manual_seed(9)
    table = W.quant_table_torch(gen, cfg["vocab"], cfg["hidden"], "q4_0", cfg["d_range"])
    ids = torch.randint(0, cfg["vocab"], (8192,), device="cuda", generator=gen, dtype=torch.int32)
    out = torch.empty((8192, cfg["hidden"]), device="cuda", dtype=torch.float16)
    torch.cuda.synchronize()
    ctx.embed_gguf_norm(table.data_ptr(), hip.GGML_Q4_0, cfg["vocab"], cfg["hidden"], ids.data_ptr(),
                        8192, 1.0, 1e-6, out.data_ptr(), hip.F16)
    ctx.sync()
    ctx.check_device()
    s = np.unique(np.concatenate([[0, 8191], np.random.default_rng(10).integers(0, 8192, 62)]))
    st = torch.from_numpy(s).cuda()
    rb = 18 * cfg["hidden"] // 32
    sub = table.view(cfg["vocab"], rb)[ids[st].long()].cpu().numpy().reshape(-1)
    want = O.embed(sub, O.Q4_0, s.size, cfg["hidden"], np.arange(s.size, dtype=np.uint32), 1.0,
                   out_dtype=np.float16, norm_eps=1e-6)
    assert_bits_equal(out[st].cpu().numpy(), want, "full table + norm")


# The gather fused with the first block's attention norm
# (cuca_hip_embed_gguf_rms): x bit-identical to the plain gather (the
# oracle's TokenEmbedding::rows), h = rms(x, w, eps) within the norm's bar
# (1e-5 relative in f32, 2 f16 ulps) of the oracle's norm of that x, and of
# the separate cuca_hip_add_rmsnorm call.
@pytest.mark.parametrize("qname", ["q4_0", "q8_0"])
@pytest.mark.parametrize("out", [np.float32, np.float16])
@pytest.mark.parametrize("hidden,eps,scale,weighted", [
    (4096, 1e-5, 1.0, True), (2048, 1e-6, 1.0, True), (3584, 1e-6, float(np.float32(np.sqrt(3584.0))), True),
    (1024, 1e-6, 1.0, False), (8192 + 96, 1e-5, 0.5, True), (96, 0.0, 2.0, True), (32, 1e-5, 1.0, True),
    (20000, 1e-6, 1.0, True)])
def test_embed_rms_matches_gather_then_norm(ctx, qname, out, hidden, eps, scale, weighted):
    """Rows of 1 to 1024 units take a workgroup per token (one unit per
    thread), 1025 to 2048 units 1024 threads of two, and wider rows the
    wave-per-token kernel (several rounds, the row re-read for h)."""
    from helpers import assert_close
    rng = np.random.default_rng(hidden * 3 + (qname == "q8_0"))
    vocab = 300
    table = W.quant_table(rng, vocab, hidden, qname, (0.001, 0.05))
    ty = W.GGML_ID[qname]
    ids = rng.integers(0, vocab, 45).astype(np.uint32)
    w = (1 + 0.02 * rng.standard_normal(hidden)).astype(np.float32) if weighted else None
    emb = ops.TokenEmbedding(ctx, ty, table, vocab, hidden)
    x, h = emb.rows_rms(ids, scale, w, eps, out_dtype=out)
    x, h = x.numpy(), h.numpy()
    ctx.check_device()
    want_x = O.embed(table, ty, vocab, hidden, ids, scale, out_dtype=out)
    assert_bits_equal(x, want_x, f"embed_rms x {qname} {hidden}")
    _, want_h = O.add_rmsnorm(want_x, None, w, eps, write_x=False)
    assert_close(h, want_h, what=f"embed_rms h {qname} {hidden}")
    # the unfused pair on the device
    _, h2 = ops.add_rms(ctx.array(want_x), None, w, eps, write_x=False)
    assert_close(h, h2.numpy(), what="embed_rms h vs add_rmsnorm")


@pytest.mark.parametrize("out", [np.float32, np.float16])
@pytest.mark.parametrize("hidden,n,weighted,bad", [
    (256, 8200, True, False), (256, 20001, False, False), (2048, 8200, True, True), (4096, 8193, True, False),
    (4096, 9000, False, True), (4128, 8200, True, False), (4096, 16384, True, True), (2048, 40000, True, False),
    (4096, 40000, False, False)])
def test_embed_rms_many_tokens(ctx, out, hidden, n, weighted, bad):
    """More than 8192 tokens: rows of 256 or 512 units (hidden 2048, 4096)
    take the persistent kernels (a thread per unit, each workgroup looping
    over 8, 16 or 32 tokens; 40000 tokens of 4096 need more than one round
    of workgroups), other rows of up to 4096 the LDS-staged kernel (weights
    in LDS once per workgroup, each wave looping over tpw tokens: 2 at 8200
    tokens, 4 at 20001, the last workgroup partial), wider rows the
    wave-per-token kernel.  An id outside the table gives zero rows of x and
    h and is reported, the other rows unchanged."""
    from helpers import assert_close
    rng = np.random.default_rng(hidden + n)
    vocab = 64
    qname = "q8_0" if hidden == 4096 else "q4_0"
    ty = W.GGML_ID[qname]
    table = W.quant_table(rng, vocab, hidden, qname, (0.001, 0.05))
    ids = rng.integers(0, vocab, n).astype(np.uint32)
    if bad:
        ids[n // 3] = vocab + 7
    w = (1 + 0.02 * rng.standard_normal(hidden)).astype(np.float32) if weighted else None
    emb = ops.TokenEmbedding(ctx, ty, table, vocab, hidden)
    dids = ctx.array(ids)
    x = ctx.empty((n, hidden), out)
    h = ctx.empty((n, hidden), out)
    dw = ctx.array(w) if weighted else None
    ctx.embed_gguf_rms(emb.table.ptr, ty, vocab, hidden, dids.ptr, n, 1.0, dw.ptr if weighted else None, 1e-6,
                       x.ptr, h.ptr, hip.F32 if out == np.float32 else hip.F16)
    if bad:
        with pytest.raises(hip.CucaError, match=f"token id {vocab + 7} outside"):
            ctx.check_device()
    else:
        ctx.check_device()
    good = np.ones(n, bool)
    if bad:
        good[n // 3] = False
        assert np.all(x.numpy()[n // 3] == 0) and np.all(h.numpy()[n // 3] == 0)
    ids_ok = np.where(good, ids, 0).astype(np.uint32)
    want_x = O.embed(table, ty, vocab, hidden, ids_ok, 1.0, out_dtype=out)[good]
    xs, hs = x.numpy()[good], h.numpy()[good]
    assert_bits_equal(xs, want_x, f"many tokens x {hidden} {n}")
    _, want_h = O.add_rmsnorm(want_x, None, w, 1e-6, write_x=False)
    assert_close(hs, want_h, what=f"many tokens h {hidden} {n}")


def test_embed_rms_bad_id_and_checks(ctx):
    rng = np.random.default_rng(11)
    table = W.quant_table(rng, 16, 256, "q8_0", (0.001, 0.05))
    emb = ops.TokenEmbedding(ctx, hip.GGML_Q8_0, table, 16, 256)
    ids = ctx.array(np.array([3, 16, 5], np.uint32))
    x = ctx.empty((3, 256), np.float16)
    h = ctx.empty((3, 256), np.float16)
    w = ctx.array(np.ones(256, np.float32))
    ctx.embed_gguf_rms(emb.table.ptr, hip.GGML_Q8_0, 16, 256, ids.ptr, 3, 1.0, w.ptr, 1e-6, x.ptr, h.ptr,
                       hip.F16)
    with pytest.raises(hip.CucaError, match="token id 16 outside the embedding table of 16 rows"):
        ctx.check_device()
    assert np.all(x.numpy()[1] == 0) and np.all(h.numpy()[1] == 0)
    want = O.embed(table, O.Q8_0, 16, 256, np.array([3, 5], np.uint32), 1.0, out_dtype=np.float16)
    assert_bits_equal(x.numpy()[[0, 2]], want)
    with pytest.raises(hip.CucaError, match="eps"):
        ctx.embed_gguf_rms(emb.table.ptr, hip.GGML_Q8_0, 16, 256, ids.ptr, 3, 1.0, w.ptr, -1.0, x.ptr, h.ptr,
                           hip.F16)
    with pytest.raises(hip.CucaError, match="null h_out"):
        ctx.embed_gguf_rms(emb.table.ptr, hip.GGML_Q8_0, 16, 256, ids.ptr, 3, 1.0, w.ptr, 1e-6, x.ptr, None,
                           hip.F16)


def test_embed_rms_full_size_config_c_sampled_rows(ctx):
    """Config C at 4096 tokens (128256 x 4096 Q8_0 table, f16), sampled rows
    against the oracle."""
    torch = pytest.importorskip("torch")
    from helpers import assert_close
    cfg = W.CONFIGS["C"]
    n, H = 4096, cfg["hidden"]
    gen = torch.Generator(device="cuda").manual_seed(21)
    table = W.quant_table_torch(gen, cfg["vocab"], H, cfg["qtype"], cfg["d_range"])
    ids = torch.randint(0, cfg["vocab"], (n,), device="cuda", generator=gen, dtype=torch.int32)
    w = (1 + 0.02 * torch.randn(H, device="cuda", generator=gen)).float()
    x = torch.empty((n, H), device="cuda", dtype=torch.float16)
    h = torch.empty_like(x)
    torch.cuda.synchronize()
    ctx.embed_gguf_rms(table.data_ptr(), W.GGML_ID[cfg["qtype"]], cfg["vocab"], H, ids.data_ptr(), n,
                       cfg["embd_scale"], w.data_ptr(), cfg["eps"], x.data_ptr(), h.data_ptr(), hip.F16)
    ctx.sync()
    ctx.check_device()
    rows = np.array([0, 1, 777, 2048, n - 1])
    sel = torch.from_numpy(rows).cuda()
    rb = W.row_bytes(cfg["qtype"], H)
    ids_np = ids.cpu().numpy().astype(np.uint32)[rows]
    tab_rows = table.view(cfg["vocab"], rb).index_select(0, torch.from_numpy(ids_np.astype(np.int64)).cuda())
    want_x = O.embed(tab_rows.cpu().numpy(), W.GGML_ID[cfg["qtype"]], rows.size, H, np.arange(rows.size, dtype=np.uint32),
                     cfg["embd_scale"], out_dtype=np.float16)
    assert_bits_equal(x.index_select(0, sel).cpu().numpy(), want_x, "C x")
    _, want_h = O.add_rmsnorm(want_x, None, w.cpu().numpy(), cfg["eps"], write_x=False)
    assert_close(h.index_select(0, sel).cpu().numpy(), want_h, what="C h")
