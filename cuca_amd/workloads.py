"""The five workload shapes of the per-layer ops and their seeded synthetic
inputs (used by bench.py and the tests; not by the ops themselves).

Shapes (A..E) are those the reference's architectures give these ops:
  A  Qwen3-0.6B layer:  H 1024, F 3072, Q 16x128 / K 8x128 NEOX theta 1e6,
     Q4_0 table 151936 x 1024, 128 tokens, f32, eps 1e-6.
  B  Llama-3-8B decode: H 4096, F 14336, Q 32x128 / K 8x128 NORM theta 5e5,
     Q8_0 table 128256 x 4096, batch 1 and 32, positions U[0, 8191], f32, eps 1e-5.
  C  Llama-3-8B prefill: as B, 4096 and 16384 tokens, f16 activations,
     positions 0..N-1.
  D  Gemma-2-9B layer: H 3584 with (1 + gamma) norms and the pre/post
     sandwich, GeGLU-tanh F 14336, Q 16x256 / K 8x256 interleaved (NORM)
     theta 1e4, Q4_0 table 256000 x 3584 scaled by sqrt(3584); 8 (f32) and
     2048 (f16) tokens; activations ~N(0, 2).
  E  Qwen3-30B-A3B MoE layer: H 2048, QK-norm + NEOX on Q 32x128 / K 4x128
     theta 1e6, SwiGLU F 768 over 8-of-128 token-expert pairs grouped by
     expert (ids ~ Zipf(1.1)), Q4_0 table 151936 x 2048; 64 (f32) and 8192
     (f16) tokens.

RoPE kinds follow the reference's architecture table (arch.rs:405-428): Llama
is NORM (adjacent pairs), Qwen is NEOX; config D asks for the interleaved
layout.

Host-side inputs (tests, small) come from numpy's PCG64 generator; full-size
inputs (bench) are generated on the device with torch's generator, so that
hundreds of MiB need not cross PCIe; the CPU baseline copies back the rows
it times.
"""

import math

import numpy as np

CONFIGS = {
    "A": dict(name="qwen3-0.6b-layer", hidden=1024, ff=3072, nq=16, nk=8, head_dim=128,
              rope="neox", theta=1e6, vocab=151936, qtype="q4_0", d_range=(0.001, 0.05),
              tokens=(128,), dtypes=("f32",), eps=1e-6, act="silu", std=1.0, seed=0,
              positions="prefix", embd_scale=1.0),
    "B": dict(name="llama3-8b-decode", hidden=4096, ff=14336, nq=32, nk=8, head_dim=128,
              rope="norm", theta=5e5, vocab=128256, qtype="q8_0", d_range=(0.001, 0.02),
              tokens=(1, 32), dtypes=("f32",), eps=1e-5, act="silu", std=1.0, seed=1,
              positions="random8192", embd_scale=1.0),
    "C": dict(name="llama3-8b-prefill", hidden=4096, ff=14336, nq=32, nk=8, head_dim=128,
              rope="norm", theta=5e5, vocab=128256, qtype="q8_0", d_range=(0.001, 0.02),
              tokens=(4096, 16384), dtypes=("f16",), eps=1e-5, act="silu", std=1.0, seed=2,
              positions="prefix", embd_scale=1.0),
    "D": dict(name="gemma2-9b-layer", hidden=3584, ff=14336, nq=16, nk=8, head_dim=256,
              rope="norm", theta=1e4, vocab=256000, qtype="q4_0", d_range=(0.001, 0.05),
              tokens=(8, 2048), dtypes=("f32", "f16"), eps=1e-6, act="gelu", std=2.0, seed=3,
              positions="prefix", sandwich=True,
              embd_scale=float(np.float32(math.sqrt(3584.0)))),
    "E": dict(name="qwen3-30b-a3b-moe-layer", hidden=2048, ff=768, nq=32, nk=4, head_dim=128,
              rope="neox", theta=1e6, vocab=151936, qtype="q4_0", d_range=(0.001, 0.05),
              tokens=(64, 8192), dtypes=("f32", "f16"), eps=1e-6, act="silu", std=1.0, seed=4,
              positions="prefix", qk_norm=True, moe=(128, 8), embd_scale=1.0),
}

BLOCK_BYTES = {"q4_0": 18, "q8_0": 34}
GGML_ID = {"q4_0": 2, "q8_0": 8}


def row_bytes(qtype, hidden):
    return hidden // 32 * BLOCK_BYTES[qtype]


def quant_table(rng, rows, hidden, qtype, d_range):
    """A Q4_0 / Q8_0 table [rows, hidden] as bytes (numpy): f16 scales
    ~U(d_range) rounded to nearest f16; Q4_0 nibble bytes uniform 0..255
    (both nibbles uniform); Q8_0 quants uniform in [-127, 127]."""
    nb = hidden // 32
    bs = BLOCK_BYTES[qtype]
    t = np.empty((rows * nb, bs), np.uint8)
    t[:, 0:2] = rng.uniform(*d_range, rows * nb).astype(np.float16).view(np.uint8).reshape(-1, 2)
    if qtype == "q4_0":
        t[:, 2:] = rng.integers(0, 256, (rows * nb, 16), dtype=np.uint8)
    else:
        t[:, 2:] = rng.integers(-127, 128, (rows * nb, 32), dtype=np.int8).view(np.uint8)
    return t.reshape(-1)


def quant_table_torch(gen, rows, hidden, qtype, d_range, device="cuda"):
    """quant_table on the device with a torch generator (full-size tables)."""
    import torch
    nb = hidden // 32
    bs = BLOCK_BYTES[qtype]
    t = torch.empty((rows * nb, bs), dtype=torch.uint8, device=device)
    d = torch.empty(rows * nb, dtype=torch.float32, device=device).uniform_(*d_range, generator=gen)
    t[:, 0:2] = d.to(torch.float16).view(torch.uint8).view(-1, 2)
    if qtype == "q4_0":
        t[:, 2:] = torch.randint(0, 256, (rows * nb, 16), dtype=torch.uint8, device=device,
                                 generator=gen)
    else:
        q = torch.randint(-127, 128, (rows * nb, 32), dtype=torch.int8, device=device, generator=gen)
        t[:, 2:] = q.view(torch.uint8)
    return t.view(-1)


def zipf_expert_rows(rng, n_tokens, n_experts, k, s=1.1):
    """MoE routing of n_tokens tokens to k distinct experts each, expert ids
    drawn from Zipf(s) over n_experts, grouped by expert in token order
    (route_with's grouping, moe.rs:39-94).  Returns (offsets int32
    [n_experts + 1], the token of every grouped row)."""
    p = 1.0 / np.arange(1, n_experts + 1, dtype=np.float64) ** s
    cdf = np.cumsum(p / p.sum())
    cdf[-1] = 1.0
    chosen = np.full((n_tokens, k), -1, np.int64)
    filled = np.zeros(n_tokens, np.int64)
    while (filled < k).any():
        todo = np.nonzero(filled < k)[0]
        e = np.searchsorted(cdf, rng.uniform(size=todo.size), side="right")
        e = np.minimum(e, n_experts - 1)
        dup = (chosen[todo] == e[:, None]).any(1)
        ok = todo[~dup]
        chosen[ok, filled[ok]] = e[~dup]
        filled[ok] += 1
    order = np.lexsort((np.repeat(np.arange(n_tokens), k), chosen.reshape(-1)))
    experts = chosen.reshape(-1)[order]
    tokens = np.repeat(np.arange(n_tokens), k)[order]
    counts = np.bincount(experts, minlength=n_experts)
    offsets = np.zeros(n_experts + 1, np.int32)
    offsets[1:] = np.cumsum(counts)
    return offsets, tokens


def positions(cfg, n, rng):
    if cfg["positions"] == "random8192":
        return rng.integers(0, 8192, n).astype(np.int32)
    return np.arange(n, dtype=np.int32)


def table_rows_needed(cfg, n):
    return 8192 if cfg["positions"] == "random8192" else max(n, 1)
