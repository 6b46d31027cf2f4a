"""Seeded synthetic workloads for the five BASELINE configurations.

Shapes follow the Qwen2 models the configurations name (layers, query heads,
KV heads, head_dim); inputs are synthetic (no weights or datasets exist on
this path): q, k, v ~ N(0, 1) fp32 from numpy's PCG64 with fixed seeds,
optionally with outlier channels or rounded to bf16-representable values.
Block tables come from the product's BlockTable (allocate/release in the
reference's LIFO order), so page ids are exactly what the table semantics
produce for the described call sequence.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

import tge_kv


@dataclass(frozen=True)
class Shape:
    name: str
    layers: int
    q_heads: int
    kv_heads: int
    head_dim: int

    @property
    def group(self):
        return self.q_heads // self.kv_heads

    @property
    def kv_dim(self):
        return self.kv_heads * self.head_dim

    @property
    def q_dim(self):
        return self.q_heads * self.head_dim


QWEN2_0_5B = Shape("Qwen2-0.5B", 24, 14, 2, 64)
QWEN2_1_5B = Shape("Qwen2-1.5B", 28, 12, 2, 128)
QWEN2_7B = Shape("Qwen2-7B", 28, 28, 4, 128)
# Attention shape of a 256-dim-head model (Gemma-2-9B: 16 query heads, 8 KV
# heads); 8 layers are enough for per-layer figures.
WIDE_HEADS = Shape("16/8 heads x 256 dims, 8 layers", 8, 16, 8, 256)


@dataclass
class Config:
    key: str
    shape: Shape
    fmt: int
    contexts: list            # initial context per session
    steps: int                # decode steps (0 for prefill)
    n_new: int = 1            # tokens appended + attended per session per step
    pool_pages: int = 0
    prefill_chunk: int = 0    # C4: chunk size of the prompt
    prompt: int = 0
    outlier_frac: float = 0.0  # fraction of kv channels scaled by outlier_gain in k
    outlier_gain: float = 8.0
    bf16_inputs: bool = False
    churn_every: int = 0
    churn_sessions: int = 0
    churn_context: int = 0
    fragmented: bool = True   # pool free list shuffled before the first session
    seed: int = 0
    note: str = field(default="")


def configs():
    """The five BASELINE.json configurations, in order."""
    rng = np.random.default_rng(2025)
    c5_ctx = [int(round(math.exp(x))) for x in rng.uniform(math.log(1024), math.log(32768), 64)]
    return {
        "c1": Config("c1", QWEN2_0_5B, tge_kv.KV_F16, [1024], steps=64, pool_pages=128, seed=1,
                     note="1 seq, f16, ctx 1024 + 64 decode steps, 128-page permuted pool"),
        "c2": Config("c2", QWEN2_0_5B, tge_kv.KV_I8, [4096], steps=128, pool_pages=272,
                     outlier_frac=0.01, fragmented=False, seed=2,
                     note="1 seq, int8+f16 scales, ctx 4096 + 128 steps, 1% outlier k channels x8"),
        "c3": Config("c3", QWEN2_1_5B, tge_kv.KV_F16, [512, 2048, 4096, 8192], steps=32,
                     pool_pages=1024, seed=3,
                     note="4 sessions 512/2048/4096/8192, f16, 32 steps, fragmented pool"),
        "c4": Config("c4", QWEN2_7B, tge_kv.KV_F16, [0], steps=0, pool_pages=128,
                     prefill_chunk=512, prompt=2048, bf16_inputs=True, seed=4,
                     note="2048-token prompt in 4 causal chunks of 512, f16, MFMA"),
        "c5": Config("c5", QWEN2_7B, tge_kv.KV_I8, c5_ctx, steps=32, n_new=4,
                     pool_pages=0, outlier_frac=0.01, churn_every=16, churn_sessions=8,
                     churn_context=2048, fragmented=False, seed=5,
                     note="64 sessions log-uniform 1k-32k, int8+f16 scales, 4-query verify, "
                          "churn 8 sessions / 16 steps"),
    }


def wide_head_configs():
    """Two legs at head_dim 256 (256-dim page blocks), beside the
    BASELINE configurations: a c5-like verify decode (32 sessions
    log-uniform 1k-32k, int8 + f16 scales, 4 queries each) and a c4-like
    prompt (2048 tokens in 4 causal chunks of 512, f16)."""
    rng = np.random.default_rng(2026)
    ctx = [int(round(math.exp(x))) for x in rng.uniform(math.log(1024), math.log(32768), 32)]
    return {
        "d256": Config("d256", WIDE_HEADS, tge_kv.KV_I8, ctx, steps=16, n_new=4, pool_pages=0,
                       outlier_frac=0.01, fragmented=True, seed=6,
                       note="head_dim 256: 32 sessions log-uniform 1k-32k, int8+f16 scales, "
                            "4-query verify, fragmented pool"),
        "p256": Config("p256", WIDE_HEADS, tge_kv.KV_F16, [0], steps=0, pool_pages=160,
                       prefill_chunk=512, prompt=2048, bf16_inputs=True, seed=7,
                       note="head_dim 256: 2048-token prompt in 4 causal chunks of 512, f16"),
    }


def pool_pages_for(cfg: Config, headroom=1.15):
    if cfg.pool_pages:
        return cfg.pool_pages
    need = sum(math.ceil((c + cfg.steps * cfg.n_new) / 16) for c in cfg.contexts)
    return int(need * headroom) + 64


def fragmented_table(pages, seed):
    """A BlockTable whose free list has been shuffled: allocate every page,
    then release them in a seeded random order. Later allocations pop the
    free list LIFO, so sessions receive scattered physical pages."""
    return tge_kv.BlockTable(pages).fragment(seed)


def normal(rng, shape):
    return rng.standard_normal(shape, dtype=np.float32)


def to_bf16_representable(x):
    """Round fp32 to the nearest bf16 value (ties to even), kept as fp32."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return rounded.astype(np.uint32).view(np.float32)


def outlier_channels(kv_dim, frac, seed):
    n = math.ceil(frac * kv_dim)
    return np.sort(np.random.default_rng(seed + 7).choice(kv_dim, size=n, replace=False))


def make_kv(rng, rows, kv_dim, cfg: Config):
    """k, v rows for `rows` tokens of one layer."""
    k = normal(rng, (rows, kv_dim))
    v = normal(rng, (rows, kv_dim))
    if cfg.outlier_frac:
        ch = outlier_channels(kv_dim, cfg.outlier_frac, cfg.seed)
        k[:, ch] *= np.float32(cfg.outlier_gain)
    if cfg.bf16_inputs:
        k, v = to_bf16_representable(k), to_bf16_representable(v)
    return k, v


def make_q(rng, rows, q_dim, cfg: Config):
    q = normal(rng, (rows, q_dim))
    return to_bf16_representable(q) if cfg.bf16_inputs else q


def algorithmic_bytes_decode(shape: Shape, fmt, spans, n_q=1):
    """Algorithmic bytes of one layer's decode attention over sessions with
    the given spans (K/V read once, q in, out, block table)."""
    total = 0
    kv = shape.kv_dim
    for s in spans:
        if fmt == tge_kv.KV_F16:
            kvb = 2 * s * kv * 2
        else:
            kvb = 2 * s * kv + 2 * s * (kv // 32) * 2
        total += kvb + 2 * n_q * shape.q_dim * 4 + math.ceil(s / 16) * 4
    return total


def algorithmic_bytes_append(shape: Shape, fmt, rows):
    kv = shape.kv_dim
    if fmt == tge_kv.KV_F16:
        return rows * (2 * kv * 4 + 2 * kv * 2)
    return rows * (2 * kv * 4 + 2 * kv + 2 * (kv // 32) * 2)


def prefill_flops(shape: Shape, ctx, n_new):
    """Useful FLOPs (QK + PV, causal) of one layer's chunk."""
    spans = sum(ctx + i + 1 for i in range(n_new))
    return 4 * shape.q_heads * shape.head_dim * spans
