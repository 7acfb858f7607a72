"""Synthetic workloads of the five benchmark configurations (host metadata only).

Each generator returns numpy arrays of the per-sequence metadata (context
lengths, block tables, slots) drawn from numpy's PCG64 with the configuration's
seed, so tests and the benchmark see identical layouts on every host.  Tensor
contents (Q/K/V) are drawn separately: numpy for the small parity cases,
torch on the GPU for full-size benchmark pools.

C1  Qwen2.5-0.5B layer: H14 Hkv2 D64 bs16, pool 256 blocks, B=4, ctx ~ U[1,512], seed 0
C2  Llama-3-8B decode:   H32 Hkv8 D128 bs16, B=64, ctx ~ U[512,4096], pool = 1.1 x need, seed 1
C3  Qwen2.5-7B mixed:    H28 Hkv4 D128 bs32, 8 x 512-token chunks on prior U[0,2048]
                         + 120 decodes with ctx ~ U[1024,8192], seed 2
C4  block ops:           32 layers x Hkv8 x D128 fp16, bs64, 4096 copy pairs, 2048 swaps, seed 3
C5  FP8 decode:          H32 Hkv8 D128 bs16, B=256, ctx = clip(lognormal(7.6,1),128,32768), seed 4
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

import numpy as np


@dataclass
class Layout:
    """Block tables of a batch over a shared, randomly permuted pool."""
    context_lens: np.ndarray      # int32 [S] keys per sequence (after this step's append)
    block_tables: np.ndarray      # int32 [S, MB]
    num_blocks: int
    block_size: int
    extra: dict = field(default_factory=dict)

    @property
    def max_blocks_per_seq(self) -> int:
        return int(self.block_tables.shape[1])

    def slots(self, positions: np.ndarray, seqs: np.ndarray) -> np.ndarray:
        """slot = block_table[s][pos // bs] * bs + pos % bs (src/layers/attention.cpp:85-94)."""
        bs = self.block_size
        return (self.block_tables[seqs, positions // bs].astype(np.int64) * bs + positions % bs).astype(np.int32)


def make_layout(context_lens: np.ndarray, block_size: int, rng: np.random.Generator,
                num_blocks: Optional[int] = None, slack: float = 0.1,
                max_blocks_per_seq: Optional[int] = None) -> Layout:
    """Assign each sequence ceil(ctx/bs) distinct blocks from one random permutation of
    the pool; unused table entries are -1."""
    context_lens = np.asarray(context_lens, dtype=np.int32)
    need = (context_lens.astype(np.int64) + block_size - 1) // block_size
    total = int(need.sum())
    if num_blocks is None:
        num_blocks = int(np.ceil(total * (1.0 + slack))) if total else 1
    if total > num_blocks:
        raise ValueError(f"pool of {num_blocks} blocks cannot hold {total}")
    mb = int(need.max()) if len(need) else 1
    if max_blocks_per_seq is not None:
        mb = max(mb, max_blocks_per_seq)
    mb = max(mb, 1)
    perm = rng.permutation(num_blocks).astype(np.int32)
    tables = np.full((len(context_lens), mb), -1, np.int32)
    off = 0
    for s, n in enumerate(need):
        tables[s, :n] = perm[off:off + n]
        off += int(n)
    return Layout(context_lens, tables, num_blocks, block_size)


@dataclass
class DecodeConfig:
    name: str
    num_heads: int
    num_kv_heads: int
    head_dim: int
    block_size: int
    seed: int
    sigma: float
    layout: Layout
    prev_lens: np.ndarray  # context before this step's appended token

    @property
    def scale(self) -> float:
        return float(1.0 / np.sqrt(np.float32(self.head_dim)))

    @property
    def num_seqs(self) -> int:
        return int(len(self.prev_lens))

    def kv_bytes(self, elem_bytes: float, scale_bytes: int = 0) -> int:
        """Algorithmic KV bytes read by one decode call: every attended token's K and V once per kv head."""
        toks = int(self.layout.context_lens.astype(np.int64).sum())
        return toks * self.num_kv_heads * (2 * self.head_dim * elem_bytes + 2 * scale_bytes)


def config1() -> DecodeConfig:
    rng = np.random.default_rng(0)
    prev = rng.integers(1, 513, size=4).astype(np.int32)
    lay = make_layout(prev + 1, 16, rng, num_blocks=256)
    return DecodeConfig("C1-qwen2.5-0.5b", 14, 2, 64, 16, 0, 0.5, lay, prev)


def config2() -> DecodeConfig:
    rng = np.random.default_rng(1)
    prev = rng.integers(512, 4097, size=64).astype(np.int32)
    lay = make_layout(prev + 1, 16, rng, slack=0.1)
    return DecodeConfig("C2-llama3-8b-decode", 32, 8, 128, 16, 1, 0.3, lay, prev)


def config5() -> DecodeConfig:
    rng = np.random.default_rng(4)
    ctx = np.clip(np.round(rng.lognormal(7.6, 1.0, size=256)), 128, 32768).astype(np.int32)
    lay = make_layout(ctx, 16, rng, slack=0.1)
    # the appended token is the last of ctx: prev = ctx - 1
    return DecodeConfig("C5-llama3-8b-fp8-decode", 32, 8, 128, 16, 4, 1.0, lay, ctx - 1)


@dataclass
class MixedConfig:
    name: str
    num_heads: int
    num_kv_heads: int
    head_dim: int
    block_size: int
    layout: Layout            # prefill sequences first, then decode sequences
    q_lens: np.ndarray        # int32 [S] query tokens per sequence this step
    prior_lens: np.ndarray    # int32 [S] keys already cached before the step

    @property
    def query_start_loc(self) -> np.ndarray:
        return np.concatenate([[0], np.cumsum(self.q_lens)]).astype(np.int32)

    @property
    def scale(self) -> float:
        return float(1.0 / np.sqrt(np.float32(self.head_dim)))


def config3(num_prefill: int = 8, chunk: int = 512, num_decode: int = 120) -> MixedConfig:
    rng = np.random.default_rng(2)
    prior_p = rng.integers(0, 2049, size=num_prefill).astype(np.int32)
    ctx_d = rng.integers(1024, 8193, size=num_decode).astype(np.int32)
    prior = np.concatenate([prior_p, ctx_d - 1]).astype(np.int32)
    q_lens = np.concatenate([np.full(num_prefill, chunk), np.ones(num_decode)]).astype(np.int32)
    lay = make_layout(prior + q_lens, 32, rng, slack=0.1)
    return MixedConfig("C3-qwen2.5-7b-mixed", 28, 4, 128, 32, lay, q_lens, prior)


@dataclass
class BlockOpsConfig:
    num_layers: int
    num_kv_heads: int
    head_dim: int
    block_size: int
    num_blocks: int
    copy_pairs: np.ndarray    # int32 [P, 2]
    swap_blocks: np.ndarray   # int32 [Q] device blocks to swap out and back

    @property
    def block_bytes(self) -> int:  # one layer, K or V, fp16
        return self.block_size * self.num_kv_heads * self.head_dim * 2


def config4(num_pairs: int = 4096, num_swap: int = 2048, num_blocks: Optional[int] = None) -> BlockOpsConfig:
    """Copy pairs have distinct destinations and no destination is a source."""
    rng = np.random.default_rng(3)
    if num_blocks is None:
        num_blocks = 2 * num_pairs
    ids = rng.permutation(num_blocks).astype(np.int32)
    src = ids[:num_pairs]
    dst = ids[num_pairs:2 * num_pairs]
    pairs = np.stack([src, dst], axis=1).astype(np.int32)
    swap = rng.choice(num_blocks, size=min(num_swap, num_blocks), replace=False).astype(np.int32)
    return BlockOpsConfig(32, 8, 128, 64, num_blocks, pairs, swap)


def fill_pool_numpy(rng: np.random.Generator, num_blocks: int, block_size: int, num_kv_heads: int,
                    head_dim: int, sigma: float) -> tuple:
    """fp16 K and V pools [N, bs, Hkv, D] ~ N(0, sigma) (numpy, for small cases)."""
    shape = (num_blocks, block_size, num_kv_heads, head_dim)
    k = (rng.standard_normal(shape, dtype=np.float32) * sigma).astype(np.float16)
    v = (rng.standard_normal(shape, dtype=np.float32) * sigma).astype(np.float16)
    return k, v
