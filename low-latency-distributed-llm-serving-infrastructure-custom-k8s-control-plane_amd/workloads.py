"""Seeded synthetic steps for the paged-attention path.

Each workload is one engine step over a paged KV pool: per sequence a start
position and a new-token count (decode = 1 token at start = context - 1,
prefill chunk = many tokens), plus a random non-contiguous block table drawn
as a seeded permutation of the pool's block ids.  Shapes and distributions:

  fp32_mha_decode       8 seqs, 8/8 heads, D=64, ctx ~ U{16..512}, pool 512
                        blocks, scale 1/8, N(0,1) values
  kv_write_pack         32 seqs: 24 decode (prior ctx ~ U{16..2047}) + 8
                        prefill (count ~ U{64..256}, start 0), 32 KV heads,
                        D=128, bf16
  llama7b_mha_decode    64 seqs, 32/32 heads, D=128, ctx ~ U{128..4096},
                        values 0.5 * N(0,1), bf16
  llama3_8b_gqa_decode  256 seqs, 32/8 heads, D=128, ctx =
                        clip(round(lognormal(ln 1024, 1.0)), 32, 8192), bf16
  mixed_step            4 prefill chunks x 512 tokens at starts
                        {0, 512, 1024, 1536} + 128 decode seqs with ctx ~
                        U{512..32768}, 32/8 heads, D=128, bf16
  PREFILL_SHAPES        prefill-only steps of four 512-token chunks (at
                        {0, 512, 1024, 1536} or all at 4096), 32/8 heads,
                        D=128, bf16 and fp32; one 128-token prompt and
                        eight 64-token prompts, bf16

Lengths and block tables come from numpy's PCG64 generator; tensor values
are drawn with torch (on the target device for the large pools).
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import List, Optional, Tuple

import numpy as np
import torch

BLOCK_SIZE = 16


@dataclass
class StepWorkload:
    name: str
    num_query_heads: int
    num_kv_heads: int
    head_dim: int
    block_size: int
    dtype: torch.dtype
    value_scale: float
    start_positions: List[int]
    new_token_counts: List[int]
    block_lists: List[List[int]]
    total_blocks: int
    num_layers: int = 1

    @property
    def num_seqs(self) -> int:
        return len(self.start_positions)

    @property
    def context_lens(self) -> List[int]:
        return [s + c for s, c in zip(self.start_positions, self.new_token_counts)]

    @property
    def num_query_tokens(self) -> int:
        return int(sum(self.new_token_counts))

    @property
    def num_context_tokens(self) -> int:
        return int(sum(self.context_lens))

    @property
    def scaling(self) -> float:
        return 1.0 / math.sqrt(self.head_dim)

    @property
    def max_blocks(self) -> int:
        return max((len(b) for b in self.block_lists), default=0)

    def block_table_array(self, width: Optional[int] = None) -> np.ndarray:
        """int32 [B, width] padded with -1 (the layout of build_block_tables)."""
        width = self.max_blocks if width is None else width
        table = np.full((self.num_seqs, width), -1, dtype=np.int32)
        for i, blocks in enumerate(self.block_lists):
            table[i, : len(blocks)] = blocks
        return table

    def kv_bytes(self) -> int:
        """Algorithmic K+V bytes read by decode: each context token once per KV head."""
        e = torch.tensor([], dtype=self.dtype).element_size()
        return self.num_context_tokens * 2 * self.num_kv_heads * self.head_dim * e


def _block_tables(rng: np.random.Generator, context_lens: List[int], block_size: int, pool: Optional[int] = None):
    need = [-(-c // block_size) for c in context_lens]
    total = sum(need) if pool is None else pool
    if total < sum(need):
        raise ValueError("pool smaller than the blocks the contexts need")
    perm = rng.permutation(total).astype(np.int64)
    lists, off = [], 0
    for n in need:
        lists.append([int(b) for b in perm[off : off + n]])
        off += n
    return lists, total


def fp32_mha_decode(seed: int = 0) -> StepWorkload:
    rng = np.random.Generator(np.random.PCG64(seed))
    ctx = [int(c) for c in rng.integers(16, 512, size=8, endpoint=True)]
    lists, total = _block_tables(rng, ctx, BLOCK_SIZE, pool=512)
    return StepWorkload("fp32_mha_decode", 8, 8, 64, BLOCK_SIZE, torch.float32, 1.0,
                        [c - 1 for c in ctx], [1] * 8, lists, total)


def kv_write_pack(seed: int = 0) -> StepWorkload:
    rng = np.random.Generator(np.random.PCG64(seed))
    prior = [int(c) for c in rng.integers(16, 2047, size=24, endpoint=True)]
    counts = [int(c) for c in rng.integers(64, 256, size=8, endpoint=True)]
    starts = prior + [0] * 8
    new = [1] * 24 + counts
    ctx = [s + c for s, c in zip(starts, new)]
    lists, total = _block_tables(rng, ctx, BLOCK_SIZE)
    return StepWorkload("kv_write_pack", 32, 32, 128, BLOCK_SIZE, torch.bfloat16, 1.0, starts, new, lists, total)


def llama7b_mha_decode(seed: int = 0) -> StepWorkload:
    rng = np.random.Generator(np.random.PCG64(seed))
    ctx = [int(c) for c in rng.integers(128, 4096, size=64, endpoint=True)]
    lists, total = _block_tables(rng, ctx, BLOCK_SIZE)
    return StepWorkload("llama7b_mha_decode", 32, 32, 128, BLOCK_SIZE, torch.bfloat16, 0.5,
                        [c - 1 for c in ctx], [1] * 64, lists, total)


def llama3_8b_gqa_decode(seed: int = 0, num_seqs: int = 256) -> StepWorkload:
    rng = np.random.Generator(np.random.PCG64(seed))
    raw = rng.lognormal(mean=math.log(1024.0), sigma=1.0, size=num_seqs)
    ctx = [int(c) for c in np.clip(np.round(raw), 32, 8192)]
    lists, total = _block_tables(rng, ctx, BLOCK_SIZE)
    return StepWorkload("llama3_8b_gqa_decode", 32, 8, 128, BLOCK_SIZE, torch.bfloat16, 1.0,
                        [c - 1 for c in ctx], [1] * num_seqs, lists, total)


def mixed_step(seed: int = 0) -> StepWorkload:
    rng = np.random.Generator(np.random.PCG64(seed))
    starts = [0, 512, 1024, 1536]
    counts = [512] * 4
    dctx = [int(c) for c in rng.integers(512, 32768, size=128, endpoint=True)]
    starts += [c - 1 for c in dctx]
    counts += [1] * 128
    ctx = [s + c for s, c in zip(starts, counts)]
    lists, total = _block_tables(rng, ctx, BLOCK_SIZE)
    return StepWorkload("mixed_step", 32, 8, 128, BLOCK_SIZE, torch.bfloat16, 1.0, starts, counts, lists, total)


def prefill_chunks(name: str, starts: List[int], counts: List[int], dtype: torch.dtype, num_query_heads: int = 32,
                   num_kv_heads: int = 8, head_dim: int = 128, seed: int = 0) -> StepWorkload:
    """A prefill-only step: one chunk of ``counts[i]`` tokens at ``starts[i]``
    per sequence, over a pool of exactly the blocks the contexts need."""
    rng = np.random.Generator(np.random.PCG64(seed))
    ctx = [s + c for s, c in zip(starts, counts)]
    lists, total = _block_tables(rng, ctx, BLOCK_SIZE)
    return StepWorkload(name, num_query_heads, num_kv_heads, head_dim, BLOCK_SIZE, dtype, 1.0, list(starts),
                        list(counts), lists, total)


def decode_layers(num_seqs: int, num_layers: int = 32, seed: int = 0) -> StepWorkload:
    """A bf16 decode step of ``num_seqs`` sequences with contexts of 256-1024
    tokens (uniform) over 32/8 heads of 128, with ``num_layers`` layers of
    cache: the step a model's layer loop runs once per layer."""
    rng = np.random.Generator(np.random.PCG64(seed))
    ctx = [int(c) for c in rng.integers(256, 1024, size=num_seqs, endpoint=True)]
    lists, total = _block_tables(rng, ctx, BLOCK_SIZE)
    return StepWorkload(f"decode_layers_{num_seqs}", 32, 8, 128, BLOCK_SIZE, torch.bfloat16, 1.0,
                        [c - 1 for c in ctx], [1] * num_seqs, lists, total, num_layers)


# Prefill kernel shapes (32/8 heads, D=128): the mixed step's four 512-token
# chunks and four chunks deep in their contexts, in both dtypes, and two
# small prompt steps (one prompt of 128 tokens, eight of 64).
PREFILL_SHAPES = {
    "chunks_0_512_1024_1536_bf16": ([0, 512, 1024, 1536], [512] * 4, torch.bfloat16),
    "chunks_at_4096_bf16": ([4096] * 4, [512] * 4, torch.bfloat16),
    "chunks_0_512_1024_1536_fp32": ([0, 512, 1024, 1536], [512] * 4, torch.float32),
    "chunks_at_4096_fp32": ([4096] * 4, [512] * 4, torch.float32),
    "one_prompt_128_bf16": ([0], [128], torch.bfloat16),
    "prompts_8x64_bf16": ([0] * 8, [64] * 8, torch.bfloat16),
}


WORKLOADS = {
    "fp32_mha_decode": fp32_mha_decode,
    "kv_write_pack": kv_write_pack,
    "llama7b_mha_decode": llama7b_mha_decode,
    "llama3_8b_gqa_decode": llama3_8b_gqa_decode,
    "mixed_step": mixed_step,
}


@dataclass
class StepTensors:
    query: torch.Tensor      # [1, H_q, T, D] (the reference layout, a view of [T, H_q, D])
    key_cache: torch.Tensor  # (L, N, bs, H_kv, D)
    value_cache: torch.Tensor
    new_keys: torch.Tensor   # [T, H_kv, D] K of the step's new tokens
    new_values: torch.Tensor


def make_tensors(w: StepWorkload, device: torch.device, seed: int = 0) -> StepTensors:
    """Random query, pool contents and new K/V rows for ``w`` on ``device``.

    Values are N(0,1) * w.value_scale, rounded to w.dtype.  Drawn with torch's
    generator on ``device`` so that multi-GB pools are filled in place.
    """
    device = torch.device(device)
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    shape = (w.num_layers, w.total_blocks, w.block_size, w.num_kv_heads, w.head_dim)

    def draw(sz):
        t = torch.randn(sz, generator=gen, device=device, dtype=torch.float32)
        if w.value_scale != 1.0:
            t.mul_(w.value_scale)
        return t.to(w.dtype)

    q_flat = draw((w.num_query_tokens, w.num_query_heads, w.head_dim))
    key_cache = draw(shape)
    value_cache = draw(shape)
    new_k = draw((w.num_query_tokens, w.num_kv_heads, w.head_dim))
    new_v = draw((w.num_query_tokens, w.num_kv_heads, w.head_dim))
    query = q_flat.transpose(0, 1).unsqueeze(0)
    return StepTensors(query, key_cache, value_cache, new_k, new_v)


def decode_bytes(w: StepWorkload) -> int:
    """Algorithmic HBM bytes of one decode launch over the single-token
    sequences of the step: K+V once per (context token, KV head) + q and out
    rows + block-table entries + one context length per sequence."""
    e = torch.tensor([], dtype=w.dtype).element_size()
    ctx = [s + n for s, n in zip(w.start_positions, w.new_token_counts) if n == 1]
    kv = sum(ctx) * 2 * w.num_kv_heads * w.head_dim * e
    qo = len(ctx) * w.num_query_heads * w.head_dim * 2 * e
    bt = sum(-(-c // w.block_size) for c in ctx) * 4
    return kv + qo + bt + 4 * len(ctx)


def decode_flops(w: StepWorkload) -> int:
    return 4 * w.num_query_heads * w.head_dim * w.num_context_tokens


def prefill_flops(w: StepWorkload) -> int:
    f = 0
    for s, n in zip(w.start_positions, w.new_token_counts):
        if n > 1:
            f += 4 * w.num_query_heads * w.head_dim * (n * s + n * (n + 1) // 2)
    return f
