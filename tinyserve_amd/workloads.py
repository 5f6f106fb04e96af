"""Seeded synthetic inputs for the hot-path kernels, in the reference's layouts.

``decode_case`` and ``prefill_case`` scatter sequences over a randomly permuted pool of
cache blocks, as the reference's kernel tests do (tests/test_triton_attention.py:63-98,
tests/test_triton_prefill.py:64-102): with ``sentinel=True`` every slot no sequence owns
holds NaN and block-table padding points at a NaN block, so a kernel that reads one slot
too many returns NaN. The benchmark sizes (a 1 GB pool) are generated on the device
without sentinels.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch


@dataclass
class DecodeCase:
    q: torch.Tensor  # [B, Hq, D]
    k_cache: torch.Tensor  # [num_slots, Hkv, D]
    v_cache: torch.Tensor
    block_tables: torch.Tensor  # [B, W] int32
    context_lens: torch.Tensor  # [B] int32
    scale: float
    block_size: int

    def args(self) -> tuple[torch.Tensor, ...]:
        return self.q, self.k_cache, self.v_cache, self.block_tables, self.context_lens


def _scatter_tables(
    lens: list[int], block_size: int, pool_blocks: int | None, g: torch.Generator
) -> tuple[torch.Tensor, list[list[int]], int, int]:
    per_seq = [math.ceil(n / block_size) for n in lens]
    need = sum(per_seq) + 1
    num_blocks = max(pool_blocks or 0, need + 2)
    order = torch.randperm(num_blocks, generator=g).tolist()
    pad_block = order.pop()  # block-table padding points here
    width = max(per_seq, default=0) + 2
    tables = torch.full((len(lens), width), pad_block, dtype=torch.int32)
    blocks = []
    for b, nb in enumerate(per_seq):
        mine = [order.pop() for _ in range(nb)]
        tables[b, :nb] = torch.tensor(mine, dtype=torch.int32)
        blocks.append(mine)
    return tables, blocks, num_blocks, pad_block


def _slots(blocks: list[int], n: int, block_size: int) -> torch.Tensor:
    pos = torch.arange(n)
    return torch.tensor(blocks, dtype=torch.int64)[pos // block_size] * block_size + pos % block_size


def decode_case(
    lens: list[int],
    num_q_heads: int = 16,
    num_kv_heads: int = 8,
    head_dim: int = 128,
    block_size: int = 16,
    dtype: torch.dtype = torch.float32,
    seed: int = 0,
    magnitude: float = 1.0,
    pool_blocks: int | None = None,
    device: str | torch.device = "cpu",
) -> DecodeCase:
    """Sequences of ``lens`` tokens on randomly scattered blocks, NaN everywhere else."""
    g = torch.Generator().manual_seed(seed)
    tables, blocks, num_blocks, _ = _scatter_tables(lens, block_size, pool_blocks, g)
    shape = (num_blocks * block_size, num_kv_heads, head_dim)
    k = torch.full(shape, float("nan"))
    v = torch.full(shape, float("nan"))
    for n, mine in zip(lens, blocks):
        s = _slots(mine, n, block_size)
        k[s] = torch.randn(n, num_kv_heads, head_dim, generator=g) * magnitude
        v[s] = torch.randn(n, num_kv_heads, head_dim, generator=g)
    q = torch.randn(len(lens), num_q_heads, head_dim, generator=g) * magnitude
    return DecodeCase(
        q.to(device, dtype), k.to(device, dtype), v.to(device, dtype), tables.to(device),
        torch.tensor(lens, dtype=torch.int32, device=device), head_dim**-0.5, block_size,
    )  # fmt: skip


def decode_bench_case(
    batch: int,
    ctx: int,
    num_q_heads: int = 16,
    num_kv_heads: int = 8,
    head_dim: int = 128,
    block_size: int = 16,
    dtype: torch.dtype = torch.float16,
    pool_blocks: int | None = None,
    seed: int = 0,
    device: str | torch.device = "cuda",
) -> DecodeCase:
    """A benchmark-sized decode batch, generated on ``device``: every sequence at ``ctx``
    tokens, block tables a random permutation of the pool (no sentinels)."""
    nb = math.ceil(ctx / block_size)
    num_blocks = max(pool_blocks or 0, batch * nb + 1)
    g = torch.Generator(device=device).manual_seed(seed)
    perm = torch.randperm(num_blocks, generator=g, device=device)
    tables = perm[: batch * nb].view(batch, nb).to(torch.int32).contiguous()
    shape = (num_blocks * block_size, num_kv_heads, head_dim)
    k = torch.randn(shape, generator=g, device=device, dtype=dtype)
    v = torch.randn(shape, generator=g, device=device, dtype=dtype)
    q = torch.randn(batch, num_q_heads, head_dim, generator=g, device=device, dtype=dtype)
    lens = torch.full((batch,), ctx, dtype=torch.int32, device=device)
    return DecodeCase(q, k, v, tables, lens, head_dim**-0.5, block_size)


@dataclass
class PrefillCase:
    q: torch.Tensor  # [T, Hq, D]
    k: torch.Tensor  # [num_slots, Hkv, D]
    v: torch.Tensor
    tables: torch.Tensor  # [R, W] int32
    starts: torch.Tensor  # [R] int32
    q_lens: torch.Tensor
    ctx_lens: torch.Tensor
    block_size: int
    max_q_len: int

    @property
    def scale(self) -> float:
        return self.q.shape[2] ** -0.5

    def args(self) -> tuple[object, ...]:
        return (self.q, self.k, self.v, self.tables, self.starts, self.q_lens, self.ctx_lens,
                self.scale, self.block_size, self.max_q_len)  # fmt: skip


def prefill_case(
    specs: list[tuple[int, int]],  # per sequence: (cached tokens, new tokens)
    num_q_heads: int = 4,
    num_kv_heads: int = 2,
    head_dim: int = 8,
    block_size: int = 4,
    dtype: torch.dtype = torch.float32,
    seed: int = 0,
    gap: int = 0,  # rows of no sequence between sequences
    sentinel: bool = True,
    device: str | torch.device = "cpu",
) -> PrefillCase:
    """Packed varlen batch over a scattered cache (tests/test_triton_prefill.py:64-102)."""
    g = torch.Generator().manual_seed(seed)
    totals = [c + n for c, n in specs]
    tables, blocks, num_blocks, _ = _scatter_tables(totals, block_size, None, g)
    shape = (num_blocks * block_size, num_kv_heads, head_dim)
    fill = float("nan") if sentinel else 0.0
    k, v = torch.full(shape, fill), torch.full(shape, fill)
    starts, row = [], 0
    for (cached, new), total, mine in zip(specs, totals, blocks):
        s = _slots(mine, total, block_size)
        k[s] = torch.randn(total, num_kv_heads, head_dim, generator=g)
        v[s] = torch.randn(total, num_kv_heads, head_dim, generator=g)
        starts.append(row)
        row += new + gap
    q = torch.randn(row, num_q_heads, head_dim, generator=g)

    def i32(xs: list[int]) -> torch.Tensor:
        return torch.tensor(xs, dtype=torch.int32, device=device)

    return PrefillCase(
        q.to(device, dtype), k.to(device, dtype), v.to(device, dtype), tables.to(device),
        i32(starts), i32([n for _, n in specs]), i32(totals), block_size,
        max((n for _, n in specs), default=0),
    )  # fmt: skip


def prefill_lengths(num_seqs: int = 32, lo: int = 16, hi: int = 2048, seed: int = 0) -> list[int]:
    """BASELINE config 3's prompt lengths: uniform on [lo, hi], seeded."""
    g = torch.Generator().manual_seed(seed)
    return torch.randint(lo, hi + 1, (num_seqs,), generator=g).tolist()


@dataclass
class FusedCase:
    x: torch.Tensor  # [T, hidden]
    norm_w: torch.Tensor  # [hidden]
    qkv: torch.Tensor  # [T, (Hq + 2 Hkv) D], q/k/v are strided views of it
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    q_w: torch.Tensor
    k_w: torch.Tensor
    cos: torch.Tensor
    sin: torch.Tensor
    slots: torch.Tensor  # [T] int64
    k_cache: torch.Tensor
    v_cache: torch.Tensor
    eps: float


def fused_case(
    tokens: int = 4096,
    hidden: int = 1024,
    num_q_heads: int = 16,
    num_kv_heads: int = 8,
    head_dim: int = 128,
    num_blocks: int = 512,
    block_size: int = 16,
    theta: float = 1.0e6,
    eps: float = 1e-6,
    dtype: torch.dtype = torch.float16,
    seed: int = 0,
    sentinel: bool = True,
    device: str | torch.device = "cpu",
    cos_sin: tuple[torch.Tensor, torch.Tensor] | None = None,
) -> FusedCase:
    """RMSNorm input, QKV projection output views, RoPE tables for
    positions ~ U[0, 4095], and an injective slot map into a num_blocks x block_size pool.
    ``cos_sin``: the tables for the case's positions (by default computed here with the
    layers.py:41-65 formula, float64 angles)."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(tokens, hidden, generator=g)
    norm_w = 1 + 0.1 * torch.randn(hidden, generator=g)
    width = (num_q_heads + 2 * num_kv_heads) * head_dim
    qkv = torch.randn(tokens, width, generator=g)
    q_w = 1 + 0.1 * torch.randn(head_dim, generator=g)
    k_w = 1 + 0.1 * torch.randn(head_dim, generator=g)
    positions = torch.randint(0, 4096, (tokens,), generator=g)
    num_slots = num_blocks * block_size
    if tokens > num_slots:
        raise ValueError(f"{tokens} tokens do not fit injectively into {num_slots} slots")
    slots = torch.randperm(num_slots, generator=g)[:tokens]
    if cos_sin is None:
        exponent = torch.arange(0, head_dim, 2, dtype=torch.float64) / head_dim
        inv_freq = torch.pow(torch.tensor(theta, dtype=torch.float64), -exponent)
        ang = positions.to(torch.float64)[:, None] * inv_freq[None, :]
        ang = torch.cat([ang, ang], dim=-1)
        cos, sin = torch.cos(ang).float(), torch.sin(ang).float()
    else:
        cos, sin = cos_sin
    fill = float("nan") if sentinel else 0.0
    cache_shape = (num_slots, num_kv_heads, head_dim)
    qkv_d = qkv.to(device, dtype)
    hq, hkv, d = num_q_heads, num_kv_heads, head_dim
    return FusedCase(
        x=x.to(device, dtype), norm_w=norm_w.to(device, dtype), qkv=qkv_d,
        q=qkv_d[:, : hq * d].view(tokens, hq, d),
        k=qkv_d[:, hq * d : (hq + hkv) * d].view(tokens, hkv, d),
        v=qkv_d[:, (hq + hkv) * d :].view(tokens, hkv, d),
        q_w=q_w.to(device, dtype), k_w=k_w.to(device, dtype),
        cos=cos.to(device), sin=sin.to(device), slots=slots.to(device),
        k_cache=torch.full(cache_shape, fill, dtype=dtype, device=device),
        v_cache=torch.full(cache_shape, fill, dtype=dtype, device=device),
        eps=eps,
    )  # fmt: skip
