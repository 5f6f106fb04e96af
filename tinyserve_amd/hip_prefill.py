"""Varlen causal prefill attention on MI355X: ``paged_prefill_attention`` of the
reference's ``tinyserve.triton_prefill`` (src/tinyserve/triton_prefill.py:128-216), same
arguments, result and errors, launching ``csrc/prefill.hip``.

fp16 / bf16 with head_dim 64 or 128 run the MFMA kernel (v_mfma_f32_32x32x16):
S^T = K.Q^T and O^T += V^T.P^T with an online softmax in fp32, K and V tiles gathered
from the paged cache into LDS by direct-to-LDS loads and shared by every wave of the
workgroup. The library compiles three workgroup shapes and picks one from the launch's
sizes: 8 waves over 64-key tiles (128 queries x 2 heads, a 3-stage ring; large launches),
8 waves over 64 queries x 2 heads with the keys split into two halves walked by waves
w and w + 4 and merged through LDS (launches too small to fill the chip), and 4 waves
over 32-key tiles, three workgroups per CU (mid-size launches). fp16 P is rounded to
fp16 before P.V, as the reference kernel rounds P to V's dtype (triton_prefill.py:118);
bf16 P is carried as a hi + lo bf16 pair (two P.V MFMAs), since one bf16 rounding moves
outputs past the tolerance. fp32 inputs (exact fp32 dots, the reference's "ieee" path)
and other head dims run the decode kernel's loop, one wave per (query row, kv head).
"""

from __future__ import annotations

import torch

from tinyserve_amd import _lib

# The reference's Triton tile (rows_per_tile, block_n, num_warps), :47. The arguments are
# validated as the reference does and otherwise unused: the HIP kernels choose their tiles.
DEFAULT_TILE = (64, 32, 8)


def paged_prefill_attention(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    q_starts: torch.Tensor,
    q_lens: torch.Tensor,
    context_lens: torch.Tensor,
    scale: float,
    block_size: int,
    max_q_len: int,
    out: torch.Tensor | None = None,
    rows_per_tile: int | None = None,
    block_n: int | None = None,
    num_warps: int | None = None,
    ieee: bool | None = None,
) -> torch.Tensor:
    """One launch of causal attention over a packed batch of R prompts (or prompt
    chunks) whose keys and values are already in the paged cache
    (triton_prefill.py:128-198).

    Prompt r contributes ``q_lens[r]`` consecutive rows of ``q``, starting at row
    ``q_starts[r]``; they are the last ``q_lens[r]`` of its ``context_lens[r]``
    positions, and each row sees the positions up to and including its own, looked up
    through ``block_tables[r]``.

    Args:
        q: ``[T, Hq, D]`` queries after RoPE; rows no prompt claims are not read.
        k_cache, v_cache: one layer of the cache, ``[num_slots, Hkv, D]``, already
            holding this step's keys and values.
        block_tables: int32 ``[R, max_blocks]``.
        q_starts, q_lens, context_lens: int32 ``[R]``.
        max_q_len: host-side maximum of ``q_lens``; it sizes the grid, so nothing is read
            back from the device.
        out: ``[T, Hq, D]`` receiving the claimed rows only (default: a new tensor like
            ``q``).
        rows_per_tile, block_n, num_warps, ieee: tuning knobs of the Triton kernel; they
            are validated with the reference's rules and then ignored, since the HIP
            kernel chooses its own tiles.

    Returns:
        ``out``.
    """
    t, num_q_heads, head_dim = q.shape
    num_kv_heads = k_cache.shape[1]
    group = num_q_heads // num_kv_heads
    rows_per_tile = max(DEFAULT_TILE[0], group) if rows_per_tile is None else rows_per_tile
    block_n = DEFAULT_TILE[1] if block_n is None else block_n
    if num_q_heads % num_kv_heads or group & (group - 1):
        raise ValueError(f"need a power-of-2 head group, got {num_q_heads} / {num_kv_heads}")
    for name, n in (("block_size", block_size), ("rows_per_tile", rows_per_tile),
                    ("block_n", block_n)):  # fmt: skip
        if n < 1 or n & (n - 1):
            raise ValueError(f"{name} must be a power of 2, got {n}")
    if rows_per_tile < max(16, group) or block_n < 16:
        raise ValueError("a tile needs at least 16 rows and 16 keys")
    if k_cache.shape != v_cache.shape or k_cache.shape[2] != head_dim:
        raise ValueError(f"cache shapes {k_cache.shape} / {v_cache.shape} vs q {q.shape}")
    if q.stride(2) != 1 or k_cache.stride(2) != 1 or v_cache.stride() != k_cache.stride():
        raise ValueError("the head dimension must be contiguous, and k/v laid out alike")
    r = block_tables.shape[0]
    for name, x in (("q_starts", q_starts), ("q_lens", q_lens), ("context_lens", context_lens)):
        if x.dtype != torch.int32 or x.shape != (r,):
            raise ValueError(f"{name} must be int32 with one entry per sequence ({r})")
    if block_tables.dtype != torch.int32:
        raise ValueError("block_tables must be int32")
    if q.dtype != k_cache.dtype or q.dtype not in _lib.DTYPES:
        raise ValueError(f"q ({q.dtype}) and the cache ({k_cache.dtype}) must share a float dtype")
    if head_dim & (head_dim - 1) or head_dim * q.element_size() < 16 or head_dim > 256:
        raise ValueError(f"head_dim {head_dim} is outside the HIP kernels' range (2^k, 8..256)")
    if out is None:
        out = torch.empty_like(q)
    elif out.shape != q.shape or out.dtype != q.dtype or out.stride(2) != 1:
        raise ValueError(f"out must be like q {tuple(q.shape)} {q.dtype}")
    if r == 0 or t == 0:
        return out
    dev = _lib.require_device(q, k_cache, v_cache, block_tables, q_starts, q_lens, context_lens, out)
    _lib.call(
        "ts_prefill_varlen",
        q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), out.data_ptr(),
        block_tables.data_ptr(), q_starts.data_ptr(), q_lens.data_ptr(), context_lens.data_ptr(),
        r, num_q_heads, num_kv_heads, head_dim, block_size, int(max_q_len), t,
        q.stride(0), q.stride(1), out.stride(0), out.stride(1),
        k_cache.stride(0), k_cache.stride(1), block_tables.stride(0),
        float(scale), _lib.dtype_code(q), _lib.stream_of(dev),
    )  # fmt: skip
    return out
