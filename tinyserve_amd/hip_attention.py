"""Paged decode attention on MI355X: the entry points of the reference's
``tinyserve.triton_attention`` (src/tinyserve/triton_attention.py:330-586), same names,
arguments, results and errors, launching the HIP kernels of ``csrc/decode.hip``.

Kernel shape (gfx950). One wave64 per (sequence, query-head tile, split): the grouped
and split launches give a wave the whole GQA group of one kv head (both query heads of
Qwen3-0.6B), so every K/V byte is read once; the per-query-head launch
(``paged_decode_attention``, any head grouping) gives it one query head. Each wave
streams 16-byte K/V vectors of its range of cache blocks, three iterations in flight, and
keeps an online softmax per token lane, merged across lanes once at the end. With more
than one split, each (sequence, head tile) workgroup walks the reference's S block
ranges, parks each range's softmax state (m, l, acc) in LDS and merges them by the
reference's merge rule (``_merge_splits_kernel``, :299-327) before one write of the
output; shapes that cannot (blocks smaller than a loop iteration's tokens, too many
states for the LDS) write the fp32 partials to HBM and a second kernel combines them.

Every launch goes on torch's current stream, never synchronises and never allocates
outside torch's caching allocator, so a HIP graph can capture the ``launch_*``
functions. ``check_decode_args`` reads ``context_lens`` back (a host sync), as the
reference's does (:361-391).
"""

from __future__ import annotations

import ctypes
import functools

import torch

from tinyserve_amd import _lib

# The reference's names for its tuning knobs. ``NO_SPECIALIZE`` and ``DECODE_TILE`` are
# Triton launch options there (:62, :73); the HIP kernels have one compiled variant per
# (dtype, head_dim, heads per wave) whatever the batch looks like, and choose their own
# tiling, so a ``tile`` argument is validated (``check_tile``) and otherwise unused.
NO_SPECIALIZE = ["stride_bt", "num_splits"]
DECODE_TILE = (1, 1)

# Split-K policy (the reference's :488-510, retuned for MI355X). On one-round launches of
# long walks the kernel runs one wave per SIMD (its heavy register budget needs more than
# 256 VGPRs; launches of several rounds, or whose waves walk under 512 tokens, run a
# light budget at two per SIMD, and so do launches whose K/V exceeds the 256 MiB
# last-level cache, with non-temporal loads), and HBM wants about four waves per CU in
# flight. The library already splits each (sequence, head tile, split) over a workgroup
# of up to 4 waves (8 under the light budget) that merge in LDS (no HBM partials, no
# second launch), so a launch of 256 workgroups (one per CU) fills the chip. Splits that
# write HBM partials are only
# added below that: the launch aims at TARGET_PROGRAMS workgroups and stops splitting
# once the batch alone gives NO_SPLIT_PROGRAMS. The reference's T4 values were 1024 and
# 256 (T4_* below).
TARGET_PROGRAMS = 256
NO_SPLIT_PROGRAMS = 256
MAX_SPLITS = 16

# Split counts from the policy up to this run as one launch: the kernel gives each
# (sequence, head tile) a workgroup of up to 4 or 8 waves over contiguous block ranges,
# merged in LDS, so there are no fp32 partials in HBM and no combine pass (at B=32 x 256
# tokens: 10.0 us against 21.5 us for 4 partials + combine). More splits, and any count
# a caller asks for, write partials and combine them.
IN_GROUP_SPLITS = 4
# A split count S > 1 runs inside the one-split grid's workgroups (the ranges' states
# merged in LDS, one launch) only when that grid occupies at least this many SIMDs (one
# wave per SIMD under the heavy budget, two under the light ones), the whole chip; a
# smaller grid leaves most of the chip idle, and S workgroups per (sequence, head tile)
# writing fp32 partials, then the combine, finish sooner.
IN_GROUP_MIN_WAVES = 1024

# Reference constants, kept for ``num_splits_for(..., target=..., no_split=...)`` callers
# that want the T4 policy exactly.
T4_TARGET_PROGRAMS = 1024
T4_NO_SPLIT_PROGRAMS = 256


def check_decode_args(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    context_lens: torch.Tensor,
    block_size: int,
) -> None:
    """Raise ValueError if the arguments do not fit together (triton_attention.py:361-391).

    The last check reads ``context_lens`` to the host (a sync), so it is separate from
    the ``launch_*`` functions, which a graph can capture."""
    b, num_q_heads, head_dim = q.shape
    num_kv_heads = k_cache.shape[1]
    if num_q_heads % num_kv_heads:
        raise ValueError(f"{num_q_heads} query heads do not split into {num_kv_heads} groups")
    for name, n in (("head_dim", head_dim), ("block_size", block_size)):
        if n < 1 or n & (n - 1):
            raise ValueError(f"{name} must be a power of 2, got {n}")
    if k_cache.shape != v_cache.shape or k_cache.shape[2] != head_dim:
        raise ValueError(f"cache shapes {k_cache.shape} / {v_cache.shape} vs q {q.shape}")
    if block_tables.dtype != torch.int32 or context_lens.dtype != torch.int32:
        raise ValueError("block_tables and context_lens must be int32")
    if context_lens.shape != (b,) or block_tables.shape[0] != b:
        raise ValueError(f"need one block-table row and one length per sequence ({b})")
    if q.stride(2) != 1 or k_cache.stride(2) != 1 or v_cache.stride() != k_cache.stride():
        raise ValueError("the head dimension must be contiguous, and k/v laid out alike")
    _check_kernel_shape(q, k_cache)
    if bool((context_lens < 1).any()):
        raise ValueError("every sequence needs at least one token")


def _check_kernel_shape(q: torch.Tensor, k_cache: torch.Tensor) -> None:
    """Shapes the compiled kernels cover (head rows of 16 bytes .. 256 elements)."""
    head_dim = q.shape[2]
    if q.dtype != k_cache.dtype:
        raise ValueError(f"q is {q.dtype} but the cache is {k_cache.dtype}")
    if q.dtype not in _lib.DTYPES:
        raise ValueError(f"unsupported dtype {q.dtype}")
    if head_dim * q.element_size() < 16 or head_dim > 256:
        raise ValueError(f"head_dim {head_dim} is outside the HIP kernels' range (8..256)")


def check_tile(tile: tuple[int, int]) -> tuple[int, int]:
    """``tile`` if both numbers are powers of 2 (the reference's check, :480-485)."""
    blocks, warps = tile
    if blocks < 1 or blocks & (blocks - 1) or warps < 1 or warps & (warps - 1):
        raise ValueError(f"tile blocks and warps must be powers of 2, got {tile}")
    return tile


def num_splits_for(
    batch: int,
    num_kv_heads: int,
    max_blocks: int,
    target: int | None = None,
    no_split: int | None = None,
) -> int:
    """Ranges to split each sequence's blocks into (triton_attention.py:499-510): enough
    for about ``target`` waves, at most ``MAX_SPLITS`` and the block-table width; 1 once
    the batch alone gives ``no_split`` waves. Its inputs are sizes only (no context
    length is read), which keeps the grid of a graph-captured launch fixed."""
    target = TARGET_PROGRAMS if target is None else target
    no_split = NO_SPLIT_PROGRAMS if no_split is None else no_split
    programs = batch * num_kv_heads
    if programs >= no_split:
        return 1
    want = -(-target // programs)
    return max(1, min(want, MAX_SPLITS, max_blocks))


BUDGETS = ("heavy", "light", "light_stream")


def decode_plan(batch: int, num_q_heads: int, num_kv_heads: int, head_dim: int, block_size: int,
                max_blocks: int, splits: int, head_tile: int = 0,
                dtype: torch.dtype = torch.float16) -> dict[str, object]:  # fmt: skip
    """How ``ts_decode_split`` runs a launch of these sizes (``splits`` as passed to it: 1
    for the policy's in-workgroup split), without launching: the register budget, waves
    per workgroup, whether workgroups take length pairs, query heads per wave, the grid
    and the LDS per workgroup. The launch shape depends on sizes only."""
    out = (ctypes.c_int32 * 8)()
    _lib.call("ts_decode_plan", batch, num_q_heads, num_kv_heads, head_dim, block_size,
              max_blocks, splits, head_tile, _lib.DTYPES[dtype], out)  # fmt: skip
    return {"budget": BUDGETS[out[0]], "waves_per_group": out[1], "by_length": bool(out[2]),
            "head_tile": out[3], "grid": (out[4], out[5], out[6]), "lds_bytes": out[7]}  # fmt: skip


@functools.lru_cache(maxsize=512)
def _one_split_waves(device: int, b: int, hq: int, hkv: int, d: int, block_size: int, width: int,
                     dtype: torch.dtype) -> int:  # fmt: skip
    """SIMDs the one-split launch of these sizes occupies on ``device`` (which sets the CU
    count): its waves, over the two waves per SIMD of the light budgets."""
    p = decode_plan(b, hq, hkv, d, block_size, width, 1, 0, dtype)
    gx, gy, gz = p["grid"]
    waves = gx * gy * gz * int(p["waves_per_group"])
    return waves // 2 if p["budget"] in ("light", "light_stream") else waves


def policy_splits(batch: int, num_q_heads: int, num_kv_heads: int, head_dim: int, block_size: int,
                  max_blocks: int, dtype: torch.dtype = torch.float16, device: int = -1) -> int:  # fmt: skip
    """The split count the launcher uses when the caller gives none. A one-split grid
    occupying at least half ``IN_GROUP_MIN_WAVES`` SIMDs keeps ``num_splits_for``'s count,
    and a count up to ``IN_GROUP_SPLITS`` becomes one launch whose workgroups split each
    sequence over their waves. A smaller grid gets enough split ranges for about twice
    the chip (at most ``MAX_SPLITS`` and the table width), as fp32 partials and the
    combine. Sizes only (``device`` sets the CU count): a graph-captured launch keeps its
    grid."""
    splits = num_splits_for(batch, num_kv_heads, max_blocks)
    simds = _one_split_waves(device, batch, num_q_heads, num_kv_heads, head_dim, block_size,
                             max_blocks, dtype)  # fmt: skip
    if simds >= IN_GROUP_MIN_WAVES // 2:
        return 1 if splits <= IN_GROUP_SPLITS else splits
    return max(splits, min(-(-2 * IN_GROUP_MIN_WAVES // max(simds, 1)), MAX_SPLITS, max_blocks))


def _policy_splits(q: torch.Tensor, k_cache: torch.Tensor, block_tables: torch.Tensor,
                   block_size: int) -> int:  # fmt: skip
    """``policy_splits`` for a launch's tensors (1 for an empty batch or CPU tensors,
    whose launch raises)."""
    b, hq, d = q.shape
    if b == 0 or not q.is_cuda:
        return 1
    return policy_splits(b, hq, k_cache.shape[1], d, block_size, block_tables.shape[1], q.dtype,
                         q.device.index)  # fmt: skip


def _launch(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    context_lens: torch.Tensor,
    scale: float,
    block_size: int,
    splits: int,
    head_tile: int,
) -> torch.Tensor:
    dev = _lib.require_device(q, k_cache, v_cache, block_tables, context_lens)
    _check_kernel_shape(q, k_cache)
    b, hq, d = q.shape
    hkv = k_cache.shape[1]
    out = torch.empty_like(q)
    if b == 0:
        return out
    stream = _lib.stream_of(dev)
    dt = _lib.dtype_code(q)
    strides = (q.stride(0), q.stride(1), out.stride(0), out.stride(1),
               k_cache.stride(0), k_cache.stride(1), block_tables.stride(0))  # fmt: skip
    width = block_tables.shape[1]  # bounds every context: picks the kernel's register budget
    if splits == 1:
        _lib.call("ts_decode_split", q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
                  block_tables.data_ptr(), context_lens.data_ptr(), out.data_ptr(),
                  None, None, None, b, hq, hkv, d, block_size, *strides, width, 1, head_tile,
                  scale, dt, stream)  # fmt: skip
        return out
    # The split ranges inside each workgroup: every range's softmax state is merged with
    # the others in LDS, and the result written once. Grids too small to fill the chip,
    # and shapes the kernel cannot cut (blocks smaller than a loop iteration's tokens, or
    # more states than its LDS holds), write fp32 partials to HBM and combine them in a
    # second launch.
    if _one_split_waves(dev, b, hq, hkv, d, block_size, width, q.dtype) >= IN_GROUP_MIN_WAVES:
        rc = _lib.call_status("ts_decode_split", q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
                              block_tables.data_ptr(), context_lens.data_ptr(), out.data_ptr(),
                              None, None, None, b, hq, hkv, d, block_size, *strides, width, splits,
                              head_tile, scale, dt, stream)  # fmt: skip
        if rc == 0:
            return out
        if rc != _lib.TS_EUNSUPPORTED:
            raise ValueError(f"ts_decode_split: {_lib.load().ts_strerror(rc).decode()}")
    m = torch.empty((b, hq, splits), dtype=torch.float32, device=q.device)
    l = torch.empty_like(m)  # noqa: E741
    acc = torch.empty((b, hq, splits, d), dtype=torch.float32, device=q.device)
    _lib.call("ts_decode_split", q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
              block_tables.data_ptr(), context_lens.data_ptr(), out.data_ptr(),
              m.data_ptr(), l.data_ptr(), acc.data_ptr(), b, hq, hkv, d, block_size,
              *strides, width, splits, head_tile, scale, dt, stream)  # fmt: skip
    _lib.call("ts_decode_combine", m.data_ptr(), l.data_ptr(), acc.data_ptr(), out.data_ptr(),
              b, hq, d, out.stride(0), out.stride(1), splits, dt, stream)  # fmt: skip
    return out


def paged_decode_attention(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    context_lens: torch.Tensor,
    scale: float,
    block_size: int,
) -> torch.Tensor:
    """Validated decode attention: one new query per sequence against its whole paged
    context, B sequences per launch (triton_attention.py:330-358).

    Args:
        q: ``[B, Hq, D]``, the rotated query of each sequence's newest token.
        k_cache, v_cache: one layer's cache, ``[num_slots, Hkv, D]``, which must already
            hold the newest tokens' keys and values.
        block_tables: int32 ``[B, max_blocks]``; row b names sequence b's blocks in
            order, and columns past its last block are ignored.
        context_lens: int32 ``[B]``, each sequence's length counting the new token; at
            least 1.
        scale: factor applied to every q.k score.
        block_size: slots per cache block.

    Returns:
        A new ``[B, Hq, D]`` tensor, q's dtype.
    """
    check_decode_args(q, k_cache, v_cache, block_tables, context_lens, block_size)
    return launch_paged_decode(q, k_cache, v_cache, block_tables, context_lens, scale, block_size)


def launch_paged_decode(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    context_lens: torch.Tensor,
    scale: float,
    block_size: int,
) -> torch.Tensor:
    """The per-query-head launch alone (:394-421): no checks, no host sync."""
    return _launch(q, k_cache, v_cache, block_tables, context_lens, scale, block_size, 1, 1)


def paged_decode_attention_grouped(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    context_lens: torch.Tensor,
    scale: float,
    block_size: int,
) -> torch.Tensor:
    """``paged_decode_attention`` with one wave per (sequence, kv head) (:424-444); needs
    ``Hq / Hkv`` to be a power of 2."""
    check_decode_args(q, k_cache, v_cache, block_tables, context_lens, block_size)
    group = q.shape[1] // k_cache.shape[1]
    if group & (group - 1):
        raise ValueError(f"the grouped kernel needs a power-of-2 head group, got {group}")
    return launch_paged_decode_grouped(
        q, k_cache, v_cache, block_tables, context_lens, scale, block_size
    )


def launch_paged_decode_grouped(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    context_lens: torch.Tensor,
    scale: float,
    block_size: int,
    tile: tuple[int, int] | None = None,
) -> torch.Tensor:
    """The grouped launch alone (:447-477): no checks, no host sync."""
    check_tile(tile or DECODE_TILE)
    return _launch(q, k_cache, v_cache, block_tables, context_lens, scale, block_size, 1, 0)


def paged_decode_attention_split(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    context_lens: torch.Tensor,
    scale: float,
    block_size: int,
) -> torch.Tensor:
    """The grouped kernel with split-K (:513-531), splits from ``num_splits_for``."""
    check_decode_args(q, k_cache, v_cache, block_tables, context_lens, block_size)
    group = q.shape[1] // k_cache.shape[1]
    if group & (group - 1):
        raise ValueError(f"the grouped kernel needs a power-of-2 head group, got {group}")
    return launch_paged_decode_split(
        q, k_cache, v_cache, block_tables, context_lens, scale, block_size
    )


def launch_paged_decode_split(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    context_lens: torch.Tensor,
    scale: float,
    block_size: int,
    num_splits: int | None = None,
    tile: tuple[int, int] | None = None,
) -> torch.Tensor:
    """The split-K launches alone (:534-586): no checks, no host sync.

    An explicit ``num_splits`` S > 1 computes what the reference computes: S block
    ranges of ``ceil(blocks / S)``, each with its own softmax state (m, l, acc), merged
    by the two-partial rule. When the one-split grid fills the chip (``IN_GROUP_MIN_WAVES``)
    the states stay in each workgroup's LDS and the merge runs in the same launch;
    smaller grids, and block sizes under a loop iteration's tokens, write fp32 partials
    to HBM and combine them in a second launch. Without a count, it comes
    from ``policy_splits``: ``num_splits_for(B, Hkv, max_blocks)``, where a count up to
    ``IN_GROUP_SPLITS`` becomes one launch whose workgroups split each sequence over
    their waves (the library sizes the workgroup to the grid), raised for grids too
    small to fill the chip."""
    if num_splits and not 1 <= num_splits <= MAX_SPLITS:
        raise ValueError(f"num_splits must be 1..{MAX_SPLITS}, got {num_splits}")
    check_tile(tile or DECODE_TILE)
    # No count given (None or 0): the policy.
    splits = num_splits or _policy_splits(q, k_cache, block_tables, block_size)
    return _launch(q, k_cache, v_cache, block_tables, context_lens, scale, block_size, splits, 0)


def launch_paged_decode_split_noalloc(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    context_lens: torch.Tensor,
    scale: float,
    block_size: int,
    out: torch.Tensor,
    num_splits: int | None = None,
) -> torch.Tensor:
    """``launch_paged_decode_split`` into a caller-owned ``out``, with nothing allocated
    on the device: the split partials go to the library's static per-device scratch
    (``ts_decode_attention_noalloc``; no reference counterpart). For callers that cannot
    allocate, such as code under graph capture. Split counts as in
    ``launch_paged_decode_split``; a launch whose partials exceed the scratch raises
    ValueError before anything runs. Calls that overlap in time on one device race."""
    b, hq, d = q.shape
    if num_splits and not 1 <= num_splits <= MAX_SPLITS:
        raise ValueError(f"num_splits must be 1..{MAX_SPLITS}, got {num_splits}")
    splits = num_splits or _policy_splits(q, k_cache, block_tables, block_size)
    if out.shape != q.shape or out.dtype != q.dtype or out.stride(2) != 1:
        raise ValueError(f"out must be like q {tuple(q.shape)} {q.dtype}")
    dev = _lib.require_device(q, k_cache, v_cache, block_tables, context_lens, out)
    _check_kernel_shape(q, k_cache)
    _lib.call("ts_decode_attention_noalloc", q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
              block_tables.data_ptr(), context_lens.data_ptr(), out.data_ptr(), b, hq,
              k_cache.shape[1], d, block_size, q.stride(0), q.stride(1), out.stride(0), out.stride(1),
              k_cache.stride(0), k_cache.stride(1), block_tables.stride(0), block_tables.shape[1],
              splits, 0, scale, _lib.dtype_code(q), _lib.stream_of(dev))  # fmt: skip
    return out
