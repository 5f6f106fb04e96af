"""The HIP paged decode-attention kernels must match the oracle (GPU).

Mirrors the reference's tests/test_triton_attention.py and tests/test_kernel_variants.py
case by case, with the oracle's ``decode_ref`` (a restatement of
``paged_decode_attention_ref``, attention.py:114-141) as the reference. Every cache slot
no sequence owns is NaN and block-table padding points at a NaN block, so a kernel that
reads one slot too many returns NaN and fails. Tolerances: tests/helpers.py.
"""

from __future__ import annotations

import math
from collections.abc import Callable

import pytest
import torch
from hypothesis import given, settings
from hypothesis import strategies as st

from oracle import ref
from tests.helpers import TOL, assert_contract, assert_matches
from tinyserve_amd import _lib
from tinyserve_amd import hip_attention as ha
from tinyserve_amd.workloads import DecodeCase, decode_bench_case, decode_case

pytestmark = pytest.mark.gpu
DEVICE = "cuda"
KERNELS = [ha.paged_decode_attention, ha.paged_decode_attention_grouped, ha.paged_decode_attention_split]


def on_gpu(c: DecodeCase) -> DecodeCase:
    return DecodeCase(*(t.to(DEVICE) for t in c.args()), c.scale, c.block_size)


def oracle32(c: DecodeCase) -> torch.Tensor:
    """The oracle's float32 result (before rounding to the case's dtype)."""
    return ref.decode_ref(c.q.float(), c.k_cache.float(), c.v_cache.float(), c.block_tables,
                          c.context_lens, c.scale, c.block_size)  # fmt: skip


def check(c: DecodeCase, kernels: list[Callable[..., torch.Tensor]] = KERNELS,
          contract: bool = False) -> torch.Tensor:  # fmt: skip
    want = oracle32(c)
    g = on_gpu(c)
    for kernel in kernels:
        out = kernel(*g.args(), g.scale, g.block_size)
        assert out.dtype == c.q.dtype and out.device.type == "cuda"
        assert torch.isfinite(out).all(), f"{kernel.__name__}: read a slot outside the sequence"
        (assert_contract if contract else assert_matches)(out, want, c.q.dtype, kernel.__name__)
    return want


def test_one_token_returns_its_value() -> None:
    c = decode_case([1], num_q_heads=4, num_kv_heads=2, head_dim=32)
    out = ha.paged_decode_attention_split(*on_gpu(c).args(), c.scale, c.block_size)
    slot = int(c.block_tables[0, 0]) * c.block_size
    torch.testing.assert_close(out[0].cpu(), c.v_cache[slot].repeat_interleave(2, dim=0),
                               atol=1e-6, rtol=1e-6)  # fmt: skip
    check(c)


def test_qwen3_shapes_across_block_boundaries() -> None:
    check(decode_case([1, 15, 16, 17, 31, 32, 33, 193]))


def test_baseline_config_1() -> None:
    # fp32, 16/8/128, contexts {17, 64, 128, 200}, a 64-block pool.
    check(decode_case([17, 64, 128, 200], pool_blocks=64), contract=True)


@pytest.mark.parametrize(("num_q_heads", "num_kv_heads"), [(4, 4), (8, 2), (8, 1), (16, 2)])
def test_head_groupings(num_q_heads: int, num_kv_heads: int) -> None:
    check(decode_case([3, 20, 47], num_q_heads, num_kv_heads, head_dim=64))


def test_a_group_that_is_not_a_power_of_2_on_the_per_head_kernel() -> None:
    check(decode_case([3, 40], 12, 4, head_dim=32), [ha.paged_decode_attention])


@pytest.mark.parametrize("block_size", [1, 2, 8, 32, 64])
def test_block_sizes(block_size: int) -> None:
    check(decode_case([1, 9, 40, 130], 4, 2, head_dim=32, block_size=block_size))


@pytest.mark.parametrize("head_dim", [8, 16, 32, 64, 128, 256])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_head_dims_and_dtypes(head_dim: int, dtype: torch.dtype) -> None:
    if head_dim * (4 if dtype == torch.float32 else 2) < 16:
        pytest.skip("rows under 16 bytes are not a kernel shape")
    check(decode_case([1, 33, 90], 4, 2, head_dim=head_dim, dtype=dtype, seed=head_dim))


def test_float16() -> None:
    check(decode_case([1, 16, 100, 193], dtype=torch.float16))


def test_bfloat16() -> None:
    check(decode_case([1, 16, 100, 193], dtype=torch.bfloat16))


def test_large_scores_do_not_overflow() -> None:
    check(decode_case([40, 70], 4, 2, head_dim=64, dtype=torch.float16, magnitude=12.0))


@pytest.mark.parametrize("kernel", KERNELS)
def test_each_sequence_only_sees_its_own_blocks(kernel: Callable[..., torch.Tensor]) -> None:
    # Running sequences together or alone gives the same rows, bit for bit.
    c = on_gpu(decode_case([7, 30, 2], 4, 2, head_dim=32, block_size=4))
    together = kernel(*c.args(), c.scale, c.block_size)
    for b in range(3):
        alone = kernel(c.q[b : b + 1], c.k_cache, c.v_cache, c.block_tables[b : b + 1],
                       c.context_lens[b : b + 1], c.scale, c.block_size)  # fmt: skip
        assert torch.equal(alone, together[b : b + 1])


@settings(max_examples=15, deadline=None)
@given(
    lens=st.lists(st.integers(1, 70), min_size=1, max_size=4),
    heads=st.sampled_from([(2, 1), (4, 2), (4, 4)]),
    head_dim=st.sampled_from([16, 32]),
    block_size=st.sampled_from([2, 4, 16]),
    seed=st.integers(0, 2**16),
)
def test_random_shapes(lens: list[int], heads: tuple[int, int], head_dim: int, block_size: int,
                       seed: int) -> None:  # fmt: skip
    check(decode_case(lens, *heads, head_dim=head_dim, block_size=block_size, seed=seed))


@pytest.mark.parametrize("splits", [1, 2, 3, 5, 16])
@pytest.mark.parametrize("lens", [[1], [17, 300, 33], [64, 2]])
def test_any_number_of_splits_gives_the_same_result(splits: int, lens: list[int]) -> None:
    # More ranges than a sequence has blocks leaves some empty: they must not count.
    c = decode_case(lens, 4, 2, head_dim=32, block_size=4, seed=splits)
    want = oracle32(c)
    g = on_gpu(c)
    out = ha.launch_paged_decode_split(*g.args(), c.scale, c.block_size, num_splits=splits)
    assert torch.isfinite(out).all()
    assert_matches(out, want, torch.float32)


@pytest.mark.parametrize("tile", [(1, 2), (2, 4), (4, 8), (8, 8)])
@pytest.mark.parametrize("splits", [1, 3])
def test_every_tile_gives_the_same_result(tile: tuple[int, int], splits: int) -> None:
    c = decode_case([17, 300, 33], 4, 2, head_dim=32, block_size=4, seed=tile[0] + splits)
    want = oracle32(c)
    g = on_gpu(c)
    out = ha.launch_paged_decode_split(*g.args(), c.scale, c.block_size, splits, tile)
    assert_matches(out, want, torch.float32)
    grouped = ha.launch_paged_decode_grouped(*g.args(), c.scale, c.block_size, tile)
    assert_matches(grouped, want, torch.float32)


WIDTHS = [1, 2, 9, 16, 32, 600]


def widened(tables: torch.Tensor, width: int) -> torch.Tensor:
    """``tables`` cut or padded to ``width`` columns (padding repeats the NaN block)."""
    if width <= tables.shape[1]:
        return tables[:, :width].contiguous()
    pad = tables[:, -1:].expand(-1, width - tables.shape[1])
    return torch.cat([tables, pad], dim=1).contiguous()


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_every_width_and_split_count_gives_the_reference(dtype: torch.dtype) -> None:
    # test_kernel_variants.py:44-58: every block-table width and every split count.
    c = decode_case([5, 12, 16], dtype=dtype, seed=7)
    want = oracle32(c)
    g = on_gpu(c)
    for w in WIDTHS:
        args = (g.q, g.k_cache, g.v_cache, widened(g.block_tables, w), g.context_lens)
        for launch in (ha.launch_paged_decode, ha.launch_paged_decode_grouped):
            assert_matches(launch(*args, c.scale, c.block_size), want, dtype, f"w={w}")
        for s in range(2, ha.MAX_SPLITS + 1):
            out = ha.launch_paged_decode_split(*args, c.scale, c.block_size, num_splits=s)
            assert_matches(out, want, dtype, f"w={w} s={s}")


def test_thirty_two_sequences_at_qwen3_shapes() -> None:
    # test_triton_attention.py:304-311: the C=32 step, 32 sequences of ~161 tokens, fp16.
    c = decode_case([161 + i for i in range(32)], dtype=torch.float16, seed=3)
    want = oracle32(c)
    g = on_gpu(c)
    for splits in (None, 1, 4):
        out = ha.launch_paged_decode_split(*g.args(), c.scale, c.block_size, splits)
        assert_matches(out, want, torch.float16, f"splits={splits}")


def test_one_long_sequence() -> None:
    check(decode_case([2048], dtype=torch.float16, seed=2))


def test_benchmark_sized_batch() -> None:
    check(decode_case([193] * 64, dtype=torch.float16, seed=1))


def hbm_split_combine(g: DecodeCase, splits: int) -> torch.Tensor:
    """The reference's two launches exactly: every split range writes its fp32 partial
    (m, l, acc) to HBM, then the combine kernel merges them."""
    b, hq, d = g.q.shape
    out = torch.empty_like(g.q)
    m = torch.empty((b, hq, splits), dtype=torch.float32, device=DEVICE)
    l = torch.empty_like(m)  # noqa: E741
    acc = torch.empty((b, hq, splits, d), dtype=torch.float32, device=DEVICE)
    dt, stream = _lib.dtype_code(g.q), _lib.stream_of(0)
    _lib.call("ts_decode_split", g.q.data_ptr(), g.k_cache.data_ptr(), g.v_cache.data_ptr(),
              g.block_tables.data_ptr(), g.context_lens.data_ptr(), None, m.data_ptr(), l.data_ptr(),
              acc.data_ptr(), b, hq, g.k_cache.shape[1], d, g.block_size, g.q.stride(0), g.q.stride(1),
              0, 0, g.k_cache.stride(0), g.k_cache.stride(1), g.block_tables.stride(0),
              g.block_tables.shape[1], splits, 0, g.scale, dt, stream)  # fmt: skip
    _lib.call("ts_decode_combine", m.data_ptr(), l.data_ptr(), acc.data_ptr(), out.data_ptr(),
              b, hq, d, out.stride(0), out.stride(1), splits, dt, stream)  # fmt: skip
    return out


def in_group_split(g: DecodeCase, splits: int) -> torch.Tensor:
    """ts_decode_split with no partial buffers: the split ranges merge in each workgroup."""
    b, hq, d = g.q.shape
    out = torch.empty_like(g.q)
    _lib.call("ts_decode_split", g.q.data_ptr(), g.k_cache.data_ptr(), g.v_cache.data_ptr(),
              g.block_tables.data_ptr(), g.context_lens.data_ptr(), out.data_ptr(), None, None,
              None, b, hq, g.k_cache.shape[1], d, g.block_size, g.q.stride(0), g.q.stride(1),
              out.stride(0), out.stride(1), g.k_cache.stride(0), g.k_cache.stride(1),
              g.block_tables.stride(0), g.block_tables.shape[1], splits, 0, g.scale,
              _lib.dtype_code(g.q), _lib.stream_of(0))  # fmt: skip
    return out


@pytest.mark.parametrize("splits", [56, 60, 100])
def test_in_group_splits_past_one_wave_of_slots(splits: int) -> None:
    # The C ABI takes any split count whose states fit the workgroup's LDS. With small
    # states (64-element rows, one query head per kv head) the split ranges plus the
    # waves' pieces can exceed 64 slots per sequence; every slot must still be merged.
    c = decode_case([3000, 1500, 4096, 77], num_q_heads=4, num_kv_heads=4, head_dim=64,
                    dtype=torch.float16, seed=9)
    want = oracle32(c)
    g = on_gpu(c)
    out = in_group_split(g, splits)
    torch.cuda.synchronize()
    assert_contract(out, want, torch.float16, f"in-group {splits} splits, D=64")


def test_baseline_config_2() -> None:
    # fp16, B=32 at context 256, a 4096-block pool, 4 splits: the
    # reference's ranges of ceil(16 / 4) = 4 blocks, each with its own softmax state, merged
    # in each workgroup's LDS (the launcher's path), and the same four states as fp32
    # partials in HBM merged by the combine pass; and the policy's one launch (no count
    # given), which splits each sequence over the waves of a workgroup.
    c = decode_case([256] * 32, dtype=torch.float16, pool_blocks=4096, seed=0)
    want = oracle32(c)
    g = on_gpu(c)
    plan = ha.decode_plan(32, 16, 8, 128, 16, g.block_tables.shape[1], 4)
    assert plan["grid"][2] == 4, plan
    out = ha.launch_paged_decode_split(*g.args(), c.scale, c.block_size, num_splits=4)
    assert torch.isfinite(out).all()
    assert_contract(out, want, torch.float16, "config 2, 4 splits merged in the workgroup")
    hbm = hbm_split_combine(g, 4)
    assert_contract(hbm, want, torch.float16, "config 2, 4 splits + combine")
    torch.testing.assert_close(out, hbm, atol=1e-3, rtol=0)
    policy = ha.launch_paged_decode_split(*g.args(), c.scale, c.block_size)
    assert_contract(policy, want, torch.float16, "config 2, policy (one launch)")


@pytest.mark.parametrize("case", [
    # (lens, heads, dtype, block_size): one-wave workgroups (512 sequences), 2-8 wave
    # workgroups, length pairs (33-64 sequences, odd and even), the heavy budget (few long
    # sequences), four query heads per wave, bf16 and fp32, more splits than blocks.
    ([1 + (97 * i) % 400 for i in range(512)], (16, 8), torch.float16, 16),
    ([256] * 32, (16, 8), torch.float16, 16),
    ([1 + (389 * i) % 1000 for i in range(45)], (16, 8), torch.float16, 16),
    ([1 + (389 * i) % 3000 for i in range(64)], (16, 8), torch.bfloat16, 16),
    ([4096, 1, 2500, 17], (16, 8), torch.float16, 16),
    ([300, 17, 64, 1000, 5], (32, 8), torch.float16, 16),
    ([300, 17, 64, 1000, 5], (16, 8), torch.float32, 16),
    ([1, 2, 17, 33], (16, 8), torch.float16, 16),
    ([700, 31, 1200], (16, 8), torch.float16, 32),
])  # fmt: skip
@pytest.mark.parametrize("splits", [2, 3, 4, 7, 16])
def test_in_workgroup_splits_match_the_hbm_partials(case: tuple, splits: int, monkeypatch) -> None:
    # An explicit split count merges the ranges' states in LDS (one launch); the same
    # ranges as HBM partials + the combine launch must give the same output up to fp32
    # summation order, and both the oracle's. The small grids here would take the HBM
    # form under the launcher's policy: the in-group path is forced for every case.
    monkeypatch.setattr(ha, "IN_GROUP_MIN_WAVES", 0)
    lens, (hq, hkv), dtype, bs = case
    c = decode_case(lens, hq, hkv, dtype=dtype, block_size=bs, seed=len(lens) + splits)
    g = on_gpu(c)
    out = ha.launch_paged_decode_split(*g.args(), c.scale, c.block_size, num_splits=splits)
    hbm = hbm_split_combine(g, splits)
    assert torch.isfinite(out).all()
    tol = {torch.float32: 2e-6, torch.float16: 1e-3, torch.bfloat16: 8e-3}[dtype]
    torch.testing.assert_close(out.float(), hbm.float(), atol=tol, rtol=0)
    rows = list(range(0, len(lens), max(1, len(lens) // 16)))
    sub = DecodeCase(c.q[rows], c.k_cache, c.v_cache, c.block_tables[rows], c.context_lens[rows],
                     c.scale, c.block_size)  # fmt: skip
    assert_matches(out[rows], oracle32(sub), dtype, f"{len(lens)} sequences, {splits} splits")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("splits,lens", [(4, [256] * 32), (16, [17, 300, 33, 1, 700, 2000]),
                                         (3, [1, 2, 47, 48, 49]), (5, [64] * 3)])  # fmt: skip
def test_split_partials_follow_the_reference_ranges(splits: int, lens: list[int], dtype: torch.dtype) -> None:
    # ts_decode_split's fp32 partials, before the combine, against the oracle's restatement
    # of _paged_decode_split_kernel (triton_attention.py:243-296): split s holds blocks
    # [s * ceil(n / S), ...) of each sequence, empty past the end (m = -inf, l = 0). m is
    # stored in base-2 units (log2 e * the max score).
    c = decode_case(lens, dtype=dtype, seed=splits)
    m_ref, l_ref, acc_ref = ref.split_partials_ref(c.q.float(), c.k_cache.float(), c.v_cache.float(),
                                                   c.block_tables, c.context_lens, c.scale, c.block_size,
                                                   splits)  # fmt: skip
    g = on_gpu(c)
    b, hq, d = g.q.shape
    m = torch.empty((b, hq, splits), dtype=torch.float32, device=DEVICE)
    l = torch.empty_like(m)  # noqa: E741
    acc = torch.empty((b, hq, splits, d), dtype=torch.float32, device=DEVICE)
    _lib.call("ts_decode_split", g.q.data_ptr(), g.k_cache.data_ptr(), g.v_cache.data_ptr(),
              g.block_tables.data_ptr(), g.context_lens.data_ptr(), None, m.data_ptr(), l.data_ptr(),
              acc.data_ptr(), b, hq, g.k_cache.shape[1], d, g.block_size, g.q.stride(0), g.q.stride(1),
              0, 0, g.k_cache.stride(0), g.k_cache.stride(1), g.block_tables.stride(0),
              g.block_tables.shape[1], splits, 0, g.scale, _lib.dtype_code(g.q),
              _lib.stream_of(0))  # fmt: skip
    torch.cuda.synchronize()
    m, l, acc = m.cpu(), l.cpu(), acc.cpu()  # noqa: E741
    empty = m_ref == float("-inf")
    assert torch.equal(m == float("-inf"), empty) and bool((l[empty] == 0).all())
    assert bool((acc[empty] == 0).all())
    full = ~empty
    torch.testing.assert_close(m[full] * math.log(2.0), m_ref[full], atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(l[full], l_ref[full], atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(acc[full], acc_ref[full], atol=1e-4, rtol=1e-5)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_metric_size_batch(dtype: torch.dtype) -> None:
    # The metric's workload, B=64 x 4096, fp16/bf16. The benched launch (one split: the
    # streaming budget on length pairs, a single launch) against the oracle on 8 of the
    # 64 sequences at the contract's bound, and every sequence for split-count
    # invariance (1 vs 8 vs 16 HBM splits).
    c = decode_bench_case(64, 4096, dtype=dtype, seed=5)
    plan = ha.decode_plan(64, 16, 8, 128, 16, c.block_tables.shape[1], 1, dtype=dtype)
    assert plan["budget"] == "light_stream" and plan["by_length"], plan
    outs = {s: ha.launch_paged_decode_split(*c.args(), c.scale, c.block_size, num_splits=s)
            for s in (1, 8, 16)}  # fmt: skip
    for s, out in outs.items():
        assert torch.isfinite(out).all(), s
    tol = TOL[dtype] * 2
    torch.testing.assert_close(outs[8], outs[1], atol=tol, rtol=tol)
    torch.testing.assert_close(outs[16], outs[1], atol=tol, rtol=tol)
    kc, vc = c.k_cache.cpu(), c.v_cache.cpu()
    rows = list(range(0, 64, 8))
    sub = DecodeCase(c.q[rows].cpu(), kc, vc, c.block_tables[rows].cpu(), c.context_lens[rows].cpu(),
                     c.scale, c.block_size)  # fmt: skip
    want = oracle32(sub)
    assert_contract(outs[1][rows], want, dtype, "metric size, the benched one-split launch")
    assert_contract(outs[8][rows], want, dtype, "metric size, 8 splits + combine")


@pytest.mark.parametrize("batch", [20, 40, 80])
@pytest.mark.parametrize("splits", [1, 3])
def test_every_workgroup_width_gives_the_reference(batch: int, splits: int) -> None:
    # The library runs each (sequence, head tile, split) on a workgroup of 1, 2 or 4 waves
    # that merge in LDS, chosen from the grid size (about 1024 waves in all on 256 CUs):
    # at Qwen3 shapes (8 head tiles) 80 sequences take 1 wave each, 40 take 2, 20 take 4.
    lens = [1 + (37 * i) % 300 for i in range(batch)]
    c = decode_case(lens, dtype=torch.float16, seed=batch + splits)
    want = oracle32(c)
    g = on_gpu(c)
    out = ha.launch_paged_decode_split(*g.args(), c.scale, c.block_size, num_splits=splits)
    assert torch.isfinite(out).all()
    assert_matches(out, want, torch.float16, f"B={batch} splits={splits}")


@pytest.mark.parametrize("batch", [33, 45, 64])
@pytest.mark.parametrize("kind", ["mixed", "equal", "one_long", "descending", "ties", "ones"])
def test_sequences_paired_by_length(batch: int, kind: str) -> None:
    # At Qwen3 shapes 33-64 sequences run paired by length: workgroup y takes the
    # sequences ranked y and B - 1 - y (longest first, ties by index) and shares its four
    # waves between them by length; an odd batch leaves the middle one alone. Lengths
    # 1 .. 1000 in a scrambled order, all equal (ties only), one long among short, already
    # in rank order (ranking skipped) with ties, five lengths scrambled, and one token each
    # (waves left with nothing to walk).
    if kind == "mixed":
        lens = [1 + (389 * i) % 1000 for i in range(batch)]
    elif kind == "equal":
        lens = [300] * batch
    elif kind == "descending":
        lens = sorted((1 + (389 * i) % 1000 for i in range(batch)), reverse=True)
        lens[5] = lens[6] = lens[7]
    elif kind == "ties":
        lens = [1 + (7 * i % 5) * 200 for i in range(batch)]
    elif kind == "ones":
        lens = [1] * batch
    else:
        lens = [7] * batch
        lens[batch // 3] = 1500
    c = decode_case(lens, dtype=torch.float16, seed=batch)
    want = oracle32(c)
    g = on_gpu(c)
    out = ha.launch_paged_decode_split(*g.args(), c.scale, c.block_size, num_splits=1)
    assert torch.isfinite(out).all()
    assert_matches(out, want, torch.float16, f"B={batch} {kind}")


def test_paired_sequences_of_2_to_the_25_tokens() -> None:
    # Contexts of 2^25 tokens and more take the pair ranking's exact comparison (its
    # packed keys hold shorter lengths only). Both long tables repeat block 0 (65,536
    # slots), so each long context is that block's keys and values repeated 512 or 513
    # times: equal weights per repeat, so the exact answer is attention over the block
    # once. The short sequences live in block 1.
    bs, hq, hkv, d, batch = 1 << 16, 16, 8, 128, 40
    g = torch.Generator().manual_seed(25)
    k = torch.randn(2 * bs, hkv, d, generator=g).half()
    v = torch.randn(2 * bs, hkv, d, generator=g).half()
    q = torch.randn(batch, hq, d, generator=g).half()
    lens = [1 + (389 * b) % 1000 for b in range(batch)]
    lens[3], lens[17] = 1 << 25, (1 << 25) + bs
    tables = torch.ones(batch, 513, dtype=torch.int32)
    tables[3, :512] = 0
    tables[17, :] = 0
    scale = d**-0.5
    out = ha.launch_paged_decode_split(q.to(DEVICE), k.to(DEVICE), v.to(DEVICE), tables.to(DEVICE),
                                       torch.tensor(lens, dtype=torch.int32, device=DEVICE), scale, bs,
                                       num_splits=1)  # fmt: skip
    once = torch.tensor([bs if n >= bs else n for n in lens], dtype=torch.int32)
    first = torch.where(torch.tensor(lens) >= bs, 0, 1).to(torch.int32)[:, None]
    want = ref.decode_ref(q.float(), k.float(), v.float(), first, once, scale, bs)
    assert torch.isfinite(out).all()
    assert_matches(out, want, torch.float16, "contexts of 2^25 tokens")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("batch,splits", [(64, 1), (45, 1), (32, 4), (4, 1), (8, 8)])
@pytest.mark.parametrize("heads", [(16, 8), (32, 8)])
def test_both_register_budgets(batch: int, splits: int, heads: tuple[int, int], dtype: torch.dtype) -> None:
    # The table width bounds the tokens a wave walks; under 512 of them the kernel runs
    # its light budget (two waves per SIMD, up to 8 a workgroup; 16 bytes a lane for tiles
    # of four query heads), else the heavy one. The same sequences through their own
    # narrow table and through one widened to 2000 blocks give the reference either way:
    # length pairs (64, 45), in-workgroup splits (32 x 4), a small batch, and HBM splits
    # with the combine (8 x 8), at GQA groups of 2 and 4.
    lens = [1 + (389 * i) % 300 for i in range(batch)]
    c = decode_case(lens, num_q_heads=heads[0], num_kv_heads=heads[1], dtype=dtype, seed=batch)
    want = oracle32(c)
    g = on_gpu(c)
    for w in (g.block_tables.shape[1], 2000):
        tables = widened(g.block_tables, w)
        out = ha.launch_paged_decode_split(g.q, g.k_cache, g.v_cache, tables, g.context_lens, c.scale,
                                           c.block_size, num_splits=splits)  # fmt: skip
        assert_matches(out, want, dtype, f"width {w}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("batch,splits,head_dim", [(256, 1, 128), (64, 16, 128), (300, 1, 64), (40, 9, 256)])
def test_launches_of_several_rounds(batch: int, splits: int, head_dim: int, dtype: torch.dtype) -> None:
    # Grids of at least 8 waves per CU (two rounds of one wave per SIMD; 2048 waves on 256
    # CUs) run the kernel's light register budget: 32 bytes of a row per lane, two waves
    # per SIMD. Here: 256 and 300 sequences at one split, 64 at the reference's 16 splits
    # (HBM partials and the combine), 40 at 9 splits with D=256; the grouped and the
    # per-head (head tile 1) launches.
    lens = [1 + (211 * i) % 900 for i in range(batch)]
    c = decode_case(lens, head_dim=head_dim, dtype=dtype, seed=batch + splits)
    want = oracle32(c)
    g = on_gpu(c)
    out = ha.launch_paged_decode_split(*g.args(), c.scale, c.block_size, num_splits=splits)
    assert torch.isfinite(out).all()
    assert_matches(out, want, dtype, f"B={batch} splits={splits} D={head_dim}")
    per_head = ha._launch(*g.args(), c.scale, c.block_size, splits, 1)
    assert_matches(per_head, want, dtype, f"head tile 1, B={batch} splits={splits} D={head_dim}")


@pytest.mark.parametrize("splits", [2, 3, 4])
def test_partials_and_combine_at_small_split_counts(splits: int) -> None:
    # An explicit count of 2-4 splits runs as HBM partials plus the combine (the policy
    # alone turns such counts into one launch split over a workgroup's waves).
    c = decode_case([17, 300, 33, 1], dtype=torch.float16, seed=splits)
    want = oracle32(c)
    g = on_gpu(c)
    assert ha.decode_plan(4, 16, 8, 128, 16, g.block_tables.shape[1], splits)["grid"][2] == splits
    out = ha.launch_paged_decode_split(*g.args(), g.scale, g.block_size, num_splits=splits)
    assert_matches(out, want, torch.float16, f"splits={splits}")
    policy = ha.launch_paged_decode_split(*g.args(), g.scale, g.block_size)
    assert_matches(policy, want, torch.float16, "policy")


@pytest.mark.parametrize("splits", [9, 64, 65, 130])
@pytest.mark.parametrize("head_dim,dtype", [(128, torch.float16), (64, torch.float32), (256, torch.bfloat16),
                                            (8, torch.float16)])  # fmt: skip
def test_combine_over_many_splits(splits: int, head_dim: int, dtype: torch.dtype) -> None:
    # The combine reduces the splits' maxima and denominators over the lanes of a wave, 64
    # splits at a time, and reads 8 splits' partials at once: split counts past one and two
    # rounds of 64, many of them empty (m = -inf, l = 0) for the short sequences, and head
    # dims of one, two and four elements per lane.
    c = decode_case([17, 3000, 33, 1, 700], num_q_heads=8, num_kv_heads=4, head_dim=head_dim, dtype=dtype,
                    seed=splits)  # fmt: skip
    want = oracle32(c)
    g = on_gpu(c)
    out = ha._launch(*g.args(), g.scale, g.block_size, splits, 0)
    assert torch.isfinite(out).all()
    assert_matches(out, want, dtype, f"splits={splits} D={head_dim}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("heads,head_tile", [((16, 8), 0), ((32, 8), 0), ((8, 8), 0), ((16, 8), 1)])
def test_streaming_launches(dtype: torch.dtype, head_dim: int, heads: tuple[int, int], head_tile: int) -> None:
    # A table wide enough to bound more than 256 MiB of K/V makes the launch stream K/V
    # with non-temporal loads (light budget, one round of workgroups; tiles of four query
    # heads and 64-element rows take the heavy budget's cached loads instead); the unused columns
    # are never read. Head groups of 2, 4 and 1 (tiles of 2, 4 and 1 query heads) and the
    # per-head launch; 32 sequences give length pairs at one split. The results match the
    # oracle and the launch over the tight table, for one split and for HBM splits.
    lens = [1, 17, 300, 64, 1000, 5, 700, 33] * 4
    c = decode_case(lens, *heads, head_dim=head_dim, dtype=dtype, seed=11)
    want = oracle32(c)
    g = on_gpu(c)
    b, w = g.block_tables.shape
    wide = torch.full((b, 8192), -1, dtype=torch.int32, device=DEVICE)  # -1: never read
    wide[:, :w] = g.block_tables
    for splits in (1, 4):
        plan = ha.decode_plan(b, *heads, head_dim, g.block_size, 8192, splits, head_tile, dtype)
        # Tiles of four query heads and rows of 64 elements run the heavy budget with cached
        # loads; the others stream.
        heavy = plan["head_tile"] == 4 or head_dim == 64
        assert plan["budget"] == ("heavy" if heavy else "light_stream"), plan
        tight = ha._launch(*g.args(), g.scale, g.block_size, splits, head_tile)
        out = ha._launch(g.q, g.k_cache, g.v_cache, wide, g.context_lens, g.scale, g.block_size, splits,
                         head_tile)  # fmt: skip
        assert torch.isfinite(out).all(), splits
        assert_matches(out, want, dtype, f"streaming, {splits} split(s)")
        torch.testing.assert_close(out, tight, atol=TOL[dtype], rtol=TOL[dtype])


def test_streaming_threshold() -> None:
    # bf16, 64 sequences, 8 kv heads of 128: each table column bounds 64 x 16 x 4 KiB =
    # 4 MiB of K/V, so a width of 64 bounds exactly 256 MiB (cached loads) and 65 just
    # over it (streaming). Both give the oracle's result on the same sequences.
    lens = [1 + (389 * i) % 1024 for i in range(64)]
    c = decode_case(lens, dtype=torch.bfloat16, seed=13)
    want = oracle32(c)
    g = on_gpu(c)
    assert int(g.context_lens.max()) <= 64 * 16  # every sequence fits a 64-column table
    assert ha.decode_plan(64, 16, 8, 128, 16, 64, 1, dtype=torch.bfloat16)["budget"] != "light_stream"
    assert ha.decode_plan(64, 16, 8, 128, 16, 65, 1, dtype=torch.bfloat16)["budget"] == "light_stream"
    for width in (64, 65):
        tables = widened(g.block_tables, width)
        out = ha.launch_paged_decode_split(g.q, g.k_cache, g.v_cache, tables, g.context_lens, g.scale,
                                           g.block_size, num_splits=1)  # fmt: skip
        assert_matches(out, want, torch.bfloat16, f"width {width}")


@pytest.mark.parametrize("splits", [4, 16])
@pytest.mark.parametrize("lens", [[256] * 32, [1 + (389 * i) % 3000 for i in range(64)], [5000]])
def test_in_workgroup_splits_replay_in_a_graph(splits: int, lens: list[int], monkeypatch) -> None:
    # The in-group split launch (its LDS slot marking, barrier and merge) captured in a HIP
    # graph: every replay, with unrelated eager work between replays, equals the eager
    # launch bit for bit. One sequence of 5000 tokens takes the heavy register budget
    # (forced in-group: the launcher's policy gives so small a grid the HBM form).
    monkeypatch.setattr(ha, "IN_GROUP_MIN_WAVES", 0)
    c = on_gpu(decode_case(lens, dtype=torch.float16, seed=len(lens) + splits))
    want = ha.launch_paged_decode_split(*c.args(), c.scale, c.block_size, num_splits=splits)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        got = ha.launch_paged_decode_split(*c.args(), c.scale, c.block_size, num_splits=splits)
    for _ in range(3):
        got.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(got, want)
        torch.randn(1 << 20, device=DEVICE).sum().item()


@pytest.mark.gpu
@pytest.mark.parametrize("lens,splits", [([8192] * 4, None), ([32768], None), ([4096] * 8, 8)])
def test_small_grids_take_the_hbm_partials(lens: list[int], splits: int | None) -> None:
    # A split count on a grid too small to fill the chip runs S workgroups per (sequence,
    # head tile) writing fp32 partials, then the combine: same output as the in-group form
    # up to fp32 summation order, and the oracle's.
    c = decode_case(lens, 16, 8, dtype=torch.float16, seed=len(lens))
    g = on_gpu(c)
    simds = ha._one_split_waves(0, len(lens), 16, 8, 128, c.block_size, g.block_tables.shape[1], torch.float16)
    assert simds < ha.IN_GROUP_MIN_WAVES
    out = ha.launch_paged_decode_split(*g.args(), c.scale, c.block_size, num_splits=splits)
    s = splits or ha._policy_splits(g.q, g.k_cache, g.block_tables, c.block_size)
    assert s > 1
    torch.testing.assert_close(out.float(), hbm_split_combine(g, s).float(), atol=0, rtol=0)
    assert_matches(out, oracle32(c), torch.float16, f"{lens} splits={splits}")


@pytest.mark.gpu
@pytest.mark.parametrize("lens", [[32768], [8192] * 4, [4096] * 8])
def test_small_grid_policy_replays_in_a_graph(lens: list[int]) -> None:
    # The policy's HBM-partials launch for a small grid (partials allocated inside the
    # capture, from the graph's pool, then the combine) captured in a HIP graph: every
    # replay, with eager work between replays, equals the eager launch bit for bit, and
    # neither form synchronizes with the host.
    c = on_gpu(decode_case(lens, dtype=torch.float16, seed=len(lens)))
    want = ha.launch_paged_decode_split(*c.args(), c.scale, c.block_size)
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        ha.launch_paged_decode_split(*c.args(), c.scale, c.block_size)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            got = ha.launch_paged_decode_split(*c.args(), c.scale, c.block_size)
    finally:
        torch.cuda.set_sync_debug_mode("default")
    for _ in range(3):
        got.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        torch.testing.assert_close(got, want, atol=0, rtol=0)
        torch.randn(1 << 20, device=DEVICE).sum()  # unrelated eager work between replays
