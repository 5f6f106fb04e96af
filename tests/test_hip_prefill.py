"""The HIP varlen prefill kernel must match the oracle (GPU).

Mirrors the reference's tests/test_triton_prefill.py: the reference result is the
oracle's ``prefill_ref`` (``paged_gqa_attention`` one sequence at a time); every cache
slot no sequence owns is NaN and block-table padding points at a NaN block. fp32 runs
the exact-fp32 path; fp16 / bf16 at head_dim 64 / 128 run the MFMA kernel, whose P is
rounded to the input dtype before P.V as in the reference kernel. Tolerances:
tests/helpers.py.
"""

from __future__ import annotations

import pytest
import torch
from hypothesis import given, settings
from hypothesis import strategies as st

from oracle import ref
from tests.helpers import assert_contract, assert_matches
from tinyserve_amd.hip_prefill import paged_prefill_attention
from tinyserve_amd.workloads import PrefillCase, prefill_case, prefill_lengths

pytestmark = pytest.mark.gpu
DEVICE = "cuda"


def on_gpu(c: PrefillCase) -> PrefillCase:
    return PrefillCase(c.q.to(DEVICE), c.k.to(DEVICE), c.v.to(DEVICE), c.tables.to(DEVICE),
                       c.starts.to(DEVICE), c.q_lens.to(DEVICE), c.ctx_lens.to(DEVICE),
                       c.block_size, c.max_q_len)  # fmt: skip


def oracle32(c: PrefillCase) -> torch.Tensor:
    return ref.prefill_ref(c.q.float(), c.k.float(), c.v.float(), c.tables, c.starts, c.q_lens,
                           c.ctx_lens, c.scale, c.block_size)  # fmt: skip


def run(c: PrefillCase, out: torch.Tensor | None = None, **kw: int) -> torch.Tensor:
    g = on_gpu(c)
    return paged_prefill_attention(*g.args(), out=out, **kw)


def check(c: PrefillCase, out: torch.Tensor) -> None:
    want = oracle32(c)
    for r in range(c.tables.shape[0]):
        s, n = int(c.starts[r]), int(c.q_lens[r])
        assert torch.isfinite(out[s : s + n]).all(), f"sequence {r} read an unowned slot"
        assert_matches(out[s : s + n], want[s : s + n], c.q.dtype, f"sequence {r}")


SHAPES = [(4, 4, 8), (4, 2, 8), (4, 1, 8), (16, 8, 128), (8, 2, 64), (16, 2, 128)]
SPECS = [
    [(0, 5)],
    [(0, 37), (0, 1), (0, 9)],
    [(12, 4), (40, 7), (3, 1)],
    [(0, 130), (70, 66), (5, 200)],  # several 64-key tiles, partial tiles, prefix hits
]


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("specs", SPECS)
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_matches_the_reference(shape: tuple[int, int, int], specs: list[tuple[int, int]],
                               dtype: torch.dtype) -> None:  # fmt: skip
    hq, hkv, d = shape
    if d * (4 if dtype == torch.float32 else 2) < 16:
        pytest.skip("rows under 16 bytes are not a kernel shape")
    c = prefill_case(specs, hq, hkv, d, block_size=16 if d >= 64 else 4, dtype=dtype)
    check(c, run(c))


@pytest.mark.parametrize("block_size", [1, 2, 4, 16, 32])
@pytest.mark.parametrize(("rows_per_tile", "block_n"), [(16, 16), (64, 32), (32, 64)])
def test_any_block_size_and_tile_shape(block_size: int, rows_per_tile: int, block_n: int) -> None:
    c = prefill_case([(9, 21), (0, 3), (30, 2)], block_size=block_size, seed=block_size)
    check(c, run(c, rows_per_tile=rows_per_tile, block_n=block_n))


@pytest.mark.parametrize("block_size", [1, 2, 4, 8, 32])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_mfma_kernel_at_any_block_size(block_size: int, dtype: torch.dtype) -> None:
    c = prefill_case([(9, 71), (0, 3), (100, 2), (0, 65)], 16, 8, 128, block_size, dtype,
                     seed=block_size)  # fmt: skip
    check(c, run(c))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_dtypes(dtype: torch.dtype) -> None:
    c = prefill_case(SPECS[2], 16, 8, 128, block_size=16, dtype=dtype)
    out = run(c)
    assert out.dtype == dtype
    check(c, out)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_rows_of_other_sequences_are_left_alone(dtype: torch.dtype) -> None:
    shape = (4, 2, 8) if dtype == torch.float32 else (16, 8, 128)
    c = prefill_case(SPECS[2], *shape, block_size=4, dtype=dtype, gap=2)
    out = torch.full_like(c.q, 7.0).to(DEVICE)
    run(c, out=out)
    check(c, out)
    mine = torch.zeros(c.q.shape[0], dtype=torch.bool)
    for s, n in zip(c.starts.tolist(), c.q_lens.tolist()):
        mine[s : s + n] = True
    assert bool((out.cpu()[~mine] == 7.0).all())


@settings(max_examples=40, deadline=None)
@given(
    specs=st.lists(st.tuples(st.integers(0, 40), st.integers(1, 40)), min_size=1, max_size=4),
    shape=st.sampled_from(SHAPES[:3]),
    block_size=st.sampled_from([1, 2, 4, 8]),
    seed=st.integers(0, 2**16),
)
def test_random_batches(specs: list[tuple[int, int]], shape: tuple[int, int, int], block_size: int,
                        seed: int) -> None:  # fmt: skip
    c = prefill_case(specs, *shape, block_size=block_size, seed=seed)
    check(c, run(c, rows_per_tile=16, block_n=16))


@settings(max_examples=60, deadline=None)
@given(
    specs=st.lists(st.tuples(st.integers(0, 150), st.integers(1, 150)), min_size=1, max_size=4),
    heads=st.sampled_from([(8, 8), (8, 4), (8, 2), (8, 1)]),
    head_dim=st.sampled_from([64, 128]),
    # The gather has three paths by block size: ids staged in LDS (a load's rows span
    # blocks: 1, 2, and 4 at head_dim 64), a scalar id per load, and one scalar id per
    # wave and tile (8 and up at the 32-key shape, 16 and up at the 4-wave 64-key shape).
    block_size=st.sampled_from([1, 2, 4, 8, 16, 32]),
    dtype=st.sampled_from([torch.float16, torch.bfloat16]),
    seed=st.integers(0, 2**16),
)
def test_random_batches_on_mfma(specs: list[tuple[int, int]], heads: tuple[int, int], head_dim: int,
                                block_size: int, dtype: torch.dtype, seed: int) -> None:  # fmt: skip
    c = prefill_case(specs, *heads, head_dim, block_size, dtype, seed=seed)
    check(c, run(c))


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32, torch.bfloat16])
def test_qwen3_shapes_with_prefix_hits(dtype: torch.dtype) -> None:
    # test_triton_prefill.py:246-252: 1,024 cached + 64 new tokens, next to a 128-token prompt.
    c = prefill_case([(1024, 64)] * 4 + [(0, 128)], 16, 8, 128, 16, dtype)
    check(c, run(c))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_baseline_config_3(dtype: torch.dtype) -> None:
    # 32 fresh prompts, L ~ U[16, 2048], packed by cu_seqlens; every
    # row within the contract's max-abs bound against the per-sequence oracle (fp16: 2e-3
    # including P's rounding to fp16 before P.V, as triton_prefill.py:118 rounds it).
    lens = prefill_lengths(32, seed=0)
    c = prefill_case([(0, n) for n in lens], 16, 8, 128, 16, dtype, seed=3)
    out = run(c)
    check(c, out)
    assert_contract(out, oracle32(c), dtype, "config 3")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_baseline_config_3_against_the_batched_path(dtype: torch.dtype) -> None:
    # The reference's other prefill path, prefill_plan + batched_prefill_attention
    # (attention.py:144-220): every sequence padded into one rectangle and attended by one
    # masked float32 SDPA call, run here on the GPU on config 3's inputs. Its padding keys
    # read slot 0 under the mask (as the reference's plan pads them), so the pool holds no
    # NaN sentinels here: 0 x NaN would poison the masked sum.
    lens = prefill_lengths(32, seed=0)
    c = prefill_case([(0, n) for n in lens], 16, 8, 128, 16, dtype, seed=3, sentinel=False)
    g = on_gpu(c)
    out = run(c)
    want = ref.batched_prefill_ref(g.q, g.k, g.v, g.tables, g.starts, g.q_lens, g.ctx_lens, g.scale,
                                   g.block_size, out=torch.empty_like(g.q, dtype=torch.float32))  # fmt: skip
    assert_contract(out, want, dtype, "config 3 vs the batched SDPA path")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_both_workgroup_shapes(dtype: torch.dtype) -> None:
    # The library picks the workgroup shape from the 8-wave grid (wg8 workgroups of 128
    # queries x 2 heads) at Qwen3 shapes on 256 CUs: 3 prompts of up to 2048 tokens make
    # 256 (under 1.5 per CU: 4 waves, 64-key tiles, two per CU); 4 prompts make 512 and 16
    # prompts of up to 512 tokens 512 (4 waves, 32-key tiles, three per CU); 24 prompts
    # of up to 1408 tokens make 2112, over 8 per CU with a mean above 1280 new tokens
    # (8 waves, 64-key tiles, many query tiles per sequence).
    for lens in ([2048, 1999, 1100, 700], [2048, 1500, 64], [512] * 15 + [77],
                 [1300 + (37 * i) % 109 for i in range(23)] + [1408]):  # fmt: skip
        c = prefill_case([(0, n) for n in lens], 16, 8, 128, 16, dtype, seed=len(lens))
        check(c, run(c))


@pytest.mark.parametrize("block_size", [1, 2, 4, 8, 16, 32, 64])
@pytest.mark.parametrize("shape", [(16, 8, 128), (8, 2, 64)])
def test_every_gather_path_on_every_workgroup_shape(block_size: int, shape: tuple[int, int, int]) -> None:
    # Each launch below runs one of the three workgroup shapes (one prompt: 4 waves,
    # 64-key tiles; 16 prompts of 512: 4 waves, 32-key tiles; 4 chunks of 128 new tokens:
    # 8 waves), with prefix hits so that tiles start mid-block, at every block size.
    for specs in ([(70, 300)], [(33, 512)] * 15 + [(5, 77)], [(100 + 300 * i, 128) for i in range(4)]):
        c = prefill_case(specs, *shape, block_size, torch.float16, seed=block_size)
        check(c, run(c))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("heads", [(16, 8, 128), (32, 8, 128), (8, 2, 64)])
def test_key_split_workgroups(dtype: torch.dtype, heads: tuple[int, int, int]) -> None:
    # One or two prompts run workgroups whose waves split the key tiles in two halves
    # and merge at the end: one key tile (the upper half empty), odd and even tile
    # counts, a query block whose keys end before the upper half, prefix hits (the
    # halves split the cached keys too; chunks of at most 64 new tokens in small launches
    # run this shape as well), and block sizes below the scalar-id gather's (the unsplit
    # 4-wave kernel).
    for specs, bs in (([(0, 1)], 16), ([(0, 64)], 16), ([(0, 65)], 16), ([(0, 200)], 16),
                      ([(0, 1000)], 32), ([(300, 37)], 16), ([(100, 2048)], 16),
                      ([(1024, 64)] * 4, 16), ([(8000, 50)], 16),
                      ([(0, 700), (9, 1300)], 64), ([(0, 500)], 2), ([(33, 400)], 1)):  # fmt: skip
        c = prefill_case(specs, *heads, bs, dtype, seed=bs + len(specs))
        check(c, run(c))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_length_ranked_sequence_groups(dtype: torch.dtype) -> None:
    # Batches of 8-16 prompts, of short ones (up to 64), of 32-64 with equal new-token
    # counts, or of 17-64 mixed ones are dispatched in groups of sequences ranked by
    # context length: 64 short prompts with ties, 12 mixed ones with prefix hits, 9 whose
    # longest is not first, 33 chunks of 600 new tokens after prefixes of different
    # lengths, 21 mixed prompts in pairs (an odd count: the last pair is one), and two
    # batches already in rank order (no ranking loop), one with ties.
    for specs in ([(0, 1 + (53 * i) % 200) for i in range(64)],
                  [((37 * i) % 300, 1 + (211 * i) % 700) for i in range(12)],
                  [(0, 40)] * 4 + [(5, 900)] + [(0, 40)] * 4,
                  [((37 * i) % 500, 600) for i in range(33)],
                  [((29 * i) % 90, 300 + (397 * i) % 1100) for i in range(21)],
                  [(0, 900 - 60 * i) for i in range(12)],
                  [(0, 500)] * 3 + [(0, 300)] * 6):  # fmt: skip
        c = prefill_case(specs, 16, 8, 128, 16, dtype, seed=len(specs), gap=1)
        out = torch.full_like(c.q, 7.0).to(DEVICE)
        run(c, out=out)
        check(c, out)
