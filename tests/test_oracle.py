"""Pins of the CPU oracle (oracle/ref.py) before anything is checked against it.

Known answers come from the reference's own tests (cited per test); PyTorch's
scaled_dot_product_attention cross-checks the attention contraction; the golden
fixtures (test_golden.py) add an independent float64 brute force. Each pin is chosen
so that a plausible slip fails it: a round-robin GQA mapping, a causal mask off by one,
a transposed contraction, a wrong slot formula, RoPE pairing neighbours instead of
i and i + D/2, a sign flip in the rotation, a missing mean in RMSNorm.
"""

from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import ref


def rand(*shape: int, seed: int = 0) -> torch.Tensor:
    return torch.randn(*shape, generator=torch.Generator().manual_seed(seed))


# --- attention (reference tests/test_attention.py) --------------------------------------


def test_first_token_sees_only_itself() -> None:  # test_attention.py:16-20
    q, k, v = rand(5, 4, 8, seed=1), rand(5, 2, 8, seed=2), rand(5, 2, 8, seed=3)
    out = ref.attend_causal(q, k, v, scale=1 / math.sqrt(8))
    torch.testing.assert_close(out[0], v[0].repeat_interleave(2, dim=0))


def test_zero_query_averages_the_past() -> None:  # test_attention.py:23-29
    t = 6
    v = rand(t, 1, 4)
    out = ref.attend_causal(torch.zeros(t, 1, 4), rand(t, 1, 4), v, scale=1.0)
    for i in range(t):
        torch.testing.assert_close(out[i, 0], v[: i + 1, 0].mean(dim=0))


def test_gqa_mapping_is_grouped_not_round_robin() -> None:  # test_attention.py:32-38
    t = 3
    v = torch.stack([torch.full((t, 4), 1.0), torch.full((t, 4), 2.0)], dim=1)
    out = ref.attend_causal(torch.zeros(t, 4, 4), torch.zeros(t, 2, 4), v, scale=1.0)
    assert out[:, 0].eq(1.0).all() and out[:, 1].eq(1.0).all()
    assert out[:, 2].eq(2.0).all() and out[:, 3].eq(2.0).all()


def test_future_tokens_do_not_leak() -> None:  # test_attention.py:41-49
    q, k, v = rand(6, 2, 8, seed=1), rand(6, 2, 8, seed=2), rand(6, 2, 8, seed=3)
    out = ref.attend_causal(q, k, v, scale=0.3)
    k2, v2 = k.clone(), v.clone()
    v2[4:] += 100.0
    k2[4:] -= 50.0
    torch.testing.assert_close(out[:4], ref.attend_causal(q, k2, v2, scale=0.3)[:4])


@pytest.mark.parametrize(("t", "hq", "hkv", "d"), [(1, 2, 2, 8), (7, 4, 2, 16), (33, 16, 8, 128)])
def test_matches_pytorch_sdpa(t: int, hq: int, hkv: int, d: int) -> None:  # :52-60
    q, k, v = rand(t, hq, d, seed=1), rand(t, hkv, d, seed=2), rand(t, hkv, d, seed=3)
    ours = ref.attend_causal(q, k, v, scale=1 / math.sqrt(d))
    want = F.scaled_dot_product_attention(
        q.transpose(0, 1), k.transpose(0, 1), v.transpose(0, 1), is_causal=True, enable_gqa=True
    ).transpose(0, 1)
    torch.testing.assert_close(ours, want, atol=1e-5, rtol=1e-4)


def test_fp16_large_scores_stay_finite() -> None:  # test_attention.py:63-70
    q = torch.full((3, 1, 64), 40.0, dtype=torch.float16)
    k = torch.full((3, 1, 64), 40.0, dtype=torch.float16)
    out = ref.attend_causal(q, k, rand(3, 1, 64).half(), scale=1.0)
    assert out.dtype == torch.float16 and torch.isfinite(out).all()


# --- the paged forms (reference tests/test_paged_attention.py) --------------------------


def scattered(k: torch.Tensor, v: torch.Tensor, bs: int, blocks: list[int], nblocks: int):
    shape = (nblocks * bs, *k.shape[1:])
    kc = torch.full(shape, float("nan"))
    vc = torch.full(shape, float("nan"))
    slots = ref.block_slots(blocks, k.shape[0], bs)
    kc[slots], vc[slots] = k, v
    return kc, vc, slots


def test_slot_table_of_the_block_table_docstring() -> None:  # block_table.py:6-12
    assert ref.block_slots([7, 2], 8, 4).tolist() == [28, 29, 30, 31, 8, 9, 10, 11]


def test_paged_prefill_equals_contiguous() -> None:  # test_paged_attention.py:98-102
    q, k, v = rand(10, 4, 8, seed=3), rand(10, 2, 8, seed=4), rand(10, 2, 8, seed=5)
    kc, vc, slots = scattered(k, v, 4, [5, 2, 7], 8)
    torch.testing.assert_close(ref.attend_paged(q, kc, vc, slots, 0.35), ref.attend_causal(q, k, v, 0.35))


def test_paged_decode_matches_last_row() -> None:  # test_paged_attention.py:105-110
    q, k, v = rand(9, 4, 8, seed=5), rand(9, 2, 8, seed=6), rand(9, 2, 8, seed=7)
    kc, vc, slots = scattered(k, v, 4, [3, 0, 6], 8)
    out = ref.attend_paged(q[-1:], kc, vc, slots, 0.35)
    torch.testing.assert_close(out, ref.attend_causal(q, k, v, 0.35)[-1:])


def test_decode_sees_every_earlier_token() -> None:  # test_paged_attention.py:113-119
    v = rand(6, 2, 8, seed=7)
    out = ref.attend_paged(torch.zeros(1, 4, 8), rand(6, 2, 8), v, torch.arange(6), 1.0)
    torch.testing.assert_close(out[0], v.mean(dim=0).repeat_interleave(2, dim=0))


def test_chunked_prefill_matches_whole() -> None:  # test_paged_attention.py:122-130
    q, k, v = rand(8, 4, 8, seed=11), rand(8, 2, 8, seed=12), rand(8, 2, 8, seed=13)
    want = ref.attend_causal(q, k, v, 0.35)
    kc, vc, slots = scattered(k, v, 2, [4, 1, 6, 0], 8)
    for lo in range(0, 8, 3):
        hi = min(lo + 3, 8)
        torch.testing.assert_close(ref.attend_paged(q[lo:hi], kc, vc, slots[:hi], 0.35), want[lo:hi])


def test_decode_ref_one_token_returns_its_value() -> None:  # test_triton_attention.py:129-135
    tables = torch.tensor([[3, 1]], dtype=torch.int32)
    kc, vc = rand(64, 2, 16, seed=1), rand(64, 2, 16, seed=2)
    out = ref.decode_ref(rand(1, 4, 16), kc, vc, tables, torch.tensor([1], dtype=torch.int32), 0.25, 16)
    torch.testing.assert_close(out[0], vc[48].repeat_interleave(2, dim=0))


def test_split_partials_hand_computed() -> None:  # triton_attention.py:283-296
    # Two tokens, one per block, two splits: each range holds one key, so m is that key's
    # score, l = 1 and acc is its value. A third split is past the end: empty.
    q = torch.tensor([[[1.0, 2.0]]])
    kc = torch.tensor([[[0.5, 0.0]], [[1.0, 1.0]], [[9.0, 9.0]]])
    vc = torch.tensor([[[3.0, 4.0]], [[5.0, 6.0]], [[7.0, 8.0]]])
    tables = torch.tensor([[2, 1]], dtype=torch.int32)  # block size 1: slots 2, 1
    m, l, acc = ref.split_partials_ref(q, kc, vc, tables, torch.tensor([2], dtype=torch.int32), 0.5, 1, 3)  # noqa: E741
    assert m[0, 0].tolist() == [13.5, 1.5, float("-inf")]
    assert l[0, 0].tolist() == [1.0, 1.0, 0.0]
    assert acc[0, 0].tolist() == [[7.0, 8.0], [5.0, 6.0], [0.0, 0.0]]


@pytest.mark.parametrize("splits", [1, 2, 3, 7, 40])
def test_split_partials_merge_to_the_decode(splits: int) -> None:
    # Any split count merges to the unsplit attention; ranges follow ceil(n / S) blocks,
    # so 40 ranges over at most 19 blocks leave trailing ones empty (m = -inf, l = 0).
    kc, vc = rand(96, 2, 8, seed=3), rand(96, 2, 8, seed=4)
    q = rand(3, 4, 8, seed=5)
    tables = torch.randperm(24, generator=torch.Generator().manual_seed(6)).to(torch.int32).view(3, 8)
    lens = torch.tensor([1, 19, 30], dtype=torch.int32)
    m, l, acc = ref.split_partials_ref(q, kc, vc, tables, lens, 0.3, 4, splits)  # noqa: E741
    want = ref.decode_ref(q, kc, vc, tables, lens, 0.3, 4)
    torch.testing.assert_close(ref.merge_partials_ref(m, l, acc), want)
    for b, n in enumerate(lens.tolist()):
        nblocks = -(-n // 4)
        per = -(-nblocks // splits)
        used = -(-nblocks // per)  # ranges holding at least one block
        assert torch.isfinite(m[b, :, :used]).all() and (l[b, :, :used] >= 1.0).all()
        assert (m[b, :, used:] == float("-inf")).all() and (l[b, :, used:] == 0).all()


def test_prefill_ref_is_per_sequence_and_leaves_other_rows() -> None:
    kc, vc = rand(64, 2, 8, seed=1), rand(64, 2, 8, seed=2)
    tables = torch.tensor([[5, 9, 0], [2, 3, 0]], dtype=torch.int32)
    q = rand(9, 4, 8, seed=3)
    out = torch.full_like(q, 7.0)
    starts, qlens, ctx = (torch.tensor(x, dtype=torch.int32) for x in ([0, 6], [5, 2], [9, 7]))
    ref.prefill_ref(q, kc, vc, tables, starts, qlens, ctx, 0.3, 4, out)
    s0 = ref.block_slots(tables[0], 9, 4)
    torch.testing.assert_close(out[0:5], ref.attend_paged(q[0:5], kc, vc, s0, 0.3))
    assert bool((out[5] == 7.0).all()) and bool((out[8] == 7.0).all())


# --- RMSNorm and RoPE (reference tests/test_layers.py) ----------------------------------


def test_rms_norm_hand_computed() -> None:  # test_layers.py:14-19
    r = math.sqrt(12.5)
    y = ref.rms_norm(torch.tensor([[3.0, 4.0]]), torch.ones(2), eps=0.0)
    torch.testing.assert_close(y, torch.tensor([[3 / r, 4 / r]]))


def test_rms_norm_weight_per_channel() -> None:  # test_layers.py:22-26
    r = math.sqrt(12.5)
    y = ref.rms_norm(torch.tensor([[3.0, 4.0]]), torch.tensor([2.0, -1.0]), eps=0.0)
    torch.testing.assert_close(y, torch.tensor([[6 / r, -4 / r]]))


def test_rms_norm_zero_row_and_fp16_overflow() -> None:  # test_layers.py:29-31, :53-59
    assert torch.equal(ref.rms_norm(torch.zeros(2, 8), torch.ones(8), 1e-6), torch.zeros(2, 8))
    x = torch.full((1, 64), 300.0, dtype=torch.float16)
    y = ref.rms_norm(x, torch.ones(64, dtype=torch.float16), 1e-6)
    assert y.dtype == torch.float16 and torch.isfinite(y).all()
    torch.testing.assert_close(y.float(), torch.ones(1, 64), atol=1e-3, rtol=0)


def test_rms_norm_rounds_before_the_weight() -> None:
    # layers.py:34-38: (x * inv) is rounded to fp16 BEFORE the weight multiply.
    x = rand(4, 32, seed=9).half() * 3
    w = (1 + 0.1 * rand(32, seed=10)).half()
    xf = x.float()
    step = (xf * torch.rsqrt(xf.square().mean(-1, keepdim=True) + 1e-6)).half()
    assert torch.equal(ref.rms_norm(x, w, 1e-6), step * w)


def test_rope_tables_hand_computed() -> None:  # test_layers.py:78-84
    p = 7
    cos, sin = ref.rope_cos_sin(4, 10000.0, torch.tensor([p]))
    angles = [p * 1.0, p * 0.01, p * 1.0, p * 0.01]
    torch.testing.assert_close(cos[0], torch.tensor([math.cos(a) for a in angles]))
    torch.testing.assert_close(sin[0], torch.tensor([math.sin(a) for a in angles]))


def test_rope_tables_accurate_at_long_positions() -> None:  # test_layers.py:87-89
    cos, _ = ref.rope_cos_sin(128, 1e6, torch.tensor([40000]))
    assert abs(cos[0, 0].item() - math.cos(40000.0)) < 1e-6


def test_rope_position_zero_is_identity() -> None:  # test_layers.py:92-95
    x = rand(1, 2, 8)
    cos, sin = ref.rope_cos_sin(8, 1e6, torch.tensor([0]))
    torch.testing.assert_close(ref.apply_rope(x, cos, sin), x)


def test_rope_pairs_i_with_i_plus_half() -> None:  # test_layers.py:98-104
    p = 3
    x = torch.tensor([[[1.0, 0.0, 0.0, 0.0]]])
    cos, sin = ref.rope_cos_sin(4, 10000.0, torch.tensor([p]))
    want = torch.tensor([[[math.cos(p), 0.0, math.sin(p), 0.0]]])
    torch.testing.assert_close(ref.apply_rope(x, cos, sin), want)


def test_rope_preserves_norm_and_relative_position() -> None:  # test_layers.py:124-147
    x = rand(1, 4, 64, seed=4)
    cos, sin = ref.rope_cos_sin(64, 1e6, torch.tensor([1234]))
    torch.testing.assert_close(ref.apply_rope(x, cos, sin).norm(dim=-1), x.norm(dim=-1))
    q, k = rand(1, 1, 32, seed=5), rand(1, 1, 32, seed=6)

    def score(a: int, b: int) -> float:
        qa = ref.apply_rope(q, *ref.rope_cos_sin(32, 1e4, torch.tensor([a])))
        kb = ref.apply_rope(k, *ref.rope_cos_sin(32, 1e4, torch.tensor([b])))
        return float((qa * kb).sum())

    assert math.isclose(score(100, 37), score(100 + 900, 37 + 900), rel_tol=1e-3, abs_tol=1e-3)


# --- the cache write (reference src/tinyserve/kv_cache.py:42-50) -------------------------


def test_kv_write_places_exactly_and_touches_nothing_else() -> None:
    kc = torch.full((16, 2, 8), float("nan"), dtype=torch.float16)
    vc = kc.clone()
    slots = torch.tensor([9, 2, 14])
    k, v = rand(3, 2, 8, seed=1), rand(3, 2, 8, seed=2)
    ref.kv_write(kc, vc, slots, k, v)
    assert torch.equal(kc[slots], k.half()) and torch.equal(vc[slots], v.half())
    others = torch.ones(16, dtype=torch.bool)
    others[slots] = False
    assert kc[others].isnan().all() and vc[others].isnan().all()


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_batched_prefill_equals_per_sequence_prefill(seed: int) -> None:
    # The reference's two prefill paths agree (test_batched_forward.py's premise): one
    # padded masked SDPA call over all sequences == paged_gqa_attention one at a time,
    # including chunked-prefill sequences (context longer than the new rows) and a gap
    # row that belongs to no sequence.
    g = torch.Generator().manual_seed(seed)
    specs = [(0, 5), (7, 3), (0, 1), (12, 9)]  # (cached, new)
    bs, hq, hkv, d = 4, 4, 2, 8
    nblk = [-(-(c + n) // bs) for c, n in specs]
    perm = torch.randperm(sum(nblk) + 2, generator=g).tolist()
    tables = torch.zeros((len(specs), max(nblk)), dtype=torch.int32)
    at = 0
    for r, k in enumerate(nblk):
        tables[r, :k] = torch.tensor(perm[at : at + k])
        at += k
    kc = torch.randn((sum(nblk) + 2) * bs, hkv, d, generator=g)
    vc = torch.randn((sum(nblk) + 2) * bs, hkv, d, generator=g)
    lens = [n for _, n in specs]
    starts = torch.tensor([sum(lens[:r]) + r for r in range(len(lens))], dtype=torch.int32)  # gaps
    q = torch.randn(int(starts[-1]) + lens[-1] + 1, hq, d, generator=g)
    ql = torch.tensor(lens, dtype=torch.int32)
    ctx = torch.tensor([c + n for c, n in specs], dtype=torch.int32)
    a = ref.prefill_ref(q, kc, vc, tables, starts, ql, ctx, 0.35, bs, torch.full_like(q, 7.0))
    b = ref.batched_prefill_ref(q, kc, vc, tables, starts, ql, ctx, 0.35, bs, torch.full_like(q, 7.0))
    torch.testing.assert_close(b, a, atol=1e-5, rtol=1e-5)
    assert (b[5] == 7.0).all()  # the gap row after sequence 0 is untouched
