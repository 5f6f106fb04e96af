"""The decode step through the HIP kernels (``tinyserve_amd.decode_step``) on the GPU.

Mirrors the reference's tests/test_decode_inputs.py:80-130, tests/test_cuda_graphs.py and
tests/test_batched_forward.py: the step's logits and cache writes against a reference step
composed from the oracle (``rms_norm``, ``rope_cos_sin``, ``qk_norm_rope_store_ref``,
``decode_ref`` / ``prefill_ref``) and plain fp32 matrix products on the CPU, on a tiny
random Qwen3 in fp32; padding rows leave real rows unchanged; a captured graph gives the
eager result on every replay, with other work between replays; a mixed prefill + decode
step (``forward_batch``) gives the oracle's logits and the same logits as each sequence
run alone.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from oracle import ref
from tinyserve_amd.decode_step import (DecodeGraph, DecodeStep, KVPool, ModelShape, random_context_tables,
                                       random_weights)  # fmt: skip
from tinyserve_amd.step_inputs import Batch, DecodeInputs, PagedTable, build_batch, fill_decode_inputs

pytestmark = pytest.mark.gpu
DEVICE = "cuda"
TINY = ModelShape(hidden=256, num_heads=4, num_kv_heads=2, head_dim=64, intermediate=512, vocab=1000,
                  num_layers=2)  # fmt: skip


def setup(lens: list[int], rows: int, dtype: torch.dtype = torch.float32, shape: ModelShape = TINY,
          block_size: int = 4, seed: int = 0):  # fmt: skip
    w = random_weights(shape, dtype, DEVICE, seed)
    blocks, nb = random_context_tables(lens, block_size, seed=seed)
    pool = KVPool(shape, nb + 3, block_size, dtype, DEVICE)  # blocks nb .. nb + 2 are spare
    g = torch.Generator(device="cpu").manual_seed(seed + 1)
    pool.k.copy_(torch.randn(pool.k.shape, generator=g).to(dtype))  # stands in for earlier steps
    pool.v.copy_(torch.randn(pool.v.shape, generator=g).to(dtype))
    tabs = [PagedTable(b, block_size, n) for b, n in zip(blocks, lens)]
    inp = DecodeInputs.empty(rows, max(len(b) for b in blocks) + 1, DEVICE)
    tokens = [(7 * i + 3) % shape.vocab for i in range(len(lens))]
    fill_decode_inputs(inp, list(zip(tokens, tabs)), pool.pad_block)
    return w, pool, tabs, inp


def reference_step(shape: ModelShape, w: dict, k: torch.Tensor, v: torch.Tensor, inp: DecodeInputs | Batch,
                   block_size: int) -> torch.Tensor:  # fmt: skip
    """The reference's forward_decode (a ``DecodeInputs``) or forward_batch (a ``Batch``:
    every sequence through the per-sequence prefill reference) composed from the oracle,
    fp32 on the CPU; logits of every row; writes k, v."""
    cw = {n: t.float().cpu() for n, t in w.items()}
    bt, lens = inp.block_tables.cpu(), inp.context_lens.cpu()
    if isinstance(inp, Batch):
        tok, pos, slots = inp.token_ids.cpu(), inp.positions.cpu(), inp.new_slots.cpu()
        qs, ql = inp.q_starts.cpu(), inp.q_lens.cpu()

        def attend(q: torch.Tensor, kc: torch.Tensor, vc: torch.Tensor) -> torch.Tensor:
            return ref.prefill_ref(q, kc, vc, bt, qs, ql, lens, shape.head_dim**-0.5, block_size)
    else:
        tok, pos, slots = inp.token_ids.cpu(), inp.positions.cpu(), inp.slots.cpu()

        def attend(q: torch.Tensor, kc: torch.Tensor, vc: torch.Tensor) -> torch.Tensor:
            return ref.decode_ref(q, kc, vc, bt, lens, shape.head_dim**-0.5, block_size)

    cos, sin = ref.rope_cos_sin(shape.head_dim, shape.rope_theta, pos)
    x = cw["model.embed_tokens.weight"][tok]
    n, s = x.shape[0], shape
    for i in range(s.num_layers):
        p = f"model.layers.{i}."
        h = ref.rms_norm(x, cw[p + "input_layernorm.weight"], s.rms_norm_eps)
        q, kk, vv = torch.split(h @ cw[p + "self_attn.qkv_proj.weight"].T, [s.q_size, s.kv_size, s.kv_size], 1)
        q = ref.qk_norm_rope_store_ref(
            q.reshape(n, s.num_heads, s.head_dim), kk.reshape(n, s.num_kv_heads, s.head_dim),
            vv.reshape(n, s.num_kv_heads, s.head_dim), cw[p + "self_attn.q_norm.weight"],
            cw[p + "self_attn.k_norm.weight"], cos, sin, slots, k[i], v[i], s.rms_norm_eps)  # fmt: skip
        attn = attend(q, k[i], v[i])
        x = x + attn.reshape(n, s.q_size) @ cw[p + "self_attn.o_proj.weight"].T
        h = ref.rms_norm(x, cw[p + "post_attention_layernorm.weight"], s.rms_norm_eps)
        gate, up = (h @ cw[p + "mlp.gate_up_proj.weight"].T).chunk(2, dim=1)
        x = x + (F.silu(gate) * up) @ cw[p + "mlp.down_proj.weight"].T
    x = ref.rms_norm(x, cw["model.norm.weight"], s.rms_norm_eps)
    return x @ cw["model.embed_tokens.weight"].T


@pytest.mark.parametrize("rows", [4, 8])  # no padding; 4 padding rows
@pytest.mark.parametrize("splits", [None, 1, 3])
def test_step_matches_the_reference_step(rows: int, splits: int | None) -> None:
    lens = [6, 1, 13, 4]
    w, pool, tabs, inp = setup(lens, rows)
    k0, v0 = pool.k.cpu(), pool.v.cpu()
    kr, vr = k0.clone(), v0.clone()
    want = reference_step(TINY, w, kr, vr, inp, pool.block_size)
    got = DecodeStep(TINY, w, pool, splits).forward(inp).cpu()
    assert got.shape == (rows, TINY.vocab) and got.dtype == torch.float32
    torch.testing.assert_close(got[: len(lens)], want[: len(lens)], atol=1e-4, rtol=1e-4)
    # The cache changed at the new tokens' slots (and the padding block) only, to the
    # reference's values.
    new = set(inp.slots.cpu().tolist())
    changed = ((pool.k.cpu() != k0) | (pool.v.cpu() != v0)).flatten(2).any(-1).any(0)
    assert set(changed.nonzero().flatten().tolist()) <= new
    real = inp.slots.cpu()[: len(lens)]
    torch.testing.assert_close(pool.k.cpu()[:, real], kr[:, real], atol=1e-5, rtol=1e-5)
    # v is the QKV product copied as is: only the GEMMs' rounding (GPU vs CPU) differs.
    torch.testing.assert_close(pool.v.cpu()[:, real], vr[:, real], atol=1e-5, rtol=1e-5)


def test_padding_rows_do_not_change_real_rows() -> None:
    outs = []
    for rows in (2, 8):
        w, pool, tabs, inp = setup([5, 2], rows, seed=4)
        outs.append(DecodeStep(TINY, w, pool).forward(inp)[:2].cpu())
    torch.testing.assert_close(outs[1], outs[0], atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_graph_replays_equal_the_eager_step(dtype: torch.dtype) -> None:
    lens = [9, 30, 2, 17, 5]
    w, pool, tabs, inp = setup(lens, 8, dtype, seed=7)
    step = DecodeStep(TINY, w, pool)
    graph = DecodeGraph(step.forward, inp)
    spare = iter(range(pool.pad_block - 3, pool.pad_block))
    for it in range(3):
        # A new step: every sequence grows by one token (the new token's block may be new).
        for t in tabs:
            t.num_tokens += 1
            if len(t.blocks) * t.block_size < t.num_tokens:
                t.blocks.append(next(spare))
        fill_decode_inputs(inp, [((it * 5 + j) % TINY.vocab, t) for j, t in enumerate(tabs)], pool.pad_block)
        k_before, v_before = pool.k.clone(), pool.v.clone()
        got = graph.replay().clone()
        torch.cuda.synchronize()
        k_after, v_after = pool.k.clone(), pool.v.clone()
        pool.k.copy_(k_before)
        pool.v.copy_(v_before)
        want = step.forward(inp)  # eager, on the same cache state
        torch.cuda.synchronize()
        torch.testing.assert_close(got, want, atol=0, rtol=0)
        assert torch.equal(pool.k, k_after) and torch.equal(pool.v, v_after)
        torch.randn(1 << 20, device=DEVICE).sum().item()  # unrelated eager work between replays


def mixed_setup(cached: list[int], new: list[int], seed: int, block_size: int = 4):
    """A tiny fp32 model, a filled pool and a ``Batch`` of ``new[b]`` tokens per sequence
    after ``cached[b]`` earlier ones (whose k/v the random pool stands in for)."""
    w, pool, tabs, _ = setup([c + n for c, n in zip(cached, new)], len(cached), seed=seed, block_size=block_size)
    g = torch.Generator(device="cpu").manual_seed(seed + 2)
    items = [(torch.randint(0, TINY.vocab, (n,), generator=g).tolist(), t) for n, t in zip(new, tabs)]
    return w, pool, tabs, items


@pytest.mark.parametrize(
    "cached,new",
    [
        ([5, 0, 9, 2, 0], [3, 7, 1, 1, 1]),  # prefill and decode sequences interleaved
        ([0, 3], [17, 40]),  # prefill only, one from scratch
        ([6, 1, 13], [1, 1, 1]),  # decode only
        ([30], [1]),
    ],
)
def test_mixed_step_matches_the_reference_step(cached: list[int], new: list[int]) -> None:
    w, pool, tabs, items = mixed_setup(cached, new, seed=11)
    batch = build_batch(items, DEVICE)
    kr, vr = pool.k.cpu(), pool.v.cpu()
    want = reference_step(TINY, w, kr, vr, batch, pool.block_size)[batch.last_rows.cpu()]
    got = DecodeStep(TINY, w, pool).forward_batch(batch).cpu()
    assert got.shape == (len(new), TINY.vocab) and got.dtype == torch.float32
    torch.testing.assert_close(got, want, atol=1e-4, rtol=1e-4)
    slots = batch.new_slots.cpu()
    torch.testing.assert_close(pool.k.cpu()[:, slots], kr[:, slots], atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(pool.v.cpu()[:, slots], vr[:, slots], atol=1e-5, rtol=1e-5)


def test_mixed_step_equals_each_sequence_alone() -> None:
    # test_batched_forward.py: a sequence's logits do not depend on what else is batched.
    cached, new = [4, 0, 11, 7], [1, 9, 1, 5]
    w, pool, tabs, items = mixed_setup(cached, new, seed=3)
    k0, v0 = pool.k.clone(), pool.v.clone()
    step = DecodeStep(TINY, w, pool)
    together = step.forward_batch(build_batch(items, DEVICE))
    for b, item in enumerate(items):
        pool.k.copy_(k0)
        pool.v.copy_(v0)
        alone = step.forward_batch(build_batch([item], DEVICE))
        torch.testing.assert_close(alone[0], together[b], atol=1e-5, rtol=1e-5)


def test_decode_only_batch_equals_the_decode_step() -> None:
    lens = [6, 1, 13, 4]
    w, pool, tabs, inp = setup(lens, len(lens), seed=5)
    k0, v0 = pool.k.clone(), pool.v.clone()
    step = DecodeStep(TINY, w, pool)
    want = step.forward(inp)
    pool.k.copy_(k0)
    pool.v.copy_(v0)
    got = step.forward_batch(build_batch([([int(t)], tab) for t, tab in zip(inp.token_ids.cpu(), tabs)], DEVICE))
    torch.testing.assert_close(got, want, atol=0, rtol=0)
