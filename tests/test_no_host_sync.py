"""No entry point on the hot path waits for the GPU (GPU).

The reference runs its decode step under ``torch.cuda.set_sync_debug_mode("error")``
after a warm-up call (tests/test_decode_inputs.py:148-161): a host sync inside a step
would break graph capture, and its launch functions are documented as sync-free
(src/tinyserve/triton_attention.py:403-406). The same check here covers every launch
entry point of the path (decode split, varlen prefill, RMSNorm rows, q/k-norm + RoPE +
KV write) and both step forms of the decode-step caller (``forward`` and
``forward_batch``). Each runs once to warm up (library load, first allocations), then
again with torch's sync debugging turned to errors.
"""

from __future__ import annotations

from collections.abc import Callable

import pytest
import torch

from tinyserve_amd import hip_attention, hip_fused, hip_prefill
from tinyserve_amd.decode_step import DecodeStep, KVPool, ModelShape, random_context_tables, random_weights
from tinyserve_amd.step_inputs import DecodeInputs, PagedTable, build_batch, fill_decode_inputs
from tinyserve_amd.workloads import decode_case, prefill_case

pytestmark = pytest.mark.gpu
DEVICE = "cuda"


def never_syncs(fn: Callable[[], object]) -> None:
    fn()
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        fn()
    finally:
        torch.cuda.set_sync_debug_mode("default")
    torch.cuda.synchronize()


@pytest.mark.parametrize("num_splits", [None, 1, 4, 16])
def test_launch_paged_decode_split_never_waits_for_the_gpu(num_splits: int | None) -> None:
    c = decode_case([17, 64, 300, 1], num_q_heads=16, num_kv_heads=8, head_dim=128, dtype=torch.float16)
    q, k, v, bt, cl = (t.to(DEVICE) for t in c.args())
    never_syncs(lambda: hip_attention.launch_paged_decode_split(q, k, v, bt, cl, c.scale, c.block_size,
                                                                num_splits))  # fmt: skip


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_paged_prefill_attention_never_waits_for_the_gpu(dtype: torch.dtype) -> None:
    c = prefill_case([(0, 130), (70, 66), (5, 200)], 16, 8, 128, block_size=16, dtype=dtype)
    args = [t.to(DEVICE) if isinstance(t, torch.Tensor) else t for t in c.args()]
    out = torch.zeros_like(args[0])
    never_syncs(lambda: hip_prefill.paged_prefill_attention(*args, out=out))


def test_fused_kernels_never_wait_for_the_gpu() -> None:
    t, hq, hkv, d = 64, 16, 8, 128
    g = torch.Generator(device=DEVICE).manual_seed(0)
    qkv = torch.randn(t, (hq + 2 * hkv) * d, generator=g, device=DEVICE).half()
    q, k, v = torch.split(qkv, [hq * d, hkv * d, hkv * d], dim=1)
    q, k, v = q.view(t, hq, d), k.view(t, hkv, d), v.view(t, hkv, d)
    w = torch.ones(d, device=DEVICE, dtype=torch.float16)
    cos, sin = hip_fused.rope_cos_sin(d, 1e6, torch.arange(t, device=DEVICE))
    slots = torch.randperm(4 * t, device=DEVICE)[:t]
    kc = torch.zeros(4 * t, hkv, d, device=DEVICE, dtype=torch.float16)
    vc = torch.zeros_like(kc)
    x = torch.randn(t, 1024, generator=g, device=DEVICE).half()
    wx = torch.ones(1024, device=DEVICE, dtype=torch.float16)
    never_syncs(lambda: hip_fused.rms_norm_rows(x, wx, 1e-6))
    never_syncs(lambda: hip_fused.qk_norm_rope_store(q, k, v, w, w, cos, sin, slots, kc, vc, 1e-6))


TINY = ModelShape(hidden=256, num_heads=4, num_kv_heads=2, head_dim=64, intermediate=512, vocab=1000,
                  num_layers=2)  # fmt: skip


@pytest.mark.parametrize(("projections", "splits"), [("rows", None), ("rows", 4), ("library", None)])
def test_decode_step_forward_never_waits_for_the_gpu(projections: str, splits: int | None) -> None:
    lens, bs = [5, 40, 12], 4
    w = random_weights(TINY, torch.float16, DEVICE, 0)
    blocks, nb = random_context_tables(lens, bs, seed=0)
    pool = KVPool(TINY, nb, bs, torch.float16, DEVICE)
    tabs = [PagedTable(b, bs, n) for b, n in zip(blocks, lens)]
    inp = DecodeInputs.empty(8, max(len(b) for b in blocks), DEVICE)
    fill_decode_inputs(inp, [(i + 1, t) for i, t in enumerate(tabs)], pool.pad_block)
    step = DecodeStep(TINY, w, pool, splits, projections)
    never_syncs(lambda: step.forward(inp))


def test_decode_step_forward_batch_never_waits_for_the_gpu() -> None:
    # A mixed step (prefill and decode sequences), its Batch built beforehand by the
    # scheduler as the reference's engine does (batch.py:60-122).
    cached, new, bs = [5, 0, 9], [3, 7, 1], 4
    w = random_weights(TINY, torch.float16, DEVICE, 1)
    lens = [c + n for c, n in zip(cached, new)]
    blocks, nb = random_context_tables(lens, bs, seed=1)
    pool = KVPool(TINY, nb, bs, torch.float16, DEVICE)
    tabs = [PagedTable(b, bs, n) for b, n in zip(blocks, lens)]
    items = [([(7 * i + j) % TINY.vocab for j in range(n)], t) for i, (n, t) in enumerate(zip(new, tabs))]
    batch = build_batch(items, DEVICE)
    step = DecodeStep(TINY, w, pool)
    never_syncs(lambda: step.forward_batch(batch))
