"""Benchmark of the attention hot path on one MI355X.

The headline ``value`` is the metric's workload: one layer's paged decode attention at
B=64 sequences x 4096 tokens, fp16, Qwen3-0.6B shapes (16 query / 8 kv heads, head_dim
128, 16-token blocks scattered over the pool), split-K + combine. One step = one call
of the attention kernel (plus the combine kernel when the launch policy splits into HBM
partials; at this batch it does not) on inputs already resident in HBM. ``value``
is the step's algorithmic bytes (K and V read once, q read, out written, block tables
and lengths read: 1,074,332,160 B) divided by the measured time per step, in GB/s.

``roofline`` covers the dominant kernel (the attention kernel): algorithmic bytes per launch
/ its average duration measured with HIP events on the launch stream, against the
8 TB/s HBM peak. ``cpu_baseline`` times the CPU oracle (the PyTorch reference path,
restated) on the same workload on this host's cores. ``extra`` adds the prefill
(MFMA-bound) and fused-kernel (HBM-bound) numbers of BASELINE configs 2-4.

    python bench.py [--gpus 1] [--steps 100] [--warmup 200] [--splits S] [--no-cpu] [--no-extra]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

from tinyserve_amd import _lib  # noqa: E402
from tinyserve_amd.hip_attention import decode_plan, launch_paged_decode_split, num_splits_for  # noqa: E402
from tinyserve_amd.hip_fused import qk_norm_rope_store, rms_norm_rows  # noqa: E402
from tinyserve_amd.hip_prefill import paged_prefill_attention  # noqa: E402
from tinyserve_amd.workloads import (  # noqa: E402
    decode_bench_case, fused_case, prefill_case, prefill_lengths)

HBM_PEAK_GBS = 8000.0
FP16_PEAK_TFLOPS = 2500.0  # dense fp16/bf16 MFMA
METRIC = "decode-attn HBM GB/s (% of peak) at B=64,ctx=4096; prefill-attn MFMA util"
HQ, HKV, D, BS = 16, 8, 128, 16


def decode_bytes(b: int, ctx: int, splits: int = 1, esize: int = 2) -> dict[str, int]:
    """Algorithmic bytes of one step, and of its attention kernel alone (the same: the
    launcher's one launch, with one split or the splits merged in each workgroup, writes
    the output itself)."""
    kv = b * ctx * HKV * D * 2 * esize
    q_io = 2 * b * HQ * D * esize
    tables = b * math.ceil(ctx / BS) * 4
    lens = b * 4
    step = kv + q_io + tables + lens
    return {"step": step, "split_kernel": step}


def split_kernel_launch(c, splits: int, m, l, acc, out, stream: int) -> None:
    """The split kernel alone, as hip_attention launches it: with ``m`` None and splits > 1
    the split ranges' states merge in each workgroup (one launch, output written);
    with partial buffers, the HBM-partials kernel that ``combine_launch`` finishes."""
    q, k = c.q, c.k_cache
    ptrs = (None, None, None) if m is None else (m.data_ptr(), l.data_ptr(), acc.data_ptr())
    _lib.call("ts_decode_split", q.data_ptr(), k.data_ptr(), c.v_cache.data_ptr(),
              c.block_tables.data_ptr(), c.context_lens.data_ptr(), out.data_ptr(),
              *ptrs, q.shape[0], HQ, HKV, D, BS,
              q.stride(0), q.stride(1), out.stride(0), out.stride(1), k.stride(0), k.stride(1),
              c.block_tables.stride(0), c.block_tables.shape[1], splits, 0, c.scale, 1, stream)  # fmt: skip


def combine_launch(splits: int, m, l, acc, out, stream: int) -> None:
    _lib.call("ts_decode_combine", m.data_ptr(), l.data_ptr(), acc.data_ptr(), out.data_ptr(),
              out.shape[0], HQ, D, out.stride(0), out.stride(1), splits, 1, stream)  # fmt: skip


def time_decode(batch: int, ctx: int, splits: int, steps: int, warmup: int) -> dict:
    dev = torch.device("cuda:0")
    c = decode_bench_case(batch, ctx, HQ, HKV, D, BS, torch.float16, device=dev)
    stream = torch.cuda.current_stream(dev)
    s = stream.cuda_stream
    out = torch.empty_like(c.q)

    def step() -> None:  # one launch: the split ranges (if any) merge in each workgroup
        split_kernel_launch(c, splits, None, None, None, out, s)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    # Timed region: exactly `steps` steps, one event pair around all of them (an event
    # per launch would add a gap between launches).
    t_start, t_end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    t_start.record(stream)
    for _ in range(steps):
        step()
    t_end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    total_ms = t_start.elapsed_time(t_end)
    split_ms = total_ms / steps  # the step is the attention kernel alone
    # The public entry point gives the same result (a check, outside the timed region).
    ref_out = launch_paged_decode_split(*c.args(), c.scale, BS, num_splits=splits)
    assert torch.equal(ref_out, out), "bench launch differs from the entry point"
    nbytes = decode_bytes(batch, ctx, splits)
    return {"ms_per_step": total_ms / steps, "wall_ms_per_step": wall * 1e3 / steps,
            "split_ms": split_ms, "bytes": nbytes, "case": c}  # fmt: skip


def loop_ms(fn, iters: int = 20, warmup: int = 3) -> float:
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(iters):
        fn()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / iters


def graph_ms(fn, launches: int = 20, replays: int = 10) -> float:
    """Mean time of one ``fn`` launch, from a captured graph of ``launches`` of them
    replayed ``replays`` times: the kernels' own rate, without the Python call overhead
    that bounds a loop of eager calls to microsecond kernels."""
    fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(launches):
            fn()
    g.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(replays):
        g.replay()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / (replays * launches)


def prefill_rates(call, flops: int) -> dict:
    """A prefill launch's rate two ways: ``ms`` / ``mfma_frac`` from graph replay (the
    kernel's own rate, what a profiler's kernel trace shows: back-to-back launches with no
    Python between them; best of 3), and ``eager_ms`` / ``eager_mfma_frac`` from a loop of
    eager calls (bounded by the host's call rate for launches of a few tens of us)."""
    eager = loop_ms(call, 20, 3)
    g = min(graph_ms(call) for _ in range(3))
    return {"ms": round(g, 4), "TFLOP/s": round(flops / g / 1e9, 1),
            "mfma_frac": round(flops / g / 1e9 / FP16_PEAK_TFLOPS, 4), "timing": "graph replay",
            "eager_ms": round(eager, 4), "eager_mfma_frac": round(flops / eager / 1e9 / FP16_PEAK_TFLOPS, 4)}


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(case, splits: int, budget_s: float = 15.0) -> dict:
    """The oracle (PyTorch reference path restated) on this host, over the same 64 x 4096
    workload, repeated until ``budget_s`` of work (at least once)."""
    from oracle import ref

    torch.set_num_threads(os.cpu_count() or 1)
    q = case.q.cpu()
    kc, vc = case.k_cache.cpu(), case.v_cache.cpu()
    bt, lens = case.block_tables.cpu(), case.context_lens.cpu()
    reps, t0 = 0, time.perf_counter()
    while True:
        ref.decode_ref(q, kc, vc, bt, lens, case.scale, BS)
        reps += 1
        if time.perf_counter() - t0 >= budget_s or reps >= 100:
            break
    dt = (time.perf_counter() - t0) / reps
    nbytes = decode_bytes(q.shape[0], int(lens[0]))["step"]
    return {"value": round(nbytes / dt / 1e9, 3), "unit": "GB/s", "cores": torch.get_num_threads(),
            "cpu_model": cpu_model(), "kind": "port",
            "sample": f"oracle.ref.decode_ref (torch CPU) over the full B={q.shape[0]} x ctx="
                      f"{int(lens[0])} fp16 workload, {reps} rep(s), {dt:.2f} s each"}  # fmt: skip


def cpu_baselines_other_configs(budget_s: float = 8.0) -> dict:
    """The oracle on this host for configs 3 (varlen prefill, fp16) and 4 (fused norm /
    RoPE / KV write, T=4096): bounded samples of the same workloads, scaled by their
    algorithmic flops or bytes."""
    from oracle import ref

    torch.set_num_threads(os.cpu_count() or 1)
    res: dict = {"cores": torch.get_num_threads(), "cpu_model": cpu_model(), "kind": "port"}
    lens = prefill_lengths(32, seed=0)
    p = prefill_case([(0, n) for n in lens], HQ, HKV, D, BS, torch.float16, seed=3, sentinel=False)
    done_flops, t0, seqs = 0, time.perf_counter(), 0
    for r, n in enumerate(lens):  # whole sequences in order until the budget is spent
        sl = slice(r, r + 1)
        ref.prefill_ref(p.q, p.k, p.v, p.tables[sl], p.starts[sl], p.q_lens[sl], p.ctx_lens[sl],
                        p.scale, BS)  # fmt: skip
        done_flops += 4 * HQ * D * n * (n + 1) // 2
        seqs += 1
        if time.perf_counter() - t0 >= budget_s:
            break
    dt = time.perf_counter() - t0
    res["prefill_varlen32_float16"] = {
        "value": round(done_flops / dt / 1e12, 4), "unit": "TFLOP/s",
        "sample": f"oracle.ref.prefill_ref on {seqs} of the 32 sequences ({done_flops / 1e9:.1f} GFLOP) "
                  f"in {dt:.2f} s"}  # fmt: skip
    f = fused_case(sentinel=False)
    reps, t0 = 0, time.perf_counter()
    while True:
        ref.rms_norm(f.x, f.norm_w, f.eps)
        ref.qk_norm_rope_store_ref(f.q, f.k, f.v, f.q_w, f.k_w, f.cos, f.sin, f.slots, f.k_cache, f.v_cache,
                                   f.eps)  # fmt: skip
        reps += 1
        if time.perf_counter() - t0 >= budget_s or reps >= 50:
            break
    dt = (time.perf_counter() - t0) / reps
    nbytes = 4096 * (1024 * 2 * 2 + 16904)
    res["fused_t4096"] = {
        "value": round(nbytes / dt / 1e9, 3), "unit": "GB/s", "ms": round(dt * 1e3, 2),
        "sample": f"oracle.ref.rms_norm + qk_norm_rope_store_ref over the full T=4096 workload, "
                  f"{reps} rep(s)"}  # fmt: skip
    return res


def check(got: torch.Tensor, want: torch.Tensor, bound: float, what: str) -> float:
    """Max-abs difference of two results of one workload by two paths (outside any
    timed region); a difference above ``bound`` stops the benchmark: a number for a
    wrong result is no number."""
    diff = float((got.float() - want.float()).abs().max())
    if not diff <= bound:
        raise SystemExit(f"bench check failed: {what}: max-abs {diff:.3g} > {bound}")
    return round(diff, 6)


def kernel_name(plan: dict, dtype: str = "f16") -> str:
    """The decode kernel instantiation the library dispatches for ``plan``."""
    budget = {"heavy": "heavy", "light": "light", "light_stream": "light-stream"}[plan["budget"]]
    return f"paged_attend_kernel<{dtype},{D},{plan['head_tile']},false,{budget}>"


def batched_sdpa_prefill(p, out: torch.Tensor) -> torch.Tensor:
    """The reference's batched prefill path on the GPU (attention.py:144-220): all
    sequences' queries and keys gathered into one padded rectangle, one masked
    scaled-dot-product call in float32 as the reference computes it. A timing
    comparison for the prefill kernel (its T4 default path), built once per call like
    the reference's ``prefill_plan`` + ``batched_prefill_attention``."""
    lens, totals, starts = p.q_lens.tolist(), p.ctx_lens.tolist(), p.starts.tolist()
    dev = p.q.device
    lq, lk, bs = max(lens), max(totals), p.block_size
    i = torch.arange(lq, device=dev)
    n = torch.tensor(lens, device=dev)[:, None]
    rows = torch.tensor(starts, device=dev)[:, None] + torch.minimum(i[None, :], n - 1)
    j = torch.arange(lk, device=dev)
    slots = p.tables.long()[:, (j // bs).clamp(max=p.tables.shape[1] - 1)] * bs + j % bs
    q_pos = torch.tensor(totals, device=dev)[:, None] - n + torch.minimum(i[None, :], n - 1)
    mask = (j[None, None, :] <= q_pos[:, :, None])[:, None]
    group = p.q.shape[1] // p.k.shape[1]
    qb = p.q[rows].float().transpose(1, 2)
    kb = p.k[slots].float().repeat_interleave(group, dim=2).transpose(1, 2)
    vb = p.v[slots].float().repeat_interleave(group, dim=2).transpose(1, 2)
    ob = torch.nn.functional.scaled_dot_product_attention(qb, kb, vb, attn_mask=mask, scale=p.scale)
    ob = ob.transpose(1, 2).to(p.q.dtype)
    for r, (st, ln) in enumerate(zip(starts, lens)):
        out[st : st + ln] = ob[r, :ln]
    return out


def extra_measurements() -> dict:
    dev = torch.device("cuda:0")
    res: dict = {}
    # Config 2: decode B=32 x 256, a 4096-block pool: 4 splits as the config states, through
    # the launcher (the four ranges' states merged in each workgroup's LDS, one launch),
    # and the policy's single launch (each sequence split over the waves of a workgroup);
    # then the same 4 splits as fp32 partials in HBM and the combine launch.
    c = decode_bench_case(32, 256, pool_blocks=4096, device=dev, seed=1)
    nb = decode_bytes(32, 256)["step"]
    outs = {}
    for key, splits in (("decode_b32_ctx256_s4", 4), ("decode_b32_ctx256_policy", None)):
        outs[key] = launch_paged_decode_split(*c.args(), c.scale, BS, num_splits=splits).clone()
        def call() -> None:
            launch_paged_decode_split(*c.args(), c.scale, BS, num_splits=splits)

        # graph_us: best of three graph replays, as for the prefill rates.
        ms, ms_g = loop_ms(call, 200, 20), min(graph_ms(call) for _ in range(3))
        plan = decode_plan(32, HQ, HKV, D, BS, c.block_tables.shape[1], 1)  # in-group splits: the one-split grid
        res[key] = {"us": round(ms * 1e3, 2), "GB/s": round(nb / ms / 1e6, 1),
                    "graph_us": round(ms_g * 1e3, 2), "graph_GB/s": round(nb / ms_g / 1e6, 1),
                    "launches": "one launch, 4 range states merged in LDS" if splits else "one launch",
                    "kernel": kernel_name(plan), "grid": plan["grid"],
                    "waves_per_group": plan["waves_per_group"]}  # fmt: skip
    res["decode_b32_ctx256_policy"]["max_abs_vs_s4"] = check(
        outs["decode_b32_ctx256_policy"], outs["decode_b32_ctx256_s4"], 4e-3, "config 2: policy vs 4 splits")
    hout = torch.empty_like(c.q)
    m = torch.empty((32, HQ, 4), dtype=torch.float32, device=dev)
    l = torch.empty_like(m)  # noqa: E741
    acc = torch.empty((32, HQ, 4, D), dtype=torch.float32, device=dev)

    def hbm() -> None:
        s = torch.cuda.current_stream(dev).cuda_stream  # a graph capture runs on its own stream
        split_kernel_launch(c, 4, m, l, acc, hout, s)
        combine_launch(4, m, l, acc, hout, s)

    ms, ms_g = loop_ms(hbm, 200, 20), min(graph_ms(hbm) for _ in range(3))
    res["decode_b32_ctx256_s4_hbm_partials"] = {
        "us": round(ms * 1e3, 2), "GB/s": round(nb / ms / 1e6, 1), "graph_us": round(ms_g * 1e3, 2),
        "graph_GB/s": round(nb / ms_g / 1e6, 1), "launches": "split kernel (fp32 partials) + combine",
        "max_abs_vs_s4": check(hout, outs["decode_b32_ctx256_s4"], 4e-3, "config 2: HBM partials vs in-group")}  # fmt: skip
    # The reference's own published decode shapes (fp16, one layer, Qwen3 heads; its T4
    # timings in BASELINE.md): B=32 x 1024, B=32 x 160, B=64 x 1024, the policy's launch.
    for b, ctx in ((32, 1024), (32, 160), (64, 1024)):
        cr = decode_bench_case(b, ctx, device=dev, seed=2)
        ms_r = graph_ms(lambda: launch_paged_decode_split(*cr.args(), cr.scale, BS))
        nb_r = decode_bytes(b, ctx)["step"]
        got = launch_paged_decode_split(*cr.args(), cr.scale, BS).clone()
        s4 = launch_paged_decode_split(*cr.args(), cr.scale, BS, num_splits=4)
        res[f"decode_b{b}_ctx{ctx}"] = {"us": round(ms_r * 1e3, 2), "GB/s": round(nb_r / ms_r / 1e6, 1),
                                        "timing": "graph replay",
                                        "max_abs_vs_s4": check(got, s4, 4e-3, f"decode {b} x {ctx}")}  # fmt: skip
    # Config 3: varlen prefill, 32 prompts L ~ U[16, 2048], fp16 and bf16.
    lens = prefill_lengths(32, seed=0)
    flops = sum(4 * HQ * D * n * (n + 1) // 2 for n in lens)
    for dt in (torch.float16, torch.bfloat16):
        p = prefill_case([(0, n) for n in lens], HQ, HKV, D, BS, dt, seed=3, sentinel=False,
                         device=dev)  # fmt: skip
        out = torch.empty_like(p.q)
        res[f"prefill_varlen32_{str(dt).split('.')[-1]}"] = {
            **prefill_rates(lambda: paged_prefill_attention(*p.args(), out=out), flops), "flops": flops}
        ms = res[f"prefill_varlen32_{str(dt).split('.')[-1]}"]["eager_ms"]
        if dt == torch.float16:  # the reference's batched SDPA path on the same input
            ref_out = torch.empty_like(p.q)
            ms_ref = loop_ms(lambda: batched_sdpa_prefill(p, ref_out), 5, 1)
            res["prefill_varlen32_reference_batched_sdpa_fp32"] = {
                "ms": round(ms_ref, 3), "TFLOP/s": round(flops / ms_ref / 1e9, 1),
                "hip_kernel_speedup": round(ms_ref / ms, 1),
                "max_abs_diff_vs_hip": check(out, ref_out, 4e-3, "config 3 vs batched SDPA")}  # fmt: skip
    # 2048-token prompts: a batch of 4 (fills the chip) and one alone (the critical path).
    four = prefill_case([(0, 2048)] * 4, HQ, HKV, D, BS, torch.float16, sentinel=False, device=dev)
    out4 = torch.empty_like(four.q)
    f4 = 4 * 4 * HQ * D * 2048 * 2049 // 2
    res["prefill_4x2048_float16"] = {**prefill_rates(lambda: paged_prefill_attention(*four.args(), out=out4), f4),
                                     "max_abs_vs_batched_sdpa": check(
                                         out4, batched_sdpa_prefill(four, torch.empty_like(four.q)), 4e-3,
                                         "prefill 4 x 2048")}  # fmt: skip
    one = prefill_case([(0, 2048)], HQ, HKV, D, BS, torch.float16, sentinel=False, device=dev)
    out = torch.empty_like(one.q)
    f1 = 4 * HQ * D * 2048 * 2049 // 2
    res["prefill_single2048_float16"] = {**prefill_rates(lambda: paged_prefill_attention(*one.args(), out=out), f1),
                                         "max_abs_vs_batched_sdpa": check(
                                             out, batched_sdpa_prefill(one, torch.empty_like(one.q)), 4e-3,
                                             "prefill 1 x 2048")}  # fmt: skip
    # Config 4: fused RMSNorm + q/k norm + RoPE + KV write, T=4096.
    f = fused_case(device=dev, sentinel=False)
    def rms() -> None:
        rms_norm_rows(f.x, f.norm_w, f.eps)

    def qk() -> None:
        qk_norm_rope_store(f.q, f.k, f.v, f.q_w, f.k_w, f.cos, f.sin, f.slots, f.k_cache, f.v_cache, f.eps)

    eager_r, eager_q = loop_ms(rms, 200, 20), loop_ms(qk, 200, 20)
    ms_r, ms_q = graph_ms(rms), graph_ms(qk)
    t = 4096
    b_r, b_q = t * 1024 * 2 * 2, t * 16904
    # layers.py:34-38 restated with torch ops on the GPU (normalise in fp32, round, times w).
    xf = f.x.float()
    want_rms = (xf * torch.rsqrt(xf.square().mean(-1, keepdim=True) + f.eps)).to(f.x.dtype) * f.norm_w
    res["fused_t4096"] = {
        "rms_max_abs_vs_torch": check(rms_norm_rows(f.x, f.norm_w, f.eps), want_rms, 2e-2, "rms_norm_rows"),
        "rms_norm_rows_us": round(ms_r * 1e3, 2), "rms_GB/s": round(b_r / ms_r / 1e6, 1),
        "qk_norm_rope_store_us": round(ms_q * 1e3, 2), "qk_GB/s": round(b_q / ms_q / 1e6, 1),
        "bytes": b_r + b_q, "timing": "graph replay of 20 launches",
        "eager_call_us": {"rms_norm_rows": round(eager_r * 1e3, 2),
                          "qk_norm_rope_store": round(eager_q * 1e3, 2)}}  # fmt: skip
    # Config 5: the 28-layer decode step.
    res["decode_step_28l_b64"] = decode_step_28l()
    res["decode_step_28l_b32_short_ctx_by_table_width"] = short_context_graph_widths()
    return res


def decode_step_28l(batch: int = 64, steps: int = 20, seed: int = 5, ctx: tuple[int, int] = (1024, 4096),
                    width: int | None = None,
                    variants: tuple = ((16, "rows"), (None, "rows"), (None, "library"))) -> dict:  # fmt: skip
    """one decode step of all 28 layers of a random-init
    Qwen3-0.6B-shaped model (fp16), B=64, contexts ~ U[1024, 4096], 16-token blocks
    scattered over the pool, replayed as a captured graph. Reported for the reference's
    16 splits and for this library's split policy: tokens/s and the decode-attention
    share of the step (a graph of the step's 28 attention launches alone, timed the
    same way). ``width``: block-table columns of the step's buffers (default: the
    longest sequence's blocks), e.g. the model's maximum position as a graph runner
    sizes them. ``variants``: (split count, projections) pairs; "rows" runs the
    projections on this library's row-batch kernels, "library" on library GEMMs (keys
    ``splits_<S>`` and ``splits_<S>_library_projections``)."""
    from tinyserve_amd.decode_step import (DecodeGraph, DecodeStep, KVPool, ModelShape,
                                           random_context_tables, random_weights)  # fmt: skip
    from tinyserve_amd.step_inputs import DecodeInputs, PagedTable, fill_decode_inputs

    dev = torch.device("cuda:0")
    shape = ModelShape()
    w = random_weights(shape, torch.float16, dev, seed)
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(ctx[0], ctx[1] + 1, (batch,), generator=g).tolist()
    blocks, nb = random_context_tables(lens, BS, seed=seed)
    pool = KVPool(shape, nb, BS, torch.float16, dev)
    gd = torch.Generator(device=dev).manual_seed(seed)
    pool.k.normal_(generator=gd)
    pool.v.normal_(generator=gd)
    tables = [PagedTable(b, BS, n) for b, n in zip(blocks, lens)]
    inp = DecodeInputs.empty(batch, width or max(len(b) for b in blocks), dev)
    fill_decode_inputs(inp, [(i % shape.vocab, t) for i, t in enumerate(tables)], pool.pad_block)
    kv_bytes = sum(lens) * shape.num_layers * 2 * shape.kv_size * 2
    res: dict = {"batch": batch, "ctx_mean": round(sum(lens) / batch, 1), "kv_read_GB": round(kv_bytes / 1e9, 2),
                 "table_width": inp.block_tables.shape[1]}  # fmt: skip
    # Each replay writes the same new tokens' k/v to the same slots, so every replay and
    # every variant sees the same cache: their logits can be compared directly.
    logits = {}
    for splits, projections in variants:
        step = DecodeStep(shape, w, pool, splits, projections)
        full = DecodeGraph(step.forward, inp)
        attn = DecodeGraph(step.attention_only, inp)
        ms_step = loop_ms(full.replay, steps, 3)
        ms_attn = loop_ms(attn.replay, steps, 3)
        logits[(splits, projections)] = full.replay().clone()
        used = splits or num_splits_for(batch, shape.num_kv_heads, inp.block_tables.shape[1])
        plan = decode_plan(batch, HQ, HKV, D, BS, inp.block_tables.shape[1], 1 if splits is None and used <= 4 else used)
        key = f"splits_{used}" + ("" if projections == "rows" else f"_{projections}_projections")
        res[key] = {"ms_per_step": round(ms_step, 3), "tok_per_s": round(batch / ms_step * 1e3, 1),
                                 "attention_ms": round(ms_attn, 3), "attention_share": round(ms_attn / ms_step, 3),
                                 "attention_GB/s": round(kv_bytes / ms_attn / 1e6, 1),
                                 "kernel": kernel_name(plan), "projections": projections}  # fmt: skip
        del full, attn
    base = logits[variants[0]]
    for key, out in list(logits.items())[1:]:
        # fp16 steps by other split counts / projection kernels: ~1e-2 of drift over 28
        # layers (the tests bound each against the fp32 composition at 0.05).
        res[f"logits_max_abs_{key[0] or 'policy'}_{key[1]}_vs_{variants[0][0] or 'policy'}_{variants[0][1]}"] = check(
            out, base, 0.1, f"decode step {key} vs {variants[0]}")  # fmt: skip
    return res


def short_context_graph_widths(batch: int = 32) -> dict:
    """The config-5 step at short contexts (B=32, contexts ~ U[192, 320]) through graph
    buffers of two widths: the batch's own longest table, and the model's maximum
    position (40,960 tokens: 2,560 blocks, as a graph runner sizes them). The wide table
    bounds more than 256 MiB of K/V, so its launches stream K/V with non-temporal loads;
    this measures what that costs inside a whole step."""
    out = {}
    for name, width in (("tight_table", None), ("max_position_table", 40960 // BS)):
        out[name] = decode_step_28l(batch=batch, steps=20, seed=7, ctx=(192, 320), width=width,
                                    variants=((None, "rows"),))  # fmt: skip
    return out


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    # The clocks ramp for the first few hundred back-to-back launches under sustained HBM
    # load (~179 us per step over the first 50, ~164 us from the 150th on, one box): the
    # untimed warmup covers the ramp, so the timed steps measure the steady state.
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--splits", type=int, default=0, help="0: the launcher's default policy")
    ap.add_argument("--batch", type=int, default=64)
    ap.add_argument("--ctx", type=int, default=4096)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--profile", choices=["prefill_varlen32", "fused_t4096", "decode_b32_ctx256",
                                          "step_projections"], default=None,
                    help="only launch one workload 3 times (for a profiler) and print what ran")
    ap.add_argument("--copy-mb", type=int, default=0,
                    help="also run 3 plain device copies of this many MiB (a known-size kernel "
                         "that calibrates the HBM byte counters of a profiler)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(run with --gpus 1)", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        sys.exit(2)
    _lib.load()
    if args.profile == "prefill_varlen32":  # config 3's fp16 prefill, nothing else
        lens = prefill_lengths(32, seed=0)
        p = prefill_case([(0, n) for n in lens], HQ, HKV, D, BS, torch.float16, seed=3, sentinel=False,
                         device=torch.device("cuda:0"))  # fmt: skip
        out = torch.empty_like(p.q)
        for _ in range(3):
            paged_prefill_attention(*p.args(), out=out)
        torch.cuda.synchronize()
        print(json.dumps({"profile": args.profile, "launches": 3, "sequences": len(lens),
                          **calibration_copies(args.copy_mb)}), flush=True)  # fmt: skip
        return
    if args.profile == "decode_b32_ctx256":  # config 2: 4 splits, then the policy's launch
        c = decode_bench_case(32, 256, pool_blocks=4096, device=torch.device("cuda:0"), seed=1)
        for splits in (4, None):
            for _ in range(20):
                launch_paged_decode_split(*c.args(), c.scale, BS, num_splits=splits)
        torch.cuda.synchronize()
        print(json.dumps({"profile": args.profile, "launches": "20 x 4 splits through the launcher (one launch, range states merged in LDS), then 20 x the policy's launch",
                          **calibration_copies(args.copy_mb)}), flush=True)  # fmt: skip
        return
    if args.profile == "step_projections":  # config 5's four projections of a layer, W cold
        print(json.dumps({"profile": args.profile, **step_projections_for_profile(),
                          **calibration_copies(args.copy_mb)}), flush=True)  # fmt: skip
        return
    if args.profile == "fused_t4096":  # config 4's two fused kernels, eager, nothing else
        f = fused_case(device=torch.device("cuda:0"), sentinel=False)
        for _ in range(3):
            rms_norm_rows(f.x, f.norm_w, f.eps)
        for _ in range(3):
            qk_norm_rope_store(f.q, f.k, f.v, f.q_w, f.k_w, f.cos, f.sin, f.slots, f.k_cache, f.v_cache, f.eps)
        torch.cuda.synchronize()
        print(json.dumps({"profile": args.profile, "launches": 3, "tokens": f.x.shape[0],
                          **calibration_copies(args.copy_mb)}), flush=True)  # fmt: skip
        return
    nb = math.ceil(args.ctx / BS)
    splits = args.splits or num_splits_for(args.batch, HKV, nb)
    r = time_decode(args.batch, args.ctx, splits, args.steps, args.warmup)
    step_bytes, split_bytes = r["bytes"]["step"], r["bytes"]["split_kernel"]
    value = step_bytes / r["ms_per_step"] / 1e6  # GB/s
    achieved = split_bytes / r["split_ms"] / 1e6
    # HBM bytes per launch come from the committed, calibrated rocprofv3 PMC run of this
    # workload (FETCH_SIZE x 2 + WRITE_SIZE; a profiler cannot run inside this process).
    traffic, traffic_src = None, None
    tf = ROOT / "profiles" / "paged_attend_decode_b64_ctx4096_traffic.json"
    if tf.exists() and (args.batch, args.ctx, splits) == (64, 4096, 1):
        traffic = json.loads(tf.read_text()).get("bytes_per_launch")
        traffic_src = "profiles/paged_attend_decode_b64_ctx4096_traffic.json (rocprofv3 --pmc, calibrated)"
    plan = decode_plan(args.batch, HQ, HKV, D, BS, nb, splits)
    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic: K/V/q ~ N(0,1), block tables a random permutation of the pool",
        "config": {"workload": f"paged decode attention, one layer, B={args.batch} x ctx={args.ctx}, "
                               f"16 q / 8 kv heads, head_dim 128, block 16, "
                               + ("one launch (in-workgroup split-K)" if splits == 1
                                  else f"split-K {splits}, range states merged in LDS (one launch)"),
                   "batch": args.batch, "ctx": args.ctx, "splits": splits,
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "kernel": kernel_name(plan), "kernel_source": "ts_decode_plan",
                     "launch": {"grid": plan["grid"], "waves_per_group": plan["waves_per_group"],
                                "length_pairs": plan["by_length"]},
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "traffic_source": traffic_src,
                     "avg_launch_us": round(r["split_ms"] * 1e3, 2),
                     "algorithmic_bytes": split_bytes},
        "frac_of_peak_step": round(value / HBM_PEAK_GBS, 4),
    }  # fmt: skip
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(r["case"], splits)
        line["cpu_baseline_other_configs"] = cpu_baselines_other_configs()
    if not args.no_extra:
        line["extra"] = extra_measurements()
    line.update(calibration_copies(args.copy_mb))
    print(json.dumps(line), flush=True)


def step_projections_for_profile(rows: int = 64, dispatches: int = 24) -> dict:
    """The config-5 layer's four projections on the row-batch kernels (qkv, o_proj with
    8 K slices, gate_up + SiLU, down_proj with 6), fp16, 64 rows, each launched
    ``dispatches`` times over as many weight copies, more than the 256 MiB last-level
    cache holds between two uses of one copy, so W comes from HBM as in the step."""
    from tinyserve_amd import hip_rows as R

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(0)
    out: dict = {}
    for name, (n, k) in {"qkv": (4096, 1024), "o_proj": (1024, 2048), "gate_up": (6144, 1024),
                         "down_proj": (1024, 3072)}.items():  # fmt: skip
        ws = [torch.randn(n, k, generator=g, device=dev).half() for _ in range(max(dispatches, (320 << 20) // (n * k * 2)))]
        x = torch.randn(rows, k, generator=g, device=dev).half()
        xt = R.Tiled.from_dense(x)
        for w in ws[:dispatches]:
            if name == "qkv":
                R.rows_linear(xt, w)
            elif name == "o_proj":
                R.rows_linear_partials(x, w)
            elif name == "gate_up":
                R.rows_silu_gate_up(xt, w)
            else:
                R.rows_linear_partials(xt, w)
        torch.cuda.synchronize()
        out[name] = {"W_bytes": n * k * 2, "dispatches": dispatches, "copies": len(ws)}
        del ws
    return out


def calibration_copies(mb: int) -> dict:
    """Three plain device copies of ``mb`` MiB (none if 0): a kernel of known traffic
    that calibrates a profiler's HBM byte counters."""
    if not mb:
        return {}
    src = torch.ones(mb << 18, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    return {"copy_calibration_bytes": {"read": src.numel() * 4, "write": dst.numel() * 4}}


if __name__ == "__main__":
    main()
