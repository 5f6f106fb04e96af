"""The C-ABI library and the host side of the entry points, on the CPU.

The library is loaded (never asked to launch): every function ``include/tinyserve_amd.h``
declares must be exported and bound. The Python entry points must raise the reference's
ValueErrors before touching the device, and must refuse CPU tensors outright (no CPU
fallback) once the arguments are valid.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch

from tinyserve_amd import _lib, hip_attention, hip_fused, hip_prefill
from tinyserve_amd.workloads import decode_case, prefill_case

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "tinyserve_amd.h"


@pytest.fixture(scope="module")
def lib() -> ctypes.CDLL:
    if not _lib.LIB_PATH.exists():
        from tinyserve_amd.build import build

        build()
    return _lib.load()


def declared() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.findall(r"\b(ts_[a-z_0-9]+)\s*\(", text)


def test_header_declares_what_the_binding_binds() -> None:
    assert sorted(declared()) == sorted(_lib.EXPORTS)


def test_library_exports_every_declared_symbol(lib: ctypes.CDLL) -> None:
    for name in declared():
        assert hasattr(lib, name), name
    assert lib.ts_version() == (0 << 16) | 1
    assert b"invalid argument" in lib.ts_strerror(-1)
    assert b"unsupported" in lib.ts_strerror(-2)


def test_c_abi_rejects_bad_sizes_before_any_launch(lib: ctypes.CDLL) -> None:
    # Hq not a multiple of Hkv, a block size that is not a power of 2, zero splits: the
    # library returns TS_EINVAL without launching (null pointers are never touched).
    null = None
    strides = (0,) * 7
    assert lib.ts_decode_split(*([null] * 9), 1, 6, 4, 32, 16, *strides, 0, 1, 0, 1.0, 0, null) == -1
    assert lib.ts_decode_split(*([null] * 9), 1, 4, 2, 32, 12, *strides, 0, 1, 0, 1.0, 0, null) == -1
    assert lib.ts_decode_split(*([null] * 9), 1, 4, 2, 32, 16, *strides, 0, 0, 0, 1.0, 0, null) == -1
    # splits > 1 needs the partial buffers
    assert lib.ts_decode_split(*([null] * 9), 1, 4, 2, 32, 16, *strides, 0, 2, 0, 1.0, 0, null) == -1
    assert lib.ts_prefill_varlen(*([null] * 8), 1, 12, 4, 32, 16, 4, 0, *strides, 1.0, 0, null) == -1
    assert lib.ts_rms_norm_rows(null, null, null, 4, 0, 0, 0, 1e-6, 0, null) == -1
    assert lib.ts_qk_norm_rope_store(*([null] * 11), 1, 4, 2, 12, *([0] * 11), 1e-6, 0, 0, null) == -1
    # the no-allocation decode refuses partials beyond its scratch (2048 x 16 x 16 x 130
    # floats > 16 MiB) before touching any pointer or device
    assert lib.ts_decode_attention_noalloc(*([null] * 5), 1, 2048, 16, 8, 128, 16, *strides, 0, 16, 0,
                                           1.0, 1, null) == -3  # fmt: skip
    assert b"scratch" in lib.ts_strerror(-3)
    # empty batches launch nothing and succeed
    assert lib.ts_decode_split(*([null] * 9), 0, 4, 2, 32, 16, *strides, 0, 1, 0, 1.0, 0, null) == 0
    assert lib.ts_rms_norm_rows(null, null, null, 0, 16, 16, 16, 1e-6, 1, null) == 0
    # RoPE tables: odd head dim, a row stride shorter than the head dim, a theta of 0
    assert lib.ts_rope_cos_sin(null, 4, 63, 1e6, null, null, 64, null) == -1
    assert lib.ts_rope_cos_sin(null, 4, 64, 1e6, null, null, 32, null) == -1
    assert lib.ts_rope_cos_sin(null, 4, 64, 0.0, null, null, 64, null) == -1
    assert lib.ts_rope_cos_sin(null, 0, 64, 1e6, null, null, 64, null) == 0
    # The decode step's projections: missing operands, an unknown epilogue, strides
    # shorter than a row, a tiled x whose width is not a multiple of 32.
    p = ctypes.c_void_p(16)  # a non-null stand-in; never dereferenced on these paths
    assert lib.ts_rows_gemm(null, 0, 64, p, 64, p, 64, null, 0, 4, 64, 64, 0, 1, null) == -1
    assert lib.ts_rows_gemm(p, 0, 64, p, 64, p, 64, null, 0, 4, 64, 64, 3, 1, null) == -1
    assert lib.ts_rows_gemm(p, 0, 32, p, 64, p, 64, null, 0, 4, 64, 64, 0, 1, null) == -1
    assert lib.ts_rows_gemm(p, 1, 0, p, 48, p, 64, null, 0, 4, 64, 48, 0, 1, null) == -1
    assert lib.ts_rows_gemm(p, 0, 64, p, 64, p, 64, null, 0, 0, 64, 64, 0, 1, null) == 0  # no rows
    # fp32 has no MFMA projection kernel
    assert lib.ts_rows_gemm(p, 0, 64, p, 64, p, 64, null, 0, 4, 64, 64, 0, 0, null) == -2
    assert lib.ts_add_rms_norm(p, 64, null, 2, p, p, 64, p, 0, 64, 4, 64, 1e-6, 1, null) == -1  # ks, no partials
    assert lib.ts_add_rms_norm(p, 32, null, 0, p, p, 64, p, 0, 64, 4, 64, 1e-6, 1, null) == -1  # short stride
    assert lib.ts_add_rms_norm(p, 64, null, 0, p, p, 64, p, 0, 64, 0, 64, 1e-6, 1, null) == 0  # no rows
    out = (ctypes.c_int * 5)()
    assert lib.ts_rows_gemm_plan(64, 4096, 48, 0, out) == -2  # K not a multiple of 32
    assert lib.ts_rows_gemm_plan(64, 4096, 1024, 7, out) == -1


def test_projection_launch_plans(lib: ctypes.CDLL) -> None:
    # The projection kernels' launch shapes at Qwen3-0.6B's sizes (64 rows): sizes only.
    out = (ctypes.c_int * 5)()
    for (n, k, epi), want in {
        (4096, 1024, 0): (8, 1, 4, 1, 1),   # qkv: one K slice, 256 workgroups
        (1024, 2048, 1): (4, 2, 2, 8, 1),   # o_proj: 8 K slices
        (3072, 1024, 2): (8, 2, 4, 1, 1),   # gate_up + SiLU
        (1024, 3072, 1): (8, 2, 2, 6, 1),   # down_proj: 6 K slices
        (64, 96, 2): (1, 2, 1, 1, 3),        # small: one wave, three 32-column chunks
    }.items():
        assert lib.ts_rows_gemm_plan(64, n, k, epi, out) == 0
        assert tuple(out) == want, (n, k, epi, tuple(out))


def test_decode_launch_plans(lib: ctypes.CDLL) -> None:
    # The launch shape is a function of sizes only (MI355X: 256 CUs; without a device the
    # library assumes that count). The metric's B=64 x 4096 streams K/V on length pairs of
    # 8 waves; an explicit count of 4 splits (config 2) runs 4 ranges in the grid's z;
    # head dims without a non-temporal kernel (256) keep cached loads however wide the
    # table; the policy's one launch at config 2 is one 8-wave workgroup per
    # (sequence, head tile).
    plan = hip_attention.decode_plan
    assert plan(64, 16, 8, 128, 16, 256, 1) == {
        "budget": "light_stream", "waves_per_group": 8, "by_length": True, "head_tile": 2,
        "grid": (8, 32, 1), "lds_bytes": 2 * 8 * 2 * 130 * 4}  # fmt: skip
    assert plan(32, 16, 8, 128, 16, 16, 4)["grid"] == (8, 32, 4)
    assert plan(32, 16, 8, 128, 16, 16, 1)["waves_per_group"] == 8
    assert plan(64, 16, 8, 256, 16, 2560, 1)["budget"] == "heavy"
    assert plan(64, 16, 8, 128, 16, 2560, 16)["budget"] == "light_stream"
    assert plan(8, 32, 8, 128, 16, 8, 1, head_tile=1)["head_tile"] == 1
    with pytest.raises(ValueError):
        plan(8, 12, 8, 128, 16, 8, 1)


def test_decode_budget_choices(lib: ctypes.CDLL) -> None:
    # Which register budget a launch runs (sizes only). Streaming launches (K/V bounded by
    # the table width above 256 MiB): light-stream for two-head tiles of 128-element rows,
    # the heavy budget's cached loads for four-head tiles and 64-element rows. Cached
    # launches of two-head 16-bit tiles: light at any walk length; fp32 and four-head
    # tiles keep the walk rule (heavy for long walks on one round of waves).
    plan = hip_attention.decode_plan
    assert plan(64, 16, 8, 128, 16, 256, 1)["budget"] == "light_stream"
    assert plan(64, 32, 8, 128, 16, 256, 1)["budget"] == "heavy"  # four-head tiles
    assert plan(64, 32, 8, 128, 16, 256, 1)["head_tile"] == 4
    assert plan(64, 16, 8, 64, 16, 512, 1)["budget"] == "heavy"  # D=64, 512 MiB bound
    assert plan(64, 16, 8, 128, 16, 64, 1)["budget"] == "light"  # 64 x 1024, cached
    assert plan(16, 16, 8, 128, 16, 128, 1, dtype=torch.bfloat16)["budget"] == "light"
    assert plan(64, 16, 8, 64, 16, 64, 1)["budget"] == "light"  # D=64, cached
    assert plan(64, 32, 8, 128, 16, 64, 1)["budget"] == "heavy"  # four heads, long walks
    assert plan(8, 16, 8, 128, 16, 256, 1, dtype=torch.float32)["budget"] == "heavy"


def test_policy_splits_for_small_grids(lib: ctypes.CDLL) -> None:
    # The launcher's split count with none given (sizes only; 256 CUs assumed without a
    # device): num_splits_for's count, one launch for counts up to 4 on grids of at least
    # half the chip's SIMDs, and more ranges (at most 16 and the table width) for smaller
    # grids.
    def policy(b: int, width: int) -> int:
        return hip_attention.policy_splits(b, 16, 8, 128, 16, width)

    assert policy(64, 256) == 1  # the metric: one launch
    assert policy(32, 16) == 1  # config 2 without a count
    assert policy(1, 2048) == 16  # one long sequence: 16 ranges of partials
    assert policy(8, 256) == 8
    assert policy(16, 128) == 1  # half the chip: one launch


# --- decode entry points: the reference's argument errors (test_triton_attention.py:201-234)


def test_rejects_empty_sequence() -> None:
    c = decode_case([3, 5], 4, 2, head_dim=32)
    c.context_lens[1] = 0
    with pytest.raises(ValueError, match="at least one token"):
        hip_attention.paged_decode_attention(*c.args(), c.scale, c.block_size)


def test_rejects_non_power_of_two_head_dim() -> None:
    c = decode_case([3], 4, 2, head_dim=24)
    with pytest.raises(ValueError, match="power of 2"):
        hip_attention.paged_decode_attention(*c.args(), c.scale, c.block_size)


def test_rejects_int64_block_tables() -> None:
    c = decode_case([3], 4, 2, head_dim=32)
    with pytest.raises(ValueError, match="int32"):
        hip_attention.paged_decode_attention(
            c.q, c.k_cache, c.v_cache, c.block_tables.long(), c.context_lens, c.scale, 16
        )


def test_rejects_heads_that_do_not_group() -> None:
    c = decode_case([3], 6, 4, head_dim=32)
    with pytest.raises(ValueError, match="groups"):
        hip_attention.paged_decode_attention(*c.args(), c.scale, c.block_size)


def test_grouped_kernels_reject_a_group_that_is_not_a_power_of_2() -> None:
    c = decode_case([3], 12, 4, head_dim=32)
    for fn in (hip_attention.paged_decode_attention_grouped, hip_attention.paged_decode_attention_split):
        with pytest.raises(ValueError, match="power-of-2 head group"):
            fn(*c.args(), c.scale, c.block_size)


def test_split_count_out_of_range_is_refused() -> None:  # test_kernel_variants.py:67-71
    c = decode_case([20], head_dim=32, block_size=4)
    for bad in (-1, hip_attention.MAX_SPLITS + 1):
        with pytest.raises(ValueError, match="num_splits"):
            hip_attention.launch_paged_decode_split(*c.args(), c.scale, c.block_size, num_splits=bad)


@pytest.mark.parametrize("tile", [(3, 4), (2, 3), (0, 4)])
def test_rejects_a_tile_that_is_not_powers_of_2(tile: tuple[int, int]) -> None:
    c = decode_case([3], 4, 2, head_dim=32, block_size=4)
    with pytest.raises(ValueError, match="powers of 2"):
        hip_attention.launch_paged_decode_split(*c.args(), c.scale, c.block_size, 2, tile)
    with pytest.raises(ValueError, match="powers of 2"):
        hip_attention.launch_paged_decode_grouped(*c.args(), c.scale, c.block_size, tile)


def test_cpu_tensors_are_refused_not_computed() -> None:
    c = decode_case([3, 9], 4, 2, head_dim=32)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        hip_attention.paged_decode_attention_split(*c.args(), c.scale, c.block_size)
    p = prefill_case([(0, 5)])
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        hip_prefill.paged_prefill_attention(*p.args())
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        hip_fused.rms_norm_rows(torch.randn(2, 16), torch.randn(16), 1e-6)


def test_split_policy_tables() -> None:
    # The reference's T4 policy, reproduced exactly with its constants
    # (test_triton_attention.py:240-249) ...
    t4 = {"target": hip_attention.T4_TARGET_PROGRAMS, "no_split": hip_attention.T4_NO_SPLIT_PROGRAMS}
    batches = (1, 2, 4, 8, 10, 16, 24, 31, 32, 64)
    assert [hip_attention.num_splits_for(b, 8, 64, **t4) for b in batches] == [
        16, 16, 16, 16, 13, 8, 6, 5, 1, 1]  # fmt: skip
    assert hip_attention.num_splits_for(1, 8, 4, **t4) == 4
    assert hip_attention.num_splits_for(1, 1, 64, **t4) == hip_attention.MAX_SPLITS
    assert hip_attention.num_splits_for(256, 1, 64, **t4) == 1
    # ... and the MI355X default: about 256 workgroups, never more than the table width.
    assert [hip_attention.num_splits_for(b, 8, 256) for b in (1, 8, 16, 32, 64, 512)] == [
        16, 4, 2, 1, 1, 1]  # fmt: skip
    assert hip_attention.num_splits_for(1, 8, 4) == 4


# --- prefill and fused argument errors (test_triton_prefill.py:173-185,
#     test_triton_fused.py:53-59, :102-111)


def test_prefill_rejects_bad_arguments() -> None:
    case = prefill_case([(0, 5)])
    args = case.args()
    with pytest.raises(ValueError):
        hip_prefill.paged_prefill_attention(*args, rows_per_tile=8)
    with pytest.raises(ValueError):
        hip_prefill.paged_prefill_attention(*args, block_n=24)
    q3 = case.q[:, :3].contiguous()
    with pytest.raises(ValueError):
        hip_prefill.paged_prefill_attention(q3, case.k, case.v, case.tables, case.starts,
                                            case.q_lens, case.ctx_lens, 1.0, 4, 5)  # fmt: skip
    with pytest.raises(ValueError):
        hip_prefill.paged_prefill_attention(case.q, case.k, case.v, case.tables, case.starts.long(),
                                            case.q_lens, case.ctx_lens, 1.0, 4, 5)  # fmt: skip


def test_rms_norm_rows_of_nothing_and_bad_shapes() -> None:
    assert hip_fused.rms_norm_rows(torch.randn(0, 16), torch.randn(16), 1e-6).shape == (0, 16)
    with pytest.raises(ValueError):
        hip_fused.rms_norm_rows(torch.randn(2, 3, 16), torch.randn(16), 1e-6)
    with pytest.raises(ValueError):
        hip_fused.rms_norm_rows(torch.randn(2, 16), torch.randn(8), 1e-6)


def test_qk_norm_rope_store_rejects_bad_shapes() -> None:
    t, hq, hkv, d = 3, 4, 2, 8
    q, k, v = torch.randn(t, hq, d), torch.randn(t, hkv, d), torch.randn(t, hkv, d)
    w = torch.randn(d)
    cos = sin = torch.randn(t, d)
    slots = torch.arange(t)
    kc = vc = torch.randn(16, hkv, d)
    with pytest.raises(ValueError):  # v with the wrong number of heads
        hip_fused.qk_norm_rope_store(q, k, q, w, w, cos, sin, slots, kc, vc, 1e-6)
    with pytest.raises(ValueError):  # tables for the wrong number of tokens
        hip_fused.qk_norm_rope_store(q, k, v, w, w, cos[:2], sin[:2], slots, kc, vc, 1e-6)
