"""The decode step's projection kernels (``hip_rows``) against PyTorch's own ops in fp32.

The reference computes these with F.linear, F.silu and the residual ``x + ...``
(src/tinyserve/model.py:137-179); no kernel of the reference corresponds, so each output
is compared with the same op evaluated in float32 and rounded as the reference's op
rounds: a projection within half an output ulp plus the fp32 summation-order term
``2^-22 * K * sum|x w|`` (a different order of the same fp32 sums), the residual add and
RMSNorm bit for bit with ``rms_norm_rows`` on the same residual.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from tests.helpers import ULP
from tinyserve_amd.hip_fused import rms_norm_rows
from tinyserve_amd.hip_rows import (ROWS_PARTIAL, ROWS_SILU, ROWS_STORE, Tiled, add_rms_norm, padded_rows,
                                    rows_linear, rows_linear_partials, rows_plan, rows_silu_gate_up)  # fmt: skip

DEVICE = "cuda"
EPS = 1e-6
DTYPES = [torch.float16, torch.bfloat16]
# (N, K) of Qwen3-0.6B's projections (qkv, o_proj, down_proj) and of a small model.
SHAPES = [(4096, 1024), (1024, 2048), (1024, 3072), (512, 256), (256, 512), (96, 64)]
ROWS = [1, 7, 64, 65, 130]


def operands(m: int, n: int, k: int, dtype: torch.dtype, seed: int = 0) -> tuple[torch.Tensor, torch.Tensor]:
    g = torch.Generator().manual_seed(seed * 1000 + m * 7 + n + k)
    x = torch.randn(m, k, generator=g).to(dtype)
    w = (torch.randn(n, k, generator=g) * 0.02).to(dtype)
    return x.to(DEVICE), w.to(DEVICE)


def linear32(x: torch.Tensor, w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """x . w^T in float64 (as float32), and the fp32 summation-order allowance."""
    ref = (x.double() @ w.double().t()).float()
    order = 2.0**-22 * x.shape[1] * (x.double().abs() @ w.double().abs().t()).float()
    return ref, order


def padding_rows(t: Tiled) -> torch.Tensor:
    """Rows ``t.rows ..`` of the padded matrix a Tiled buffer holds."""
    return Tiled(t.buf, padded_rows(t.rows), t.cols).to_dense()[t.rows :]


# ---- layout (CPU) ---------------------------------------------------------------------------
@pytest.mark.parametrize(("m", "k"), [(1, 32), (64, 64), (65, 96), (130, 1024)])
def test_tiled_layout_round_trip_and_index_formula(m: int, k: int) -> None:
    x = torch.arange(m * k, dtype=torch.float32).view(m, k).to(torch.float16 if m * k < 2048 else torch.float32)
    t = Tiled.from_dense(x)
    assert t.buf.numel() == padded_rows(m) * k
    assert torch.equal(t.to_dense(), x)
    # The documented formula, element by element on a sample of positions.
    for mm, kk in [(0, 0), (m - 1, k - 1), (m // 2, k // 3), (min(m - 1, 17), min(k - 1, 40))]:
        idx = ((((mm // 64) * (k // 32) + kk // 32) * 4 + (mm % 64) // 16) * 64 + ((kk % 32) // 8) * 16 + mm % 16) * 8 + kk % 8
        assert t.buf[idx] == x[mm, kk]
    assert torch.equal(padding_rows(t), torch.zeros_like(padding_rows(t)))


def test_tiled_needs_32_column_multiples() -> None:
    with pytest.raises(ValueError, match="multiple of 32"):
        Tiled.empty(4, 48, torch.float16, torch.device("cpu"))


# ---- projections (GPU) ------------------------------------------------------------------------
@pytest.mark.gpu
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize(("n", "k"), SHAPES)
@pytest.mark.parametrize("m", ROWS)
@pytest.mark.parametrize("tiled", [False, True])
def test_rows_linear_equals_f_linear(m: int, n: int, k: int, dtype: torch.dtype, tiled: bool) -> None:
    x, w = operands(m, n, k, dtype)
    got = rows_linear(Tiled.from_dense(x) if tiled else x, w)
    assert got.shape == (m, n) and got.dtype == dtype
    ref, order = linear32(x, w)
    err = (got.float() - ref).abs()
    bound = ULP[dtype] / 2 * ref.abs() + order + 1e-30
    print(f"[rows_linear] m={m} n={n} k={k} {dtype} tiled={tiled} max_abs={err.max().item():.3g}")
    assert bool((err <= bound).all()), (err - bound).max().item()


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize(("n", "k"), SHAPES)
@pytest.mark.parametrize("m", ROWS)
def test_partials_sum_to_f_linear(m: int, n: int, k: int, dtype: torch.dtype) -> None:
    x, w = operands(m, n, k, dtype, seed=1)
    part, ks = rows_linear_partials(x, w)
    assert part.shape == (ks, m, n) and ks == rows_plan(m, n, k, ROWS_PARTIAL)["k_splits"]
    ref, order = linear32(x, w)
    err = (part.sum(0) - ref).abs()
    print(f"[partials] m={m} n={n} k={k} ks={ks} max_abs={err.max().item():.3g}")
    assert bool((err <= order + 1e-30).all())


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize(("n", "k"), [(3072, 1024), (512, 256), (64, 96)])
@pytest.mark.parametrize("m", [1, 33, 64, 100])
def test_silu_gate_up_equals_torch(m: int, n: int, k: int, dtype: torch.dtype) -> None:
    x, w = operands(m, 2 * n, k, dtype, seed=2)
    got = rows_silu_gate_up(Tiled.from_dense(x), w)
    assert (got.rows, got.cols) == (m, n)
    ref, order = linear32(x, w)
    # The reference's ops on the gate / up sums: F.linear rounds, F.silu rounds, * rounds.
    gate, up = ref[:, :n], ref[:, n:]
    want = (F.silu(gate.to(dtype).float()).to(dtype).float() * up.to(dtype).float())
    dense = got.to_dense().float()
    # A gate or up sum within the summation-order term of a rounding boundary may round
    # the other way: one ulp of gate (carried through silu, slope < 1.1, and silu's own
    # rounding) or of up, times the other factor.
    slack = ULP[dtype] * up.abs() * (3.5 * gate.abs() + 1.0) + 2 * (order[:, :n] + order[:, n:])
    err = (dense - want).abs()
    bound = ULP[dtype] / 2 * want.abs() + slack + 1e-30
    print(f"[silu] m={m} n={n} k={k} {dtype} max_abs={err.max().item():.3g}")
    assert bool((err <= bound).all()), (err - bound).max().item()
    assert torch.equal(padding_rows(got), torch.zeros_like(padding_rows(got)))


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("n", [256, 1024, 4096])
@pytest.mark.parametrize("m", [1, 64, 70])
@pytest.mark.parametrize("ks", [0, 1, 6])
@pytest.mark.parametrize("tiled", [False, True])
def test_add_rms_norm_is_the_residual_add_then_rms_norm_rows(m: int, n: int, ks: int, dtype: torch.dtype,
                                                             tiled: bool) -> None:  # fmt: skip
    g = torch.Generator().manual_seed(m * 31 + n + ks)
    x0 = (torch.randn(m, n, generator=g) * 3).to(dtype).to(DEVICE)
    w = torch.randn(n, generator=g).to(dtype).to(DEVICE)
    part = (torch.randn(ks, m, n, generator=g) * 2).to(DEVICE) if ks else None
    x = x0.clone()
    h = add_rms_norm(x, part, w, EPS, tiled=tiled)
    if ks:
        s = part[0].clone()
        for z in range(1, ks):
            s += part[z]
        want_x = (s.to(dtype).float() + x0.float()).to(dtype)
    else:
        want_x = x0
    assert torch.equal(x, want_x), "the residual add: sum of partials in order rounded, plus x, rounded (model.py:172,179)"
    dense = h.to_dense() if tiled else h
    assert torch.equal(dense, rms_norm_rows(want_x, w, EPS)), "RMSNorm as rms_norm_rows computes it"
    if tiled:
        assert torch.equal(padding_rows(h), torch.zeros_like(padding_rows(h)))


@pytest.mark.gpu
def test_plans_at_the_qwen3_shapes() -> None:
    """The launch shapes the kernel comments quote for 64 rows."""
    assert rows_plan(64, 4096, 1024, ROWS_STORE) == {"waves": 8, "tiles_per_wave": 1, "steps": 4, "k_splits": 1, "chunks": 1}
    assert rows_plan(64, 1024, 2048, ROWS_PARTIAL) == {"waves": 4, "tiles_per_wave": 2, "steps": 2, "k_splits": 8, "chunks": 1}
    assert rows_plan(64, 3072, 1024, ROWS_SILU) == {"waves": 8, "tiles_per_wave": 2, "steps": 4, "k_splits": 1, "chunks": 1}
    assert rows_plan(64, 1024, 3072, ROWS_PARTIAL) == {"waves": 8, "tiles_per_wave": 2, "steps": 2, "k_splits": 6, "chunks": 1}


@pytest.mark.gpu
def test_arguments_are_checked() -> None:
    x, w = operands(4, 64, 64, torch.float16)
    with pytest.raises(ValueError, match="columns"):
        rows_linear(x, w[:, :32].contiguous())
    with pytest.raises(ValueError, match="dtype"):
        rows_linear(x.float(), w.float())
    with pytest.raises(ValueError, match="dtype"):
        add_rms_norm(x, None, w[0].float(), EPS)
    with pytest.raises(ValueError, match="KS"):
        add_rms_norm(x, torch.zeros(2, 4, 32, device=DEVICE), w[0], EPS)
    # Caller-provided outputs must be exactly what the kernel writes.
    with pytest.raises(ValueError, match="out must be"):
        rows_linear(x, w, out=torch.empty(4, 32, dtype=torch.float16, device=DEVICE))
    with pytest.raises(ValueError, match="out must be"):
        rows_linear(x, w, out=torch.empty(4, 64, dtype=torch.float32, device=DEVICE))
    with pytest.raises(ValueError, match="partial"):
        rows_linear_partials(x, w, torch.empty(4 * 64 * 16, dtype=torch.float16, device=DEVICE))
    with pytest.raises(ValueError, match="Tiled"):
        rows_silu_gate_up(x, w, out=torch.empty(4, 32, dtype=torch.float16, device=DEVICE))
    with pytest.raises(ValueError, match="operand-tiled"):
        rows_silu_gate_up(x, w, out=Tiled.empty(4, 64, torch.float16, torch.device(DEVICE)))
    with pytest.raises(ValueError, match="h must be"):
        add_rms_norm(x, None, w[0], EPS, tiled=True, h=torch.empty_like(x))
    with pytest.raises(ValueError, match="h must be"):
        add_rms_norm(x, None, w[0], EPS, tiled=True, h=Tiled.empty(8, 64, torch.float16, torch.device(DEVICE)))


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(12))
def test_random_shapes_through_every_epilogue(seed: int) -> None:
    # Seeded sizes that reach the planner's other shapes (one-wave workgroups, several K
    # chunks per workgroup, uneven K splits): rows 1..200, N a multiple of 32, K of 32.
    g = torch.Generator().manual_seed(1000 + seed)
    m = int(torch.randint(1, 201, (1,), generator=g))
    n = 32 * int(torch.randint(1, 65, (1,), generator=g))
    k = 32 * int(torch.randint(1, 97, (1,), generator=g))
    dtype = DTYPES[seed % 2]
    x, w = operands(m, n, k, dtype, seed=seed)
    ref, order = linear32(x, w)
    plans = {e: rows_plan(m, n, k, e) for e in (ROWS_STORE, ROWS_PARTIAL)}
    print(f"[random] m={m} n={n} k={k} {dtype} plans={plans}")
    got = rows_linear(x if seed % 3 else Tiled.from_dense(x), w)
    assert bool(((got.float() - ref).abs() <= ULP[dtype] / 2 * ref.abs() + order + 1e-30).all())
    part, ks = rows_linear_partials(Tiled.from_dense(x) if seed % 3 else x, w)
    assert bool(((part.sum(0) - ref).abs() <= order + 1e-30).all())
    # The SiLU epilogue on [gate; up] = the first and second half of w's rows.
    half = n // 2
    if half % 32 == 0:
        act = rows_silu_gate_up(Tiled.from_dense(x), w).to_dense().float()
        gate, up = ref[:, :half], ref[:, half:]
        want = F.silu(gate.to(dtype).float()).to(dtype).float() * up.to(dtype).float()
        slack = ULP[dtype] * up.abs() * (3.5 * gate.abs() + 1.0) + 2 * (order[:, :half] + order[:, half:])
        assert bool(((act - want).abs() <= ULP[dtype] / 2 * want.abs() + slack + 1e-30).all())


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(8))
def test_add_rms_norm_random_widths_and_partial_counts(seed: int) -> None:
    # Widths up to 4096 (8 chunks of 8 per lane) and up to 16 partials: the partial loads
    # then take several groups; the result stays the ordered sum and rms_norm_rows.
    g = torch.Generator().manual_seed(2000 + seed)
    m = int(torch.randint(1, 150, (1,), generator=g))
    n = 32 * int(torch.randint(1, 129, (1,), generator=g))
    ks = int(torch.randint(0, 17, (1,), generator=g))
    dtype = DTYPES[seed % 2]
    x0 = (torch.randn(m, n, generator=g) * 2).to(dtype).to(DEVICE)
    w = torch.randn(n, generator=g).to(dtype).to(DEVICE)
    part = torch.randn(ks, m, n, generator=g).to(DEVICE) if ks else None
    x = x0.clone()
    h = add_rms_norm(x, part, w, EPS, tiled=bool(seed % 2))
    want_x = x0
    if ks:
        s = part[0].clone()
        for z in range(1, ks):
            s += part[z]
        want_x = (s.to(dtype).float() + x0.float()).to(dtype)
    print(f"[add_rms random] m={m} n={n} ks={ks} {dtype}")
    assert torch.equal(x, want_x)
    dense = h.to_dense() if seed % 2 else h
    assert torch.equal(dense, rms_norm_rows(want_x, w, EPS))
