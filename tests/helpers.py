"""Tolerances and comparison helpers shared by the GPU parity tests.

Tolerance policy (the reference's, tests/test_triton_attention.py:6-11, extended to bf16
with the north-star bound of 2e-3). ``ref32`` is always the oracle's float32 result
computed from the same inputs, before its final rounding to the kernel's dtype:

    float32   atol = rtol = 1e-5 (torch.testing.assert_close);
    float16   |out - ref32| <= 1e-3 + 1e-3 |ref32| + 2^-11 |ref32|;
    bfloat16  |out - ref32| <= 2e-3 + 2e-3 |ref32| + 2^-8 |ref32|.

The last term is the output format's own rounding, at most half an ulp (2^-11 relative
for fp16, 2^-8 for bf16): a 16-bit output cannot be closer than that to the float32
value, and for bf16 half an ulp exceeds 2e-3 already at |x| = 0.5. Kernels whose
numerics contract rounds an intermediate to the input dtype (RMSNorm rounds x/rms
before the weight multiply, layers.py:34-38) may land that intermediate on the other
neighbour when their float32 sum of squares differs in the last bit from PyTorch's
(summation order); callers pass that allowance, one intermediate ulp propagated to the
output, as ``extra``.
"""

from __future__ import annotations

import torch

TOL = {torch.float32: 1e-5, torch.float16: 1e-3, torch.bfloat16: 2e-3}
HALF_ULP = {torch.float32: 0.0, torch.float16: 2.0**-11, torch.bfloat16: 2.0**-8}
ULP = {torch.float32: 2.0**-23, torch.float16: 2.0**-10, torch.bfloat16: 2.0**-7}


def assert_matches(
    out: torch.Tensor,
    ref32: torch.Tensor,
    dtype: torch.dtype,
    msg: str = "",
    extra: torch.Tensor | None = None,
) -> None:
    """``out`` (kernel result, any device) against ``ref32`` (oracle, float32)."""
    out = out.detach().cpu()
    ref32 = ref32.detach().cpu().float()
    assert out.dtype == dtype, (out.dtype, dtype)
    assert out.shape == ref32.shape, (out.shape, ref32.shape)
    tol = TOL[dtype]
    o = out.float()
    bound = tol + (tol + HALF_ULP[dtype]) * ref32.abs()
    if extra is not None:
        bound = bound + extra.detach().cpu().float()
    err = (o - ref32).abs()
    bad = ~(err <= bound)
    if bool(bad.any()):
        i = int(bad.flatten().nonzero()[0])
        raise AssertionError(
            f"{msg}: {int(bad.sum())} of {bad.numel()} elements outside the {dtype} bound "
            f"(max err {float(err.max()):.3g}); first at flat index {i}: "
            f"got {o.flatten()[i].item()!r}, want {ref32.flatten()[i].item()!r}"
        )


# The north-star contract: max-abs error against the reference's float32 math.
CONTRACT = {torch.float32: 1e-5, torch.float16: 2e-3, torch.bfloat16: 2e-3}


def assert_contract(
    out: torch.Tensor,
    ref32: torch.Tensor,
    dtype: torch.dtype,
    msg: str = "",
    extra: torch.Tensor | None = None,
) -> float:
    """Max-abs error of ``out`` against ``ref32`` within the contract (1e-5 float32,
    2e-3 float16), on top of ``assert_matches``; returns the max-abs error, which is
    printed. bfloat16 keeps the half-ulp allowance of ``assert_matches`` only: half an
    ulp of a bf16 output in [1, 2) is 3.9e-3, above 2e-3 whatever the kernel does.

    ``extra`` (kernels that round an intermediate to the input dtype, as RMSNorm rounds
    x/rms) is the one-ulp allowance of that intermediate: an element may exceed the
    contract by no more than it, which is the intermediate landing on the other
    neighbour of a near-tie, and such elements must be rare (at most 1 in 10^4)."""
    assert_matches(out, ref32, dtype, msg, extra)
    o = out.detach().cpu().float()
    r = ref32.detach().cpu().float()
    err = (o - r).abs()
    worst = float(err.max()) if err.numel() else 0.0
    print(f"[contract] {msg or 'result'} {dtype}: max-abs {worst:.3g} (bound {CONTRACT[dtype]:.0e})")
    if dtype == torch.bfloat16 or not err.numel():
        return worst
    bound = torch.full_like(err, CONTRACT[dtype])
    if extra is not None:
        over = err > bound
        assert int(over.sum()) <= max(1, err.numel() // 10_000), (
            f"{msg}: {int(over.sum())} of {err.numel()} elements above the contract's {CONTRACT[dtype]:.0e}"
        )
        bound = bound + extra.detach().cpu().float()
    bad = ~(err <= bound)
    if bool(bad.any()):
        i = int(bad.flatten().nonzero()[0])
        raise AssertionError(
            f"{msg}: max-abs {worst:.3g} above the contract's {CONTRACT[dtype]:.0e} for {dtype} "
            f"({int(bad.sum())} elements; first at flat index {i}: got {o.flatten()[i].item()!r}, "
            f"want {r.flatten()[i].item()!r})"
        )
    return worst


def max_abs_err(out: torch.Tensor, ref32: torch.Tensor) -> float:
    return float((out.detach().cpu().float() - ref32.detach().cpu().float()).abs().max())
