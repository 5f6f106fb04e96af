"""The HIP fused norm / RoPE / KV-write kernels must match the oracle (GPU).

Mirrors the reference's tests/test_triton_fused.py: ``rms_norm_rows`` against
``rms_norm`` (including x300 inputs whose squares overflow fp16), and
``qk_norm_rope_store`` against ``apply_rope(rms_norm(.))`` + ``KVCache.write`` with the v
scatter exact (atol = rtol = 0) and every other cache slot still NaN. Tolerances:
tests/helpers.py; the slot placement and the v copy are compared bit for bit.
"""

from __future__ import annotations

import pytest
import torch

from oracle import ref
from tests.helpers import ULP, assert_contract, assert_matches
from tinyserve_amd.hip_fused import qk_norm_rope_store, rms_norm_rows, rope_cos_sin
from tinyserve_amd.workloads import fused_case

pytestmark = pytest.mark.gpu
DEVICE = "cuda"
EPS = 1e-6
DTYPES = [torch.float32, torch.float16, torch.bfloat16]


def randn(*shape: int, dtype: torch.dtype = torch.float32, scale: float = 1.0) -> torch.Tensor:
    return (torch.randn(shape) * scale).to(dtype)


def rms32(x: torch.Tensor, w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """The oracle's rms_norm before its final rounding (the in-dtype weight multiply is
    exact in fp32 for 16-bit inputs), and the allowance for the intermediate rounding of
    x/rms: one ulp of it, times |w|."""
    xf = x.float()
    xn = xf * torch.rsqrt(xf.square().mean(-1, keepdim=True) + EPS)
    return xn.to(x.dtype).float() * w.float(), ULP[x.dtype] * xn.abs() * w.float().abs()


@pytest.mark.parametrize("n", [16, 24, 1024, 4096, 5000])
@pytest.mark.parametrize("dtype", DTYPES)
def test_rms_norm_rows_equals_rms_norm(n: int, dtype: torch.dtype) -> None:
    torch.manual_seed(n)
    x = randn(7, n, dtype=dtype, scale=300.0)  # 300**2 overflows fp16: must upcast first
    w = randn(n, dtype=dtype)
    got = rms_norm_rows(x.to(DEVICE), w.to(DEVICE), EPS)
    assert got.dtype == dtype and torch.isfinite(got).all()
    want, extra = rms32(x, w)
    assert_matches(got, want, dtype, extra=extra)


def test_rms_norm_rows_strided_rows() -> None:
    x = randn(6, 2048, dtype=torch.float16)[:, :1024]  # row stride 2048
    w = randn(1024, dtype=torch.float16)
    got = rms_norm_rows(x.to(DEVICE), w.to(DEVICE), EPS)
    want, extra = rms32(x, w)
    assert_matches(got, want, torch.float16, extra=extra)


def qk_case(t: int, hq: int, hkv: int, d: int, dtype: torch.dtype, seed: int = 0) -> dict[str, torch.Tensor]:
    torch.manual_seed(seed)
    num_slots = 4 * t + 8
    return {
        "q": randn(t, hq, d, dtype=dtype, scale=30.0),
        "k": randn(t, hkv, d, dtype=dtype, scale=30.0),
        "v": randn(t, hkv, d, dtype=dtype),
        "qw": randn(d, dtype=dtype),
        "kw": randn(d, dtype=dtype),
        "pos": torch.randint(0, 40_000, (t,)),
        "slots": torch.randperm(num_slots)[:t],
        "k_cache": torch.full((num_slots, hkv, d), float("nan"), dtype=dtype),
        "v_cache": torch.full((num_slots, hkv, d), float("nan"), dtype=dtype),
    }


def rope32(x: torch.Tensor, w: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor):
    """apply_rope(rms_norm(x)) before its final rounding, and the allowance for the
    normalised intermediate's rounding: one ulp of each element of a rotate-half pair."""
    n = ref.rms_norm(x, w, EPS).float()
    h = n.shape[-1] // 2
    e = ULP[x.dtype] * (n[..., :h].abs() + n[..., h:].abs())
    return ref.apply_rope(n, cos, sin), torch.cat([e, e], dim=-1)


def run_qk(c: dict[str, torch.Tensor], cos: torch.Tensor, sin: torch.Tensor) -> tuple[torch.Tensor, ...]:
    g = {k: v.to(DEVICE) for k, v in c.items()}
    q = qk_norm_rope_store(g["q"], g["k"], g["v"], g["qw"], g["kw"], cos.to(DEVICE), sin.to(DEVICE),
                           g["slots"], g["k_cache"], g["v_cache"], EPS)  # fmt: skip
    return q.cpu(), g["k_cache"].cpu(), g["v_cache"].cpu()


@pytest.mark.parametrize(("hq", "hkv", "d"), [(4, 2, 8), (4, 4, 16), (16, 8, 128), (8, 2, 64), (4, 1, 256)])
@pytest.mark.parametrize("dtype", DTYPES)
def test_qk_norm_rope_store_equals_the_pytorch_ops(hq: int, hkv: int, d: int, dtype: torch.dtype) -> None:
    c = qk_case(9, hq, hkv, d, dtype, seed=d)
    cos, sin = ref.rope_cos_sin(d, 1e6, c["pos"])
    q, kc, vc = run_qk(c, cos, sin)
    want_q, extra_q = rope32(c["q"], c["qw"], cos, sin)
    want_k, extra_k = rope32(c["k"], c["kw"], cos, sin)
    assert_matches(q, want_q, dtype, "q", extra_q)
    assert_matches(kc[c["slots"]], want_k, dtype, "k", extra_k)
    assert torch.equal(vc[c["slots"]], c["v"])  # the v scatter is an exact copy
    others = torch.ones(kc.shape[0], dtype=torch.bool)
    others[c["slots"]] = False
    assert kc[others].isnan().all() and vc[others].isnan().all()


def test_qk_norm_rope_store_into_a_float32_cache() -> None:
    # KVCache.write casts to the cache dtype: k after its rounding to k's dtype, v as is.
    c = qk_case(5, 4, 2, 64, torch.float16, seed=3)
    c["k_cache"] = c["k_cache"].float()
    c["v_cache"] = c["v_cache"].float()
    cos, sin = ref.rope_cos_sin(64, 1e6, c["pos"])
    _, kc, vc = run_qk(c, cos, sin)
    # fp16 k rounded once more to the (float32) cache: exactly the fp16 value.
    want_k, extra_k = rope32(c["k"], c["kw"], cos, sin)
    got_k = kc[c["slots"]]
    assert torch.equal(got_k, got_k.half().float())
    assert_matches(got_k.half(), want_k, torch.float16, "k", extra_k)
    assert torch.equal(vc[c["slots"]], c["v"].float())


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_baseline_config_4(dtype: torch.dtype) -> None:
    # T=4096, hidden 1024, q/k/v as strided views of the QKV
    # projection output, an injective slot map into a 512 x 16 pool; scatter bit-exact.
    # Values within the contract's max-abs bound (fp16 2e-3), except where the rounding
    # of x/rms to the input dtype (layers.py:34-38) lands on the other neighbour of a
    # near-tie: one ulp of that intermediate, rare, allowed by ``extra``.
    cpu = fused_case(dtype=dtype, device="cpu")
    dev = fused_case(dtype=dtype, device=DEVICE)
    x = rms_norm_rows(dev.x, dev.norm_w, dev.eps)
    want, extra = rms32(cpu.x, cpu.norm_w)
    assert_contract(x, want, dtype, "config 4 rms_norm_rows", extra)
    q = qk_norm_rope_store(dev.q, dev.k, dev.v, dev.q_w, dev.k_w, dev.cos, dev.sin, dev.slots,
                           dev.k_cache, dev.v_cache, dev.eps)  # fmt: skip
    want_q, extra_q = rope32(cpu.q, cpu.q_w, cpu.cos, cpu.sin)
    assert_contract(q, want_q, dtype, "config 4 q", extra_q)
    kc, vc = dev.k_cache.cpu(), dev.v_cache.cpu()
    want_k, extra_k = rope32(cpu.k, cpu.k_w, cpu.cos, cpu.sin)
    assert_contract(kc[cpu.slots], want_k, dtype, "config 4 k", extra_k)
    assert torch.equal(vc[cpu.slots], cpu.v)
    # Placement: the oracle's KVCache.write of the kernel's own k rows lands bit-identically.
    kc_ref = torch.full_like(kc, float("nan"))
    vc_ref = torch.full_like(vc, float("nan"))
    ref.kv_write(kc_ref, vc_ref, cpu.slots, kc[cpu.slots], cpu.v)
    assert torch.equal(kc.isnan(), kc_ref.isnan()) and torch.equal(vc.isnan(), vc_ref.isnan())
    assert torch.equal(torch.nan_to_num(kc), torch.nan_to_num(kc_ref))
    assert torch.equal(torch.nan_to_num(vc), torch.nan_to_num(vc_ref))


@pytest.mark.parametrize("head_dim", [2, 64, 128, 256])
@pytest.mark.parametrize("theta", [10_000.0, 1_000_000.0])
def test_rope_cos_sin_equals_the_reference_tables(head_dim: int, theta: float) -> None:
    # layers.py:41-65 in float64 on the CPU (the oracle) against the one-launch kernel:
    # the same float64 angles, cos / sin rounded once to float32. Both libms are within
    # an ulp of float64, so a table entry may differ only where the float64 result lies
    # within that of a float32 rounding boundary: at most one float32 ulp, rarely.
    g = torch.Generator().manual_seed(head_dim)
    pos = torch.cat([torch.arange(0, 70), torch.randint(0, 40960, (500,), generator=g), torch.tensor([40959])])
    want_c, want_s = ref.rope_cos_sin(head_dim, theta, pos)
    got_c, got_s = rope_cos_sin(head_dim, theta, pos.to(DEVICE))
    for got, want in ((got_c.cpu(), want_c), (got_s.cpu(), want_s)):
        assert got.shape == want.shape == (pos.numel(), head_dim) and got.dtype == torch.float32
        assert torch.equal(got[:, : head_dim // 2], got[:, head_dim // 2 :])
        diff = got != want
        ulp = torch.finfo(torch.float32).eps * want.abs().clamp_min(2.0**-126)
        assert bool(((got - want).abs() <= ulp).all())
        assert int(diff.sum()) <= max(1, want.numel() // 10_000), int(diff.sum())


def test_rope_cos_sin_rejects_bad_arguments() -> None:
    with pytest.raises(ValueError, match="int64"):
        rope_cos_sin(64, 1e6, torch.arange(4, dtype=torch.int32, device=DEVICE))
    with pytest.raises(ValueError, match="even"):
        rope_cos_sin(63, 1e6, torch.arange(4, device=DEVICE))
    c, s = rope_cos_sin(64, 1e6, torch.empty(0, dtype=torch.int64, device=DEVICE))
    assert c.shape == s.shape == (0, 64)
