"""The oracle against the golden fixtures of tests/golden/ (float64 brute force written
independently of the oracle; see tests/golden/make_golden.py)."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

from oracle import ref

GOLDEN = Path(__file__).resolve().parent / "golden"


def load(name: str) -> dict[str, np.ndarray]:
    with np.load(GOLDEN / f"{name}.npz") as z:  # allow_pickle stays False
        return {k: z[k] for k in z.files}


def t(x: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(x))


def test_decode_oracle_matches_golden() -> None:
    g = load("decode")
    d = g["q"].shape[-1]
    out = ref.decode_ref(t(g["q"]), t(g["k_cache"]), t(g["v_cache"]), t(g["block_tables"]),
                         t(g["context_lens"]), d**-0.5, int(g["block_size"]))  # fmt: skip
    assert torch.isfinite(out).all()
    torch.testing.assert_close(out.double(), t(g["out"]), atol=1e-5, rtol=1e-5)


def test_prefill_oracle_matches_golden() -> None:
    g = load("prefill")
    d = g["q"].shape[-1]
    out = ref.prefill_ref(t(g["q"]), t(g["k_cache"]), t(g["v_cache"]), t(g["block_tables"]),
                          t(g["q_starts"]), t(g["q_lens"]), t(g["context_lens"]), d**-0.5,
                          int(g["block_size"]))  # fmt: skip
    torch.testing.assert_close(out.double(), t(g["out"]), atol=1e-5, rtol=1e-5)


def test_fused_oracle_matches_golden() -> None:
    g = load("fused")
    eps = float(g["eps"])
    torch.testing.assert_close(ref.rms_norm(t(g["x"]), t(g["w"]), eps).double(), t(g["x_out"]),
                               atol=1e-5, rtol=1e-5)  # fmt: skip
    d = g["q"].shape[-1]
    cos, sin = ref.rope_cos_sin(d, float(g["theta"]), t(g["positions"]))
    torch.testing.assert_close(cos.double(), t(g["cos"]), atol=1e-7, rtol=0)
    torch.testing.assert_close(sin.double(), t(g["sin"]), atol=1e-7, rtol=0)
    kc = torch.full((4 * g["q"].shape[0], g["k"].shape[1], d), float("nan"))
    vc = kc.clone()
    slots = t(g["slots"])
    q_out = ref.qk_norm_rope_store_ref(t(g["q"]), t(g["k"]), t(g["v"]), t(g["q_w"]), t(g["k_w"]),
                                       cos, sin, slots, kc, vc, eps)  # fmt: skip
    torch.testing.assert_close(q_out.double(), t(g["q_out"]), atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(kc[slots].double(), t(g["k_out"]), atol=1e-5, rtol=1e-5)
    assert torch.equal(vc[slots], t(g["v"]))
