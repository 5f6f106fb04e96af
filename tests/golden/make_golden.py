"""Write the golden fixtures in this folder: seeded inputs plus expected outputs computed
by a float64 brute force in numpy, written independently of ``oracle/ref.py`` (explicit
loops over positions, slots from the block-table formula of the reference's
src/tinyserve/block_table.py:74-82, scores/softmax/weighted sums of
src/tinyserve/attention.py:62-141, RMSNorm and RoPE of src/tinyserve/layers.py:14-91).

The reference's own tests hold no stored vectors for this path (they draw seeded inputs
at run time), so these fixtures pin the oracle against a second implementation.

    python tests/golden/make_golden.py     # rewrites decode.npz, prefill.npz, fused.npz
"""

from __future__ import annotations

import math
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent


def slot(table: np.ndarray, pos: int, bs: int) -> int:
    return int(table[pos // bs]) * bs + pos % bs


def attend_one(qv: np.ndarray, kc: np.ndarray, vc: np.ndarray, slots: list[int], kvh: int, scale: float) -> np.ndarray:
    """softmax over keys of q.k * scale, then the weighted sum of v, all float64."""
    scores = np.array([float(np.dot(qv, kc[s, kvh])) * scale for s in slots])
    w = np.exp(scores - scores.max())
    w /= w.sum()
    return sum(wi * vc[s, kvh] for wi, s in zip(w, slots))


def scatter(rng: np.random.Generator, totals: list[int], bs: int, hkv: int, d: int):
    per = [math.ceil(t / bs) for t in totals]
    nblocks = sum(per) + 3
    order = list(rng.permutation(nblocks))
    pad = order.pop()
    tables = np.full((len(totals), max(per) + 2), pad, dtype=np.int32)
    k = np.full((nblocks * bs, hkv, d), np.nan, dtype=np.float32)
    v = np.full_like(k, np.nan)
    for r, (t, nb) in enumerate(zip(totals, per)):
        tables[r, :nb] = [order.pop() for _ in range(nb)]
        for p in range(t):
            s = slot(tables[r], p, bs)
            k[s] = rng.standard_normal((hkv, d)).astype(np.float32)
            v[s] = rng.standard_normal((hkv, d)).astype(np.float32)
    return tables, k, v


def make_decode() -> dict[str, np.ndarray]:
    rng = np.random.default_rng(1234)
    lens, hq, hkv, d, bs = [17, 64, 128, 200], 4, 2, 32, 16
    tables, k, v = scatter(rng, lens, bs, hkv, d)
    q = rng.standard_normal((len(lens), hq, d)).astype(np.float32)
    scale = d**-0.5
    out = np.zeros((len(lens), hq, d))
    kd, vd = k.astype(np.float64), v.astype(np.float64)
    for b, n in enumerate(lens):
        slots = [slot(tables[b], p, bs) for p in range(n)]
        for h in range(hq):
            out[b, h] = attend_one(q[b, h].astype(np.float64), kd, vd, slots, h // (hq // hkv), scale)
    return {"q": q, "k_cache": k, "v_cache": v, "block_tables": tables,
            "context_lens": np.array(lens, dtype=np.int32), "block_size": np.int32(bs),
            "out": out}  # fmt: skip


def make_prefill() -> dict[str, np.ndarray]:
    rng = np.random.default_rng(99)
    specs, hq, hkv, d, bs = [(0, 37), (12, 4), (40, 7), (3, 1)], 4, 2, 8, 4
    totals = [c + n for c, n in specs]
    tables, k, v = scatter(rng, totals, bs, hkv, d)
    starts = np.cumsum([0] + [n for _, n in specs])[:-1].astype(np.int32)
    t = sum(n for _, n in specs)
    q = rng.standard_normal((t, hq, d)).astype(np.float32)
    scale = d**-0.5
    out = np.zeros((t, hq, d))
    kd, vd = k.astype(np.float64), v.astype(np.float64)
    for r, ((cached, new), total) in enumerate(zip(specs, totals)):
        for i in range(new):
            pos = cached + i  # the sequence's newest positions
            slots = [slot(tables[r], p, bs) for p in range(pos + 1)]
            for h in range(hq):
                out[starts[r] + i, h] = attend_one(q[starts[r] + i, h].astype(np.float64), kd, vd,
                                                   slots, h // (hq // hkv), scale)  # fmt: skip
    return {"q": q, "k_cache": k, "v_cache": v, "block_tables": tables, "q_starts": starts,
            "q_lens": np.array([n for _, n in specs], dtype=np.int32),
            "context_lens": np.array(totals, dtype=np.int32), "block_size": np.int32(bs),
            "out": out}  # fmt: skip


def make_fused() -> dict[str, np.ndarray]:
    rng = np.random.default_rng(7)
    t, hq, hkv, d, n, eps, theta = 9, 4, 2, 16, 48, 1e-6, 1e6
    x = (rng.standard_normal((t, n)) * 3).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    q = (rng.standard_normal((t, hq, d)) * 5).astype(np.float32)
    kk = (rng.standard_normal((t, hkv, d)) * 5).astype(np.float32)
    vv = rng.standard_normal((t, hkv, d)).astype(np.float32)
    qw = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    kw = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    pos = rng.integers(0, 40000, t)
    slots = rng.permutation(4 * t)[:t].astype(np.int64)

    def norm(vec: np.ndarray, wt: np.ndarray) -> np.ndarray:
        vec = vec.astype(np.float64)
        return vec / math.sqrt(float(np.mean(vec * vec)) + eps) * wt.astype(np.float64)

    cos = np.zeros((t, d))
    sin = np.zeros((t, d))
    for i in range(t):
        for j in range(d // 2):
            ang = float(pos[i]) * theta ** (-2.0 * j / d)
            cos[i, j] = cos[i, j + d // 2] = math.cos(ang)
            sin[i, j] = sin[i, j + d // 2] = math.sin(ang)

    def rope(vec: np.ndarray, i: int) -> np.ndarray:
        h = d // 2
        a, b = vec[:h], vec[h:]
        return np.concatenate([a * cos[i, :h] - b * sin[i, :h], b * cos[i, :h] + a * sin[i, :h]])

    x_out = np.stack([norm(x[i], w) for i in range(t)])
    q_out = np.stack([[rope(norm(q[i, h], qw), i) for h in range(hq)] for i in range(t)])
    k_out = np.stack([[rope(norm(kk[i, h], kw), i) for h in range(hkv)] for i in range(t)])
    return {"x": x, "w": w, "q": q, "k": kk, "v": vv, "q_w": qw, "k_w": kw,
            "positions": pos, "slots": slots, "eps": np.float64(eps), "theta": np.float64(theta),
            "cos": cos, "sin": sin, "x_out": x_out, "q_out": q_out, "k_out": k_out}  # fmt: skip


def main() -> None:
    for name, fn in (("decode", make_decode), ("prefill", make_prefill), ("fused", make_fused)):
        np.savez_compressed(HERE / f"{name}.npz", **fn())
        print("wrote", HERE / f"{name}.npz")


if __name__ == "__main__":
    main()
