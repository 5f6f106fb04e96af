"""CPU oracle: a restatement of the reference's PyTorch paths for TinyServe's attention
hot path. TEST INFRASTRUCTURE ONLY -- the HIP kernels are checked against it; nothing in
the product imports it.

Each function follows one reference function (paths relative to the reference repo):

    block_slots         src/tinyserve/block_table.py:74-82   slot = table[p // bs] * bs + p % bs
    attend_causal       src/tinyserve/attention.py:16-59     causal_gqa_attention
    attend_paged        src/tinyserve/attention.py:62-111    paged_gqa_attention
    decode_ref          src/tinyserve/attention.py:114-141   paged_decode_attention_ref
    split_partials_ref  src/tinyserve/triton_attention.py:243-296  each split's (m, l, acc)
    merge_partials_ref  src/tinyserve/triton_attention.py:299-327  their combine
    prefill_ref         tests/test_triton_prefill.py:57-61   paged_gqa_attention per sequence
    batched_prefill_ref src/tinyserve/attention.py:144-220   prefill_plan + batched SDPA
    rms_norm            src/tinyserve/layers.py:14-38
    rope_cos_sin        src/tinyserve/layers.py:41-65        (angles in float64)
    apply_rope          src/tinyserve/layers.py:68-91
    kv_write            src/tinyserve/kv_cache.py:42-50      cache[slots] = x.to(cache dtype)
    qk_norm_rope_store_ref   the composition triton_fused.py:129-177 replaces

The functions compute on the device their inputs live on: the CPU in the oracle's own
tests, the GPU where a large parity test runs the oracle there as its checker (float32,
the same operations).

Numerics contract (the reference's): attention scores, softmax and the weighted sum in
float32, one rounding to the query dtype at the end; RMSNorm normalises in float32,
rounds to the input dtype, then multiplies by the weight in that dtype; RoPE rotates in
float32 and rounds once.

How each function is pinned (tests/test_oracle.py): hand-computed values from the
reference's own tests (one token returns its v, q = 0 averages the past, GQA grouping,
RMSNorm of [3, 4], RoPE at D = 4, theta = 1e4, p = 7, pairing i with i + D/2, the slot
table of block_table.py:6-12), PyTorch's scaled_dot_product_attention, and a float64
brute force over positions and slots written independently in tests/golden/.
"""

from __future__ import annotations

import torch


def block_slots(table_row: torch.Tensor | list[int], n: int, block_size: int) -> torch.Tensor:
    """int64 ``[n]``: the cache slot of each position 0 .. n-1 of one sequence."""
    row = torch.as_tensor(table_row, dtype=torch.int64).flatten().cpu()
    pos = torch.arange(n, dtype=torch.int64)
    return row[pos // block_size] * block_size + pos % block_size


def _scores_softmax_values(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, allowed: torch.Tensor, scale: float
) -> torch.Tensor:
    """softmax(q k^T * scale, masked) v per query head, in float32.

    q ``[n, Hq, D]``; k, v ``[m, Hkv, D]``; allowed ``[n, m]`` bool. Query head h reads kv
    head ``h // (Hq // Hkv)`` (consecutive groups, attention.py:23-25). Returns float32
    ``[n, Hq, D]``."""
    hq, hkv = q.shape[1], k.shape[1]
    group = hq // hkv
    qh = q.float().permute(1, 0, 2)  # [Hq, n, D]
    kh = k.float().permute(1, 0, 2).repeat_interleave(group, dim=0)  # [Hq, m, D]
    vh = v.float().permute(1, 0, 2).repeat_interleave(group, dim=0)
    s = torch.matmul(qh, kh.transpose(1, 2)) * scale  # [Hq, n, m]
    s = s.masked_fill(~allowed.to(s.device), float("-inf"))
    p = torch.softmax(s, dim=-1)
    return torch.matmul(p, vh).permute(1, 0, 2)


def attend_causal(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float) -> torch.Tensor:
    """Causal GQA attention of one contiguous sequence (attention.py:16-59)."""
    t = q.shape[0]
    pos = torch.arange(t)
    allowed = pos[None, :] <= pos[:, None]
    return _scores_softmax_values(q, k, v, allowed, scale).to(q.dtype)


def attend_paged(
    q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, slots: torch.Tensor, scale: float
) -> torch.Tensor:
    """Attention of the newest ``n = len(q)`` positions of a sequence whose keys and
    values sit at ``slots`` (one per position, in order) of a cache layer
    (attention.py:62-111)."""
    n, total = q.shape[0], slots.shape[0]
    slots = slots.to(torch.int64).to(k_cache.device)
    k = k_cache.index_select(0, slots)
    v = v_cache.index_select(0, slots)
    q_pos = torch.arange(total - n, total)
    allowed = torch.arange(total)[None, :] <= q_pos[:, None]
    return _scores_softmax_values(q, k, v, allowed, scale).to(q.dtype)


def decode_ref(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    context_lens: torch.Tensor,
    scale: float,
    block_size: int,
) -> torch.Tensor:
    """One decode query per sequence over its paged context (attention.py:114-141)."""
    rows = []
    for b, n in enumerate(context_lens.tolist()):
        slots = block_slots(block_tables[b], n, block_size)
        rows.append(attend_paged(q[b : b + 1], k_cache, v_cache, slots, scale))
    return torch.cat(rows) if rows else torch.empty_like(q)


def split_partials_ref(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    context_lens: torch.Tensor,
    scale: float,
    block_size: int,
    splits: int,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """The partial results of the split-K decode (triton_attention.py:243-296): sequence
    b's ``n = ceil(len / bs)`` blocks are cut into ranges of ``ceil(n / splits)`` blocks
    (``first = split * per_split``, ``last = min(first + per_split, n)``, :283-286), and
    each (sequence, query head, range) gives its maximum score ``m`` (natural units),
    ``l = sum exp(s - m)`` and the unnormalised ``acc = sum exp(s - m) v`` over the keys
    of its range. An empty range has m = -inf, l = 0, acc = 0. float32
    ``[B, Hq, S]``, ``[B, Hq, S]``, ``[B, Hq, S, D]``."""
    b_count, hq, d = q.shape
    group = hq // k_cache.shape[1]
    m = torch.full((b_count, hq, splits), float("-inf"))
    l = torch.zeros((b_count, hq, splits))  # noqa: E741
    acc = torch.zeros((b_count, hq, splits, d))
    for b, n in enumerate(context_lens.tolist()):
        slots = block_slots(block_tables[b], n, block_size)
        nblocks = -(-n // block_size)
        per = -(-nblocks // splits)
        for s in range(splits):
            t0, t1 = min(s * per, nblocks) * block_size, min((s + 1) * per * block_size, n)
            if t0 >= t1:
                continue
            idx = slots[t0:t1]
            k = k_cache.index_select(0, idx).float()  # [t, Hkv, D]
            v = v_cache.index_select(0, idx).float()
            for h in range(hq):
                sc = (k[:, h // group] @ q[b, h].float()) * scale  # [t]
                mx = sc.max()
                p = torch.exp(sc - mx)
                m[b, h, s], l[b, h, s] = mx, p.sum()
                acc[b, h, s] = p @ v[:, h // group]
    return m, l, acc


def merge_partials_ref(m: torch.Tensor, l: torch.Tensor, acc: torch.Tensor) -> torch.Tensor:  # noqa: E741
    """The combine of split partials (triton_attention.py:299-327): weights
    ``w_s = exp(m_s - max_s m_s)``, ``out = sum w_s acc_s / sum w_s l_s``; float32."""
    w = torch.exp(m - m.max(dim=-1, keepdim=True).values)
    return (w[..., None] * acc).sum(dim=-2) / (w * l).sum(dim=-1)[..., None]


def prefill_ref(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    q_starts: torch.Tensor,
    q_lens: torch.Tensor,
    context_lens: torch.Tensor,
    scale: float,
    block_size: int,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Varlen prefill: sequence r's rows ``q_starts[r] ..`` attend causally to its
    ``context_lens[r]`` keys (the per-sequence reference of
    tests/test_triton_prefill.py:57-61). Rows of no sequence are left as in ``out``."""
    out = torch.empty_like(q) if out is None else out
    for r, (s, n, total) in enumerate(zip(q_starts.tolist(), q_lens.tolist(), context_lens.tolist())):
        slots = block_slots(block_tables[r], total, block_size)
        out[s : s + n] = attend_paged(q[s : s + n], k_cache, v_cache, slots, scale)
    return out


def batched_prefill_ref(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    q_starts: torch.Tensor,
    q_lens: torch.Tensor,
    context_lens: torch.Tensor,
    scale: float,
    block_size: int,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """The reference's batched prefill path (attention.py:144-220, ``prefill_plan`` +
    ``batched_prefill_attention``): every sequence's queries and keys gathered into one
    padded rectangle and attended by a single masked scaled-dot-product call in float32.
    Padded query rows repeat the sequence's last query (their results are dropped);
    padded keys are masked out by causality. A second, independently structured oracle
    for ``prefill_ref``; rows of no sequence are left as in ``out``."""
    out = torch.empty_like(q) if out is None else out
    starts, lens, totals = q_starts.tolist(), q_lens.tolist(), context_lens.tolist()
    if not lens:
        return out
    dev = q.device  # runs where the inputs are (the GPU tests run it on the device)
    lq, lk = max(lens), max(totals)
    i = torch.arange(lq)
    rows = torch.stack([s + torch.clamp(i, max=n - 1) for s, n in zip(starts, lens)])  # [R, Lq]
    slots = torch.zeros((len(lens), lk), dtype=torch.int64)
    for r, total in enumerate(totals):
        slots[r, :total] = block_slots(block_tables[r].cpu(), total, block_size)
    first = torch.tensor([t - n for t, n in zip(totals, lens)])[:, None]  # position of query 0
    q_pos = first + torch.clamp(i[None, :], max=torch.tensor(lens)[:, None] - 1)
    mask = (torch.arange(lk)[None, None, :] <= q_pos[:, :, None]).to(dev)  # [R, Lq, Lk]
    rows, slots = rows.to(dev), slots.to(dev)
    group = q.shape[1] // k_cache.shape[1]
    qb = q[rows].float().transpose(1, 2)  # [R, Hq, Lq, D]
    kb = k_cache[slots].float().repeat_interleave(group, dim=2).transpose(1, 2)
    vb = v_cache[slots].float().repeat_interleave(group, dim=2).transpose(1, 2)
    ob = torch.nn.functional.scaled_dot_product_attention(qb, kb, vb, attn_mask=mask[:, None], scale=scale)
    ob = ob.transpose(1, 2)  # [R, Lq, Hq, D] float32
    for r, (s, n) in enumerate(zip(starts, lens)):
        out[s : s + n] = ob[r, :n].to(out.dtype)
    return out


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """RMSNorm over the last dim (layers.py:14-38): fp32 normalise, round, weight in x's dtype."""
    xf = x.float()
    inv = torch.rsqrt(xf.square().mean(dim=-1, keepdim=True) + eps)
    return (xf * inv).to(x.dtype) * weight


def rope_cos_sin(head_dim: int, theta: float, positions: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """RoPE tables ``[T, D]`` float32 (layers.py:41-65): pair i turns by
    p * theta^(-2i/D), angles in float64, both halves hold the same angles."""
    exponent = torch.arange(0, head_dim, 2, dtype=torch.float64) / head_dim
    inv_freq = torch.pow(torch.tensor(theta, dtype=torch.float64), -exponent)
    ang = positions.to(torch.float64).cpu()[:, None] * inv_freq[None, :]
    ang = torch.cat([ang, ang], dim=-1)
    return torch.cos(ang).float(), torch.sin(ang).float()


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Rotate-half RoPE (layers.py:68-91): pair (i, i + D/2), fp32 math, one rounding."""
    half = x.shape[-1] // 2
    xf = x.float()
    a, b = xf[..., :half], xf[..., half:]
    c = cos[:, None, :half].to(xf.device)
    s = sin[:, None, :half].to(xf.device)
    return torch.cat([a * c - b * s, b * c + a * s], dim=-1).to(x.dtype)


def kv_write(
    k_cache: torch.Tensor, v_cache: torch.Tensor, slots: torch.Tensor, k: torch.Tensor, v: torch.Tensor
) -> None:
    """``KVCache.write`` for one layer (kv_cache.py:42-50): an indexed store with a cast."""
    idx = slots.to(torch.int64)
    k_cache[idx] = k.to(k_cache.dtype)
    v_cache[idx] = v.to(v_cache.dtype)


def qk_norm_rope_store_ref(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    q_weight: torch.Tensor,
    k_weight: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    slots: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    eps: float,
) -> torch.Tensor:
    """What ``qk_norm_rope_store`` fuses (model.py's unfused path): returns the rotated,
    normalised q and writes rotated, normalised k and v into the caches at ``slots``."""
    q_out = apply_rope(rms_norm(q, q_weight, eps), cos, sin)
    k_rot = apply_rope(rms_norm(k, k_weight, eps), cos, sin)
    kv_write(k_cache, v_cache, slots, k_rot, v)
    return q_out
