"""Fused per-layer kernels around attention on MI355X: ``rms_norm_rows`` and
``qk_norm_rope_store`` of the reference's ``tinyserve.triton_fused``
(src/tinyserve/triton_fused.py:116-177), same arguments, results and errors, launching
``csrc/fused.hip``; and ``rope_cos_sin``, the reference's per-step RoPE tables
(layers.py:41-65) as one launch.

``rms_norm_rows``: one wave64 per row, the row held in registers as 16-byte vectors,
one HBM read and one write per element.

``qk_norm_rope_store``: one lane group per (token, head); each lane holds a pair of
16-byte chunks i and i + D/2, so the rotate-half pairs never leave the lane and the
per-head norm is a reduction over 8 lanes (D = 128, fp16). Query heads go to the
returned tensor; key heads and value heads are written straight into their cache slots
(``k_cache[slots[t]]``, ``v_cache[slots[t]]``). Numerics follow layers.py:14-91 step by
step: fp32 sum of squares, ``1 / sqrt`` (correctly rounded), round to the input dtype,
multiply by the weight in the input dtype, rotate in fp32 without fused multiply-adds
(``a*cos - b*sin`` as two rounded products and a difference, like PyTorch), round once.
"""

from __future__ import annotations

import torch

from tinyserve_amd import _lib


def rms_norm_rows(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """RMSNorm (``layers.rms_norm``) applied to each of the T rows of ``x [T, N]``,
    all rows in a single launch (:116-126)."""
    if x.dim() != 2 or x.stride(1) != 1 or weight.shape != (x.shape[1],):
        raise ValueError(f"need a row-contiguous [T, N] tensor and an [N] weight: {x.shape}")
    if weight.dtype != x.dtype or weight.stride(0) != 1:
        raise ValueError(f"the weight must be a contiguous {x.dtype} vector, got {weight.dtype}")
    out = torch.empty_like(x)
    if x.shape[0]:
        dev = _lib.require_device(x, weight)
        _lib.call("ts_rms_norm_rows", x.data_ptr(), weight.data_ptr(), out.data_ptr(),
                  x.shape[0], x.shape[1], x.stride(0), out.stride(0), float(eps),
                  _lib.dtype_code(x), _lib.stream_of(dev))  # fmt: skip
    return out


def qk_norm_rope_store(
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
    """Per-head RMSNorm of q and k, rotary embedding of both, and the cache store of
    this step's k and v, as a single launch for one layer (:129-177).

    The returned tensor is ``apply_rope(rms_norm(q, q_weight, eps), cos, sin)``. As a
    side effect, row t of ``apply_rope(rms_norm(k, k_weight, eps), cos, sin)`` and of
    ``v`` go to cache slot ``slots[t]`` of ``k_cache`` / ``v_cache``, converted to the
    cache's dtype; no other slot is touched and the host never waits on the device.

    Args:
        q: ``[T, Hq, D]``; k, v: ``[T, Hkv, D]``. Only the head dimension must be
            contiguous, so views into one fused QKV projection output work directly.
        q_weight, k_weight: ``[D]`` in q's dtype.
        cos, sin: float32 ``[T, D]`` tables from ``rope_cos_sin``; the kernel reads
            their first D/2 columns.
        slots: ``[T]`` int64 destination slots (int32 is accepted and widened).
        k_cache, v_cache: ``[num_slots, Hkv, D]``, the layer's cache.
    """
    t, num_q_heads, head_dim = q.shape
    num_kv_heads = k.shape[1]
    if head_dim % 2 or (head_dim // 2) & (head_dim // 2 - 1):
        raise ValueError(f"head_dim must be twice a power of 2, got {head_dim}")
    if k.shape != v.shape or k.shape[0] != t or k_cache.shape[1:] != k.shape[1:]:
        raise ValueError(f"shapes q {q.shape}, k {k.shape}, v {v.shape}, cache {k_cache.shape}")
    if any(x.stride(2) != 1 for x in (q, k, v, k_cache)) or v_cache.stride() != k_cache.stride():
        raise ValueError("the head dimension must be contiguous, and k/v caches laid out alike")
    if cos.shape != (t, head_dim) or cos.stride() != sin.stride() or cos.stride(1) != 1:
        raise ValueError(f"cos and sin must be [T, D] = {(t, head_dim)}, laid out alike")
    if cos.dtype != torch.float32 or sin.dtype != torch.float32:
        raise ValueError("cos and sin must be float32 (rope_cos_sin)")
    if head_dim < 8 or head_dim > 256:
        raise ValueError(f"head_dim {head_dim} is outside the HIP kernels' range (8..256)")
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError(f"q, k and v must share a dtype: {q.dtype}, {k.dtype}, {v.dtype}")
    for w in (q_weight, k_weight):
        if w.shape != (head_dim,) or w.dtype != q.dtype or w.stride(0) != 1:
            raise ValueError(f"q/k norm weights must be contiguous [{head_dim}] {q.dtype}")
    if k_cache.dtype != v_cache.dtype:
        raise ValueError("k_cache and v_cache must share a dtype")
    if slots.shape != (t,):
        raise ValueError(f"slots must be [T] = [{t}]")
    out = torch.empty_like(q)
    if t:
        dev = _lib.require_device(q, k, v, q_weight, k_weight, cos, sin, slots, k_cache, v_cache)
        if slots.dtype != torch.int64:
            slots = slots.to(torch.int64)
        _lib.call(
            "ts_qk_norm_rope_store",
            q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
            q_weight.data_ptr(), k_weight.data_ptr(), cos.data_ptr(), sin.data_ptr(),
            slots.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
            t, num_q_heads, num_kv_heads, head_dim,
            q.stride(0), q.stride(1), k.stride(0), k.stride(1), v.stride(0), v.stride(1),
            out.stride(0), out.stride(1), cos.stride(0), k_cache.stride(0), k_cache.stride(1),
            float(eps), _lib.dtype_code(q), _lib.dtype_code(k_cache), _lib.stream_of(dev),
        )  # fmt: skip
    return out


def rope_cos_sin(head_dim: int, theta: float, positions: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """``layers.rope_cos_sin`` in one launch: ``(cos, sin)``, each ``[T, head_dim]``
    float32, ``cat([angles, angles], -1)`` with angles in float64."""
    if positions.dim() != 1 or positions.dtype != torch.int64:
        raise ValueError(f"positions must be a [T] int64 tensor, got {positions.dtype} {tuple(positions.shape)}")
    if head_dim < 2 or head_dim % 2:
        raise ValueError(f"head_dim must be even, got {head_dim}")
    t = positions.shape[0]
    cos = torch.empty(t, head_dim, dtype=torch.float32, device=positions.device)
    sin = torch.empty_like(cos)
    if t:
        dev = _lib.require_device(positions)
        pos = positions.contiguous()
        _lib.call("ts_rope_cos_sin", pos.data_ptr(), t, head_dim, float(theta),
                  cos.data_ptr(), sin.data_ptr(), cos.stride(0), _lib.stream_of(dev))  # fmt: skip
    return cos, sin
