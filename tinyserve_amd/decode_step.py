"""A Qwen3-0.6B-shaped decode step for many sequences through the HIP kernels: the
reference's ``Qwen3.forward_decode`` with its fused kernels and a kernel decode
(src/tinyserve/model.py:137-179, 332-356), and a captured graph of it like the
reference's ``DecodeGraphs`` (src/tinyserve/cuda_graphs.py:135-173).

Per layer, on the flat ``[N]`` rows of a ``DecodeInputs`` (step_inputs.py), with the
projections on the row-batch kernels (hip_rows.py; fp16/bf16, up to 256 rows):

    h    = add_rms_norm(x += previous layer's down partials, input_layernorm)  HIP (rows.hip)
    qkv  = rows_linear(h, W_qkv)                                              HIP (rows.hip)
    q    = qk_norm_rope_store(q, k, v, ...) -> K/V cache at slots             HIP (fused.hip)
    attn = paged decode attention over the block tables                       HIP (decode.hip)
    part = rows_linear_partials(attn, W_o)                                    HIP (rows.hip)
    h    = add_rms_norm(x += part, post_attention_layernorm)                  HIP
    act  = rows_silu_gate_up(h, W_gate_up)      (silu(gate) * up)             HIP
    part = rows_linear_partials(act, W_down)    (added by the next add_rms_norm)

then the final norm (adding the last layer's down partials) and the tied output head
(``[vocab, hidden]``, a library GEMM), padded to 8 rows as the reference pads it
(model.py:214-221). Other dtypes and larger row counts (a mixed prefill step) take the
projections through library GEMMs instead:

    h = rms_norm_rows(x); qkv = h @ W_qkv^T; ...; x += attn @ W_o^T (rounded, then added in place);
    h = rms_norm_rows(x); x += (silu(gate) * up) @ W_down^T

Weights are random (no checkpoints here): linear weights ~ N(0, 0.02) in the model dtype,
norm weights 1 + 0.1 N(0, 1). The KV pool has the reference's layout (kv_cache.py:20-50):
per layer ``[num_blocks * block_size + block_size, Hkv, D]``, the last block being the
padding block that padding rows write and read.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F

from collections.abc import Callable

from tinyserve_amd import hip_attention, hip_fused, hip_prefill, hip_rows
from tinyserve_amd.step_inputs import Batch, DecodeInputs, host_ints

HEAD_MIN_ROWS = 8  # the output head runs on at least this many rows (model.py:64)
ROWS_MAX = 256  # steps of more rows take the projections through library GEMMs


@dataclass(frozen=True)
class ModelShape:
    """Qwen3-0.6B by default (config.py of the reference)."""

    hidden: int = 1024
    num_heads: int = 16
    num_kv_heads: int = 8
    head_dim: int = 128
    intermediate: int = 3072
    vocab: int = 151936
    num_layers: int = 28
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1_000_000.0

    @property
    def q_size(self) -> int:
        return self.num_heads * self.head_dim

    @property
    def kv_size(self) -> int:
        return self.num_kv_heads * self.head_dim


def random_weights(shape: ModelShape, dtype: torch.dtype = torch.float16,
                   device: torch.device | str = "cuda", seed: int = 0) -> dict[str, torch.Tensor]:  # fmt: skip
    """Random weights under the reference's names, q/k/v and gate/up already merged
    (model.py:94-127, ``merge_projections``)."""
    device = torch.device(device)
    g = torch.Generator(device=device).manual_seed(seed)  # drawn where the weights live

    def lin(rows: int, cols: int) -> torch.Tensor:
        return (torch.randn(rows, cols, generator=g, device=device) * 0.02).to(dtype)

    def norm(n: int) -> torch.Tensor:
        return (1.0 + 0.1 * torch.randn(n, generator=g, device=device)).to(dtype)

    s = shape
    w = {"model.embed_tokens.weight": lin(s.vocab, s.hidden), "model.norm.weight": norm(s.hidden)}
    for i in range(s.num_layers):
        p = f"model.layers.{i}."
        w[p + "input_layernorm.weight"] = norm(s.hidden)
        w[p + "post_attention_layernorm.weight"] = norm(s.hidden)
        w[p + "self_attn.qkv_proj.weight"] = lin(s.q_size + 2 * s.kv_size, s.hidden)
        w[p + "self_attn.o_proj.weight"] = lin(s.hidden, s.q_size)
        w[p + "self_attn.q_norm.weight"] = norm(s.head_dim)
        w[p + "self_attn.k_norm.weight"] = norm(s.head_dim)
        w[p + "mlp.gate_up_proj.weight"] = lin(2 * s.intermediate, s.hidden)
        w[p + "mlp.down_proj.weight"] = lin(s.hidden, s.intermediate)
    return w


class KVPool:
    """The KV cache tensors (kv_cache.py:20-50): ``k``, ``v`` of shape
    ``[L, num_blocks * block_size + block_size, Hkv, D]``; block ``num_blocks`` is the
    padding block."""

    def __init__(self, shape: ModelShape, num_blocks: int, block_size: int,
                 dtype: torch.dtype = torch.float16, device: torch.device | str = "cuda") -> None:  # fmt: skip
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.num_slots = num_blocks * block_size
        self.pad_block = num_blocks
        dims = (shape.num_layers, self.num_slots + block_size, shape.num_kv_heads, shape.head_dim)
        self.k = torch.zeros(dims, dtype=dtype, device=device)
        self.v = torch.zeros(dims, dtype=dtype, device=device)

    @property
    def memory_bytes(self) -> int:
        return 2 * self.k.numel() * self.k.element_size()


def rope_tables(head_dim: int, theta: float, positions: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """``[T, D]`` float32 cos / sin on the positions' device, angles in float64 (the
    reference's ``rope_cos_sin``, layers.py:41-65; positions reach 40960): one launch of
    ``hip_fused.rope_cos_sin``."""
    return hip_fused.rope_cos_sin(head_dim, theta, positions.to(torch.int64))


class DecodeStep:
    """``forward(inputs)`` -> ``[N, vocab]`` float32 logits, writing each row's new k/v
    into the pool (the reference's ``forward_decode``). Nothing in it waits for the GPU,
    so a graph can capture it.

    ``num_splits``: the decode kernel's split count (None: the launcher's policy; the
    reference's config-5 step forces 16). ``projections``: "rows" (the row-batch HIP
    kernels), "library" (library GEMMs) or "auto" (rows where the dtype and shapes allow,
    for steps of up to ``ROWS_MAX`` rows)."""

    def __init__(self, shape: ModelShape, weights: dict[str, torch.Tensor], pool: KVPool,
                 num_splits: int | None = None, projections: str = "auto") -> None:  # fmt: skip
        self.shape = shape
        self.w = weights
        self.pool = pool
        self.num_splits = num_splits
        self.scale = shape.head_dim**-0.5
        dtype = weights["model.embed_tokens.weight"].dtype
        fits = (hip_rows.supported(dtype) and shape.hidden % 32 == 0 and shape.intermediate % 32 == 0
                and shape.q_size % 32 == 0 and shape.hidden <= 4096)  # fmt: skip
        if projections not in ("auto", "rows", "library"):
            raise ValueError(f"projections must be 'auto', 'rows' or 'library', got {projections!r}")
        if projections == "rows" and not fits:
            raise ValueError(f"the row-batch projections need fp16/bf16 and 32-aligned widths (hidden <= 4096), "
                             f"got {dtype} and {shape}")  # fmt: skip
        self.projections = projections if projections != "auto" else ("rows" if fits else "library")

    def _attention(self, i: int, q: torch.Tensor, inputs: DecodeInputs) -> torch.Tensor:
        return hip_attention.launch_paged_decode_split(
            q, self.pool.k[i], self.pool.v[i], inputs.block_tables, inputs.context_lens,
            self.scale, self.pool.block_size, self.num_splits)  # fmt: skip

    def layer(self, i: int, x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, slots: torch.Tensor,
              attend: Callable[[int, torch.Tensor], torch.Tensor]) -> torch.Tensor:  # fmt: skip
        """One decoder layer (model.py:137-179, the fused path): the new tokens' k/v go to
        the pool at ``slots``; ``attend(i, q)`` returns the attention output for ``q``."""
        s, w, p = self.shape, self.w, f"model.layers.{i}."
        n = x.shape[0]
        h = hip_fused.rms_norm_rows(x, w[p + "input_layernorm.weight"], s.rms_norm_eps)
        qkv = F.linear(h, w[p + "self_attn.qkv_proj.weight"])
        q, k, v = torch.split(qkv, [s.q_size, s.kv_size, s.kv_size], dim=1)
        q = hip_fused.qk_norm_rope_store(
            q.view(n, s.num_heads, s.head_dim), k.view(n, s.num_kv_heads, s.head_dim),
            v.view(n, s.num_kv_heads, s.head_dim), w[p + "self_attn.q_norm.weight"],
            w[p + "self_attn.k_norm.weight"], cos, sin, slots, self.pool.k[i],
            self.pool.v[i], s.rms_norm_eps)  # fmt: skip
        attn = attend(i, q)
        # Residual adds as model.py:172,179 writes them: the projection is rounded to the
        # model dtype, then the sum (in place: x is this step's own activation).
        x.add_(F.linear(attn.reshape(n, s.q_size), w[p + "self_attn.o_proj.weight"]))
        h = hip_fused.rms_norm_rows(x, w[p + "post_attention_layernorm.weight"], s.rms_norm_eps)
        gate, up = F.linear(h, w[p + "mlp.gate_up_proj.weight"]).chunk(2, dim=1)
        return x.add_(F.linear(F.silu(gate) * up, w[p + "mlp.down_proj.weight"]))

    def _layers_rows(self, x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, slots: torch.Tensor,
                     attend: Callable[[int, torch.Tensor], torch.Tensor]) -> torch.Tensor:  # fmt: skip
        """Every layer and the final norm with the row-batch projection kernels: returns
        the final-normed rows. ``x`` (this step's embedded rows) is updated in place: each
        residual add happens in the ``add_rms_norm`` that follows it."""
        s, w = self.shape, self.w
        n = x.shape[0]
        eps = s.rms_norm_eps
        pending = None  # the previous layer's down_proj partials, not yet added to x
        for i in range(s.num_layers):
            p = f"model.layers.{i}."
            h = hip_rows.add_rms_norm(x, pending, w[p + "input_layernorm.weight"], eps)
            qkv = hip_rows.rows_linear(h, w[p + "self_attn.qkv_proj.weight"])
            q, k, v = torch.split(qkv, [s.q_size, s.kv_size, s.kv_size], dim=1)
            q = hip_fused.qk_norm_rope_store(
                q.view(n, s.num_heads, s.head_dim), k.view(n, s.num_kv_heads, s.head_dim),
                v.view(n, s.num_kv_heads, s.head_dim), w[p + "self_attn.q_norm.weight"],
                w[p + "self_attn.k_norm.weight"], cos, sin, slots, self.pool.k[i],
                self.pool.v[i], eps)  # fmt: skip
            attn = attend(i, q)
            part, _ = hip_rows.rows_linear_partials(attn.reshape(n, s.q_size), w[p + "self_attn.o_proj.weight"])
            h = hip_rows.add_rms_norm(x, part, w[p + "post_attention_layernorm.weight"], eps)
            act = hip_rows.rows_silu_gate_up(h, w[p + "mlp.gate_up_proj.weight"])
            pending, _ = hip_rows.rows_linear_partials(act, w[p + "mlp.down_proj.weight"])
        return hip_rows.add_rms_norm(x, pending, w["model.norm.weight"], eps, tiled=False)

    def _run(self, token_ids: torch.Tensor, positions: torch.Tensor, slots: torch.Tensor,
             attend: Callable[[int, torch.Tensor], torch.Tensor],
             rows: torch.Tensor | None = None) -> torch.Tensor:  # fmt: skip
        """Logits of every token, or of ``rows`` only (model.py:181-211)."""
        s = self.shape
        cos, sin = rope_tables(s.head_dim, s.rope_theta, positions)
        x = self.w["model.embed_tokens.weight"][token_ids]
        if self.projections == "rows" and x.shape[0] <= ROWS_MAX:
            x = self._layers_rows(x, cos, sin, slots, attend)
        else:
            for i in range(s.num_layers):
                x = self.layer(i, x, cos, sin, slots, attend)
            x = hip_fused.rms_norm_rows(x, self.w["model.norm.weight"], s.rms_norm_eps)
        if rows is not None:
            x = x[rows]
        n = x.shape[0]
        if n < HEAD_MIN_ROWS:
            x = F.pad(x, (0, 0, 0, HEAD_MIN_ROWS - n))
        return F.linear(x, self.w["model.embed_tokens.weight"])[:n].float()

    def forward(self, inputs: DecodeInputs) -> torch.Tensor:
        """One decode step for every row of ``inputs`` (model.py:332-356)."""
        return self._run(inputs.token_ids, inputs.positions, inputs.slots,
                         lambda i, q: self._attention(i, q, inputs))  # fmt: skip

    def forward_batch(self, batch: Batch) -> torch.Tensor:
        """``[B, vocab]`` logits of each sequence's last new token for a mixed step
        (model.py:255-323 with the kernels): one-token sequences attend through the
        decode kernel in one launch, the others through the varlen prefill kernel in one
        launch, both on the rows of one flat batch. Reads the query lengths on the host."""
        qlens = batch.query_lens
        starts = [0]
        for n in qlens[:-1]:
            starts.append(starts[-1] + n)
        dev = batch.token_ids.device
        one = [b for b, n in enumerate(qlens) if n == 1]
        rest = [b for b, n in enumerate(qlens) if n != 1]
        scale, bs = self.scale, self.pool.block_size

        def ints(xs: list[int]) -> torch.Tensor:
            return host_ints(xs, torch.int32, dev)

        if one:
            d_idx = host_ints(one, torch.int64, dev)
            d_rows = host_ints([starts[b] for b in one], torch.int64, dev)
            d_tables, d_lens = batch.block_tables[d_idx], batch.context_lens[d_idx]
        if rest:
            p_idx = host_ints(rest, torch.int64, dev)
            p_starts, p_qlens = ints([starts[b] for b in rest]), ints([qlens[b] for b in rest])
            p_tables, p_lens = batch.block_tables[p_idx], batch.context_lens[p_idx]
            max_q = max(qlens[b] for b in rest)

        def attend(i: int, q: torch.Tensor) -> torch.Tensor:
            k, v = self.pool.k[i], self.pool.v[i]
            if not rest:  # all decode: the rows are the sequences, in order
                return hip_attention.launch_paged_decode_split(
                    q, k, v, batch.block_tables, batch.context_lens, scale, bs, self.num_splits)
            out = torch.empty_like(q)
            if one:
                out[d_rows] = hip_attention.launch_paged_decode_split(
                    q[d_rows], k, v, d_tables, d_lens, scale, bs, self.num_splits)  # fmt: skip
            hip_prefill.paged_prefill_attention(q, k, v, p_tables, p_starts, p_qlens, p_lens, scale, bs,
                                                max_q, out)  # fmt: skip
            return out

        return self._run(batch.token_ids, batch.positions, batch.new_slots, attend, rows=batch.last_rows)

    def attention_only(self, inputs: DecodeInputs) -> torch.Tensor:
        """The step's decode-attention launches alone (one per layer, on the current
        cache contents and a fixed q): for measuring the attention share of a step."""
        s = self.shape
        q = torch.zeros(inputs.num_rows, s.num_heads, s.head_dim, dtype=self.pool.k.dtype,
                        device=self.pool.k.device)  # fmt: skip
        out = q
        for i in range(s.num_layers):
            out = self._attention(i, q, inputs)
        return out


class DecodeGraph:
    """One captured graph of ``fn(inputs)`` on fixed ``inputs`` buffers (the reference's
    ``DecodeGraphs`` for one bucket, cuda_graphs.py:135-173): ``replay()`` re-runs it on
    whatever the buffers hold and returns the output buffer (overwritten by the next
    replay). The pass runs twice on a side stream first, so every library handle and
    kernel is loaded before capture."""

    def __init__(self, fn, inputs: DecodeInputs) -> None:  # noqa: ANN001
        dev = inputs.token_ids.device
        side = torch.cuda.Stream(dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            for _ in range(2):
                fn(inputs)
        torch.cuda.current_stream(dev).wait_stream(side)
        torch.cuda.synchronize(dev)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.output = fn(inputs)
        torch.cuda.synchronize(dev)

    def replay(self) -> torch.Tensor:
        self.graph.replay()
        return self.output


def random_context_tables(lens: list[int], block_size: int, num_blocks: int | None = None,
                          seed: int = 0) -> tuple[list[list[int]], int]:  # fmt: skip
    """Block lists for sequences of ``lens`` tokens, scattered over a pool by a seeded
    permutation (the synthetic input of the config-5 step). Returns the lists and the
    pool's block count."""
    need = [math.ceil(n / block_size) for n in lens]
    total = sum(need)
    num_blocks = num_blocks or total
    if num_blocks < total:
        raise ValueError(f"{total} blocks needed, the pool has {num_blocks}")
    perm = torch.randperm(num_blocks, generator=torch.Generator().manual_seed(seed)).tolist()
    out, at = [], 0
    for k in need:
        out.append(perm[at : at + k])
        at += k
    return out, num_blocks
