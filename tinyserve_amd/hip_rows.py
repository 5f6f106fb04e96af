"""Projections of a decode step, and the residual add + RMSNorm between them, on the
HIP kernels of ``csrc/rows.hip``.

A decode step multiplies a few rows (one token per sequence) by each weight matrix of a
layer, so every projection is a stream of its weights from HBM. These wrappers replace
the decoder layer's ``F.linear`` calls and the residual adds around them
(src/tinyserve/model.py:137-179) on that path:

    h    = rms_norm(x)                       add_rms_norm(x, None, ...)      -> h tiled
    qkv  = F.linear(h, W_qkv)                rows_linear(h, W_qkv)
    x    = x + F.linear(attn, W_o)           rows_linear_partials(attn, W_o)  -> partials
    h    = rms_norm(x)                       add_rms_norm(x, partials, ...)  (x updated)
    act  = silu(gate) * up                   rows_silu_gate_up(h, W_gate_up) -> act tiled
    x    = x + F.linear(act, W_down)         rows_linear_partials(act, W_down), added by
                                             the next add_rms_norm

``Tiled`` holds a matrix in the operand-tiled layout the projections read fastest (each
MFMA operand load one contiguous 1 KB read): element (m, k) of an [M, K] matrix, with M
padded to a multiple of 64, sits at
``((((m//64) * (K//32) + k//32) * 4 + (m%64)//16) * 64 + ((k%32)//8) * 16 + m%16) * 8 + k%8``.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib

ROWS_STORE, ROWS_PARTIAL, ROWS_SILU = 0, 1, 2
ROW_BLOCK = 64


def padded_rows(m: int) -> int:
    """Rows of an operand-tiled matrix of ``m`` rows: ``m`` rounded up to 64."""
    return (m + ROW_BLOCK - 1) // ROW_BLOCK * ROW_BLOCK


@dataclass
class Tiled:
    """An operand-tiled ``[rows, cols]`` matrix in the flat buffer ``buf`` of
    ``padded_rows(rows) * cols`` elements (padding rows hold zeros once written)."""

    buf: torch.Tensor
    rows: int
    cols: int

    @staticmethod
    def empty(rows: int, cols: int, dtype: torch.dtype, device: torch.device) -> Tiled:
        if cols % 32:
            raise ValueError(f"an operand-tiled matrix needs a multiple of 32 columns, got {cols}")
        return Tiled(torch.empty(padded_rows(rows) * cols, dtype=dtype, device=device), rows, cols)

    @property
    def dtype(self) -> torch.dtype:
        return self.buf.dtype

    def _view6(self) -> torch.Tensor:
        mb = padded_rows(self.rows) // ROW_BLOCK
        # buffer order (row block, column chunk, 16-row tile, 8-column group, row, element)
        return self.buf.view(mb, self.cols // 32, 4, 4, 16, 8)

    def to_dense(self) -> torch.Tensor:
        """The ``[rows, cols]`` matrix, row-major (a copy)."""
        d = self._view6().permute(0, 2, 4, 1, 3, 5).reshape(padded_rows(self.rows), self.cols)
        return d[: self.rows].clone()

    @staticmethod
    def from_dense(x: torch.Tensor) -> Tiled:
        """``x`` [M, K] in the operand-tiled layout (padding rows zero)."""
        m, k = x.shape
        t = Tiled.empty(m, k, x.dtype, x.device)
        full = torch.zeros(padded_rows(m), k, dtype=x.dtype, device=x.device)
        full[:m] = x
        mb = padded_rows(m) // ROW_BLOCK
        t.buf.copy_(full.view(mb, 4, 16, k // 32, 4, 8).permute(0, 3, 1, 4, 2, 5).reshape(-1))
        return t


def rows_plan(m: int, n: int, k: int, epilogue: int) -> dict | None:
    """The launch shape ``ts_rows_gemm`` takes for these sizes, or None if it has none."""
    out = (_lib.ctypes.c_int * 5)()
    if _lib.load().ts_rows_gemm_plan(m, n, k, epilogue, out) != 0:
        return None
    return {"waves": out[0], "tiles_per_wave": out[1], "steps": out[2], "k_splits": out[3], "chunks": out[4]}


def supported(dtype: torch.dtype) -> bool:
    """Whether the projection kernels take this dtype (MFMA fp16 / bf16)."""
    return dtype in (torch.float16, torch.bfloat16)


def _x_args(x: torch.Tensor | Tiled) -> tuple[int, int, int, int, int]:
    """(pointer, tiled, row stride, rows, cols) of a projection's input."""
    if isinstance(x, Tiled):
        if x.cols % 32 or x.buf.numel() < padded_rows(x.rows) * x.cols or not x.buf.is_contiguous():
            raise ValueError(f"x: an operand-tiled [{x.rows}, {x.cols}] needs a contiguous buffer of "
                             f"{padded_rows(x.rows) * x.cols} elements and a multiple of 32 columns")  # fmt: skip
        return x.buf.data_ptr(), 1, 0, x.rows, x.cols
    if x.dim() != 2 or x.stride(1) != 1:
        raise ValueError("x must be [M, K] with unit column stride")
    return x.data_ptr(), 0, x.stride(0), x.shape[0], x.shape[1]


def _check_out(t: torch.Tensor | Tiled, rows: int, cols: int, dtype: torch.dtype, dev: int, what: str) -> None:
    """A caller-provided output must be exactly what the kernel writes: the kernels see
    raw pointers and would write past a smaller buffer."""
    if isinstance(t, Tiled):
        if (t.rows, t.cols) != (rows, cols) or t.buf.numel() < padded_rows(rows) * cols:
            raise ValueError(f"{what} must be an operand-tiled [{rows}, {cols}], got [{t.rows}, {t.cols}]")
        if not t.buf.is_contiguous():
            raise ValueError(f"{what}'s buffer must be contiguous")
        t = t.buf
    elif tuple(t.shape) != (rows, cols) or t.stride(1) != 1:
        raise ValueError(f"{what} must be [{rows}, {cols}] with unit column stride, got {tuple(t.shape)}")
    if t.dtype != dtype:
        raise ValueError(f"{what} must be {dtype}, got {t.dtype}")
    if _lib.require_device(t) != dev:
        raise ValueError(f"{what} is on another device")


def _check(x: torch.Tensor | Tiled, w: torch.Tensor) -> int:
    xt = x.buf if isinstance(x, Tiled) else x
    if w.dim() != 2 or w.stride(1) != 1:
        raise ValueError("w must be [N, K] with unit column stride")
    if xt.dtype != w.dtype or not supported(w.dtype):
        raise ValueError(f"x and w must share dtype float16 or bfloat16, got {xt.dtype} and {w.dtype}")
    return _lib.require_device(xt, w)


def rows_linear(x: torch.Tensor | Tiled, w: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """``F.linear(x, w)`` for the few rows of a decode step: [M, N] in x's dtype."""
    dev = _check(x, w)
    xp, xt, xs, m, k = _x_args(x)
    n = w.shape[0]
    if w.shape[1] != k:
        raise ValueError(f"x has {k} columns but w is {tuple(w.shape)}")
    if out is None:
        out = torch.empty(m, n, dtype=w.dtype, device=w.device)
    _check_out(out, m, n, w.dtype, dev, "out")
    _lib.call("ts_rows_gemm", xp, xt, xs, w.data_ptr(), w.stride(0), out.data_ptr(), out.stride(0), None, 0,
              m, n, k, ROWS_STORE, _lib.dtype_code(w), _lib.stream_of(dev))  # fmt: skip
    return out


def rows_linear_partials(x: torch.Tensor | Tiled, w: torch.Tensor,
                         partial: torch.Tensor | None = None) -> tuple[torch.Tensor, int]:  # fmt: skip
    """fp32 partial sums of ``F.linear(x, w)`` over KS slices of K: ``(partial, KS)`` with
    ``partial[:KS]`` [KS, M, N]; ``add_rms_norm`` adds them to the residual."""
    dev = _check(x, w)
    xp, xt, xs, m, k = _x_args(x)
    n = w.shape[0]
    if w.shape[1] != k:
        raise ValueError(f"x has {k} columns but w is {tuple(w.shape)}")
    plan = rows_plan(m, n, k, ROWS_PARTIAL)
    if plan is None:
        raise ValueError(f"no projection shape for M={m}, N={n}, K={k}")
    ks = plan["k_splits"]
    if partial is not None and (partial.dtype != torch.float32 or not partial.is_contiguous()
                                or _lib.require_device(partial) != dev):  # fmt: skip
        raise ValueError("partial must be a contiguous float32 buffer on x's device")
    if partial is None:
        partial = torch.empty(ks * m * n, dtype=torch.float32, device=w.device)
    elif partial.numel() < ks * m * n:
        raise ValueError(f"partial holds {partial.numel()} floats; this projection needs {ks * m * n}")
    _lib.call("ts_rows_gemm", xp, xt, xs, w.data_ptr(), w.stride(0), None, 0, partial.data_ptr(),
              partial.numel(), m, n, k, ROWS_PARTIAL, _lib.dtype_code(w), _lib.stream_of(dev))  # fmt: skip
    return partial.view(-1)[: ks * m * n].view(ks, m, n), ks


def rows_silu_gate_up(x: torch.Tensor | Tiled, w_gate_up: torch.Tensor, out: Tiled | None = None) -> Tiled:
    """``silu(gate) * up`` with ``[gate | up] = F.linear(x, w_gate_up)`` (gate the first
    half of the weight's rows), operand-tiled for the down projection."""
    dev = _check(x, w_gate_up)
    xp, xt, xs, m, k = _x_args(x)
    if w_gate_up.shape[1] != k or w_gate_up.shape[0] % 2:
        raise ValueError(f"x has {k} columns but w_gate_up is {tuple(w_gate_up.shape)}")
    n = w_gate_up.shape[0] // 2
    if out is None:
        out = Tiled.empty(m, n, w_gate_up.dtype, w_gate_up.device)
    if not isinstance(out, Tiled):
        raise ValueError("out must be a Tiled (the SiLU epilogue writes the operand-tiled layout)")
    _check_out(out, m, n, w_gate_up.dtype, dev, "out")
    _lib.call("ts_rows_gemm", xp, xt, xs, w_gate_up.data_ptr(), w_gate_up.stride(0), out.buf.data_ptr(), 0,
              None, 0, m, n, k, ROWS_SILU, _lib.dtype_code(w_gate_up), _lib.stream_of(dev))  # fmt: skip
    return out


def add_rms_norm(x: torch.Tensor, partial: torch.Tensor | None, weight: torch.Tensor, eps: float,
                 tiled: bool = True, h: torch.Tensor | Tiled | None = None) -> torch.Tensor | Tiled:  # fmt: skip
    """``x += partial.sum(0)`` (rounded once, in place; skipped for ``partial`` None), then
    ``rms_norm(x, weight, eps)``, operand-tiled or row-major."""
    if x.dim() != 2 or x.stride(1) != 1:
        raise ValueError("x must be [M, N] with unit column stride")
    m, n = x.shape
    if not supported(x.dtype) or weight.dtype != x.dtype or weight.numel() != n:
        raise ValueError("x and weight must share dtype float16 or bfloat16, weight of x's width")
    ks = 0
    if partial is not None:
        if partial.dim() != 3 or tuple(partial.shape[1:]) != (m, n) or partial.dtype != torch.float32:
            raise ValueError(f"partial must be fp32 [KS, {m}, {n}], got {tuple(partial.shape)}")
        if not partial.is_contiguous():
            raise ValueError("partial must be contiguous")
        ks = partial.shape[0]
    dev = _lib.require_device(x, weight, *(() if partial is None else (partial,)))
    if h is None:
        h = Tiled.empty(m, n, x.dtype, x.device) if tiled else torch.empty_like(x)
    if isinstance(h, Tiled) != tiled:
        raise ValueError(f"h must be {'a Tiled' if tiled else 'a row-major tensor'} (tiled={tiled})")
    _check_out(h, m, n, x.dtype, dev, "h")
    hp = h.buf.data_ptr() if isinstance(h, Tiled) else h.data_ptr()
    hs = 0 if isinstance(h, Tiled) else h.stride(0)
    _lib.call("ts_add_rms_norm", x.data_ptr(), x.stride(0), None if partial is None else partial.data_ptr(), ks,
              weight.data_ptr(), x.data_ptr(), x.stride(0), hp, int(isinstance(h, Tiled)), hs, m, n, eps,
              _lib.dtype_code(x), _lib.stream_of(dev))  # fmt: skip
    return h
