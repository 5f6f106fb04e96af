"""The no-allocation decode entry point (``ts_decode_attention_noalloc``) against the
allocating one (GPU).

The variant runs the same split and combine kernels as the allocating HBM-partials path
(``ts_decode_split`` with caller partial buffers, then ``ts_decode_combine``), with the
fp32 split partials in the library's static per-device scratch array instead of caller
buffers, so its output must equal that path's at the same split count bit for bit (and,
at one split, ``launch_paged_decode_split``'s). Two calls in a row, the second smaller,
share the scratch: nothing the first call left may leak into the second.
"""

from __future__ import annotations

import pytest
import torch

from tinyserve_amd import _lib
from tinyserve_amd import hip_attention as ha
from tinyserve_amd.workloads import DecodeCase, decode_case

pytestmark = pytest.mark.gpu
DEVICE = "cuda"


def on_gpu(c: DecodeCase) -> DecodeCase:
    return DecodeCase(*(t.to(DEVICE) for t in c.args()), c.scale, c.block_size)


def noalloc(c: DecodeCase, splits: int) -> torch.Tensor:
    """One call of the C entry point, into a NaN-filled output."""
    out = torch.full_like(c.q, float("nan"))
    b, hq, d = c.q.shape
    _lib.call("ts_decode_attention_noalloc", c.q.data_ptr(), c.k_cache.data_ptr(), c.v_cache.data_ptr(),
              c.block_tables.data_ptr(), c.context_lens.data_ptr(), out.data_ptr(), b, hq,
              c.k_cache.shape[1], d, c.block_size, c.q.stride(0), c.q.stride(1), out.stride(0),
              out.stride(1), c.k_cache.stride(0), c.k_cache.stride(1), c.block_tables.stride(0),
              c.block_tables.shape[1], splits, 0, c.scale, _lib.dtype_code(c.q),
              _lib.stream_of(0))  # fmt: skip
    return out


def allocating(c: DecodeCase, splits: int) -> torch.Tensor:
    """The allocating entry points with caller buffers: fp32 partials in torch-allocated
    HBM and the combine launch (one split: the launcher's single launch)."""
    if splits == 1:
        return ha.launch_paged_decode_split(*c.args(), c.scale, c.block_size, num_splits=1)
    b, hq, d = c.q.shape
    out = torch.empty_like(c.q)
    m = torch.empty((b, hq, splits), dtype=torch.float32, device=DEVICE)
    l = torch.empty_like(m)  # noqa: E741
    acc = torch.empty((b, hq, splits, d), dtype=torch.float32, device=DEVICE)
    dt, stream = _lib.dtype_code(c.q), _lib.stream_of(0)
    _lib.call("ts_decode_split", c.q.data_ptr(), c.k_cache.data_ptr(), c.v_cache.data_ptr(),
              c.block_tables.data_ptr(), c.context_lens.data_ptr(), None, m.data_ptr(), l.data_ptr(),
              acc.data_ptr(), b, hq, c.k_cache.shape[1], d, c.block_size, c.q.stride(0), c.q.stride(1),
              0, 0, c.k_cache.stride(0), c.k_cache.stride(1), c.block_tables.stride(0),
              c.block_tables.shape[1], splits, 0, c.scale, dt, stream)  # fmt: skip
    _lib.call("ts_decode_combine", m.data_ptr(), l.data_ptr(), acc.data_ptr(), out.data_ptr(),
              b, hq, d, out.stride(0), out.stride(1), splits, dt, stream)  # fmt: skip
    return out


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_noalloc_equals_the_allocating_entry_point(dtype: torch.dtype) -> None:
    # First call: 64 sequences of mixed lengths at the reference's 16 splits (8.5 MB of
    # partials at fp32 D=128); second call: 6 sequences at 3 splits, then one split (no
    # scratch at all).
    big = on_gpu(decode_case([1 + (389 * i) % 1500 for i in range(64)], dtype=dtype, seed=21))
    small = on_gpu(decode_case([1, 40, 17, 300, 2, 99], dtype=dtype, seed=22))
    for c, splits in ((big, 16), (small, 3), (small, 1)):
        got = noalloc(c, splits)
        want = allocating(c, splits)
        torch.cuda.synchronize()
        assert torch.isfinite(got).all(), splits
        assert torch.equal(got, want), f"B={c.q.shape[0]} splits={splits}"
    # And through the Python wrapper, into a caller-owned output.
    out = torch.empty_like(small.q)
    got = ha.launch_paged_decode_split_noalloc(*small.args(), small.scale, small.block_size, out, num_splits=5)
    want = allocating(small, 5)
    assert got is out and torch.equal(got, want)


def test_noalloc_rejects_partials_beyond_the_scratch() -> None:
    # 2048 sequences x 16 heads x 16 splits x 130 floats = 272 MB > 16 MiB: refused before
    # any launch, with the library's own error.
    c = on_gpu(decode_case([1, 2], dtype=torch.float16, seed=3))
    q = c.q[:1].expand(2048, -1, -1)
    lens = c.context_lens.repeat(1024)
    tables = c.block_tables.repeat(1024, 1)
    out = torch.empty(q.shape, dtype=q.dtype, device=DEVICE)
    with pytest.raises(ValueError, match="scratch"):
        ha.launch_paged_decode_split_noalloc(q, c.k_cache, c.v_cache, tables, lens, c.scale, c.block_size,
                                             out, num_splits=16)  # fmt: skip
