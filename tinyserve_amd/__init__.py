"""tinyserve_amd: TinyServe's attention hot path as hand-written HIP kernels for MI355X
(gfx950), behind the reference's Python kernel entry points.

Modules (each mirrors one reference module, same function names and arguments):
    hip_attention  -- paged decode attention, split-K and combine (triton_attention.py)
    hip_prefill    -- varlen causal prefill attention (triton_prefill.py)
    hip_fused      -- rms_norm_rows, qk_norm_rope_store (triton_fused.py)
The kernels live in ``libtinyserve_amd.so`` (C ABI: include/tinyserve_amd.h), built by
``python -m tinyserve_amd.build``.
"""

__version__ = "0.1.0"
