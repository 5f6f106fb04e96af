"""ctypes binding of ``libtinyserve_amd.so`` (the C ABI in ``include/tinyserve_amd.h``).

``torch`` is imported first on purpose: it loads the HIP runtime it ships
(``libamdhip64.so.7``), and the library then binds to that same runtime instead of a
second copy, so both share one device context, one allocator and torch's streams.

There is no fallback: if the library is missing, or a tensor is not on a HIP device,
the entry points raise instead of computing anything on the CPU.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch

# The in-tree build; TINYSERVE_AMD_LIB may name another build of the same sources.
LIB_PATH = Path(os.environ.get("TINYSERVE_AMD_LIB") or Path(__file__).resolve().with_name("libtinyserve_amd.so"))

_c_i32p = ctypes.POINTER(ctypes.c_int32)
_c_i64p = ctypes.POINTER(ctypes.c_int64)
_vp, _i, _i64, _f = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float

# Every exported function and its argument types, in header order.
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "ts_version": (_i, []),
    "ts_strerror": (ctypes.c_char_p, [_i]),
    "ts_decode_split": (
        _i,
        [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,  # q k v bt lens out m l acc
         _i, _i, _i, _i, _i,  # B Hq Hkv D block_size
         _i64, _i64, _i64, _i64, _i64, _i64, _i64,  # strides
         _i, _i, _i, _f, _i, _vp],  # max_blocks splits head_tile scale dtype stream
    ),
    "ts_decode_plan": (_i, [_i, _i, _i, _i, _i, _i, _i, _i, _i, _c_i32p]),
    "ts_decode_attention_noalloc": (
        _i,
        [_vp, _vp, _vp, _vp, _vp, _vp,  # q k v bt lens out
         _i, _i, _i, _i, _i,  # B Hq Hkv D block_size
         _i64, _i64, _i64, _i64, _i64, _i64, _i64,  # strides
         _i, _i, _i, _f, _i, _vp],  # max_blocks splits head_tile scale dtype stream
    ),
    "ts_decode_combine": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i64, _i64, _i, _i, _vp]),
    "ts_prefill_varlen": (
        _i,
        [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,  # q k v out bt q_starts q_lens ctx_lens
         _i, _i, _i, _i, _i, _i, _i64,  # R Hq Hkv D block_size max_q_len n_rows
         _i64, _i64, _i64, _i64, _i64, _i64, _i64,  # strides
         _f, _i, _vp],
    ),
    "ts_rms_norm_rows": (_i, [_vp, _vp, _vp, _i, _i, _i64, _i64, _f, _i, _vp]),
    "ts_qk_norm_rope_store": (
        _i,
        [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,  # tensors
         _i, _i, _i, _i,  # T Hq Hkv D
         *([_i64] * 11),  # strides
         _f, _i, _i, _vp],
    ),
    "ts_rope_cos_sin": (_i, [_vp, _i, _i, ctypes.c_double, _vp, _vp, _i64, _vp]),
    "ts_rows_gemm": (_i, [_vp, _i, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _i, _i, _i, _i, _i, _vp]),
    "ts_rows_gemm_plan": (_i, [_i, _i, _i, _i, _c_i32p]),
    "ts_add_rms_norm": (_i, [_vp, _i64, _vp, _i, _vp, _vp, _i64, _vp, _i, _i64, _i, _i, _f, _i, _vp]),
}  # fmt: skip

EXPORTS = tuple(SIGNATURES)

DTYPES = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """The loaded library (raises RuntimeError if it has not been built)."""
    global _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH.name} is not built: run `python -m tinyserve_amd.build` "
                    "(the HIP kernels have no CPU fallback)"
                )
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


_fns: dict[str, object] = {}


def call(name: str, *args: object) -> None:
    """Call entry point ``name``; raise on a non-zero status."""
    fn = _fns.get(name)
    if fn is None:
        fn = _fns[name] = getattr(load(), name)
    rc = fn(*args)
    if rc != 0:
        msg = load().ts_strerror(rc).decode()
        if rc < 0:
            raise ValueError(f"{name}: {msg}")
        raise RuntimeError(f"{name}: HIP error {rc}: {msg}")


def call_status(name: str, *args: object) -> int:
    """Call entry point ``name`` and return its status; raise only on a HIP error (a
    positive status), so the caller can take another path on a TS_E* code."""
    fn = _fns.get(name)
    if fn is None:
        fn = _fns[name] = getattr(load(), name)
    rc = fn(*args)
    if rc > 0:
        raise RuntimeError(f"{name}: HIP error {rc}: {load().ts_strerror(rc).decode()}")
    return rc


TS_EUNSUPPORTED = -2


def dtype_code(t: torch.Tensor) -> int:
    try:
        return DTYPES[t.dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {t.dtype}: float32, float16 or bfloat16") from None


def require_device(*tensors: torch.Tensor) -> int:
    """Index of the common HIP device of ``tensors``; RuntimeError for CPU tensors (no
    fallback)."""
    idx = -1
    for t in tensors:
        if not t.is_cuda:
            raise RuntimeError(
                "tinyserve_amd kernels run on a HIP device only (no CPU fallback); "
                f"got a tensor on {t.device}"
            )
        i = t.get_device()
        if idx < 0:
            idx = i
        elif i != idx:
            raise ValueError(f"tensors on different devices: cuda:{idx} and cuda:{i}")
    return idx


def stream_of(dev: int) -> int:
    """Handle of torch's current stream on device ``dev`` (the kernels launch there)."""
    return torch._C._cuda_getCurrentRawStream(dev)


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()
