"""ctypes binding of ``libedgerag_amd.so`` -- the only way Python reaches the HIP kernels.

``torch`` is imported before the library is opened. torch bundles its own HIP runtime, and a
library opened first would pull the system runtime in beside it; importing torch first makes the
dynamic loader resolve ``libamdhip64.so.7`` to the copy torch already mapped, so tensors, streams
and kernels all live in one runtime.

There is no fallback: if the library is missing, or a tensor is not on a HIP device, the call
raises. Every entry point returns a status code that is turned into :class:`EdgeragError` here.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch  # noqa: F401  -- must precede loading the library (single HIP runtime)

from edgerag_amd._build import LIB_PATH

c_i32 = ctypes.c_int32
c_i64 = ctypes.c_int64
c_f32 = ctypes.c_float
c_vp = ctypes.c_void_p
c_i32p = ctypes.POINTER(ctypes.c_int32)
c_i64p = ctypes.POINTER(ctypes.c_int64)

EDGERAG_OK = 0
EDGERAG_EINVAL = 1
EDGERAG_EHIP = 2
EDGERAG_EWORKSPACE = 3
EDGERAG_EUNSUPPORTED = 4

ATTN_TILES, ATTN_ROWS, ATTN_COMBINE, ATTN_ALL = 1, 2, 4, 7
ATTN_TILES_SHARED = 8  # modifier of ATTN_TILES: one tile workgroup per CU, beside decode rows
PLAN_SPLIT_ROWS = 1  # edgerag_attn_plan_ex flag: decode rows as KV splits merged by a launch
PLAN_OVERLAP = 2  # edgerag_attn_plan_ex flag: plan tiles beside rows (two streams) whenever both
PLAN_WORD_OVERLAP = 20  # plan word: 1 when the plan is for tiles and rows on two streams
QUANT_WORKSPACE_MAX = 8 * 1024 * 1024  # bound of edgerag_quant_linear_workspace_bytes
ATTN_SCRATCH_BYTES = 32 * 1024 * 1024  # static partials of edgerag_paged_attention_noalloc

DTYPE_CODES = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}

#: name -> (argtypes, restype). Mirrors the declarations of include/*.h one to one.
SIGNATURES: dict[str, tuple[list, object]] = {
    "edgerag_last_error": ([], ctypes.c_char_p),
    "edgerag_version": ([], ctypes.c_char_p),
    "edgerag_kv_append": (
        [c_vp, c_vp, c_i32, c_i64, c_i64, c_vp, c_i32, c_vp, c_vp, c_i32, c_i32, c_i32, c_i32,
         c_i32, c_vp],
        c_i32,
    ),
    "edgerag_kv_gather": ([c_vp, c_i32, c_i32, c_i32, c_i32, c_i32, c_vp, c_i32, c_vp, c_vp], c_i32),
    "edgerag_kv_copy_blocks": (
        [c_vp, c_i32, c_i32, c_i32, c_i32, c_i32, c_vp, c_vp, c_i32, c_vp],
        c_i32,
    ),
    "edgerag_attn_plan": (
        [c_vp, c_vp, c_i32, c_i32, c_i32, c_i32, c_i32, c_i32, c_i32, c_vp, c_i64, c_i64p, c_i64p],
        c_i32,
    ),
    "edgerag_attn_plan_ex": (
        [c_vp, c_vp, c_i32, c_i32, c_i32, c_i32, c_i32, c_i32, c_i32, c_i32, c_vp, c_i64, c_i64p,
         c_i64p],
        c_i32,
    ),
    "edgerag_paged_attention": (
        [c_vp, c_vp, c_i64, c_vp, c_i64, c_i64, c_vp, c_vp, c_i32, c_vp, c_i64, c_vp, c_vp, c_i32,
         c_i32, c_i32, c_i32, c_i32, c_i32, c_i32, c_f32, c_vp, c_i64, c_i64, c_vp, c_i64, c_i32,
         c_vp],
        c_i32,
    ),
    "edgerag_paged_attention_noalloc": (
        [c_vp, c_vp, c_i64, c_vp, c_i64, c_i64, c_vp, c_vp, c_i32, c_vp, c_i64, c_vp, c_vp, c_i32,
         c_i32, c_i32, c_i32, c_i32, c_i32, c_i32, c_f32, c_vp, c_i64, c_i64, c_i32, c_vp],
        c_i32,
    ),
    "edgerag_paged_attention_append": (
        [c_vp, c_vp, c_i32, c_i64, c_i64, c_vp, c_vp, c_vp, c_i64, c_vp, c_i64, c_i64, c_vp, c_vp,
         c_i32, c_vp, c_i64, c_vp, c_vp, c_i32, c_i32, c_i32, c_i32, c_i32, c_i32, c_i32, c_f32,
         c_vp, c_i64, c_i64, c_vp, c_i64, c_vp],
        c_i32,
    ),
    "edgerag_paged_attention_fixed": (
        [c_vp, c_i32, c_i32, c_i32, c_i64, c_i32, c_i32, c_vp, c_i64, c_i64, c_vp, c_vp, c_i32,
         c_vp, c_i64,
         c_vp, c_vp, c_i32, c_i32, c_i32, c_i32, c_i32, c_f32, c_vp, c_i64, c_i64, c_vp, c_i64,
         c_vp],
        c_i32,
    ),
    "edgerag_rmsnorm": (
        [c_vp, c_i64, c_vp, c_i64, c_vp, c_vp, c_i64, c_vp, c_i64, c_i32, c_i32, c_f32, c_i32,
         c_vp],
        c_i32,
    ),
    "edgerag_embed_rmsnorm": (
        [c_vp, c_i32, c_vp, c_i64, c_i32, c_vp, c_vp, c_i64, c_vp, c_i64, c_i32, c_f32,
         c_vp, c_vp, c_vp, c_i32, c_i32, c_vp, c_vp, c_i32, c_vp],
        c_i32,
    ),
    "edgerag_rope_append": (
        [c_vp, c_i64, c_vp, c_vp, c_vp, c_i32, c_i32, c_i32, c_i32, c_i32, c_vp, c_i64, c_vp,
         c_vp, c_vp, c_i32, c_i32, c_i32, c_vp],
        c_i32,
    ),
    "edgerag_rope_rows": ([c_vp, c_i32, c_vp, c_vp, c_i32, c_i32, c_i32, c_vp, c_vp, c_vp],
                          c_i32),
    "edgerag_silu_mul": ([c_vp, c_i64, c_i32, c_i32, c_vp, c_i64, c_i32, c_vp], c_i32),
    "edgerag_argmax_rows": ([c_vp, c_i32, c_i32, c_i32, c_i64, c_vp, c_vp], c_i32),
    "edgerag_lm_head_argmax": (
        [c_vp, c_i64, c_i32, c_i32, c_vp, c_i32, c_vp, c_i64, c_vp, c_vp, c_i64, c_vp], c_i32,
    ),
    "edgerag_lm_head_workspace_bytes": ([c_i32, c_i32], c_i64),
    "edgerag_attn_fixed_row_items": ([c_i32, c_i32, c_i32, c_i32], c_i64),
    "edgerag_lm_head_argmax_supported": ([c_i32, c_i32], c_i32),
    "edgerag_quantize": ([c_vp, c_i32, c_i32, c_i32, c_i32, c_i32, c_vp, c_vp, c_vp], c_i32),
    "edgerag_dequantize": ([c_vp, c_vp, c_i32, c_i32, c_i32, c_i32, c_vp, c_vp], c_i32),
    "edgerag_quant_linear": (
        [c_vp, c_i32, c_i64, c_i32, c_i32, c_vp, c_vp, c_vp, c_i32, c_i32, c_i32, c_vp, c_i64,
         c_vp],
        c_i32,
    ),
    "edgerag_quant_linear_ws": (
        [c_vp, c_i32, c_i64, c_i32, c_i32, c_vp, c_vp, c_vp, c_i32, c_i32, c_i32, c_vp, c_i64,
         c_vp, c_i64, c_vp],
        c_i32,
    ),
    "edgerag_quant_linear_workspace_bytes": ([c_i32, c_i32, c_i32, c_i32, c_i32], c_i64),
    "edgerag_quant_linear_swiglu": (
        [c_vp, c_i32, c_i64, c_i32, c_i32, c_vp, c_vp, c_vp, c_i32, c_i32, c_i32, c_vp, c_i64,
         c_vp, c_i32, c_f32, c_vp],
        c_i32,
    ),
    "edgerag_quant_linear_swiglu_supported": (
        [c_i32, c_i32, c_i32, c_i32, c_i32, c_i32, c_i32], c_i32,
    ),
    "edgerag_quant_linear_rope_append": (
        [c_vp, c_i32, c_i64, c_i32, c_i32, c_vp, c_vp, c_vp, c_i32, c_i32, c_vp, c_vp, c_i32,
         c_i32, c_i32, c_vp, c_i64, c_vp, c_vp, c_vp, c_i32, c_i32, c_vp, c_i32, c_f32, c_vp],
        c_i32,
    ),
    "edgerag_quant_linear_rope_append_supported": (
        [c_i32, c_i32, c_i32, c_i32, c_i32, c_i32, c_i32, c_i32, c_i32], c_i32,
    ),
    "edgerag_quant_linear_residual": (
        [c_vp, c_i32, c_i64, c_i32, c_i32, c_vp, c_vp, c_vp, c_i32, c_i32, c_i32, c_vp, c_i64,
         c_vp, c_i64, c_vp, c_vp, c_vp, c_i64, c_vp],
        c_i32,
    ),
    "edgerag_quant_linear_residual_parts": ([c_i32, c_i32, c_i32, c_i32, c_i32, c_i32], c_i32),
}


class EdgeragError(RuntimeError):
    """A non-zero status from the native library, carrying its message."""

    def __init__(self, fn: str, code: int, message: str) -> None:
        super().__init__(f"{fn} failed ({code}): {message}")
        self.code = code


_LIB: ctypes.CDLL | None = None


def library_path() -> Path:
    return Path(os.environ.get("EDGERAG_AMD_LIB", LIB_PATH))


def load() -> ctypes.CDLL:
    """Open the library once and attach the C signatures. Raises if it has not been built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    path = library_path()
    if not path.exists():
        raise RuntimeError(
            f"{path} is missing: build it with `python -m edgerag_amd._build` (needs hipcc). "
            "edgerag_amd has no CPU fallback."
        )
    lib = ctypes.CDLL(str(path))
    for name, (argtypes, restype) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = restype
    _LIB = lib
    return lib


_FNS: dict = {}  # entry point name -> its bound ctypes function


def call(name: str, *args) -> None:
    """Invoke an entry point and raise EdgeragError on a non-zero status."""
    fn = _FNS.get(name)
    if fn is None:
        fn = _FNS[name] = getattr(load(), name)
    rc = fn(*args)
    if rc != EDGERAG_OK:
        message = load().edgerag_last_error().decode(errors="replace")
        raise EdgeragError(name, rc, message)


def version() -> str:
    return load().edgerag_version().decode()


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return DTYPE_CODES[dtype]
    except KeyError:
        raise TypeError(f"edgerag_amd supports float32/float16/bfloat16, not {dtype}") from None


def require_device(*tensors: torch.Tensor | None) -> None:
    """Every tensor handed to a kernel must live on the HIP device: there is no CPU path."""
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise ValueError(
                "edgerag_amd runs on the MI355X only: tensor on "
                f"{t.device} (move it to the HIP device first)"
            )


# torch's raw current-stream query: one C call where torch.cuda.current_stream builds a Stream
# object (a few microseconds of host time per launch).
_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_ptr(device: torch.device | None = None) -> int:
    """The current torch stream on ``device`` as a raw hipStream_t."""
    if _RAW_STREAM is not None:
        if isinstance(device, str):
            device = torch.device(device)
        index = device.index if isinstance(device, torch.device) else device
        return _RAW_STREAM(torch.cuda.current_device() if index is None else index)
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()
