"""ctypes binding of librlt_kv.so (declared in include/rlt_kv.h).

torch is imported first so the library binds to the HIP runtime torch already
loaded (one runtime, one set of streams).  There is no fallback: if the
library is missing every operation raises.
"""

from __future__ import annotations

import ctypes
import functools
from ctypes import POINTER, c_char_p, c_float, c_int, c_int64, c_void_p
from pathlib import Path

import torch  # noqa: F401  (binds the shared HIP runtime before the library loads)

LIBRARY_PATH = Path(__file__).resolve().parent / "librlt_kv.so"

RLT_OK = 0
RLT_EINVAL = -1
RLT_EUNSUPPORTED = -2
RLT_ELAUNCH = -3
RLT_EWORKSPACE = -4

RLT_FLOAT32 = 0
RLT_FLOAT16 = 1
RLT_BFLOAT16 = 2

DTYPE_CODES = {torch.float32: RLT_FLOAT32, torch.float16: RLT_FLOAT16, torch.bfloat16: RLT_BFLOAT16}

_i64p = POINTER(c_int64)

# name -> (restype, argtypes); one entry per function of include/rlt_kv.h.
SIGNATURES = {
    "rlt_last_error": (c_char_p, []),
    "rlt_version": (c_char_p, []),
    "rlt_kv_append": (
        c_int,
        [c_void_p, c_void_p, _i64p, c_void_p, _i64p, c_void_p, _i64p, c_void_p, c_void_p]
        + [c_int64] * 7
        + [c_int, c_void_p],
    ),
    "rlt_rope_kv_append": (
        c_int,
        [c_void_p, c_void_p, _i64p, c_void_p, _i64p, c_void_p, _i64p, c_void_p, _i64p, c_void_p, c_void_p, _i64p]
        + [c_void_p, _i64p, c_void_p, c_void_p]
        + [c_int64] * 9
        + [c_int, c_void_p],
    ),
    "rlt_gather_rows": (
        c_int,
        [c_void_p, c_int64, c_int64, c_void_p, c_int64, c_int64, c_void_p, c_int64, c_int64, c_void_p],
    ),
    "rlt_scatter_rows": (
        c_int,
        [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64, c_int64, c_int64, c_void_p],
    ),
    "rlt_patch_tables": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p]),
    "rlt_kv_export_pages": (
        c_int,
        [c_void_p, c_void_p, c_int64, c_int64, c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_int64, c_void_p],
    ),
    "rlt_kv_import_pages": (
        c_int,
        [c_void_p, c_void_p, c_int64, c_int64, c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_int64, c_void_p],
    ),
    "rlt_copy_segments": (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_void_p]),
    "rlt_paged_decode_workspace_bytes": (c_int64, [c_int64] * 4),
    "rlt_paged_decode": (
        c_int,
        [c_void_p, _i64p, c_void_p, c_void_p, _i64p, c_void_p, c_int64, c_int64, c_void_p, c_void_p, _i64p]
        + [c_int64] * 6
        + [c_float, c_int, c_void_p, c_int64, c_void_p],
    ),
    "rlt_paged_decode_append": (
        c_int,
        [c_void_p, _i64p, c_void_p, c_void_p, _i64p, c_void_p, c_int64, c_int64, c_void_p, c_void_p, _i64p]
        + [c_int64] * 6
        + [c_float, c_int, c_void_p, _i64p, c_void_p, _i64p, c_void_p, c_void_p, c_int64, c_void_p, c_int64, c_void_p],
    ),
    "rlt_paged_decode_no_alloc": (
        c_int,
        [c_void_p, _i64p, c_void_p, c_void_p, _i64p, c_void_p, c_int64, c_int64, c_void_p, c_void_p, _i64p]
        + [c_int64] * 6
        + [c_float, c_int, c_void_p],
    ),
    "rlt_paged_decode_no_alloc_rows_per_launch": (c_int64, [c_int64] * 3),
    "rlt_static_device_bytes": (c_int64, []),
    "rlt_paged_decode_shared_prefix": (
        c_int,
        [c_void_p, _i64p, c_void_p, c_void_p, _i64p, c_void_p, c_int64, c_int64, c_void_p, c_void_p, _i64p]
        + [c_int64] * 6
        + [c_float, c_int, c_void_p, _i64p, c_void_p, _i64p, c_void_p, c_void_p, c_int64]
        + [c_void_p] + [c_int64] * 4
        + [c_void_p, c_int64, c_void_p],
    ),
    "rlt_paged_prefill_workspace_bytes": (c_int64, [c_int64] * 7 + [c_int]),
    "rlt_paged_prefill": (
        c_int,
        [c_void_p, _i64p, c_void_p, c_void_p, _i64p, c_void_p, c_int64, c_int64, c_void_p, c_void_p]
        + [c_int64] * 3
        + [c_void_p, _i64p]
        + [c_int64] * 5
        + [c_float, c_int, c_void_p, c_int64, c_void_p],
    ),
    "rlt_kv_finalize": (
        c_int,
        [c_void_p, c_int64, c_void_p, c_int64, c_int64, c_int64, c_void_p, c_void_p, _i64p]
        + [c_int64] * 6
        + [c_int, c_void_p],
    ),
    "rlt_kv_copy_token": (
        c_int,
        [c_void_p, c_void_p, _i64p, c_int64, _i64p, c_int64, c_int64] + [c_int64] * 5 + [c_int, c_void_p],
    ),
    "rlt_kv_gather": (
        c_int,
        [c_void_p, c_void_p, _i64p, c_int64, c_void_p, c_int64, c_void_p, c_void_p]
        + [c_int64] * 5
        + [c_int, c_void_p],
    ),
    "rlt_build_decode_metadata": (
        c_int,
        [c_void_p, c_int64, c_int64, c_void_p, c_int64, c_int64, c_int64, c_int64]
        + [c_void_p] * 6
        + [c_int64, c_int64, c_void_p],
    ),
    "rlt_stage_prefill": (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_void_p]),
    "rlt_expand_prefill": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int64, c_void_p, c_void_p, c_int64, c_void_p],
    ),
}

_lib = None


def load(path: Path | str = LIBRARY_PATH) -> ctypes.CDLL:
    """Load (once) and type the library; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    path = Path(path)
    if not path.exists():
        raise RuntimeError(
            f"{path} is missing: build the HIP library first (python __graft_entry__.py build "
            "or python -m vllm_rlt_amd._build); there is no non-HIP fallback"
        )
    lib = ctypes.CDLL(str(path))
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    _lib = lib
    return lib


def last_error() -> str:
    return load().rlt_last_error().decode()


def check(rc: int, name: str) -> None:
    """Turn a status code into the reference's exception types."""
    if rc == RLT_OK:
        return
    message = last_error() or name
    if rc in (RLT_EINVAL, RLT_EUNSUPPORTED, RLT_EWORKSPACE):
        raise ValueError(message)
    raise RuntimeError(message)


@functools.lru_cache(maxsize=1024)
def _short_int64_array(values: tuple) -> ctypes.Array:
    return (c_int64 * len(values))(*values)


def int64_array(values) -> ctypes.Array:
    """A C int64 array holding `values`.  Short ones (tensor strides) are built
    once per distinct value and shared between calls: every entry point takes
    them as `const int64_t*` and only reads them."""
    if type(values) is not tuple:  # tensor strides already are tuples of ints
        values = tuple(int(v) for v in values)
    if len(values) <= 8:
        return _short_int64_array(values)
    return (c_int64 * len(values))(*values)


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return DTYPE_CODES[dtype]
    except KeyError:
        raise ValueError("KV dtype must be float32, float16, or bfloat16") from None


# The current stream's raw handle without building a Stream object per call.
_raw_current_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_handle(device: torch.device) -> int:
    """The HIP stream torch currently issues to on `device`."""
    if _raw_current_stream is not None:
        return _raw_current_stream(device.index if device.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(device).cuda_stream
