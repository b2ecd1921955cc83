"""ctypes binding of ``libtorque_hip.so`` (the C ABI declared in include/torque_hip.h).

torch is imported before the library is opened: torch ships its own HIP
runtime (soname ``libamdhip64.so.7``) and the library must bind to that same
runtime so that torch's streams and device pointers are valid in it.

There is no CPU fallback: if the library is missing or no GPU is visible the
entry points raise.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch  # noqa: F401  -- load torch's HIP runtime first

LIB_NAME = "libtorque_hip.so"
LIB_PATH = Path(__file__).resolve().with_name(LIB_NAME)

ABI_VERSION = 4

TQ_OK = 0
TQ_ERR_BAD_ARG = -1
TQ_ERR_UNSUPPORTED = -2
TQ_ERR_LAUNCH = -3

TQ_F32 = 0
TQ_F16 = 1

TQ_ROTATE_KEYS = 1
TQ_ROTATE_VALUES = 2
TQ_ROTATE_QUERY = 1
TQ_INVERSE_OUTPUT = 2
TQ_F32_PRODUCTS = 4
TQ_MATRIX_PRODUCTS = 8

_p = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64
_f = ctypes.c_float
_sz = ctypes.c_size_t

# name -> (restype, argtypes)
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "tq_abi_version": (_i, []),
    "tq_last_error": (ctypes.c_char_p, []),
    "tq_fwht": (_i, [_p, _i, _p, _i64, _i, _p, _p, _i, _p]),
    "tq_quantize_pack": (_i, [_p, _i64, _i, _i, _p, _p, _p]),
    "tq_append": (_i, [_p, _p, _i, _i, _i, _i64, _i, _i, _p, _p, _i, _p, _p, _p, _p, _i64, _i64, _p]),
    "tq_append_scaled": (_i, [_p, _p, _i, _i, _i, _i64, _i, _i, _p, _p, _i, _p, _p, _p, _p, _p, _p, _i64, _i64, _p]),
    "tq_quantize_dequantize": (_i, [_p, _p, _i, _i64, _i, _i, _p, _p, _i, _p, _p, _p, _p, _p, _p, _p]),
    "tq_quantize_dequantize_scaled": (_i, [_p, _p, _i, _i64, _i, _i, _p, _p, _i, _p, _p, _p, _p, _p, _p, _p]),
    "tq_unpack_dequantize": (_i, [_p, _i64, _i64, _i64, _i, _i, _p, _p, _p]),
    "tq_unpack_dequantize_scaled": (_i, [_p, _p, _i64, _i64, _i64, _i, _i, _p, _p, _p]),
    "tq_decode_default_splits": (_i, [_i, _i, _i, _i, _i, _i, _i64, _i]),
    "tq_decode_split_kernel": (ctypes.c_char_p, [_i, _i, _i, _i, _i, _i, _i, _i64, _i, _i]),
    "tq_decode_workspace_bytes": (_sz, [_i, _i, _i, _i, _i, _i]),
    "tq_decode": (
        _i,
        [_p, _i, _i, _i, _i, _i, _i, _p, _p, _i64, _i64, _p, _p, _p, _p, _i, _p, _p, _i, _p, _sz, _p, _p],
    ),
    "tq_decode_noalloc": (
        _i,
        [_p, _i, _i, _i, _i, _i, _i, _p, _p, _i64, _i64, _p, _p, _p, _p, _i, _p, _p, _i, _p, _p],
    ),
    "tq_decode_scaled": (
        _i,
        [_p, _i, _i, _i, _i, _i, _i, _p, _p, _p, _p, _i64, _i64, _p, _p, _p, _p, _i, _p, _p, _i, _p, _sz, _p, _p],
    ),
    "tq_decode_scaled_timed": (
        _i,
        [_p, _i, _i, _i, _i, _i, _i, _p, _p, _p, _p, _i64, _i64, _p, _p, _p, _p, _i, _p, _p, _i, _p, _sz, _p, _p, _p,
         _p],
    ),
    "tq_decode_timed": (
        _i,
        [_p, _i, _i, _i, _i, _i, _i, _p, _p, _i64, _i64, _p, _p, _p, _p, _i, _p, _p, _i, _p, _sz, _p, _p, _p, _p],
    ),
    "tq_decode_step_timed": (
        _i,
        [_p, _i, _i, _i, _i, _i, _i, _p, _p, _i64, _i64, _p, _p, _p, _p, _i, _p, _p, _i, _p, _sz, _p, _p, _p, _p, _p,
         _p],
    ),
    "tq_decode_append": (
        _i,
        [_p, _i, _p, _p, _i, _i, _i, _i, _i, _i, _p, _p, _i64, _i64, _p, _p, _p, _p, _p, _p, _i, _i, _i, _p, _sz, _p,
         _p],
    ),
    "tq_decode_dense": (_i, [_p, _i, _p, _p, _i, _i, _i, _i, _i, _i64, _i64, _p, _p, _i, _i, _p, _sz, _p, _p]),
    "tq_decode_dense_timed": (
        _i,
        [_p, _i, _p, _p, _i, _i, _i, _i, _i, _i64, _i64, _p, _p, _i, _i, _p, _sz, _p, _p, _p, _p],
    ),
    "tq_score_packed": (_i, [_p, _p, _i, _i64, _i, _i, _p, _p, _p]),
    "tq_softmax_rows": (_i, [_p, _i, _i64, _f, _p, _p]),
    "tq_accumulate_packed": (_i, [_p, _p, _i, _i64, _i, _i, _p, _p, _p]),
    "tq_stream_read": (_i, [_p, _sz, _p, _i, _p, _p, _p]),
}

_LIB: ctypes.CDLL | None = None


class TorqueHIPError(RuntimeError):
    """A HIP launch failed inside libtorque_hip."""


def library_path() -> Path:
    override = os.environ.get("TORQUE_HIP_LIB")
    return Path(override) if override else LIB_PATH


def load() -> ctypes.CDLL:
    """Open the library once and declare every C entry point."""
    global _LIB
    if _LIB is not None:
        return _LIB
    path = library_path()
    if not path.exists():
        raise RuntimeError(
            f"{path} is not built; run `python -c 'import __graft_entry__ as g; g.build()'` from the repository root"
        )
    lib = ctypes.CDLL(str(path))
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    version = lib.tq_abi_version()
    if version != ABI_VERSION:
        raise RuntimeError(f"libtorque_hip ABI version {version} does not match the bindings ({ABI_VERSION})")
    _LIB = lib
    return lib


def check(rc: int) -> None:
    """Map a TQ_* status to the reference's exception types."""
    if rc == TQ_OK:
        return
    message = load().tq_last_error().decode("utf-8", "replace")
    if rc in (TQ_ERR_BAD_ARG, TQ_ERR_UNSUPPORTED):
        raise ValueError(message)
    raise TorqueHIPError(message or f"libtorque_hip error {rc}")


_NOT_STATUS = {"tq_abi_version", "tq_last_error", "tq_decode_workspace_bytes", "tq_decode_split_kernel"}


def call(name: str, *args) -> int:
    """Call an entry point; negative int results raise (ValueError / TorqueHIPError)."""
    fn = getattr(load(), name)
    rc = fn(*args)
    if name not in _NOT_STATUS and rc < 0:
        check(rc)
    return rc


def split_kernel(kv_heads: int, query_heads: int, head_dim: int, bits: int, flags: int, query_dtype: int,
                 seq_len: int, num_layers: int = 1, n_splits: int = 0, num_cus: int = 0) -> str:
    """Name of the split kernel tq_decode launches for this call shape (tq_decode_split_kernel; n_splits 0
    is the default plan, num_cus 0 the current device's compute units)."""
    name = load().tq_decode_split_kernel(num_layers, kv_heads, query_heads, head_dim, bits, flags, query_dtype,
                                         seq_len, n_splits, num_cus)
    if name is None:
        raise ValueError(load().tq_last_error().decode("utf-8", "replace"))
    return name.decode()


def hip_available() -> bool:
    """True when the library is built and a HIP device is visible."""
    try:
        load()
    except (OSError, RuntimeError):
        return False
    return bool(torch.cuda.is_available())
