"""ctypes binding of libresident_epoch.so (include/resident_epoch.h).

The library is the product path: if it is missing the import fails loudly,
there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

LIBRARY_PATH = Path(__file__).resolve().parent / "lib" / "libresident_epoch.so"

_c_i32p = ctypes.POINTER(ctypes.c_int32)
_c_i64p = ctypes.POINTER(ctypes.c_int64)

# Every symbol declared in include/resident_epoch.h with (restype, argtypes).
SIGNATURES: dict[str, tuple] = {
    "resident_epoch_create": (
        ctypes.c_void_p,
        [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p, _c_i32p],
    ),
    "resident_epoch_execute": (
        ctypes.c_int32,
        [
            ctypes.c_void_p,  # opaque
            ctypes.c_int32,  # request_count
            ctypes.c_int32,  # max_steps
            _c_i64p,  # input_token_ids
            _c_i64p,  # input_positions
            _c_i32p,  # input_sequence_lengths
            _c_i32p,  # input_eos_token_ids
            _c_i32p,  # input_row_generations
            _c_i64p,  # output_token_ids
            _c_i32p,  # output_executed
            _c_i32p,  # output_row_generations
            _c_i32p,  # output_model_calls
            _c_i32p,  # output_device_status
            _c_i32p,  # output_feed_calls
            _c_i32p,  # output_fetch_calls
            _c_i32p,  # output_commit_state
            _c_i32p,  # output_kv_import_checksum
            _c_i64p,  # output_wall_us
            _c_i64p,  # output_native_cpu_us
            _c_i64p,  # output_declared_input_bytes
            _c_i64p,  # output_declared_output_bytes
            ctypes.c_char_p,  # transfer_path
            ctypes.c_uint64,  # transfer_id
            ctypes.c_void_p,  # ipc metadata
        ],
    ),
    "resident_epoch_destroy": (None, [ctypes.c_void_p]),
    "resident_epoch_proc": (
        ctypes.c_int32,
        [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64],
    ),
    "resident_decoder_step": (
        ctypes.c_int32,
        [ctypes.c_void_p] + [ctypes.c_void_p] * 11,
    ),
    "resident_epoch_prefill": (
        ctypes.c_int32,
        [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p, ctypes.c_int32, ctypes.c_void_p],
    ),
    "resident_epoch_prefill_batch": (
        ctypes.c_int32,
        [ctypes.c_void_p, ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
         ctypes.c_void_p],
    ),
    "resident_epoch_prefill_batch_noalloc": (
        ctypes.c_int32,
        [ctypes.c_void_p, ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
         ctypes.c_void_p],
    ),
    "resident_epoch_read_state": (
        ctypes.c_int32,
        [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_void_p, ctypes.c_int64],
    ),
    "resident_epoch_write_state": (
        ctypes.c_int32,
        [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_void_p, ctypes.c_int64],
    ),
    "resident_epoch_info": (ctypes.c_int32, [ctypes.c_void_p, ctypes.c_char_p, _c_i64p]),
    "resident_epoch_kernel_timing": (ctypes.c_int32, [ctypes.c_void_p, ctypes.c_int32]),
    "resident_epoch_read_kernel_timing": (
        ctypes.c_int32,
        [ctypes.c_void_p, ctypes.POINTER(ctypes.c_float), ctypes.c_int32],
    ),
    "resident_epoch_time_ops": (
        ctypes.c_int32,
        [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.POINTER(ctypes.c_float)],
    ),
    "resident_epoch_time_layer_op": (
        ctypes.c_int32,
        [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32, ctypes.POINTER(ctypes.c_float)],
    ),
    "resident_epoch_gemm": (
        ctypes.c_int32,
        [ctypes.c_void_p] * 5 + [ctypes.c_int32] * 5,
    ),
}

_LIB: ctypes.CDLL | None = None


def library_path() -> Path:
    override = os.getenv("CRUISE_RESIDENT_EPOCH_LIBRARY")
    return Path(override) if override else LIBRARY_PATH


def load(path: Path | None = None) -> ctypes.CDLL:
    """Load the HIP library (once per path) and bind every declared symbol.
    ``path`` defaults to the in-tree build (or CRUISE_RESIDENT_EPOCH_LIBRARY)."""
    global _LIB
    if path is not None and Path(path).resolve() != library_path().resolve():
        return _bind(Path(path))
    if _LIB is not None:
        return _LIB
    _LIB = _bind(library_path())
    return _LIB


BRIDGE_SYMBOLS = ("resident_epoch_create", "resident_epoch_execute", "resident_epoch_destroy")


def load_bridge(path: Path) -> ctypes.CDLL:
    """A library that exports the three bridge entry points (the reference
    bridge's whole C-ABI), bound without the engine's other symbols."""
    return _bind(Path(path), BRIDGE_SYMBOLS)


def _bind(path: Path, symbols=None) -> ctypes.CDLL:
    # PyTorch-ROCm ships its own libamdhip64.so.7.  Importing it first makes
    # the library bind that same HIP runtime (same soname), so torch tensors
    # and the engine share one runtime and one device context per process.
    try:
        import torch  # noqa: F401
    except ImportError:  # pragma: no cover - torch is part of this image
        pass
    if not path.is_file():
        raise RuntimeError(
            f"libresident_epoch.so is not built ({path}); run `python -m cruise_amd.build` "
            "or __graft_entry__.build() first"
        )
    lib = ctypes.CDLL(str(path))
    for name in symbols or SIGNATURES:
        restype, argtypes = SIGNATURES[name]
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    return lib
