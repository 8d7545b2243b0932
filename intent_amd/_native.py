"""ctypes binding of ``libintent_amd.so`` (the C ABI in ``include/intent_amd.h``).

The reference binds natively compiled entries the same way: ``ctypes.CDLL``
plus one flat C symbol per entry with pointer / int64 extent slots
(python/intent/runtime/native_artifact.py:194-262, runtime/native.py:14-120).
There is no fallback: if the library is missing every call raises.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

from .errors import INTENT_OK, NativeLibraryError, status_error

PACKAGE = Path(__file__).resolve().parent
# INTENT_AMD_LIBRARY names another build of the same library (the host-side
# AddressSanitizer build the sanitizer test loads); the in-tree build otherwise.
LIBRARY_PATH = Path(os.environ.get("INTENT_AMD_LIBRARY") or PACKAGE / "_lib" / "libintent_amd.so")
ABI_VERSION = 1

P = ctypes.c_void_p
I64 = ctypes.c_int64
INT = ctypes.c_int
SIZE = ctypes.c_size_t
F32 = ctypes.c_float

# Entry -> (argtypes, restype). Mirrors include/intent_amd.h.
SIGNATURES: dict[str, tuple[list, object]] = {
    "intent_amd_abi_version": ([], INT),
    "intent_amd_last_error": ([], ctypes.c_char_p),
    "intent_amd_last_kernel": ([], ctypes.c_char_p),
    "intent_amd_device_arch": ([INT, ctypes.c_char_p, I64], INT),
    "intent_w8a16_matmul": ([P, I64, I64, I64, P, I64, I64, P, P, I64, P], INT),
    "intent_w4a16_matmul": ([P, I64, I64, I64, P, I64, I64, P, P, I64, I64, P, I64, P], INT),
    "intent_w4a16_gemv": ([P, I64, I64, I64, P, I64, I64, P, P, I64, I64, P, I64, P], INT),
    "intent_w4a16_gemm": ([P, I64, I64, I64, P, I64, I64, P, P, I64, I64, P, I64, P], INT),
    "intent_w8a8_gemm": ([P, I64, I64, I64, P, P, I64, I64, P, P, I64, P], INT),
    "intent_i8_gemm_i32": ([P, I64, I64, I64, P, I64, I64, P, P, I64, P], INT),
    "intent_i8_gemm_i32_kn": ([P, I64, I64, I64, P, I64, I64, P, P, I64, P], INT),
    "intent_moe_route": ([P, I64, I64, I64, INT, P, P, P], INT),
    "intent_moe_align": ([P, I64, I64, I64, I64, P, I64, P, I64, P, P, P], INT),
    "intent_moe_gate_up_w4": ([P, I64, I64, I64, P, P, I64, I64, I64, P, P, P, I64, I64, I64, P, I64, P], INT),
    "intent_moe_down_w4": ([P, I64, P, P, I64, I64, I64, P, P, P, I64, I64, I64, I64, P, I64, P], INT),
    "intent_moe_combine": ([P, I64, P, I64, I64, P, I64, I64, P], INT),
    "intent_q8k_quantize": ([P, I64, I64, P, I64, P], INT),
    "intent_q4k_q8k_gemv": ([P, I64, I64, I64, P, P, P], INT),
    "intent_q4k_projection": ([P, I64, I64, I64, P, I64, P, P, P], INT),
    "intent_q4k_projection_noalloc": ([P, I64, I64, I64, P, I64, P, P], INT),
    "intent_fp8_groupwise_quantize": ([P, INT, I64, I64, I64, P, I64, P, I64, I64, P], INT),
    "intent_w4a8_gemm": ([P, I64, I64, I64, P, I64, I64, P, I64, P], INT),
    "intent_bitnet_int2_gemm": ([P, I64, I64, I64, P, I64, I64, P, I64, P], INT),
    "intent_mxfp8_gemm": ([P, I64, I64, I64, P, I64, P, I64, I64, P, I64, P, I64, P], INT),
    "intent_fp8_transpose": ([P, I64, I64, I64, P, I64, P], INT),
    "intent_scaled_fp8_gemm": ([P, I64, I64, I64, P, I64, I64, F32, F32, I64, INT, P, I64, P], INT),
    "intent_scaled_fp8_gemm_kn": ([P, I64, I64, I64, P, I64, I64, F32, F32, I64, INT, P, I64, P], INT),
    "intent_w4_sym_repack": ([P, I64, I64, I64, P, I64, I64, P, I64, P, P, I64, P], INT),
    "intent_w4a16_sym_gemv": ([P, I64, I64, I64, P, I64, I64, P, I64, P, I64, P], INT),
    "intent_w4a16_sym_gemm": ([P, I64, I64, I64, P, I64, I64, P, I64, P, I64, P], INT),
    "intent_f16_transpose": ([P, I64, I64, I64, P, I64, P], INT),
    "intent_quantized_gemm": ([P, I64, I64, I64, P, I64, I64, P, P, I64, P, P, I64, P], INT),
    "intent_f16_transpose_batched": ([P, I64, I64, I64, I64, I64, P, I64, I64, P], INT),
    "intent_grouped_gemm": ([P, I64, I64, I64, P, I64, P, I64, P, I64, I64, I64, INT, P, I64, P], INT),
    "intent_grouped_gemm_kn": ([P, I64, I64, I64, P, I64, P, I64, I64, I64, INT, P, I64, P], INT),
    "intent_moe_expert_ffn_workspace_size": ([I64, I64, I64, I64], SIZE),
    "intent_moe_expert_ffn": ([P, I64, I64, I64, P, I64, P, I64, P, P, I64, P, P, I64, P, I64, P, SIZE, P], INT),
    "intent_f16_gemm": ([P, I64, I64, I64, P, I64, I64, INT, P, I64, P], INT),
    "intent_f16_gemm_kn": ([P, I64, I64, I64, P, I64, I64, INT, P, I64, P], INT),
    "intent_quantized_gemm_kn": ([P, I64, I64, I64, P, I64, I64, P, P, I64, P, P, I64, P], INT),
    "intent_nvfp4_quantize": ([P, I64, I64, I64, P, P, I64, P, P], INT),
    "intent_fp4_bf16_matmul": ([P, I64, I64, I64, P, I64, I64, P, I64, P], INT),
    "intent_fp8_gemm": ([P, I64, I64, I64, P, I64, I64, INT, P, I64, P], INT),
    "intent_deepgemm_fp8": ([P, I64, I64, I64, P, I64, P, I64, I64, P, I64, P, I64, P], INT),
    "intent_moe_workspace_size": ([I64, I64, I64, I64, I64, I64], SIZE),
    "intent_moe_expert_ffn_w4": ([P, P, I64, I64, I64, I64, INT, P, P, P, P, P, P, I64, I64, P, P, SIZE, P, P, P],
                                 INT),
    "intent_i8_per_token_quantize": ([P, INT, I64, I64, I64, P, I64, P, P], INT),
    "intent_hbm_read_probe": ([P, I64, INT, INT, P, I64, P], INT),
    "intent_mfma_peak_probe": ([INT, I64, I64, P, P], INT),
}

_lock = threading.Lock()
_library: ctypes.CDLL | None = None


def library() -> ctypes.CDLL:
    """Load (once) and return the gfx950 library; raises if it is not built."""
    global _library
    if _library is not None:
        return _library
    with _lock:
        if _library is not None:
            return _library
        if not LIBRARY_PATH.exists():
            raise NativeLibraryError(
                f"{LIBRARY_PATH} is not built; run `python -m intent_amd.build` (hipcc, gfx950). "
                "There is no CPU fallback for the quantized-contraction kernels.")
        lib = ctypes.CDLL(str(LIBRARY_PATH))
        for name, (argtypes, restype) in SIGNATURES.items():
            try:
                fn = getattr(lib, name)
            except AttributeError as error:
                raise NativeLibraryError(f"{LIBRARY_PATH} does not export {name}") from error
            fn.argtypes = argtypes
            fn.restype = restype
        version = lib.intent_amd_abi_version()
        if version != ABI_VERSION:
            raise NativeLibraryError(f"ABI version {version} != expected {ABI_VERSION}")
        _library = lib
        return lib


def last_error() -> str:
    raw = library().intent_amd_last_error()
    return raw.decode("utf-8", "replace") if raw else ""


def last_kernel() -> str:
    """The kernel variant the calling thread's latest launch dispatched to."""
    raw = library().intent_amd_last_kernel()
    return raw.decode("utf-8", "replace") if raw else ""


def call(entry: str, *arguments) -> None:
    """Invoke an int-status entry and raise the mapped exception on failure."""
    status = getattr(library(), entry)(*arguments)
    if status != INTENT_OK:
        raise status_error(status, entry, last_error())


def device_arch(device: int) -> str:
    buf = ctypes.create_string_buffer(128)
    call("intent_amd_device_arch", device, buf, len(buf))
    return buf.value.decode()
