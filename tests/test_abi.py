"""The C ABI: every symbol declared in include/*.h is exported, and the
argument checks that run before any HIP call return the documented status codes.
CPU only: no call here reaches a kernel launch."""
import ctypes
import re
from pathlib import Path

import pytest

from intent_amd import _native
from intent_amd import errors

HEADERS = sorted((Path(__file__).resolve().parent.parent / "include").glob("*.h"))


def declared_symbols():
    text = "\n".join(h.read_text() for h in HEADERS)
    return sorted(set(re.findall(r"^\s*(?:int|size_t|const char\*)\s+(intent_\w+)\s*\(", text, re.M)))


def test_header_declares_expected_entries():
    names = declared_symbols()
    assert len(names) >= 16
    assert set(names) == set(_native.SIGNATURES), "ctypes signature table and header disagree"


def test_library_exports_every_declared_symbol():
    lib = _native.library()
    for name in declared_symbols():
        assert hasattr(lib, name), name
    assert lib.intent_amd_abi_version() == _native.ABI_VERSION


def status(entry, *args):
    return getattr(_native.library(), entry)(*args)


P = ctypes.c_void_p
FAKE = 0x1000  # a 16-byte aligned non-null address; never dereferenced by the checks


def test_w4a16_argument_checks():
    # Shapes outside the tiled kernels (K not a multiple of 128, groups of other sizes, unaligned
    # rows) run the generic kernel (GPU tests); here only calls that are invalid, which fail before
    # any launch. K odd:
    assert status("intent_w4a16_matmul", FAKE, 1, 101, 101, FAKE, 8, 51, FAKE, FAKE, 1, 101, FAKE, 8, None) == \
        errors.INTENT_ERR_INVALID_ARGUMENT
    assert "even" in _native.last_error()
    # K not a multiple of the group size
    assert status("intent_w4a16_gemv", FAKE, 1, 96, 96, FAKE, 8, 48, FAKE, FAKE, 2, 64, FAKE, 8, None) == \
        errors.INTENT_ERR_INVALID_ARGUMENT
    # group size 0
    assert status("intent_w4a16_gemm", FAKE, 4, 256, 256, FAKE, 8, 128, FAKE, FAKE, 2, 0, FAKE, 8, None) == \
        errors.INTENT_ERR_INVALID_ARGUMENT
    # null pointer
    assert status("intent_w4a16_gemm", None, 4, 256, 256, FAKE, 8, 128, FAKE, FAKE, 2, 128, FAKE, 8, None) == \
        errors.INTENT_ERR_INVALID_ARGUMENT
    # row stride smaller than the row
    assert status("intent_w4a16_gemm", FAKE, 4, 256, 128, FAKE, 8, 128, FAKE, FAKE, 2, 128, FAKE, 8, None) == \
        errors.INTENT_ERR_INVALID_ARGUMENT
    # GEMV covers M <= 16 only
    assert status("intent_w4a16_gemv", FAKE, 17, 256, 256, FAKE, 8, 128, FAKE, FAKE, 2, 128, FAKE, 8, None) == \
        errors.INTENT_ERR_UNSUPPORTED
    # empty problems are a no-op success
    assert status("intent_w4a16_matmul", FAKE, 0, 256, 256, FAKE, 8, 128, FAKE, FAKE, 2, 128, FAKE, 8, None) == 0


def test_int8_and_w8a16_checks():
    # any K and any alignment run (the generic kernel off the tiled shapes); invalid calls fail first
    assert status("intent_w8a8_gemm", FAKE, 4, 128, 128, None, FAKE, 4, 128, FAKE, FAKE, 4, None) == \
        errors.INTENT_ERR_INVALID_ARGUMENT
    assert status("intent_w8a8_gemm", FAKE, 4, 100, 90, FAKE, FAKE, 4, 100, FAKE, FAKE, 4, None) == \
        errors.INTENT_ERR_INVALID_ARGUMENT  # a_ld < K
    assert status("intent_i8_gemm_i32", FAKE, 4, 128, 136, FAKE, 4, 100, None, FAKE, 4, None) == \
        errors.INTENT_ERR_INVALID_ARGUMENT  # w_ld < K
    assert status("intent_w8a16_matmul", FAKE, 4, 96, 96, None, 4, 96, FAKE, FAKE, 4, None) == \
        errors.INTENT_ERR_INVALID_ARGUMENT
    assert status("intent_w8a16_matmul", FAKE, 4, 96, 96, FAKE, 4, 96, FAKE, FAKE, 3, None) == \
        errors.INTENT_ERR_INVALID_ARGUMENT  # y_ld < N
    assert status("intent_i8_gemm_i32", FAKE, 0, 128, 128, FAKE, 4, 128, None, FAKE, 4, None) == 0


def test_moe_checks():
    assert status("intent_moe_route", FAKE, 8, 8, 9, 1, FAKE, FAKE, None) == errors.INTENT_ERR_UNSUPPORTED
    assert status("intent_moe_route", FAKE, 8, 0, 1, 1, FAKE, FAKE, None) == errors.INTENT_ERR_INVALID_ARGUMENT
    assert status("intent_moe_route", FAKE, 0, 8, 2, 1, FAKE, FAKE, None) == 0
    # capacity below R + E*(B-1)
    assert status("intent_moe_align", FAKE, 16, 2, 4, 128, FAKE, 100, FAKE, 10, FAKE, FAKE, None) == \
        errors.INTENT_ERR_INVALID_ARGUMENT
    assert "needs" in _native.last_error()
    assert status("intent_moe_align", FAKE, 16, 2, 3000, 128, FAKE, 10 ** 6, FAKE, 10 ** 4, FAKE, FAKE, None) == \
        errors.INTENT_ERR_UNSUPPORTED  # more than 2048 experts
    # other block sizes and dimensions off the tiles run the generic kernels (GPU tests); invalid calls:
    assert status("intent_moe_gate_up_w4", FAKE, 4, 256, 256, FAKE, FAKE, 2, 0, 2, FAKE, FAKE, FAKE, 2, 128, 128,
                  FAKE, 128, None) == errors.INTENT_ERR_INVALID_ARGUMENT  # block size 0
    assert status("intent_moe_gate_up_w4", FAKE, 4, 250, 256, FAKE, FAKE, 2, 32, 2, FAKE, FAKE, FAKE, 2, 128, 128,
                  FAKE, 128, None) == errors.INTENT_ERR_INVALID_ARGUMENT  # group 128 does not divide H = 250
    assert status("intent_moe_down_w4", FAKE, 95, FAKE, FAKE, 2, 128, 8, FAKE, FAKE, FAKE, 2, 256, 95, 32,
                  FAKE, 256, None) == errors.INTENT_ERR_INVALID_ARGUMENT  # F odd
    assert _native.library().intent_moe_workspace_size(512, 2, 8, 4096, 14336, 128) >= \
        16 * 128 * 14336 * 2 + 1024 * 4096 * 4  # block 128: padded activations + route outputs
    need = _native.library().intent_moe_workspace_size(512, 2, 8, 4096, 14336, 0)  # composite plan
    # 128 routes per expert: the composite may take 128- or 160-row blocks and sizes for either
    assert need == max(_native.library().intent_moe_workspace_size(512, 2, 8, 4096, 14336, b) for b in (128, 160))
    # 8 routes per expert: 128-row blocks only
    assert _native.library().intent_moe_workspace_size(32, 2, 8, 4096, 14336, 0) == \
        _native.library().intent_moe_workspace_size(32, 2, 8, 4096, 14336, 128)
    assert status("intent_moe_expert_ffn_w4", FAKE, FAKE, 512, 4096, 8, 2, 1, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE,
                  14336, 128, FAKE, FAKE, need - 1, None, None, None) == errors.INTENT_ERR_WORKSPACE
    assert _native.library().intent_moe_workspace_size(-1, 2, 8, 64, 64, 128) == 0


def test_kquant_checks():
    # Q8_K: x must be 16-byte aligned; rows of at least 256 values / 292 bytes
    assert status("intent_q8k_quantize", FAKE + 4, 3, 256, FAKE, 292, None) == errors.INTENT_ERR_ALIGNMENT
    assert status("intent_q8k_quantize", FAKE, 3, 128, FAKE, 292, None) == errors.INTENT_ERR_INVALID_ARGUMENT
    assert status("intent_q8k_quantize", FAKE, 3, 256, FAKE, 291, None) == errors.INTENT_ERR_INVALID_ARGUMENT
    assert status("intent_q8k_quantize", None, 0, 256, None, 292, None) == 0  # G = 0: nothing to do
    # Q4_K rows: stride below G records, misaligned rows, null inputs
    assert status("intent_q4k_q8k_gemv", FAKE, 4, 3, 400, FAKE, FAKE, None) == errors.INTENT_ERR_INVALID_ARGUMENT
    assert status("intent_q4k_q8k_gemv", FAKE, 4, 3, 440, FAKE, FAKE, None) == errors.INTENT_ERR_ALIGNMENT
    assert status("intent_q4k_q8k_gemv", FAKE, 4, 3, 432, FAKE + 2, FAKE, None) == errors.INTENT_ERR_ALIGNMENT
    assert status("intent_q4k_q8k_gemv", None, 4, 3, 432, FAKE, FAKE, None) == errors.INTENT_ERR_INVALID_ARGUMENT
    assert status("intent_q4k_q8k_gemv", FAKE, 0, 3, 432, FAKE, FAKE, None) == 0  # N = 0
    assert status("intent_q4k_projection", FAKE, 4, 3, 432, FAKE + 8, 256, FAKE, FAKE, None) == \
        errors.INTENT_ERR_ALIGNMENT


def test_probe_checks():
    e = errors
    rp = "intent_hbm_read_probe"
    assert status(rp, P(FAKE), 4095, 1, 0, P(FAKE), 256, None) == e.INTENT_ERR_INVALID_ARGUMENT  # bytes % 16
    assert status(rp, P(FAKE), 4096, 3, 0, P(FAKE), 256, None) == e.INTENT_ERR_UNSUPPORTED  # unroll
    assert status(rp, P(FAKE), 4096, 1, 4, P(FAKE), 256, None) == e.INTENT_ERR_INVALID_ARGUMENT  # store mode 0..3
    assert status(rp, P(FAKE), 4096, 1, 0, P(FAKE), 255, None) == e.INTENT_ERR_INVALID_ARGUMENT  # sink < 256
    # store mode: one workgroup of four waves per 4096 bytes at unroll 1, two words per wave
    assert status(rp, P(FAKE), 65536, 1, 1, P(FAKE), 127, None) == e.INTENT_ERR_INVALID_ARGUMENT
    assert status(rp, P(FAKE + 8), 4096, 1, 0, P(FAKE), 256, None) == e.INTENT_ERR_ALIGNMENT
    assert status("intent_mfma_peak_probe", 0, 0, 1, P(FAKE), None) == e.INTENT_ERR_INVALID_ARGUMENT


def test_status_mapping():
    assert isinstance(errors.status_error(-1, "e", "m"), ValueError)
    assert isinstance(errors.status_error(-2, "e", "m"), ValueError)
    assert isinstance(errors.status_error(-3, "e", "m"), NotImplementedError)
    assert isinstance(errors.status_error(-4, "e", "m"), RuntimeError)
    assert isinstance(errors.status_error(-5, "e", "m"), ValueError)
    with pytest.raises(NotImplementedError, match="M <= 16"):
        _native.call("intent_w4a16_gemv", FAKE, 17, 256, 256, FAKE, 8, 128, FAKE, FAKE, 2, 128, FAKE, 8, None)
    with pytest.raises(ValueError, match="multiple of group_size"):
        _native.call("intent_w4a16_matmul", FAKE, 1, 100, 100, FAKE, 8, 50, FAKE, FAKE, 4, 32, FAKE, 8, None)
