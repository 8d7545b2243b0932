"""CPU oracle for the quantized-contraction hot path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this package, and only as the checker (never as the thing
measured or shipped). The product path in ``intent_amd`` never touches it.

Two layers:
  * ``liboracle.so`` (``oracle.c``): the plain-C restatement of the reference's
    CPU numerics, one function per hot-path function (each cites the reference
    file:line it follows). Built by ``oracle/Makefile``.
  * numpy restatements in this module, written independently of the C file,
    used to pin the C oracle (tests compare the two and compare both with
    float64 / int64 brute force, closed forms and known answers).

Parity status of every function is pinned by tests in ``tests/test_oracle.py``:
  w8a16, w4a16, i8_gemm_i32, w8a8, moe_route, moe_align, moe_ffn_w4 and the
  f16/bf16 conversions all have independent checks (numpy float64 / int64
  brute force, known-answer vectors, invariants, and the committed fixtures in
  ``tests/golden/``). No function is "parity unpinned".
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
# ORACLE_LIBRARY names another build of oracle.c (the sanitizer test's
# AddressSanitizer / UBSan build); the in-tree liboracle.so otherwise.
LIBRARY = Path(os.environ.get("ORACLE_LIBRARY") or HERE / "liboracle.so")

_lib = None


def build() -> Path:
    """Compile oracle.c with the committed Makefile."""
    proc = subprocess.run(["make", "-s", "-C", str(HERE)], capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{proc.stdout}\n{proc.stderr}")
    return LIBRARY


def lib():
    global _lib
    if _lib is None:
        if not LIBRARY.exists():
            build()
        _lib = ctypes.CDLL(str(LIBRARY))
        i64, ci = ctypes.c_int64, ctypes.c_int
        p = ctypes.c_void_p
        _lib.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        _lib.orc_f16_to_f32.restype = ctypes.c_float
        _lib.orc_f32_to_f16.argtypes = [ctypes.c_float]
        _lib.orc_f32_to_f16.restype = ctypes.c_uint16
        _lib.orc_f32_to_bf16.argtypes = [ctypes.c_float]
        _lib.orc_f32_to_bf16.restype = ctypes.c_uint16
        _lib.orc_w8a16.argtypes = [p, i64, i64, p, i64, p, p, ci]
        _lib.orc_w4a16.argtypes = [p, i64, i64, p, i64, p, p, i64, p, ci]
        _lib.orc_i8_gemm_i32.argtypes = [p, i64, i64, p, i64, p, p, ci]
        _lib.orc_w8a8.argtypes = [p, i64, i64, p, p, i64, p, p, ci]
        _lib.orc_moe_route.argtypes = [p, i64, i64, i64, ci, p, p]
        _lib.orc_moe_align.argtypes = [p, i64, i64, i64, i64, p, i64, p, i64, p, p]
        _lib.orc_moe_ffn_w4.argtypes = [p, i64, i64, p, p, i64, i64, p, p, p, p, p, p, i64, i64, p, ci]
        _lib.orc_q8k_quantize.argtypes = [p, i64, p]
        _lib.orc_q4k_q8k_dot.argtypes = [p, p, i64]
        _lib.orc_q4k_q8k_dot.restype = ctypes.c_float
        _lib.orc_q4k_gemv.argtypes = [p, i64, i64, i64, p, p, ci]
        _lib.orc_f32_to_e4m3fn.argtypes = [ctypes.c_float]
        _lib.orc_f32_to_e4m3fn.restype = ctypes.c_uint8
        _lib.orc_fp8_groupwise_quantize.argtypes = [p, i64, i64, i64, i64, ctypes.c_float, p, i64, p, i64]
        _lib.orc_fp8_groupwise_quantize.restype = None
        _lib.orc_i8_per_token_quantize.argtypes = [p, i64, i64, i64, p, i64, p]
        _lib.orc_i8_per_token_quantize.restype = None
        _lib.orc_w4a8.argtypes = [p, i64, i64, p, i64, p, ci]
        _lib.orc_bitnet_int2.argtypes = [p, i64, i64, p, i64, p, ci]
        _lib.orc_w4a8.restype = None
        _lib.orc_e4m3fn_to_f32.argtypes = [ctypes.c_uint8]
        _lib.orc_e4m3fn_to_f32.restype = ctypes.c_float
        _lib.orc_e8m0_to_f32.argtypes = [ctypes.c_uint8]
        _lib.orc_e8m0_to_f32.restype = ctypes.c_float
        _lib.orc_mxfp8_gemm.argtypes = [p, p, i64, i64, p, p, i64, p, ci]
        _lib.orc_mxfp8_gemm.restype = None
        _lib.orc_scaled_fp8_gemm.argtypes = [p, i64, i64, p, i64, ctypes.c_float, ctypes.c_float, i64, ci, p, ci]
        _lib.orc_scaled_fp8_gemm.restype = None
        _lib.orc_deepgemm_fp8.argtypes = [p, p, i64, i64, p, p, i64, p, ci]
        _lib.orc_deepgemm_fp8.restype = None
        _lib.orc_e5m2_to_f32.argtypes = [ctypes.c_uint8]
        _lib.orc_e5m2_to_f32.restype = ctypes.c_float
        _lib.orc_f32_to_e5m2.argtypes = [ctypes.c_float]
        _lib.orc_f32_to_e5m2.restype = ctypes.c_uint8
        _lib.orc_fp8_gemm.argtypes = [ci, p, i64, i64, p, i64, p, ci]
        _lib.orc_fp8_gemm.restype = None
        _lib.orc_fp4_decode.argtypes = [p, i64]
        _lib.orc_fp4_decode.restype = ctypes.c_float
        _lib.orc_fp4_bf16_matmul.argtypes = [p, i64, i64, p, i64, p, ci]
        _lib.orc_fp4_bf16_matmul.restype = None
        _lib.orc_w4_sym.argtypes = [p, i64, i64, p, p, i64, p, ci]
        _lib.orc_w4_sym.restype = None
        _lib.orc_quantized_gemm.argtypes = [p, i64, i64, p, i64, p, p, p, p, ci]
        _lib.orc_quantized_gemm.restype = None
        _lib.orc_grouped_gemm.argtypes = [p, ci, i64, p, i64, p, i64, p, i64, p, ci]
        _lib.orc_grouped_gemm.restype = None
        _lib.orc_float_gemm.argtypes = [p, i64, i64, p, i64, ci, ci, p, ci]
        _lib.orc_float_gemm.restype = None
        _lib.orc_moe_expert_ffn.argtypes = [p, i64, i64, p, i64, p, p, p, p, p, i64, p, p, ctypes.c_int]
        _lib.orc_moe_expert_ffn.restype = None
        _lib.orc_nvfp4_quantize.argtypes = [p, i64, i64, ctypes.c_float, p, p]
        _lib.orc_nvfp4_quantize.restype = None
        _lib.orc_bitnet_int2.restype = None
        for name in ("orc_w8a16", "orc_w4a16", "orc_i8_gemm_i32", "orc_w8a8", "orc_moe_route", "orc_moe_align",
                     "orc_moe_ffn_w4", "orc_q8k_quantize", "orc_q4k_gemv"):
            getattr(_lib, name).restype = None
    return _lib


def _ptr(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"], "oracle inputs must be C-contiguous"
    return a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ---- C oracle wrappers --------------------------------------------------------

def w8a16(x, w, scales, threads: int = 1) -> np.ndarray:
    x, w, s = _c(x, np.float16), _c(w, np.int8), _c(scales, np.float16)
    M, K = x.shape
    N = w.shape[0]
    y = np.empty((M, N), np.float16)
    lib().orc_w8a16(_ptr(x), M, K, _ptr(w), N, _ptr(s), _ptr(y), threads)
    return y


def w4a16(x, packed, scales, zeros, threads: int = 1) -> np.ndarray:
    x, q = _c(x, np.float16), _c(packed, np.uint8)
    s, z = _c(scales, np.float16), _c(zeros, np.uint8)
    M, K = x.shape
    N = q.shape[0]
    gs = K // s.shape[1]
    y = np.empty((M, N), np.float16)
    lib().orc_w4a16(_ptr(x), M, K, _ptr(q), N, _ptr(s), _ptr(z), gs, _ptr(y), threads)
    return y


def i8_gemm_i32(a, w, bias=None, threads: int = 1) -> np.ndarray:
    a, w = _c(a, np.int8), _c(w, np.int8)
    M, K = a.shape
    N = w.shape[0]
    c = np.empty((M, N), np.int32)
    b = None if bias is None else _c(bias, np.int32)
    lib().orc_i8_gemm_i32(_ptr(a), M, K, _ptr(w), N, None if b is None else _ptr(b), _ptr(c), threads)
    return c


def w8a8(a, sa, w, sw, threads: int = 1) -> np.ndarray:
    """Returns the bf16 bit patterns (uint16) of the W8A8 output."""
    a, w = _c(a, np.int8), _c(w, np.int8)
    sa, sw = _c(sa, np.float32), _c(sw, np.float32)
    M, K = a.shape
    N = w.shape[0]
    out = np.empty((M, N), np.uint16)
    lib().orc_w8a8(_ptr(a), M, K, _ptr(sa), _ptr(w), N, _ptr(sw), _ptr(out), threads)
    return out


def moe_route(logits, top_k: int, renormalize: bool = True):
    lg = _c(logits, np.float32)
    T, E = lg.shape
    ids = np.empty((T, top_k), np.int32)
    wts = np.empty((T, top_k), np.float32)
    lib().orc_moe_route(_ptr(lg), T, E, top_k, int(renormalize), _ptr(ids), _ptr(wts))
    return ids, wts


def align_sizes(routes: int, experts: int, block: int) -> tuple[int, int]:
    capacity = routes + experts * (block - 1)
    return capacity, (capacity + block - 1) // block


def moe_align(ids, experts: int, block: int):
    ids = _c(ids, np.int32)
    T, k = ids.shape
    cap, nb = align_sizes(T * k, experts, block)
    sorted_ids = np.empty(cap, np.int32)
    blocks = np.empty(nb, np.int32)
    offsets = np.empty(experts + 1, np.int32)
    total = np.empty(1, np.int32)
    lib().orc_moe_align(_ptr(ids), T, k, experts, block, _ptr(sorted_ids), cap, _ptr(blocks), nb, _ptr(offsets),
                        _ptr(total))
    return sorted_ids, blocks, offsets, total


def moe_ffn_w4(x, ids, weights, wgu, sgu, zgu, wd, sd, zd, y=None, threads: int = 1) -> np.ndarray:
    """y (f32 [T,H]) accumulated in place; a zero y is created when None."""
    x = _c(x, np.float16)
    ids, weights = _c(ids, np.int32), _c(weights, np.float32)
    wgu, sgu, zgu = _c(wgu, np.uint8), _c(sgu, np.float16), _c(zgu, np.uint8)
    wd, sd, zd = _c(wd, np.uint8), _c(sd, np.float16), _c(zd, np.uint8)
    T, H = x.shape
    top_k = ids.shape[1]
    E, F2, _ = wgu.shape
    F = F2 // 2
    gs = H // sgu.shape[2]
    assert F // sd.shape[2] == gs, "gate/up and down must share the group size"
    y = np.zeros((T, H), np.float32) if y is None else y
    assert y.dtype == np.float32 and y.flags["C_CONTIGUOUS"]
    lib().orc_moe_ffn_w4(_ptr(x), T, H, _ptr(ids), _ptr(weights), top_k, E, _ptr(wgu), _ptr(sgu), _ptr(zgu),
                         _ptr(wd), _ptr(sd), _ptr(zd), F, gs, _ptr(y), threads)
    return y


Q4K_BYTES = 144
Q8K_BYTES = 292


def q8k_quantize(x) -> np.ndarray:
    """f32 [G, 256] -> Q8_K records uint8 [G, 292]."""
    x = _c(x, np.float32)
    G = x.shape[0]
    assert x.shape == (G, 256)
    out = np.empty((G, Q8K_BYTES), np.uint8)
    lib().orc_q8k_quantize(_ptr(x), G, _ptr(out))
    return out


def q4k_q8k_dot(w, xq) -> np.float32:
    """Q4_K records [G, 144] . Q8_K records [G, 292] -> f32."""
    w, xq = _c(w, np.uint8), _c(xq, np.uint8)
    G = w.shape[0]
    assert w.shape == (G, Q4K_BYTES) and xq.shape == (G, Q8K_BYTES)
    return np.float32(lib().orc_q4k_q8k_dot(_ptr(w), _ptr(xq), G))


def q4k_gemv(w, xq, threads: int = 1) -> np.ndarray:
    """Rows of Q4_K records [N, G, 144] against one Q8_K vector [G, 292] -> f32 [N]."""
    w, xq = _c(w, np.uint8), _c(xq, np.uint8)
    N, G, _ = w.shape
    y = np.empty(N, np.float32)
    lib().orc_q4k_gemv(_ptr(w), N, G, G * Q4K_BYTES, _ptr(xq), _ptr(y), threads)
    return y


FP8_EPS = {"bf16": 1.0e-12, "f32": 1.0e-4}  # examples/kernels/quantization/fp8.py:33,63


def fp8_groupwise_quantize(x, groups: int | None = None, source: str = "f32"):
    """[M, N] values (f32, or bf16 widened exactly to f32) -> (E4M3FN bits uint8 [M, N],
    scales f32 [M, groups]); groups defaults to ceil(N / 128)."""
    x = _c(x, np.float32)
    M, N = x.shape
    G = groups if groups is not None else (N + 127) // 128
    q = np.empty((M, N), np.uint8)
    sc = np.empty((M, G), np.float32)
    lib().orc_fp8_groupwise_quantize(_ptr(x), M, N, N, G, FP8_EPS[source], _ptr(q), N, _ptr(sc), G)
    return q, sc


def i8_per_token_quantize(x):
    """[M, K] values (f16 / bf16 widened exactly to f32, or f32) -> (int8 [M, K], scales f32 [M])."""
    x = _c(x, np.float32)
    M, K = x.shape
    q = np.empty((M, K), np.int8)
    sc = np.empty((M,), np.float32)
    lib().orc_i8_per_token_quantize(_ptr(x), M, K, K, _ptr(q), K, _ptr(sc))
    return q, sc


def i8_per_token_quantize_np(x):
    """numpy restatement, written apart from the C one: np.rint is round-half-even."""
    x = np.asarray(x, np.float32)
    amax = np.max(np.abs(x), axis=1) if x.shape[1] else np.zeros(x.shape[0], np.float32)
    amax = amax.astype(np.float32)
    zero = amax == 0
    safe = np.where(zero, np.float32(1), amax)
    scale = np.where(zero, np.float32(0), safe / np.float32(127)).astype(np.float32)
    inv = np.where(zero, np.float32(0), np.float32(127) / safe).astype(np.float32)
    t = np.clip(x * inv[:, None], np.float32(-128), np.float32(127))
    return np.rint(t).astype(np.int8), scale


def f32_to_e4m3fn(values) -> np.ndarray:
    v = np.asarray(values, np.float32).reshape(-1)
    return np.array([lib().orc_f32_to_e4m3fn(float(f)) for f in v], np.uint8)


def w4a8(a, packed, threads: int = 1) -> np.ndarray:
    """int8 a [M, K] x signed-nibble weights [N, K/2] -> int32 [N, M]."""
    a, packed = _c(a, np.int8), _c(packed, np.uint8)
    M, K = a.shape
    N = packed.shape[0]
    out = np.empty((N, M), np.int32)
    lib().orc_w4a8(_ptr(a), M, K, _ptr(packed), N, _ptr(out), threads)
    return out


def bitnet_int2(a, packed, threads: int = 1) -> np.ndarray:
    """int8 a [M, K] x interleaved 2-bit weights [N, K/4] -> int32 [M, N]."""
    a, packed = _c(a, np.int8), _c(packed, np.uint8)
    M, K = a.shape
    N = packed.shape[0]
    out = np.empty((M, N), np.int32)
    lib().orc_bitnet_int2(_ptr(a), M, K, _ptr(packed), N, _ptr(out), threads)
    return out


def mxfp8_gemm(a, sa, b, sb, threads: int = 1) -> np.ndarray:
    """E4M3FN bytes a [M, K], b [N, K] with E8M0 scales [M, K/32], [N, K/32] -> f32 [M, N]."""
    a, sa, b, sb = (_c(t, np.uint8) for t in (a, sa, b, sb))
    M, K = a.shape
    N = b.shape[0]
    out = np.empty((M, N), np.float32)
    lib().orc_mxfp8_gemm(_ptr(a), _ptr(sa), M, K, _ptr(b), _ptr(sb), N, _ptr(out), threads)
    return out


def scaled_fp8_gemm(a, b, lhs_scale, rhs_scale, splits=1, out=None, threads: int = 1) -> np.ndarray:
    """E4M3FN bytes a [M, K] and b [K, N] (N contiguous) -> f16 [M, N]:
    f16((acc * lhs_scale) * rhs_scale) per split, added in split order into
    out when out is given (split-K form), else the plain form."""
    a, b = _c(a, np.uint8), _c(b, np.uint8)
    M, K = a.shape
    N = b.shape[1]
    accumulate = out is not None
    res = _c(out, np.float16).copy() if accumulate else np.zeros((M, N), np.float16)
    lib().orc_scaled_fp8_gemm(_ptr(a), M, K, _ptr(b), N, float(lhs_scale), float(rhs_scale), int(splits),
                              int(accumulate), _ptr(res), threads)
    return res


def deepgemm_fp8(a, sa, b, sb, threads: int = 1) -> np.ndarray:
    """E4M3FN bytes a [M, KB*128], b [N, KB*128]; f32 scales sa [M, KB], sb [N/128, KB]
    -> bf16 bits (uint16) [M, N]."""
    a, b = _c(a, np.uint8), _c(b, np.uint8)
    sa, sb = _c(sa, np.float32), _c(sb, np.float32)
    M, K = a.shape
    N = b.shape[0]
    out = np.empty((M, N), np.uint16)
    lib().orc_deepgemm_fp8(_ptr(a), _ptr(sa), M, K // 128, _ptr(b), _ptr(sb), N, _ptr(out), threads)
    return out


def fp8_gemm(a, bt, fmt: str, threads: int = 1) -> np.ndarray:
    """FP8 bytes a [M, K], bt [N, K] ("e4m3fn" or "e5m2") -> FP8 bytes [M, N]."""
    a, bt = _c(a, np.uint8), _c(bt, np.uint8)
    M, K = a.shape
    N = bt.shape[0]
    out = np.empty((M, N), np.uint8)
    lib().orc_fp8_gemm(1 if fmt == "e5m2" else 0, _ptr(a), M, K, _ptr(bt), N, _ptr(out), threads)
    return out


def f32_to_e5m2(values) -> np.ndarray:
    return np.array([lib().orc_f32_to_e5m2(float(v)) for v in np.asarray(values, np.float32).reshape(-1)], np.uint8)


def e5m2_to_f32(bits) -> np.ndarray:
    return np.array([lib().orc_e5m2_to_f32(int(v)) for v in np.asarray(bits, np.uint8).reshape(-1)], np.float32)


def fp4_decode_row(row) -> np.ndarray:
    """Decoded E2M1 values of one packed FP4 row (K = 2 * len(row))."""
    row = _c(row, np.uint8)
    return np.array([lib().orc_fp4_decode(_ptr(row), k) for k in range(2 * row.shape[0])], np.float32)


def fp4_bf16_matmul(x_bits, packed, threads: int = 1) -> np.ndarray:
    """bf16 bits x [M, K] and packed FP4 [N, K/2] -> bf16 bits [M, N]."""
    x, packed = _c(x_bits, np.uint16), _c(packed, np.uint8)
    M, K = x.shape
    N = packed.shape[0]
    out = np.empty((M, N), np.uint16)
    lib().orc_fp4_bf16_matmul(_ptr(x), M, K, _ptr(packed), N, _ptr(out), threads)
    return out


def w4_sym(x, packed, scales, threads: int = 1) -> np.ndarray:
    """The reference's weight_only_int4_matmul: f16 x [M, K], int32 packed [K/8, N],
    f16 scales [K/64, N] -> f16 [M, N]."""
    x, packed, scales = _c(x, np.float16), _c(packed, np.int32), _c(scales, np.float16)
    M, K = x.shape
    N = packed.shape[1]
    y = np.empty((M, N), np.float16)
    lib().orc_w4_sym(_ptr(x), M, K, _ptr(packed), _ptr(scales), N, _ptr(y), threads)
    return y


def quantized_gemm(a, b, bias, residual, output_scale, threads: int = 1) -> np.ndarray:
    """f16 a [M, K], b [K, N], f32 bias [N], f16 residual [M, N], f32 scale [N] -> int8 [M, N]."""
    a, b, r = _c(a, np.float16), _c(b, np.float16), _c(residual, np.float16)
    bias, sc = _c(bias, np.float32), _c(output_scale, np.float32)
    M, K = a.shape
    N = b.shape[1]
    out = np.empty((M, N), np.int8)
    lib().orc_quantized_gemm(_ptr(a), M, K, _ptr(b), N, _ptr(bias), _ptr(r), _ptr(sc), _ptr(out), threads)
    return out


def grouped_gemm(x_bits, bf16: bool, offsets, w_bits, out_rows: int, routes=None, top_k: int = 1,
                 threads: int = 1) -> np.ndarray:
    """16-bit element bits: x [rows, K]; w [G, K, N] (ragged) or [G, N, K] (routed).
    Returns the [out_rows, N] bits; rows no group writes stay 0."""
    x, w = _c(x_bits, np.uint16), _c(w_bits, np.uint16)
    offs = _c(offsets, np.int32)
    K = x.shape[1]
    G = offs.shape[0] - 1
    N = w.shape[2] if routes is None else w.shape[1]
    out = np.zeros((out_rows, N), np.uint16)
    r = None if routes is None else _c(routes, np.int32)
    lib().orc_grouped_gemm(_ptr(x), int(bf16), K, _ptr(offs), G, None if r is None else _ptr(r), top_k, _ptr(w), N,
                           _ptr(out), threads)
    return out


def moe_expert_ffn(x, route_offsets, member_routes, route_token, route_weights, w1, w2, y=None, tokens=None,
                   threads: int = 1) -> np.ndarray:
    """f16 x [T, D], i32 route_offsets [E+1], member_routes [R], route_token [NR], f32 route_weights [NR],
    f16 w1 [E, D, F], w2 [E, F, D] -> f32 y [T, D] (y += ..., from zeros if y is None). tokens: optional
    indices whose rows are computed (others keep y's values)."""
    x, w1, w2 = _c(x, np.float16), _c(w1, np.float16), _c(w2, np.float16)
    offs, mem, tok = _c(route_offsets, np.int32), _c(member_routes, np.int32), _c(route_token, np.int32)
    rw = _c(route_weights, np.float32)
    T, D = x.shape
    E, _, F = w1.shape
    out = np.zeros((T, D), np.float32) if y is None else _c(y, np.float32).copy()
    sel = None
    if tokens is not None:
        sel = np.zeros(T, np.uint8)
        sel[np.asarray(tokens)] = 1
    lib().orc_moe_expert_ffn(_ptr(x), T, D, _ptr(offs), E, _ptr(mem), _ptr(tok), _ptr(rw), _ptr(w1), _ptr(w2), F,
                             _ptr(out), None if sel is None else _ptr(sel), threads)
    return out


def float_gemm(a_bits, b_bits, bf16: bool, relu: bool = False, threads: int = 1) -> np.ndarray:
    """16-bit element bits a [M, K], b [K, N] -> c bits [M, N] (f16 or bf16)."""
    a, b = _c(a_bits, np.uint16), _c(b_bits, np.uint16)
    M, K = a.shape
    N = b.shape[1]
    c = np.empty((M, N), np.uint16)
    lib().orc_float_gemm(_ptr(a), M, K, _ptr(b), N, int(bf16), int(relu), _ptr(c), threads)
    return c


def nvfp4_quantize(x_bits, global_scale: float, packed=None, scales=None):
    """bf16 bits x [M, N] -> (packed [M, N/2], scales [ceil(M/128), ceil(N/64), 32, 4, 4]);
    entries no group writes keep the given (or zero) contents."""
    x = _c(x_bits, np.uint16)
    M, N = x.shape
    p = np.zeros((M, N // 2), np.uint8) if packed is None else _c(packed, np.uint8).copy()
    s = np.zeros(((M + 127) // 128, (N // 16 + 3) // 4, 32, 4, 4), np.uint8) if scales is None else \
        _c(scales, np.uint8).copy()
    lib().orc_nvfp4_quantize(_ptr(x), M, N, float(global_scale), _ptr(p), _ptr(s))
    return p, s


def e4m3fn_to_f32(bits) -> np.ndarray:
    return np.array([lib().orc_e4m3fn_to_f32(int(v)) for v in np.asarray(bits, np.uint8).reshape(-1)], np.float32)


def e8m0_to_f32(bits) -> np.ndarray:
    return np.array([lib().orc_e8m0_to_f32(int(v)) for v in np.asarray(bits, np.uint8).reshape(-1)], np.float32)


# ---- independent numpy restatements (used to pin the C oracle) ------------------

def w4a8_int64(a, packed) -> np.ndarray:
    """The reference's CPU formula (cpu_runtime.py:105-108) in int64 numpy."""
    p = np.asarray(packed, np.int64)
    nib = np.stack((p & 15, p >> 4), axis=-1).reshape(p.shape[0], -1)
    signed = nib - ((nib & 8) << 1)
    return signed @ np.asarray(a, np.int64).T


def bitnet_int2_int64(a, packed) -> np.ndarray:
    """The reference's CPU formula (cpu_runtime.py:111-114) in int64 numpy."""
    p = np.asarray(packed, np.int64)
    groups = p.reshape(p.shape[0], -1, 4)
    logical = np.stack(tuple((groups >> (lane * 2)) & 3 for lane in range(4)), axis=2).reshape(p.shape[0], -1)
    return np.asarray(a, np.int64) @ logical.T


def q4k_pack(d, dmin, sc, m, q) -> np.ndarray:
    """Build Q4_K records from fields (the inverse of the spec's unpacking,
    doc/dsl/quantized-operations.en.md:28-36): d, dmin f16 [G]; sc, m 6-bit [G, 8];
    q 4-bit [G, 256]."""
    d = np.asarray(d, np.float16).reshape(-1)
    G = d.size
    sc, m, q = (np.asarray(a, np.int64) for a in (sc, m, q))
    rec = np.zeros((G, Q4K_BYTES), np.uint8)
    rec[:, 0:2] = d.view(np.uint8).reshape(G, 2)
    rec[:, 2:4] = np.asarray(dmin, np.float16).reshape(-1).view(np.uint8).reshape(G, 2)
    for r, f in enumerate((sc, m)):
        for i in range(4):
            rec[:, 4 + 4 * r + i] |= (f[:, i] & 63).astype(np.uint8)
            rec[:, 4 + 4 * r + i] |= ((f[:, 4 + i] >> 4) << 6).astype(np.uint8)
            rec[:, 12 + i] |= ((f[:, 4 + i] & 15) << (4 * r)).astype(np.uint8)
    for g in range(4):  # 64 elements per 32-byte group: low nibbles then high nibbles
        lo = q[:, 64 * g:64 * g + 32]
        hi = q[:, 64 * g + 32:64 * g + 64]
        rec[:, 16 + 32 * g:48 + 32 * g] = (lo | (hi << 4)).astype(np.uint8)
    return rec


def q8k_fields(xq):
    """Q8_K records [G, 292] -> ds f32 [G], q int64 [G, 256], bsum int64 [G, 16]."""
    xq = np.asarray(xq, np.uint8)
    ds = xq[:, 0:4].copy().view(np.float32).reshape(-1)
    q = xq[:, 4:260].view(np.int8).astype(np.int64)
    bsum = xq[:, 260:292].copy().view(np.int16).astype(np.int64)
    return ds, q, bsum


def q4k_q8k_dot_f64(wfields, xq) -> float:
    """float64 dot of the dequantised vectors: sum_i (d*sc*q - dmin*m) * (ds*q8).
    Equal to the record formula up to f32 rounding (bsum replaces sum(q8))."""
    d, dmin, sc, m, q = wfields
    ds, q8, _ = q8k_fields(xq)
    sub = np.repeat(np.arange(8), 32)
    w = (np.asarray(d, np.float16).astype(np.float64)[:, None] * sc[:, sub] * q
         - np.asarray(dmin, np.float16).astype(np.float64)[:, None] * m[:, sub])
    return float(np.sum(w * (ds.astype(np.float64)[:, None] * q8)))




def unpack_nibbles(packed: np.ndarray) -> np.ndarray:
    """[N, K/2] uint8 -> [N, K] uint8; even k = low nibble."""
    packed = np.asarray(packed, np.uint8)
    out = np.empty((packed.shape[0], packed.shape[1] * 2), np.uint8)
    out[:, 0::2] = packed & 15
    out[:, 1::2] = packed >> 4
    return out


def dequant_w4_f64(packed, scales, zeros) -> np.ndarray:
    q = unpack_nibbles(packed).astype(np.float64)
    gs = q.shape[1] // scales.shape[1]
    z = np.repeat(np.asarray(zeros, np.float64), gs, axis=1)
    s = np.repeat(np.asarray(scales, np.float16).astype(np.float64), gs, axis=1)
    return (q - z) * s


def w4a16_f64(x, packed, scales, zeros) -> np.ndarray:
    """float64 brute force (no rounding until the caller's comparison)."""
    return np.asarray(x, np.float16).astype(np.float64) @ dequant_w4_f64(packed, scales, zeros).T


def w8a16_f64(x, w, scales) -> np.ndarray:
    acc = np.asarray(x, np.float16).astype(np.float64) @ np.asarray(w, np.int8).astype(np.float64).T
    return acc * np.asarray(scales, np.float16).astype(np.float64)[None, :]


def i8_gemm_i64(a, w, bias=None) -> np.ndarray:
    acc = np.asarray(a, np.int64) @ np.asarray(w, np.int64).T
    if bias is not None:
        acc = acc + np.asarray(bias, np.int64)[None, :]
    return acc


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(f: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 in numpy (independent of oracle.c)."""
    u = np.asarray(f, np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def w8a8_numpy(a, sa, w, sw) -> np.ndarray:
    acc = i8_gemm_i64(a, w).astype(np.int32)  # exact: |acc| < 2^31 for these ranges
    f = acc.astype(np.float32) * np.asarray(sa, np.float32)[:, None]
    f = f * np.asarray(sw, np.float32)[None, :]
    return f32_to_bf16_bits(f)


def moe_route_numpy(logits, top_k: int, renormalize: bool = True):
    lg = np.asarray(logits, np.float64)
    order = np.argsort(-lg, axis=1, kind="stable")[:, :top_k]  # ties: lower index first
    p = np.exp(lg - lg.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    w = np.take_along_axis(p, order, axis=1)
    if renormalize:
        w = w / w.sum(axis=1, keepdims=True)
    return order.astype(np.int32), w


def moe_align_numpy(ids, experts: int, block: int):
    """Direct restatement of moe_align_block_size (cpu_runtime.py:1081-1098)."""
    flat = np.asarray(ids, np.int64).reshape(-1)
    R = flat.size
    valid = (flat >= 0) & (flat < experts)
    counts = np.bincount(flat[valid], minlength=experts)
    padded = (counts + block - 1) // block * block
    offsets = np.concatenate(([0], np.cumsum(padded))).astype(np.int32)
    routes = np.argsort(np.where(valid, flat, experts), kind="stable")
    cap, nb = align_sizes(R, experts, block)
    sorted_ids = np.full(cap, R, np.int32)
    blocks = np.full(nb, -1, np.int32)
    src = 0
    for e in range(experts):
        b, c = int(offsets[e]), int(counts[e])
        sorted_ids[b:b + c] = routes[src:src + c]
        blocks[b // block:int(offsets[e + 1]) // block] = e
        src += c
    return sorted_ids, blocks, offsets, np.array([offsets[-1]], np.int32)


def moe_ffn_f64(x, ids, weights, wgu, sgu, zgu, wd, sd, zd) -> np.ndarray:
    """float64 brute force of the SiLU-gated W4 expert FFN (hidden kept in f64)."""
    x = np.asarray(x, np.float16).astype(np.float64)
    T, H = x.shape
    top_k = ids.shape[1]
    F = wgu.shape[1] // 2
    y = np.zeros((T, H), np.float64)
    for e in range(wgu.shape[0]):
        toks, slots = np.nonzero(ids == e)
        if toks.size == 0:
            continue
        gu = dequant_w4_f64(wgu[e], sgu[e], zgu[e])
        dn = dequant_w4_f64(wd[e], sd[e], zd[e])
        h = x[toks] @ gu.T
        g, u = h[:, :F], h[:, F:]
        a = g / (1.0 + np.exp(-g)) * u
        o = a @ dn.T
        np.add.at(y, toks, np.asarray(weights, np.float64)[toks, slots][:, None] * o)
    return y
