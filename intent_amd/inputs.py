"""Seeded synthetic inputs for the five benchmark configurations.

Draws use ``numpy.random.default_rng(seed)`` in the order each configuration
lists its tensors (the reference seeds its example inputs the same way,
examples/programs/inputs.py:27-41: float32 standard normal then cast).
W4 weights are drawn as nibbles [N, K] then packed two per byte, even k in the
low nibble. All arrays are host numpy arrays; ``to_device`` moves them.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np


def pack_nibbles(nibbles: np.ndarray) -> np.ndarray:
    """[..., K] uint8 (0..15) -> [..., K/2] uint8, even k in the low nibble."""
    nibbles = np.asarray(nibbles, np.uint8)
    if nibbles.shape[-1] % 2:
        raise ValueError("K must be even to pack nibbles")
    return (nibbles[..., 0::2] & 15) | ((nibbles[..., 1::2] & 15) << 4)


def w4_weight(rng: np.random.Generator, rows: int, k: int, group: int = 128,
              scale_range=(0.005, 0.02)) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Asymmetric uint4 group-quant weight: (packed [rows,k/2], scales f16, zeros u8)."""
    nib = rng.integers(0, 16, size=(rows, k), dtype=np.uint8)
    packed = pack_nibbles(nib)
    del nib
    scales = rng.uniform(scale_range[0], scale_range[1], size=(rows, k // group)).astype(np.float32).astype(np.float16)
    zeros = rng.integers(0, 16, size=(rows, k // group), dtype=np.uint8)
    return packed, scales, zeros


def normal_f16(rng: np.random.Generator, shape) -> np.ndarray:
    return rng.standard_normal(shape, dtype=np.float32).astype(np.float16)


def config0_w8a16(seed: int = 0, M: int = 16, K: int = 1024, N: int = 1024) -> dict:
    rng = np.random.default_rng(seed)
    x = normal_f16(rng, (M, K))
    w = rng.integers(-127, 128, size=(N, K), dtype=np.int8)
    s = rng.uniform(0.002, 0.02, size=N).astype(np.float32).astype(np.float16)
    return {"x": x, "w": w, "scales": s}


def config1_w4a16_decode(seed: int = 0, M: int = 1, K: int = 4096, N: int = 4096, group: int = 128) -> dict:
    rng = np.random.default_rng(seed)
    x = normal_f16(rng, (M, K))
    packed, scales, zeros = w4_weight(rng, N, K, group)
    return {"x": x, "packed": packed, "scales": scales, "zeros": zeros}


def config2_w4a16_prefill(seed: int = 0, M: int = 2048, K: int = 4096, N: int = 11008, group: int = 128) -> dict:
    return config1_w4a16_decode(seed, M=M, K=K, N=N, group=group)


def config3_w8a8(seed: int = 0, M: int = 4096, K: int = 8192, N: int = 8192) -> dict:
    rng = np.random.default_rng(seed)
    a = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
    sa = rng.uniform(0.005, 0.05, size=M).astype(np.float32)
    w = rng.integers(-127, 128, size=(N, K), dtype=np.int8)
    sw = rng.uniform(0.001, 0.01, size=N).astype(np.float32)
    return {"a": a, "a_scales": sa, "w": w, "w_scales": sw}


def _config4_logits(rng, T: int, E: int) -> np.ndarray:
    return rng.standard_normal((T, E), dtype=np.float32)


def config4_logits(seed: int = 0, T: int = 512, E: int = 8) -> np.ndarray:
    """The router logits of config4_moe(seed, T=T, E=E) (its first draw), without
    drawing the expert weights."""
    return _config4_logits(np.random.default_rng(seed), T, E)


def config4_moe(seed: int = 0, T: int = 512, H: int = 4096, E: int = 8, top_k: int = 2, F: int = 14336,
                group: int = 128) -> dict:
    rng = np.random.default_rng(seed)
    logits = _config4_logits(rng, T, E)
    x = normal_f16(rng, (T, H))
    wgu = np.empty((E, 2 * F, H // 2), np.uint8)
    sgu = np.empty((E, 2 * F, H // group), np.float16)
    zgu = np.empty((E, 2 * F, H // group), np.uint8)
    wd = np.empty((E, H, F // 2), np.uint8)
    sd = np.empty((E, H, F // group), np.float16)
    zd = np.empty((E, H, F // group), np.uint8)
    for e in range(E):
        wgu[e], sgu[e], zgu[e] = w4_weight(rng, 2 * F, H, group)
        wd[e], sd[e], zd[e] = w4_weight(rng, H, F, group)
    return {"logits": logits, "x": x, "top_k": top_k, "wgu": wgu, "sgu": sgu, "zgu": zgu,
            "wd": wd, "sd": sd, "zd": zd}


def moe_routes(T: int, top_k: int, E: int, kind: str = "reference", seed: int = 0) -> dict:
    """Ragged routing of the reference's f16 MoE FFN (moe.py:12-53).

    kind "reference": the construction of experiments/_common/support.py:113-130 (route r =
    token r // top_k, weight 1/top_k, expert r % E, members = stable argsort by expert);
    kind "random": top-k experts of seeded N(0,1) logits per token with their renormalised
    softmax weights, members stable-sorted by expert (the moe_align order)."""
    R = T * top_k
    route_token = np.repeat(np.arange(T, dtype=np.int32), top_k)
    if kind == "reference":
        experts = (np.arange(R) % E).astype(np.int64)
        weights = np.full(R, 1.0 / top_k, np.float32)
    else:
        rng = np.random.default_rng(seed)
        logits = rng.standard_normal((T, E)).astype(np.float32)
        ids = np.argsort(-logits, axis=1, kind="stable")[:, :top_k]
        p = np.exp(logits - logits.max(axis=1, keepdims=True))
        p /= p.sum(axis=1, keepdims=True)
        pw = np.take_along_axis(p, ids, axis=1)
        weights = (pw / pw.sum(axis=1, keepdims=True)).astype(np.float32).reshape(-1)
        experts = ids.reshape(-1).astype(np.int64)
    members = np.argsort(experts, kind="stable").astype(np.int32)
    counts = np.bincount(experts, minlength=E)
    offsets = np.concatenate(([0], np.cumsum(counts))).astype(np.int32)
    return {"route_offsets": offsets, "member_routes": members, "route_token": route_token,
            "route_weights": weights}


def moe_ffn_f16(seed: int = 0, T: int = 512, D: int = 4096, E: int = 8, top_k: int = 2, F: int = 14336,
                kind: str = "reference") -> dict:
    """Inputs of the reference's f16 moe_expert_ffn: x [T, D], w1 [E, D, F], w2 [E, F, D] ~ N(0,1)
    scaled by 1/sqrt(fan-in) (keeps f16 hidden values in range), f32 y [T, D] zeros."""
    rng = np.random.default_rng(seed)
    d = moe_routes(T, top_k, E, kind, seed)
    d["x"] = normal_f16(rng, (T, D))
    d["w1"] = (rng.standard_normal((E, D, F), dtype=np.float32) / np.sqrt(D)).astype(np.float16)
    d["w2"] = (rng.standard_normal((E, F, D), dtype=np.float32) / np.sqrt(F)).astype(np.float16)
    d["y"] = np.zeros((T, D), np.float32)
    return d


def q4k_records(rng: np.random.Generator, shape, d_range=(0.0005, 0.005)) -> np.ndarray:
    """Random Q4_K records uint8 [*shape, 144]: f16 d and dmin drawn from d_range;
    every other byte (6-bit sc/m fields, nibbles) uniform, which is always a
    legal record (doc/dsl/quantized-operations.en.md:21-36)."""
    shape = tuple(shape)
    rec = rng.integers(0, 256, size=shape + (144,), dtype=np.uint8)
    d = rng.uniform(d_range[0], d_range[1], size=shape + (2,)).astype(np.float32).astype(np.float16)
    rec[..., 0:4] = d.view(np.uint8).reshape(shape + (4,))
    return rec


def kquant_projection(seed: int = 0, N: int = 4096, K: int = 4096) -> dict:
    """quantized_projection inputs (examples/kernels/quantization/quantized_projection.py):
    Q4_K weight records [N, K/256, 144] and f32 activations [K/256, 256] ~ N(0,1)."""
    if K % 256:
        raise ValueError("K must be a multiple of 256")
    rng = np.random.default_rng(seed)
    w = q4k_records(rng, (N, K // 256))
    x = rng.standard_normal((K // 256, 256), dtype=np.float32)
    return {"w": w, "x": x}


def to_device(arrays: dict, device="cuda") -> dict:
    import torch

    out = {}
    for key, value in arrays.items():
        out[key] = torch.from_numpy(np.ascontiguousarray(value)).to(device) if isinstance(value, np.ndarray) else value
    return out


@dataclass(frozen=True)
class Workload:
    name: str
    flops: int
    bytes: int


def w4a16_work(M: int, K: int, N: int, group: int = 128) -> Workload:
    """Algorithmic flops and bytes (every tensor touched once)."""
    g = K // group
    b = M * K * 2 + N * K // 2 + N * g * 2 + N * g + M * N * 2
    return Workload(f"w4a16 M{M} K{K} N{N} g{group}", 2 * M * N * K, b)


def w8a16_work(M: int, K: int, N: int) -> Workload:
    return Workload(f"w8a16 M{M} K{K} N{N}", 2 * M * N * K, M * K * 2 + N * K + N * 2 + M * N * 2)


def w8a8_work(M: int, K: int, N: int) -> Workload:
    return Workload(f"w8a8 M{M} K{K} N{N}", 2 * M * N * K, M * K + N * K + M * 4 + N * 4 + M * N * 2)


def kquant_work(N: int, K: int) -> Workload:
    """Q4_K weights (144 B per 256) + f32 activations + Q8_K records written and
    read once + f32 outputs; flops count one multiply-add per weight."""
    G = K // 256
    return Workload(f"q4k projection N{N} K{K}", 2 * N * K, N * G * 144 + K * 4 + 2 * G * 292 + N * 4)


def moe_work(T: int, H: int, E: int, top_k: int, F: int, group: int = 128) -> Workload:
    R = T * top_k
    flops = 2 * R * H * (2 * F) + 2 * R * F * H
    weights = E * (2 * F * H // 2 + 2 * F * (H // group) * 3 + H * F // 2 + H * (F // group) * 3)
    acts = T * E * 4 + T * H * 2 + 2 * T * H * 4  # logits, x, y read and written
    return Workload(f"moe T{T} H{H} E{E} top{top_k} F{F} g{group}", flops, weights + acts)
