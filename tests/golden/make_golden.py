"""Writes the committed golden fixtures (small inputs + expected outputs).

The reference ships no golden vectors for this path (its comparisons are live
runs against PyTorch eager), so the fixtures here come from this repo's C
oracle, cross-checked at generation time against the independent numpy
float64 / int64 restatements in ``oracle/__init__.py``. Tests then pin both
the C oracle (exact regression) and the GPU kernels against these files.

Run: ``python tests/golden/make_golden.py`` (rewrites tests/golden/*.npz).
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))

import oracle  # noqa: E402
from intent_amd import inputs  # noqa: E402


def rms(a):
    return float(np.sqrt(np.mean(np.asarray(a, np.float64) ** 2)))


def f16_close(y, y64) -> bool:
    """Within half an f16 ulp of the float64 value plus a small fp32-accumulation slack."""
    err = np.abs(y.astype(np.float64) - y64)
    return bool(np.all(err <= 2.0 ** -11 * np.abs(y64) + 1e-5 * rms(y64) + 2.0 ** -25))


def main() -> None:
    # W4A16: two shapes, group 128 and 64 (natural packing, asymmetric zeros).
    for name, (M, K, N, g) in {"w4a16_m3_k256_n40_g128": (3, 256, 40, 128),
                               "w4a16_m17_k512_n24_g64": (17, 512, 24, 64)}.items():
        d = inputs.config1_w4a16_decode(11, M=M, K=K, N=N, group=g)
        y = oracle.w4a16(d["x"], d["packed"], d["scales"], d["zeros"])
        y64 = oracle.w4a16_f64(d["x"], d["packed"], d["scales"], d["zeros"])
        assert f16_close(y, y64)
        np.savez(HERE / f"{name}.npz", x=d["x"], packed=d["packed"], scales=d["scales"], zeros=d["zeros"], y=y,
                 y_f64=y64)
    # W8A16
    d = inputs.config0_w8a16(12, M=5, K=192, N=33)
    y = oracle.w8a16(d["x"], d["w"], d["scales"])
    y64 = oracle.w8a16_f64(d["x"], d["w"], d["scales"])
    assert f16_close(y, y64)
    np.savez(HERE / "w8a16_m5_k192_n33.npz", x=d["x"], w=d["w"], scales=d["scales"], y=y, y_f64=y64)
    # W8A8 (bf16 bits) and the raw int32 contraction with bias
    d = inputs.config3_w8a8(13, M=9, K=256, N=20)
    out = oracle.w8a8(d["a"], d["a_scales"], d["w"], d["w_scales"])
    assert np.array_equal(out, oracle.w8a8_numpy(d["a"], d["a_scales"], d["w"], d["w_scales"]))
    bias = np.random.default_rng(13).integers(-1000, 1000, 20).astype(np.int32)
    acc = oracle.i8_gemm_i32(d["a"], d["w"], bias)
    assert np.array_equal(acc.astype(np.int64), oracle.i8_gemm_i64(d["a"], d["w"], bias))
    np.savez(HERE / "w8a8_m9_k256_n20.npz", a=d["a"], a_scales=d["a_scales"], w=d["w"], w_scales=d["w_scales"],
             out_bf16_bits=out, bias=bias, acc_i32=acc)
    # K-quant projection: Q4_K rows x Q8_K records (bit-exact f32), with the
    # float64 dequantised dot as the generation-time cross-check.
    d = inputs.kquant_projection(14, N=7, K=768)
    xq = oracle.q8k_quantize(d["x"])
    y = oracle.q4k_gemv(d["w"], xq)
    ds, q8, bsum = oracle.q8k_fields(xq)
    assert np.array_equal(bsum, q8.reshape(-1, 16, 16).sum(-1))
    np.savez(HERE / "q4k_n7_g3.npz", w=d["w"], x=d["x"], xq=xq, y=y)
    # MoE routing + alignment (exact) and a tiny expert FFN
    m = inputs.config4_moe(14, T=24, H=128, E=4, top_k=2, F=128)
    ids, wts = oracle.moe_route(m["logits"], 2, True)
    nid, _ = oracle.moe_route_numpy(m["logits"], 2, True)
    assert np.array_equal(ids, nid)
    sorted_ids, blocks, offsets, total = oracle.moe_align(ids, 4, 16)
    for got, ref in zip((sorted_ids, blocks, offsets, total), oracle.moe_align_numpy(ids, 4, 16)):
        assert np.array_equal(got, ref)
    y = oracle.moe_ffn_w4(m["x"], ids, wts, m["wgu"], m["sgu"], m["zgu"], m["wd"], m["sd"], m["zd"])
    y64 = oracle.moe_ffn_f64(m["x"], ids, wts, m["wgu"], m["sgu"], m["zgu"], m["wd"], m["sd"], m["zd"])
    assert np.max(np.abs(y - y64)) <= 1e-2 * rms(y64)
    np.savez(HERE / "moe_t24_h128_e4_f128.npz", logits=m["logits"], x=m["x"], wgu=m["wgu"], sgu=m["sgu"],
             zgu=m["zgu"], wd=m["wd"], sd=m["sd"], zd=m["zd"], topk_ids=ids, topk_weights=wts,
             sorted_ids_b16=sorted_ids, blocks_b16=blocks, offsets_b16=offsets, total_b16=total, y=y, y_f64=y64)
    print("golden fixtures written to", HERE)


if __name__ == "__main__":
    main()
