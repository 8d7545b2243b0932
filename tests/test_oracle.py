"""Pins the C oracle (oracle/oracle.c) with checks a plausible mistake would fail.

Each function is checked against (a) the committed golden fixtures, (b) an
independent numpy float64 / int64 restatement, and (c) closed forms and
known answers (all-equal nibbles and zeros give 0, one-hot activations pick a
single dequantized column, nibble order, integer wraparound, tie-breaking,
stable scatter order). CPU only.
"""
from itertools import permutations
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from intent_amd import inputs

GOLDEN = Path(__file__).resolve().parent / "golden"


def rms(a):
    return float(np.sqrt(np.mean(np.asarray(a, np.float64) ** 2)))


def f16_close(y, y64):
    err = np.abs(np.asarray(y, np.float64) - y64)
    bound = 2.0 ** -11 * np.abs(y64) + 1e-5 * rms(y64) + 2.0 ** -25
    assert np.all(err <= bound), f"max excess {np.max(err - bound)}"


# ---- scalar conversions ----------------------------------------------------------

def test_f16_to_f32_all_patterns():
    lib = oracle.lib()
    bits = np.arange(65536, dtype=np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([lib.orc_f16_to_f32(int(b)) for b in bits], np.float32)
    same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    assert same.all()


def test_f32_to_f16_round_to_nearest_even():
    lib = oracle.lib()
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-9, 6, 20000),
        np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 65536.0, 1e9, -1e9, np.inf, -np.inf,
                  2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26, 2.0 ** -14, 2.0 ** -14 - 2.0 ** -25,
                  1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11], np.float32),
        # exact halfway points between adjacent f16 values
        ((np.arange(-300, 300, dtype=np.float32) + 0.5) * 2.0 ** -10 + 1.0).astype(np.float32),
    ])
    want = vals.astype(np.float16).view(np.uint16)
    got = np.array([lib.orc_f32_to_f16(float(v)) for v in vals], np.uint16)
    assert np.array_equal(got, want)
    assert lib.orc_f32_to_f16(float("nan")) & 0x7C00 == 0x7C00


def test_f32_to_bf16_matches_torch():
    lib = oracle.lib()
    rng = np.random.default_rng(1)
    vals = np.concatenate([rng.standard_normal(5000).astype(np.float32) * 1e3,
                           np.array([1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8, 3.3895314e38, np.inf, -0.0], np.float32)])
    want = torch.from_numpy(vals).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = np.array([lib.orc_f32_to_bf16(float(v)) for v in vals], np.uint16)
    assert np.array_equal(got, want)
    assert np.array_equal(oracle.f32_to_bf16_bits(vals), want)


# ---- W4A16 ------------------------------------------------------------------------

@pytest.mark.parametrize("name", ["w4a16_m3_k256_n40_g128", "w4a16_m17_k512_n24_g64"])
def test_w4a16_golden(name):
    g = np.load(GOLDEN / f"{name}.npz")
    y = oracle.w4a16(g["x"], g["packed"], g["scales"], g["zeros"], threads=2)
    assert np.array_equal(y.view(np.uint16), g["y"].view(np.uint16))
    f16_close(y, g["y_f64"])


@pytest.mark.parametrize("M,K,N,group", [(1, 4096, 64, 128), (4, 384, 16, 32), (2, 1024, 8, 256)])
def test_w4a16_vs_float64(M, K, N, group):
    d = inputs.config1_w4a16_decode(3, M=M, K=K, N=N, group=group)
    y = oracle.w4a16(d["x"], d["packed"], d["scales"], d["zeros"])
    f16_close(y, oracle.w4a16_f64(d["x"], d["packed"], d["scales"], d["zeros"]))


def test_w4a16_known_answers():
    K, N = 256, 4
    rng = np.random.default_rng(2)
    nib = rng.integers(0, 16, (N, K), dtype=np.uint8)
    zeros = rng.integers(0, 16, (N, 2), dtype=np.uint8)
    scales = np.full((N, 2), 0.5, np.float16)
    # q == z everywhere -> exactly zero whatever x is
    q_eq = np.repeat(zeros, 128, axis=1)
    x = inputs.normal_f16(rng, (3, K))
    y = oracle.w4a16(x, inputs.pack_nibbles(q_eq), scales, zeros)
    assert np.all(y == 0)
    # one-hot activation picks (q[n,k] - z[n,g]) * s[n,g] exactly; covers nibble order (even k low)
    for k in (0, 1, 2, 127, 128, 129, 255):
        xo = np.zeros((1, K), np.float16)
        xo[0, k] = 1
        y = oracle.w4a16(xo, inputs.pack_nibbles(nib), scales, zeros)
        want = (nib[:, k].astype(np.float32) - zeros[:, k // 128]) * 0.5
        assert np.array_equal(y[0].astype(np.float32), want), k
    # packed byte 0x21 holds k=0 -> 1 and k=1 -> 2
    packed = np.zeros((1, K // 2), np.uint8)
    packed[0, 0] = 0x21
    xo = np.zeros((1, K), np.float16)
    xo[0, 1] = 1
    y = oracle.w4a16(xo, packed, np.ones((1, 2), np.float16), np.zeros((1, 2), np.uint8))
    assert y[0, 0] == 2


# ---- W8A16 ------------------------------------------------------------------------

def test_w8a16_golden_and_f64():
    g = np.load(GOLDEN / "w8a16_m5_k192_n33.npz")
    y = oracle.w8a16(g["x"], g["w"], g["scales"])
    assert np.array_equal(y.view(np.uint16), g["y"].view(np.uint16))
    d = inputs.config0_w8a16(4, M=3, K=1024, N=16)
    f16_close(oracle.w8a16(d["x"], d["w"], d["scales"]), oracle.w8a16_f64(d["x"], d["w"], d["scales"]))
    # one-hot: y[n] = w[n,k] * s[n]
    xo = np.zeros((1, 1024), np.float16)
    xo[0, 7] = 1
    y = oracle.w8a16(xo, d["w"], d["scales"])
    want = (d["w"][:, 7].astype(np.float32) * d["scales"].astype(np.float32)).astype(np.float16)
    assert np.array_equal(y[0], want)


# ---- int8 -------------------------------------------------------------------------

def test_i8_golden_and_exact():
    g = np.load(GOLDEN / "w8a8_m9_k256_n20.npz")
    assert np.array_equal(oracle.i8_gemm_i32(g["a"], g["w"], g["bias"]), g["acc_i32"])
    assert np.array_equal(oracle.w8a8(g["a"], g["a_scales"], g["w"], g["w_scales"]), g["out_bf16_bits"])
    rng = np.random.default_rng(5)
    a = rng.integers(-128, 128, (7, 320), dtype=np.int8)
    w = rng.integers(-128, 128, (11, 320), dtype=np.int8)
    assert np.array_equal(oracle.i8_gemm_i32(a, w).astype(np.int64), oracle.i8_gemm_i64(a, w))


def test_i8_wraps_modulo_2_32():
    K = 140000  # 127*127*K exceeds 2^31
    a = np.full((1, K), 127, np.int8)
    w = np.full((1, K), 127, np.int8)
    exact = 127 * 127 * K
    wrapped = (exact + 2 ** 31) % 2 ** 32 - 2 ** 31
    assert oracle.i8_gemm_i32(a, w)[0, 0] == wrapped
    assert oracle.i8_gemm_i32(-a, w)[0, 0] == (-exact + 2 ** 31) % 2 ** 32 - 2 ** 31


def test_w8a8_epilogue_order_matches_torch():
    d = inputs.config3_w8a8(6, M=16, K=512, N=24)
    acc = torch.from_numpy(oracle.i8_gemm_i64(d["a"], d["w"]).astype(np.float32))
    f = acc * torch.from_numpy(d["a_scales"])[:, None]
    f = f * torch.from_numpy(d["w_scales"])[None, :]
    want = f.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(oracle.w8a8(d["a"], d["a_scales"], d["w"], d["w_scales"]), want)
    assert np.array_equal(oracle.w8a8_numpy(d["a"], d["a_scales"], d["w"], d["w_scales"]), want)


# ---- MoE routing ------------------------------------------------------------------

def test_route_vs_numpy_and_ties():
    rng = np.random.default_rng(7)
    logits = rng.standard_normal((300, 8), dtype=np.float32)
    logits[::3, 5] = logits[::3, 2]  # ties -> lower index first
    logits[::7] = 0.5  # all-equal rows -> experts 0, 1
    for k, renorm in ((2, True), (3, False), (1, True)):
        ids, w = oracle.moe_route(logits, k, renorm)
        nid, nw = oracle.moe_route_numpy(logits, k, renorm)
        assert np.array_equal(ids, nid)
        np.testing.assert_allclose(w, nw, rtol=1e-5)
    ids, w = oracle.moe_route(logits[::7], 2, True)
    assert np.all(ids == [0, 1]) and np.allclose(w, 0.5)


def test_route_brute_force_orderings():
    base = np.array([0.1, 0.7, -0.4, 1.3], np.float32)
    for perm in permutations(range(4)):
        lg = base[list(perm)][None, :]
        ids, w = oracle.moe_route(lg, 2, True)
        order = sorted(range(4), key=lambda e: -lg[0, e])
        assert list(ids[0]) == order[:2]
        p = np.exp(lg[0] - lg[0].max())
        assert abs(w[0, 0] - p[order[0]] / (p[order[0]] + p[order[1]])) < 1e-6


# ---- MoE alignment ----------------------------------------------------------------

@pytest.mark.parametrize("T,k,E,B", [(24, 2, 4, 16), (4096, 2, 64, 128), (333, 3, 7, 32), (1, 1, 1, 128)])
def test_align_vs_numpy_and_invariants(T, k, E, B):
    rng = np.random.default_rng(T + E)
    ids = rng.integers(0, E, (T, k), dtype=np.int32)
    if T > 4:
        ids[0, 0], ids[2, 0] = -1, E  # dropped
    got = oracle.moe_align(ids, E, B)
    for g, r in zip(got, oracle.moe_align_numpy(ids, E, B)):
        assert np.array_equal(g, r)
    sorted_ids, blocks, offsets, total = got
    R = T * k
    flat = ids.reshape(-1)
    valid = np.nonzero((flat >= 0) & (flat < E))[0]
    assert sorted(sorted_ids[sorted_ids < R].tolist()) == valid.tolist()  # each valid route exactly once
    assert np.all(offsets % B == 0) and total[0] == offsets[-1]
    for e in range(E):
        seg = sorted_ids[offsets[e]:offsets[e + 1]]
        live = seg[seg < R]
        assert np.all(flat[live] == e) and np.all(np.diff(live) > 0)  # stable order
        assert np.all(seg[len(live):] == R)  # padding after the routes
        assert np.all(blocks[offsets[e] // B:offsets[e + 1] // B] == e)
    assert np.all(blocks[total[0] // B:] == -1)


def test_align_reference_case_canonical():
    """The reference's moe_alignment case: ids = arange(T*k) % E (routing.py:46-115)."""
    T, k, E, B = 4096, 2, 64, 128
    ids = (np.arange(T * k) % E).astype(np.int32).reshape(T, k)
    sorted_ids, blocks, offsets, total = oracle.moe_align(ids, E, B)
    assert total[0] == E * B and np.array_equal(blocks[:E], np.arange(E))
    for e in range(E):
        assert np.array_equal(sorted_ids[e * B:(e + 1) * B], np.arange(e, T * k, E))


def test_align_golden():
    g = np.load(GOLDEN / "moe_t24_h128_e4_f128.npz")
    got = oracle.moe_align(g["topk_ids"], 4, 16)
    for a, name in zip(got, ("sorted_ids_b16", "blocks_b16", "offsets_b16", "total_b16")):
        assert np.array_equal(a, g[name])


# ---- MoE expert FFN ---------------------------------------------------------------

def test_moe_ffn_golden_and_f64():
    g = np.load(GOLDEN / "moe_t24_h128_e4_f128.npz")
    ids, w = oracle.moe_route(g["logits"], 2, True)
    assert np.array_equal(ids, g["topk_ids"])
    y = oracle.moe_ffn_w4(g["x"], ids, w, g["wgu"], g["sgu"], g["zgu"], g["wd"], g["sd"], g["zd"], threads=2)
    assert np.array_equal(y, g["y"])
    assert np.max(np.abs(y - g["y_f64"])) <= 1e-2 * rms(g["y_f64"])


def test_moe_ffn_accumulates_in_slot_order():
    m = inputs.config4_moe(8, T=4, H=128, E=3, top_k=2, F=128)
    ids, w = oracle.moe_route(m["logits"], 2, True)
    zero = oracle.moe_ffn_w4(m["x"], ids, w, m["wgu"], m["sgu"], m["zgu"], m["wd"], m["sd"], m["zd"])
    y0 = np.full((4, 128), 3.0, np.float32)
    acc = oracle.moe_ffn_w4(m["x"], ids, w, m["wgu"], m["sgu"], m["zgu"], m["wd"], m["sd"], m["zd"], y=y0.copy())
    np.testing.assert_allclose(acc - 3.0, zero, atol=1e-5)
    # a single expert with weight 1 equals the dense SiLU-gated FFN brute force
    ids1 = np.zeros((4, 1), np.int32)
    w1 = np.ones((4, 1), np.float32)
    y = oracle.moe_ffn_w4(m["x"], ids1, w1, m["wgu"], m["sgu"], m["zgu"], m["wd"], m["sd"], m["zd"])
    y64 = oracle.moe_ffn_f64(m["x"], ids1, w1, m["wgu"], m["sgu"], m["zgu"], m["wd"], m["sd"], m["zd"])
    assert np.max(np.abs(y - y64)) <= 1e-2 * rms(y64)


# ---- K-quant records (doc/dsl/quantized-operations.en.md:11-70) -------------------

def _q4k_fields(rng, G):
    d = rng.uniform(0.001, 0.05, G).astype(np.float16)
    dmin = rng.uniform(0.001, 0.05, G).astype(np.float16)
    sc = rng.integers(0, 64, (G, 8))
    m = rng.integers(0, 64, (G, 8))
    q = rng.integers(0, 16, (G, 256))
    return d, dmin, sc, m, q


def _q8k_record(ds, q8):
    """Q8_K records from ds f32 [G] and q int [G,256] (bsum = exact sums)."""
    q8 = np.asarray(q8, np.int64)
    G = q8.shape[0]
    rec = np.zeros((G, oracle.Q8K_BYTES), np.uint8)
    rec[:, 0:4] = np.asarray(ds, np.float32).reshape(G, 1).view(np.uint8)
    rec[:, 4:260] = q8.astype(np.int8).view(np.uint8)
    rec[:, 260:292] = q8.reshape(G, 16, 16).sum(-1).astype(np.int16).view(np.uint8).reshape(G, 32)
    return rec


def test_q4k_nibble_and_field_layout_known_answers():
    # One nonzero weight at element e, one nonzero activation at the same e:
    # the dot is d * sc[e // 32] * q * x exactly, which pins the nibble placement
    # (quantized-operations.en.md:31-36) and the 6-bit field unpacking.
    for e in (0, 1, 31, 32, 33, 63, 64, 100, 127, 128, 191, 200, 255):
        for s_val in (1, 5, 63):
            sc = np.zeros((1, 8), np.int64)
            sc[0, e // 32] = s_val
            q = np.zeros((1, 256), np.int64)
            q[0, e] = 11
            w = oracle.q4k_pack(np.float16(0.5), np.float16(0.0), sc, np.zeros((1, 8)), q)
            q8 = np.zeros((1, 256), np.int64)
            q8[0, e] = -3
            xq = _q8k_record(np.float32(2.0), q8)
            assert oracle.q4k_q8k_dot(w, xq) == np.float32(0.5 * s_val * 11 * -3 * 2.0)
            q8[0, e] = 0
            q8[0, e ^ 1] = 7  # a neighbouring element contributes nothing
            assert oracle.q4k_q8k_dot(w, _q8k_record(np.float32(2.0), q8)) == 0.0


def test_q4k_min_term_uses_bsum_pairs():
    # d = 0: the result is -ds * dmin * sum_s m[s] * (bsum[2s] + bsum[2s+1]).
    rng = np.random.default_rng(5)
    m = rng.integers(0, 64, (1, 8))
    q8 = rng.integers(-127, 128, (1, 256))
    w = oracle.q4k_pack(np.float16(0.0), np.float16(0.25), np.zeros((1, 8)), m, np.zeros((1, 256)))
    xq = _q8k_record(np.float32(0.125), q8)
    T = int(sum(m[0, s] * q8[0, 64 * s // 2:64 * s // 2 + 32].sum() for s in range(8)))
    assert oracle.q4k_q8k_dot(w, xq) == np.float32(-0.125 * np.float32(0.25 * T))


def test_q4k_zero_records_are_zero():
    # examples/programs/matrix.py:48-52: a zero-filled record has zero scales.
    xq = oracle.q8k_quantize(np.random.default_rng(1).standard_normal((3, 256)).astype(np.float32))
    r = oracle.q4k_q8k_dot(np.zeros((3, 144), np.uint8), xq)
    assert r == 0.0 and not np.signbit(r)
    assert oracle.q4k_q8k_dot(np.zeros((0, 144), np.uint8), np.zeros((0, 292), np.uint8)) == 0.0


def test_q4k_dot_matches_float64_dequantised_dot():
    rng = np.random.default_rng(7)
    for G in (1, 2, 5, 16):
        f = _q4k_fields(rng, G)
        w = oracle.q4k_pack(*f)
        xq = oracle.q8k_quantize(rng.standard_normal((G, 256)).astype(np.float32))
        got = float(oracle.q4k_q8k_dot(w, xq))
        ref = oracle.q4k_q8k_dot_f64(f, xq)
        assert abs(got - ref) <= 1e-5 * max(1.0, abs(ref)), (G, got, ref)


def test_q4k_record_order_and_rounding():
    # The result is ((+0 + v0) + v1) + ... in f32: per-record values from
    # single-record calls, summed in order with numpy f32, give the same bits.
    rng = np.random.default_rng(9)
    G = 11
    w = oracle.q4k_pack(*_q4k_fields(rng, G))
    xq = oracle.q8k_quantize((rng.standard_normal((G, 256)) * 10).astype(np.float32))
    acc = np.float32(0.0)
    for b in range(G):
        acc = np.float32(acc + oracle.q4k_q8k_dot(w[b:b + 1], xq[b:b + 1]))
    assert oracle.q4k_q8k_dot(w, xq).view(np.uint32) == acc.view(np.uint32)


def test_q4k_gemv_rows_match_single_dots():
    rng = np.random.default_rng(3)
    w = rng.integers(0, 256, (6, 4, 144), dtype=np.uint8)
    w[..., 0:4] = rng.uniform(0.001, 0.01, (6, 4, 2)).astype(np.float16).view(np.uint8).reshape(6, 4, 4)
    xq = oracle.q8k_quantize(rng.standard_normal((4, 256)).astype(np.float32))
    y = oracle.q4k_gemv(w, xq, threads=2)
    assert all(y[n].view(np.uint32) == oracle.q4k_q8k_dot(w[n], xq).view(np.uint32) for n in range(6))


def test_q8k_quantize_properties():
    rng = np.random.default_rng(11)
    x = (rng.standard_normal((64, 256)) * rng.uniform(0.01, 100, (64, 1))).astype(np.float32)
    xq = oracle.q8k_quantize(x)
    ds, q, bsum = oracle.q8k_fields(xq)
    assert np.array_equal(bsum, q.reshape(64, 16, 16).sum(-1))
    # The extreme value maps to -127 (its sign flips through the negative inverse).
    ext = np.where(np.abs(x.max(1)) > np.abs(x.min(1)), x.max(1), x.min(1))
    idx = np.argmax(x == ext[:, None], axis=1)
    assert np.all(q[np.arange(64), idx] == -127)
    # Reconstruction error is at most half a step.
    err = np.abs(ds[:, None].astype(np.float64) * q - x)
    assert np.all(err <= 0.5 * np.abs(ds[:, None]) * (1 + 1e-5))
    # ds is exactly 1 / inverse with inverse = -127 / extreme (two f32 divisions).
    inv = np.float32(-127.0) / ext.astype(np.float32)
    assert np.array_equal(ds, (np.float32(1.0) / inv).astype(np.float32))


def test_q8k_quantize_ties_zero_block_and_rounding():
    x = np.zeros((3, 256), np.float32)
    x[0, 3], x[0, 9] = 2.0, -2.0  # |max| == |min|: the minimum is the extreme
    x[2, :] = np.linspace(-1, 1, 256, dtype=np.float32)
    xq = oracle.q8k_quantize(x)
    ds, q, bsum = oracle.q8k_fields(xq)
    assert q[0, 9] == -127 and q[0, 3] == 127 and ds[0] > 0
    assert not xq[1].any()  # all-zero block: ds=+0, q=0, bsum=0
    # Half-way products round to even: x = k + 0.5 steps.
    y = np.zeros((1, 256), np.float32)
    y[0, 0] = -127.0  # inverse = 1, ds = 1
    y[0, 1:6] = [0.5, 1.5, 2.5, -0.5, -1.5]
    _, q1, _ = oracle.q8k_fields(oracle.q8k_quantize(y))
    assert list(q1[0, :6]) == [-127, 0, 2, 2, 0, -2]


def test_kquant_golden():
    g = np.load(GOLDEN / "q4k_n7_g3.npz")
    assert np.array_equal(oracle.q8k_quantize(g["x"]), g["xq"])
    assert np.array_equal(oracle.q4k_gemv(g["w"], g["xq"]).view(np.uint32), g["y"].view(np.uint32))


# ---- groupwise FP8 quantizers (examples/kernels/quantization/fp8.py:11-69) ---------

def test_e4m3fn_conversion_matches_torch():
    # torch's float8_e4m3fn cast (round to nearest even) is an independent routine.
    rng = np.random.default_rng(2)
    grid = np.concatenate([
        np.linspace(-448, 448, 20001, dtype=np.float32),
        (rng.standard_normal(20000) * np.exp2(rng.uniform(-12, 8, 20000))).astype(np.float32),
        np.float32([0.0, -0.0, 2.0 ** -9, 2.0 ** -10, 3 * 2.0 ** -11, 2.0 ** -6, 448.0, -448.0, 1.0625, 1.1875]),
    ])
    grid = np.clip(grid, -448, 448).astype(np.float32)
    want = torch.from_numpy(grid).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(oracle.f32_to_e4m3fn(grid), want)


@pytest.mark.parametrize("M,N", [(3, 256), (5, 300), (2, 129)])
def test_fp8_groupwise_matches_reference_cpu_formula(M, N):
    # experiments/cpu/baselines/pytorch/cpu_runtime.py:142-147 restated with torch
    # (padding the last group with zeros leaves its max unchanged for |x| >= 0).
    rng = np.random.default_rng(M * N)
    x = (rng.standard_normal((M, N)) * rng.uniform(1e-6, 1e3, (M, 1))).astype(np.float32)
    x[0, :7] = 0.0
    q, sc = oracle.fp8_groupwise_quantize(x)
    G = (N + 127) // 128
    t = torch.zeros(M, G * 128)
    t[:, :N] = torch.from_numpy(x)
    v = t.reshape(M, G, 128)
    scale = v.abs().amax(dim=-1).clamp_min(1e-4) / 448.0
    ref = (v / scale[:, :, None]).clamp(-448.0, 448.0).to(torch.float8_e4m3fn).reshape(M, -1)[:, :N]
    assert np.array_equal(sc, scale.numpy())
    assert np.array_equal(q, ref.view(torch.uint8).numpy())


def test_fp8_groupwise_bf16_eps_and_zero_group():
    x = np.zeros((1, 256), np.float32)
    q, sc = oracle.fp8_groupwise_quantize(x, source="bf16")
    assert not q.any() and np.all(sc == np.float32(np.float32(1e-12) / np.float32(448.0)))
    x[0, 130] = -3.5  # group 1's extreme maps to -448 exactly
    q, sc = oracle.fp8_groupwise_quantize(x, source="bf16")
    assert q[0, 130] == 0xFE and sc[0, 1] == np.float32(3.5) / np.float32(448.0)


# ---- W4A8 and BitNet int2 (examples/kernels/contraction/weight_only_int4.py:54-124) -

@pytest.mark.parametrize("M,K,N", [(3, 64, 5), (16, 256, 33), (1, 512, 7)])
def test_w4a8_and_bitnet_match_reference_formulas(M, K, N):
    rng = np.random.default_rng(M + K + N)
    a = rng.integers(-128, 128, (M, K), dtype=np.int8)
    p4 = rng.integers(0, 256, (N, K // 2), dtype=np.uint8)
    p2 = rng.integers(0, 256, (N, K // 4), dtype=np.uint8)
    assert np.array_equal(oracle.w4a8(a, p4).astype(np.int64), oracle.w4a8_int64(a, p4))
    assert np.array_equal(oracle.bitnet_int2(a, p2).astype(np.int64), oracle.bitnet_int2_int64(a, p2))


def test_w4a8_and_bitnet_known_answers():
    # Nibble 0x8 is -8, 0xF is -1, 0x7 is +7; low nibble = even k.
    a = np.zeros((1, 4), np.int8)
    a[0] = [1, 10, 100, -1]
    p4 = np.array([[0x8F, 0x07]], np.uint8)  # k0 = 0xF (-1), k1 = 0x8 (-8), k2 = 7, k3 = 0
    assert oracle.w4a8(a, p4)[0, 0] == -1 * 1 + -8 * 10 + 7 * 100
    # int2 interleaving: k = 16c + 4a + b lives in byte 4c + b at bits 2a.
    K = 32
    for k in (0, 1, 3, 4, 5, 15, 16, 21, 31):
        p2 = np.zeros((1, K // 4), np.uint8)
        p2[0, (k // 16) * 4 + k % 4] = 3 << (2 * ((k // 4) % 4))
        act = np.zeros((1, K), np.int8)
        act[0, k] = 5
        assert oracle.bitnet_int2(act, p2)[0, 0] == 15
        act[0, k], act[0, (k + 1) % K] = 0, 5
        assert oracle.bitnet_int2(act, p2)[0, 0] == 0


# ---- MX block-scaled FP8 (examples/kernels/contraction/block_scaled.py:11-39) -------

def test_e4m3fn_and_e8m0_decode():
    bits = np.arange(256, dtype=np.uint8)
    want = torch.from_numpy(bits).view(torch.float8_e4m3fn).float().numpy()
    got = oracle.e4m3fn_to_f32(bits)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    assert np.array_equal(got[ok].view(np.uint32), want[ok].view(np.uint32))
    s = oracle.e8m0_to_f32(bits)
    assert s[0] == np.float32(2.0 ** -127) and np.isnan(s[255])
    assert np.array_equal(s[1:255], np.exp2(np.arange(1, 255) - 127.0).astype(np.float32))


def test_mxfp8_gemm_matches_reference_formula():
    # experiments/cpu/baselines/pytorch/cpu_runtime.py:1025-1032 restated with torch
    # in float64 (products of e4m3 values and power-of-two scales are exact).
    rng = np.random.default_rng(4)
    M, K, N = 5, 128, 7
    a = rng.integers(0, 256, (M, K), dtype=np.uint8)
    b = rng.integers(0, 256, (N, K), dtype=np.uint8)
    a[(a & 0x7F) == 0x7F] = 0x10  # no NaN codes
    b[(b & 0x7F) == 0x7F] = 0x10
    sa = rng.integers(118, 136, (M, K // 32), dtype=np.uint8)
    sb = rng.integers(118, 136, (N, K // 32), dtype=np.uint8)
    got = oracle.mxfp8_gemm(a, sa, b, sb)
    fa = torch.from_numpy(a).view(torch.float8_e4m3fn).double() * torch.exp2(torch.from_numpy(sa).double() - 127).repeat_interleave(32, 1)
    fb = torch.from_numpy(b).view(torch.float8_e4m3fn).double() * torch.exp2(torch.from_numpy(sb).double() - 127).repeat_interleave(32, 1)
    ref = (fa @ fb.T).numpy()
    assert np.allclose(got, ref, rtol=1e-5, atol=1e-6 * np.abs(ref).max())


# ---- per-tensor scaled FP8 (plain and split-K) and DeepGEMM-style FP8 -------------

def _fp8_randn(gen, shape, scale=1.0):
    return (torch.randn(shape, generator=gen) * scale).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def _f8(bits):
    return torch.from_numpy(np.ascontiguousarray(bits)).view(torch.float8_e4m3fn).double().numpy()


def test_scaled_fp8_gemm_closed_form():
    # block_scaled.py:42-63: f16((acc * lhs_scale) * rhs_scale); the f32 sum in k
    # order differs from the exact float64 sum only by rounding.
    g = torch.Generator().manual_seed(11)
    a, b = _fp8_randn(g, (6, 768)), _fp8_randn(g, (768, 9))
    got = oracle.scaled_fp8_gemm(a, b, 0.75, 1.5).astype(np.float64)
    ref = (_f8(a) @ _f8(b)) * 0.75 * 1.5
    assert np.max(np.abs(got - ref)) <= 2e-3 * np.abs(ref).max()


def test_scaled_fp8_splitk_matches_reference_formula():
    # experiments/cpu/baselines/pytorch/cpu_runtime.py:133-139 restated with torch:
    # per split an f32 matmul, scaled, rounded to f16, added to the f16 output.
    g = torch.Generator().manual_seed(12)
    M, IT, SP, N = 5, 2, 3, 7
    K = IT * SP * 256
    a, b = _fp8_randn(g, (M, K)), _fp8_randn(g, (K, N))
    out0 = (torch.randn(M, N, generator=g) * 4).half().numpy()
    got = oracle.scaled_fp8_gemm(a, b, 0.5, 1.25, splits=SP, out=out0)
    lhs = torch.from_numpy(a).view(torch.float8_e4m3fn).view(M, IT, SP, 256)
    rhs = torch.from_numpy(b).view(torch.float8_e4m3fn).view(IT, SP, 256, N)
    ref = torch.from_numpy(out0.copy())
    for s in range(SP):
        left = lhs[:, :, s, :].float().flatten(1)
        right = rhs[:, s, :, :].float().flatten(0, 1)
        ref.add_(((left @ right) * 0.5 * 1.25).half())
    ref = ref.numpy().astype(np.float64)
    # f32 sums in a different order may round to a neighbouring f16
    assert np.max(np.abs(got.astype(np.float64) - ref)) <= 2e-3 * np.abs(ref).max()


def test_scaled_fp8_splitk_known_answers():
    M, N, SP, IT = 2, 3, 4, 1
    K = SP * IT * 256
    one = np.uint8(0x38)  # E4M3FN 1.0
    a = np.zeros((M, K), np.uint8)
    b = np.zeros((K, N), np.uint8)
    # one-hot k in split 2 (k = 2*256 + 5): out = f16(b[k, n] * ls * rs)
    a[:, 2 * 256 + 5] = one
    b[2 * 256 + 5, :] = [0x40, 0xC8, 0x30]  # 2.0, -4.0, 0.5
    got = oracle.scaled_fp8_gemm(a, b, 3.0, 0.5, splits=SP, out=np.zeros((M, N), np.float16))
    assert np.array_equal(got, np.tile(np.array([3.0, -6.0, 0.75], np.float16), (M, 1)))
    # additions happen split by split in f16: 2048 + 1 + 1 stays 2048 (ties to
    # even), while a single sum of the partials would give 2050
    a = np.zeros((1, K), np.uint8)
    b = np.zeros((K, 1), np.uint8)
    a[0, 0 * 256] = a[0, 1 * 256] = one
    b[0 * 256, 0] = b[1 * 256, 0] = one
    got = oracle.scaled_fp8_gemm(a, b, 1.0, 1.0, splits=SP, out=np.full((1, 1), 2048, np.float16))
    assert got[0, 0] == np.float16(2048)


def test_deepgemm_fp8_matches_reference_formula():
    # cpu_runtime.py:127-131 restated in float64: operands scaled per (row, 128-k
    # block) and per (128-row block of rhs, 128-k block), then a matmul, then bf16.
    g = torch.Generator().manual_seed(13)
    M, KB, N = 4, 3, 256
    a, b = _fp8_randn(g, (M, KB * 128)), _fp8_randn(g, (N, KB * 128))
    sa = torch.rand(M, KB, generator=g).numpy().astype(np.float32) + 0.25
    sb = torch.rand(N // 128, KB, generator=g).numpy().astype(np.float32) + 0.25
    got = torch.from_numpy(oracle.deepgemm_fp8(a, sa, b, sb).view(np.int16)).view(torch.bfloat16).double().numpy()
    left = _f8(a) * np.repeat(sa.astype(np.float64), 128, axis=1)
    right = _f8(b) * np.repeat(np.repeat(sb.astype(np.float64), 128, axis=0), 128, axis=1)
    ref = left @ right.T
    assert np.max(np.abs(got - ref)) <= 8e-3 * np.abs(ref).max()
    # one-hot known answer: a single product lhs*sa * rhs*sb, exact in bf16
    a1 = np.zeros((1, 128), np.uint8)
    b1 = np.zeros((128, 128), np.uint8)
    a1[0, 7] = 0x40  # 2.0
    b1[5, 7] = 0x44  # 3.0
    y = oracle.deepgemm_fp8(a1, np.array([[0.5]], np.float32), b1, np.array([[4.0]], np.float32))
    vals = torch.from_numpy(y.view(np.int16)).view(torch.bfloat16).float().numpy()
    assert vals[0, 5] == 12.0 and np.count_nonzero(vals) == 1


# ---- FP8 x FP8 -> FP8 ------------------------------------------------------------

def test_e5m2_conversions_match_torch():
    codes = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(codes).view(torch.float8_e5m2).float().numpy()
    got = oracle.e5m2_to_f32(codes)
    finite = np.isfinite(ref)
    assert np.array_equal(got[finite], ref[finite]) and np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(np.isinf(got), np.isinf(ref))
    g = torch.Generator().manual_seed(21)
    vals = torch.cat([
        torch.randn(20000, generator=g) * 100,
        torch.randn(20000, generator=g) * 1e-5,                 # subnormals
        torch.from_numpy(ref[finite]).float(),                  # every finite code
        torch.from_numpy((ref[finite][:-1] + ref[finite][1:]) / 2).float(),  # half-way points
        torch.tensor([57344.0, 61439.0, 61440.0, 1e6, -1e6, float("inf"), -float("inf"), 0.0, -0.0]),
    ])
    want = vals.to(torch.float8_e5m2).view(torch.uint8).numpy()
    assert np.array_equal(oracle.f32_to_e5m2(vals.numpy()), want)


@pytest.mark.parametrize("fmt,tdt", [("e4m3fn", torch.float8_e4m3fn), ("e5m2", torch.float8_e5m2)])
def test_fp8_gemm_closed_form(fmt, tdt):
    g = torch.Generator().manual_seed(22)
    M, K, N = 6, 384, 9
    a = (torch.randn(M, K, generator=g) * 0.5).to(tdt)
    b = (torch.randn(N, K, generator=g) * 0.5).to(tdt)
    got = oracle.fp8_gemm(a.view(torch.uint8).numpy(), b.view(torch.uint8).numpy(), fmt)
    exact = a.double() @ b.double().T
    want = exact.float().to(tdt).view(torch.uint8).numpy()
    # the f32 sum in k order may round to the neighbouring code in rare cases
    assert np.mean(got == want) >= 0.95
    dec = torch.from_numpy(got).view(tdt).double()
    step = 2.0 ** -2 if fmt == "e5m2" else 2.0 ** -3
    assert torch.all((dec - exact).abs() <= step * exact.abs() + 2.0 ** -9)
    # one-hot known answer: a single product, exact in the format
    a1 = torch.zeros(1, 128, dtype=tdt)
    b1 = torch.zeros(2, 128, dtype=tdt)
    a1[0, 3], b1[1, 3] = 1.5, -2.0
    y = oracle.fp8_gemm(a1.view(torch.uint8).numpy(), b1.view(torch.uint8).numpy(), fmt)
    assert torch.from_numpy(y).view(tdt).float().tolist() == [[0.0, -3.0]]


# ---- FP4 (E2M1) x bf16 ---------------------------------------------------------------

def _fp4_reference_decode(packed):
    # cpu_runtime.py:117-124 restated with torch (the reference's own recipe)
    p = torch.from_numpy(np.ascontiguousarray(packed))
    word = (p[:, 0::2].int() << 8) | p[:, 1::2].int()
    bits = torch.stack((word & 0x81C0, (word << 3) & 0x81C0, (word << 6) & 0x81C0,
                        ((word << 1) & 0x8000) | ((word >> 3) & 0x0180) | ((word >> 7) & 0x0040)),
                       dim=-1).flatten(1).to(torch.int16)
    return (bits.view(torch.bfloat16).float() * (2.0 ** 126)).bfloat16().float().numpy()


def test_fp4_decode_matches_reference_recipe():
    words = np.arange(65536, dtype=np.uint32)  # every 16-bit word once
    packed = np.stack(((words >> 8) & 255, words & 255), axis=1).astype(np.uint8).reshape(1, -1)
    ref = _fp4_reference_decode(packed)[0]
    got = oracle.fp4_decode_row(packed[0])
    assert np.array_equal(got, ref)
    # the values are exactly the E2M1 set
    assert set(np.unique(np.abs(got)).tolist()) == {0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0}


def test_fp4_nibble_gather_in_kernel_source():
    # The FP4 kernel gathers each dword's eight codes into standard E2M1 nibbles
    # (sign, e1, e0, m0) with rotate-and-mask terms, then converts nibble pairs
    # from bytes 2, 1, 0, 3. Read those terms from the kernel source and check
    # them, with the OCP E2M1 value table, against the oracle on every word.
    import re
    src = (Path(__file__).resolve().parents[1] / "intent_amd" / "csrc" / "dense_gemm.hip").read_text()
    body = src[src.index("INTENT_DEVICE u32x4 fp4x8_to_bf16"):]
    body = body[:body.index("u32x4 out;")]
    terms = [(0, int(m, 16)) for m in re.findall(r"\(d & (0x[0-9a-f]+)u\)", body)]
    terms += [(int(r), int(m, 16)) for r, m in re.findall(r"rotl32\(d, (\d+)\) & (0x[0-9a-f]+)u", body)]
    sels = [int(v) for v in re.findall(r"cvt_scalef32_pk_bf16_fp4\(n, 1\.0f, (\d)\)", src)]
    assert len(terms) == 9 and sels == [2, 1, 0, 3]
    e2m1 = np.array([0, 0.5, 1, 1.5, 2, 3, 4, 6, -0.0, -0.5, -1, -1.5, -2, -3, -4, -6], np.float32)
    words = np.arange(65536, dtype=np.uint32)
    for shift in (0, 1):  # every word in the low and in the high half of a dword
        w = np.roll(words, shift)
        packed = np.stack(((w >> 8) & 255, w & 255), axis=1).astype(np.uint8).reshape(-1)
        d = packed.view("<u4").astype(np.uint64)
        n = np.zeros_like(d)
        for r, m in terms:
            n |= (((d << r) | (d >> ((32 - r) % 32))) & 0xFFFFFFFF) & m
        nib = np.stack([(n >> (8 * s + 4 * h)) & 15 for s in sels for h in (0, 1)], axis=1)
        got = e2m1[nib.astype(np.int64)].reshape(-1)
        assert np.array_equal(got, oracle.fp4_decode_row(packed))
        assert np.array_equal(np.signbit(got), np.signbit(oracle.fp4_decode_row(packed)))


def test_fp4_bf16_matmul_closed_form():
    g = torch.Generator().manual_seed(32)
    M, K, N = 5, 256, 7
    x = torch.randn(M, K, generator=g).bfloat16()
    packed = torch.randint(0, 256, (N, K // 2), generator=g, dtype=torch.uint8).numpy()
    got = oracle.fp4_bf16_matmul(x.view(torch.int16).numpy().view(np.uint16), packed)
    ref = x.double().numpy() @ _fp4_reference_decode(packed).astype(np.float64).T
    dec = torch.from_numpy(got.view(np.int16)).view(torch.bfloat16).double().numpy()
    assert np.max(np.abs(dec - ref)) <= 8e-3 * np.abs(ref).max()


# ---- the reference's own weight_only_int4_matmul layout --------------------------------

def _w4_sym_case(seed, M, K, N):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((M, K)).astype(np.float16)
    packed = rng.integers(-2**31, 2**31, (K // 8, N), dtype=np.int64).astype(np.int32)
    scales = rng.uniform(0.005, 0.02, (K // 64, N)).astype(np.float16)
    return x, packed, scales


def test_w4_sym_matches_reference_formula():
    # cpu_runtime.py:97-102 restated with torch
    x, packed, scales = _w4_sym_case(41, 4, 256, 9)
    got = oracle.w4_sym(x, packed, scales).astype(np.float64)
    p = torch.from_numpy(packed)
    positions = torch.arange(x.shape[1])
    nibble = (p[positions // 8] >> ((positions % 8) * 4)[:, None]) & 15
    signed = nibble - ((nibble & 8) << 1)
    deq = signed.float() * torch.from_numpy(scales).float().repeat_interleave(64, dim=0)
    ref = (torch.from_numpy(x).float() @ deq).half().double().numpy()
    assert np.max(np.abs(got - ref)) <= 2e-3 * np.abs(ref).max()


def test_w4_sym_known_answers():
    # one nibble per position: word 0x8000000F at [0, n] puts 15 -> -1 at k = 0 and
    # 8 -> -8 at k = 7; x one-hot at k = 7 picks -8 * scale
    K, N = 64, 2
    packed = np.zeros((K // 8, N), np.int32)
    packed[0, 1] = np.int32(-0x7FFFFFF1)  # bits 0x8000000F
    scales = np.full((1, N), 0.5, np.float16)
    x = np.zeros((2, K), np.float16)
    x[0, 7] = 1.0
    x[1, 0] = 2.0
    y = oracle.w4_sym(x, packed, scales)
    assert y.tolist() == [[0.0, -4.0], [0.0, -1.0]]


# ---- quantized_gemm ---------------------------------------------------------------------

def test_quantized_gemm_matches_reference_formula():
    # cpu_runtime.py:91-94 restated with torch, on the reference's input construction
    # (experiments/cpu/providers/mojo/contraction.py:177-186) at a small size
    g = torch.Generator().manual_seed(51)
    M, K, N = 6, 128, 40
    a = torch.randn((M, K), generator=g).half() / (K ** 0.5)
    b = torch.randn((K, N), generator=g).half()
    bias = torch.randn((N,), generator=g) * 0.25
    residual = (torch.randn((M, N), generator=g) * 0.25).half()
    scale = torch.linspace(1.0 / 48.0, 1.0 / 24.0, N)
    got = oracle.quantized_gemm(a.numpy(), b.numpy(), bias.numpy(), residual.numpy(), scale.numpy())
    acc = a.float() @ b.float()
    ref = ((torch.relu(acc + bias) + residual.float()) / scale).clamp(-128.0, 127.0).to(torch.int8).numpy()
    # the f32 sum in another order can move a value across an integer boundary
    assert np.max(np.abs(got.astype(np.int32) - ref.astype(np.int32))) <= 1
    assert np.mean(got == ref) >= 0.95


def test_quantized_gemm_known_answers():
    # relu, residual, division, clamp and truncation toward zero
    K, N = 64, 5
    a = np.zeros((1, K), np.float16)
    a[0, 0] = 1.0
    b = np.zeros((K, N), np.float16)
    b[0, :] = [2.0, -3.0, 1000.0, -1000.0, 1.5]
    bias = np.array([0.5, 0.0, 0.0, 0.0, 0.0], np.float32)
    residual = np.array([[0.25, 0.5, 0.0, -2.0, -3.0]], np.float16)
    scale = np.array([1.0, 0.25, 1.0, 1.0, 1.0], np.float32)
    got = oracle.quantized_gemm(a, b, bias, residual, scale)
    # 2.75 -> 2; relu(-3)+0.5 = 0.5, /0.25 = 2; 1000 -> 127; relu(-1000)-2 = -2; 1.5-3 = -1.5 -> -1
    assert got.tolist() == [[2, 2, 127, -2, -1]]


# ---- f16 / bf16 grouped GEMMs ------------------------------------------------------------

def _u16(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def test_grouped_gemm_ragged_and_routed_closed_form():
    g = torch.Generator().manual_seed(71)
    K, N = 128, 12
    x = torch.randn(10, K, generator=g).half()
    w = (torch.randn(3, K, N, generator=g) / 8).half()
    offsets = np.array([0, 4, 4, 10], np.int32)          # group 1 empty
    y = oracle.grouped_gemm(_u16(x), False, offsets, _u16(w), 10)
    yy = torch.from_numpy(y.view(np.int16)).view(torch.float16).double()
    for gi, (b, e) in enumerate(zip(offsets[:-1], offsets[1:])):
        if b == e:
            continue  # an empty group writes nothing
        ref = x[b:e].double() @ w[gi].double()
        assert torch.allclose(yy[b:e], ref, rtol=2e-3, atol=2e-3 * max(1.0, ref.abs().max().item()))
    # routed: route r of expert e reads token r // top_k and writes row r
    xb = torch.randn(3, K, generator=g).bfloat16()
    wb = (torch.randn(2, N, K, generator=g) / 8).bfloat16()
    routes = np.array([5, 0, 3, 1, 2, 4], np.int32)      # expert 0: routes 5, 0; expert 1: 3, 1, 2, 4
    offs = np.array([0, 2, 6], np.int32)
    out = oracle.grouped_gemm(_u16(xb), True, offs, _u16(wb), 6, routes=routes, top_k=2)
    ob = torch.from_numpy(out.view(np.int16)).view(torch.bfloat16).double()
    for i, r in enumerate(routes):
        e = 0 if i < 2 else 1
        ref = xb[r // 2].double() @ wb[e].double().T
        assert torch.allclose(ob[r], ref, rtol=1e-2, atol=1e-2 * max(1.0, ref.abs().max().item()))


def test_float_gemm_closed_form_and_relu():
    g = torch.Generator().manual_seed(81)
    for bf16 in (False, True):
        tdt = torch.bfloat16 if bf16 else torch.float16
        a = torch.randn(5, 128, generator=g).to(tdt)
        b = (torch.randn(128, 7, generator=g) / 8).to(tdt)
        for relu in (False, True):
            c = oracle.float_gemm(_u16(a), _u16(b), bf16, relu)
            got = torch.from_numpy(c.view(np.int16)).view(tdt).double()
            ref = a.double() @ b.double()
            if relu:
                ref = ref.clamp_min(0.0)
            assert torch.allclose(got, ref, rtol=1e-2, atol=1e-2)
            if relu:
                assert (got >= 0).all()


# ---- NVFP4 quantizer ----------------------------------------------------------------------

@pytest.mark.parametrize("gsv", [0.75, 300.0])
def test_nvfp4_quantize_matches_reference_formula(gsv):
    # cpu_runtime.py:1325-1340 restated with torch (elementwise f32: bit-exact). At gs = 300
    # many group scales pass 464, where torch's E4M3FN cast gives NaN (0x7f) and every code
    # of the group becomes 0; scales in [448, 464] round to 448.
    g = torch.Generator().manual_seed(91)
    M, N = 256, 128
    x = (torch.randn(M, N, generator=g) * torch.rand(M, 1, generator=g) * 4).bfloat16()
    x[3, :16] = 0.0                                  # a zero group: scale clamps to its minimum
    x[5, 16:32] = -0.0
    x[7, 32:48] = 9.25                               # (9.25 / 6) * 300 = 462.5: rounds to 448
    gs = torch.tensor([gsv])
    packed, scales = oracle.nvfp4_quantize(_u16(x), gsv)
    groups = x.float().reshape(M, N // 16, 16)
    scale = ((groups.abs().amax(-1) / 6.0) * gs[0]).clamp_min(1.5258789e-5).to(torch.float8_e4m3fn)
    values = groups * (gs[0] / scale.float())[..., None]
    mag = values.abs()
    enc = (mag > 0.25).to(torch.uint8)
    for code, t in enumerate((0.75, 1.25, 1.75, 2.5, 3.5, 5.0), start=2):
        sel = mag >= t if code % 2 == 0 else mag > t
        enc = torch.where(sel, code, enc)
    enc |= torch.signbit(values).to(torch.uint8) << 3
    pairs = enc.reshape(M, N // 2, 2)
    ref_packed = (pairs[..., 0] | (pairs[..., 1] << 4)).numpy()
    ref_scales = scale.view(torch.uint8).reshape(M // 128, 4, 32, N // 64, 4).permute(0, 3, 2, 1, 4).numpy()
    if gsv > 100:
        assert (ref_scales == 0x7f).any() and (ref_scales == 0x7e).any()
    assert np.array_equal(packed, ref_packed)
    assert np.array_equal(scales, ref_scales)


# ---- per-token int8 quantizer ---------------------------------------------------------

def test_i8_per_token_known_answers():
    # amax 127 makes 127/amax exactly 1, so q is x rounded half to even
    x = np.zeros((3, 16), np.float32)
    x[0, :10] = [127.0, 2.5, 3.5, -2.5, -3.5, 0.5, -0.5, 1.5, 126.5, -127.0]
    x[2, 3] = -0.25  # lone value: amax 0.25, q -127, scale 0.25/127
    q, s = oracle.i8_per_token_quantize(x)
    assert list(q[0, :10]) == [127, 2, 4, -2, -4, 0, 0, 2, 126, -127]
    assert s[0] == np.float32(1.0)
    assert s[1] == 0 and not q[1].any()  # zero row: scale 0, codes 0
    assert q[2, 3] == -127 and s[2] == np.float32(0.25) / np.float32(127)
    assert not np.delete(q[2], 3).any()


@pytest.mark.parametrize("M,K", [(7, 64), (33, 1000), (4, 8200)])
def test_i8_per_token_matches_numpy_and_bounds(M, K):
    rng = np.random.default_rng(M + K)
    x = (rng.standard_normal((M, K)) * rng.uniform(1e-4, 1e3, (M, 1))).astype(np.float16).astype(np.float32)
    x[0] = 0.0
    q, s = oracle.i8_per_token_quantize(x)
    qn, sn = oracle.i8_per_token_quantize_np(x)
    assert np.array_equal(q, qn) and np.array_equal(s.view(np.uint32), sn.view(np.uint32))
    # every code is the nearest level: |x - q*scale| <= scale/2 (float64, a little slack for the f32 inverse)
    err = np.abs(x.astype(np.float64) - q.astype(np.float64) * s[:, None].astype(np.float64))
    assert np.all(err <= s[:, None] * (0.5 + 1e-5) + 1e-30)
    # the largest magnitude of every non-zero row lands on +-127 and nothing leaves [-127, 127]
    nz = s > 0
    assert np.all(np.abs(q[nz]).max(axis=1) == 127) and np.abs(q.astype(np.int32)).max() <= 127


def test_i8_per_token_brute_force_tiny():
    # python float64 restatement of every step on a handful of values, including ties
    rng = np.random.default_rng(3)
    x = (rng.integers(-300, 301, (5, 8)) / 4.0).astype(np.float32)
    q, s = oracle.i8_per_token_quantize(x)
    for m in range(5):
        amax = float(np.float32(max(abs(float(v)) for v in x[m])))
        inv = float(np.float32(127.0) / np.float32(amax)) if amax else 0.0
        for k in range(8):
            t = float(np.float32(np.float32(x[m, k]) * np.float32(inv)))
            t = min(max(t, -128.0), 127.0)
            lo = np.floor(t)
            frac = t - lo
            r = lo + (1 if frac > 0.5 or (frac == 0.5 and int(lo) % 2 != 0) else 0)
            assert q[m, k] == int(r), (m, k, x[m, k], t)


# ---- f16 MoE expert FFN (moe.py:12-53) --------------------------------------------------

@pytest.mark.parametrize("kind", ["reference", "random"])
def test_moe_expert_ffn_oracle_matches_restatements(kind):
    # float64 restatement of the kernel's formula (hidden rounded to f16 after the f32 ReLU) and the
    # reference's host formula experiments/_common/support.py:133-151 (hidden kept in f32)
    d = inputs.moe_ffn_f16(3, T=12, D=64, E=4, top_k=2, F=96, kind=kind)
    y0 = np.random.default_rng(1).standard_normal((12, 64)).astype(np.float32)
    got = oracle.moe_expert_ffn(d["x"], d["route_offsets"], d["member_routes"], d["route_token"], d["route_weights"],
                                d["w1"], d["w2"], y=y0, threads=2)
    x = d["x"].astype(np.float64)
    want = y0.astype(np.float64).copy()
    host = y0.astype(np.float64).copy()
    offs = d["route_offsets"]
    for e in range(4):
        routes = d["member_routes"][offs[e]:offs[e + 1]]
        tok = d["route_token"][routes]
        h32 = np.maximum(x[tok] @ d["w1"][e].astype(np.float64), 0.0)
        h16 = h32.astype(np.float16).astype(np.float64)
        wts = d["route_weights"][routes].astype(np.float64)[:, None]
        np.add.at(want, tok, wts * (h16 @ d["w2"][e].astype(np.float64)))
        np.add.at(host, tok, wts * (h32 @ d["w2"][e].astype(np.float64)))
    assert np.max(np.abs(got - want)) <= 1e-4 * np.abs(want).max()
    assert np.max(np.abs(got - host)) <= 1e-2 * np.sqrt(np.mean(host ** 2))
    # every route lands once: with zero w2 the output is y0 exactly
    z = oracle.moe_expert_ffn(d["x"], d["route_offsets"], d["member_routes"], d["route_token"], d["route_weights"],
                              d["w1"], np.zeros_like(d["w2"]), y=y0)
    assert np.array_equal(z, y0)


def test_moe_routes_reference_construction():
    # support.py:113-130 at its own T/E/top_k ratio: expert r % E, members grouped by expert
    d = inputs.moe_routes(16, 2, 8)
    assert d["route_offsets"].tolist() == list(range(0, 33, 4))
    exp = np.arange(32) % 8
    for e in range(8):
        mem = d["member_routes"][d["route_offsets"][e]:d["route_offsets"][e + 1]]
        assert (exp[mem] == e).all() and (np.diff(mem) > 0).all()
    assert np.allclose(d["route_weights"], 0.5) and (d["route_token"] == np.arange(32) // 2).all()
