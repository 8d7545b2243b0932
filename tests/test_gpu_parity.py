"""GPU parity of every hot-path entry against the CPU oracle (C restatement).

Float outputs: max|y - y_ref| <= 1e-2 * RMS(y_ref) with equal finite masks
(the north-star tolerance for f16 outputs). Integer / index outputs
(int32 accumulators, W8A8 bf16 epilogue, routing ids, alignment): bit-exact.
Full BASELINE sizes whose oracle cost is large are checked on a row subset
against the oracle and at full size against an exact or float64 GPU
restatement (int products summed in float64 are exact below 2^53).
"""
import numpy as np
import pytest
import torch

import intent_amd as intent
import oracle
from intent_amd import _native, inputs

pytestmark = pytest.mark.gpu

REL_TOL = 1e-2  # max-abs-err <= REL_TOL * RMS(reference), f16 outputs


def assert_close_rms(got, ref, rel=REL_TOL, what=""):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.array_equal(np.isfinite(got), np.isfinite(ref)), f"{what}: finite masks differ"
    fin = np.isfinite(ref)
    rms = np.sqrt(np.mean(ref[fin] ** 2)) if fin.any() else 0.0
    err = np.max(np.abs(got[fin] - ref[fin])) if fin.any() else 0.0
    assert err <= rel * rms + 1e-12, f"{what}: max_abs_err={err:.4g} > {rel}*rms={rel * rms:.4g}"
    return err, rms


_artifacts = {}


def art(defn, **constexprs):
    key = (defn.name, tuple(sorted(constexprs.items())))
    if key not in _artifacts:
        _artifacts[key] = intent.compile(defn, target=intent.MI355XTarget(0), constexprs=constexprs or None)
    return _artifacts[key]


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _sample_rows(M):
    """Output rows checked against the oracle when a whole matrix would take it too long: the
    first and last 40 (every lane row of the first and last 32-row blocks) and every 37th
    between them (coprime with 32, so every row position of a block in some middle tile)."""
    return np.unique(np.r_[0:min(M, 40), max(0, M - 40):M, np.arange(40, max(40, M - 40), 37)])


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def w4_case(seed, M, K, N, group):
    d = inputs.config1_w4a16_decode(seed, M=M, K=K, N=N, group=group)
    return d["x"], d["packed"], d["scales"], d["zeros"]


# ---- W4A16 --------------------------------------------------------------------------

@pytest.mark.parametrize("M", [1, 2, 3, 4, 8, 16])
def test_w4a16_decode_config1(gpu, threads, M):
    x, q, s, z = w4_case(0, M, 4096, 4096, 128)
    y = art(intent.weight_only_int4_asym_matmul).run(dev(x), dev(q), dev(s), dev(z))
    ref = oracle.w4a16(x, q, s, z, threads)
    assert_close_rms(host(y), ref.astype(np.float32), what=f"gemv M={M}")
    assert art(intent.weight_only_int4_asym_matmul).observation.entry == "intent_w4a16_gemv"


@pytest.mark.parametrize("M,K,N,group", [(16, 4096, 4100, 128), (6, 2048, 64, 256), (7, 8192, 100, 32),
                                         (16, 8192, 333, 512), (9, 384, 31, 128), (12, 1152, 50, 64),
                                         (16, 16384, 40, 128), (4, 4096, 77, 128), (5, 2048, 129, 64)])
def test_w4a16_gemv_kernel_choices(gpu, threads, M, K, N, group):
    # M >= 6 with K <= 8192 and at most 256 groups per row: the MFMA GEMV with its loads issued up
    # front (1, 2 or 4 steps per wave, steps past K zero-scaled); K = 16384 takes the looping MFMA
    # kernel; M = 4, 5 the dot-product kernel. N not a multiple of 16 exercises the clamped tail rows.
    x, q, s, z = w4_case(3, M, K, N, group)
    a = art(intent.weight_only_int4_asym_matmul, KERNEL="gemv")
    y = a.run(dev(x), dev(q), dev(s), dev(z))
    want = ("w4a16_gemv_dot_shared_kernel" if M <= 5 else
            "w4a16_gemv_kernel" if K > 8192 else "w4a16_gemv_front_kernel")
    assert a.observation.kernel.startswith(want), a.observation.kernel
    assert_close_rms(host(y), oracle.w4a16(x, q, s, z, threads), what=f"gemv {M}x{K}x{N} g{group}")


@pytest.mark.parametrize("M,K,N,group", [(3, 256, 100, 64), (1, 384, 48, 32), (16, 128, 17, 128),
                                         (5, 2048, 1000, 256), (1, 8192, 64, 128),
                                         (2, 8192, 33, 128), (1, 16384, 24, 128), (2, 384, 40, 128),
                                         (1, 1024, 20, 64), (3, 3072, 77, 128), (3, 8192, 40, 128),
                                         (1, 8192, 100, 32), (1, 4224, 50, 96), (1, 2944, 30, 128),
                                         (2, 16384, 20, 32), (1, 4096, 4100, 128)])
def test_w4a16_gemv_shapes(gpu, threads, M, K, N, group):
    # G = K/group even and small: the workgroup-shared kernel (1..4 scale pairs per thread);
    # odd G (2944/128) or 512 groups (16384/32): the per-wave kernel
    x, q, s, z = w4_case(1, M, K, N, group)
    y = art(intent.weight_only_int4_asym_matmul, KERNEL="gemv").run(dev(x), dev(q), dev(s), dev(z))
    assert_close_rms(host(y), oracle.w4a16(x, q, s, z, threads), what="gemv shapes")


@pytest.mark.parametrize("M,K,N,group", [(1, 4096, 300, 128), (3, 2048, 70, 64), (8, 2048, 200, 128)])
def test_w4a16_gemv_strided_operands(gpu, threads, M, K, N, group):
    # x rows and scale/zero rows with leading strides wider than the row
    x, q, s, z = w4_case(2, M, K, N, group)
    G = K // group
    xw = torch.zeros(M, K + 64, dtype=torch.float16)
    xw[:, :K] = torch.from_numpy(x)
    sw = torch.zeros(N, G + 6, dtype=torch.float16)
    sw[:, :G] = torch.from_numpy(s)
    zw = torch.zeros(N, G + 6, dtype=torch.uint8)
    zw[:, :G] = torch.from_numpy(z)
    xd, sd, zd = xw.cuda(), sw.cuda(), zw.cuda()
    y = art(intent.weight_only_int4_asym_matmul, KERNEL="gemv").run(xd[:, :K], dev(q), sd[:, :G], zd[:, :G])
    assert_close_rms(host(y), oracle.w4a16(x, q, s, z, threads), what="gemv strided")


# M > 128 with group sizes that are multiples of 64 and K / group a multiple of 4 load scales
# and zeros once per pair of groups (64, 128, 192 with three stages per group, 256);
# (300, 384, 130, 192) has two groups per row and takes the per-stage loads.
@pytest.mark.parametrize("M,K,N,group", [(16, 4096, 4096, 128), (17, 512, 200, 128), (130, 256, 64, 64),
                                         (256, 1024, 384, 128), (1, 128, 128, 32), (40, 512, 256, 32),
                                         (300, 384, 130, 192), (300, 768, 130, 192), (200, 2048, 96, 256)])
def test_w4a16_gemm_shapes(gpu, threads, M, K, N, group):
    x, q, s, z = w4_case(2, M, K, N, group)
    y = art(intent.weight_only_int4_asym_matmul, KERNEL="gemm").run(dev(x), dev(q), dev(s), dev(z))
    assert_close_rms(host(y), oracle.w4a16(x, q, s, z, threads), what="gemm shapes")


def test_w4a16_prefill_config2(gpu, threads):
    d = inputs.config2_w4a16_prefill(0)
    x, q, s, z = d["x"], d["packed"], d["scales"], d["zeros"]
    X, Q, S, Z = dev(x), dev(q), dev(s), dev(z)
    y = art(intent.weight_only_int4_asym_matmul).run(X, Q, S, Z)
    assert art(intent.weight_only_int4_asym_matmul).observation.entry == "intent_w4a16_gemm"
    yh = host(y)
    rows = np.r_[0:32, 1000:1016, 2032:2048]
    ref = oracle.w4a16(x[rows], q, s, z, threads)
    assert_close_rms(yh[rows], ref, what="prefill rows vs oracle")
    # full size against a float64 restatement on the GPU
    nib = torch.stack((Q & 15, Q >> 4), dim=-1).reshape(Q.shape[0], -1).double()
    deq = (nib - Z.double().repeat_interleave(128, 1)) * S.double().repeat_interleave(128, 1)
    full = (X.double() @ deq.T).cpu().numpy()
    assert_close_rms(yh, full, what="prefill full vs f64")


@pytest.mark.parametrize("M,K,N,group", [(8192, 256, 2000, 128), (4096, 512, 3400, 64)])
def test_w4a16_gemm_many_row_tiles(gpu, threads, M, K, N, group):
    """The windowed W4 GEMM with 16 and 32 row tiles of 256 and a last column tile partly
    outside N: every output against a float64 restatement on the GPU, sampled rows
    against the oracle."""
    x, q, s, z = w4_case(3, M, K, N, group)
    X, Q, S, Z = dev(x), dev(q), dev(s), dev(z)
    y = art(intent.weight_only_int4_asym_matmul, KERNEL="gemm").run(X, Q, S, Z)
    yh = host(y)
    rows = np.r_[0:16, M - 16:M]
    assert_close_rms(yh[rows], oracle.w4a16(x[rows], q, s, z, threads), what="row tiles vs oracle")
    nib = torch.stack((Q & 15, Q >> 4), dim=-1).reshape(Q.shape[0], -1).double()
    deq = (nib - Z.double().repeat_interleave(group, 1)) * S.double().repeat_interleave(group, 1)
    assert_close_rms(yh, (X.double() @ deq.T).cpu().numpy(), what="row tiles full vs f64")


# ---- W8A16 --------------------------------------------------------------------------

@pytest.mark.parametrize("M,K,N", [(16, 1024, 1024), (1, 64, 10), (200, 320, 130)])
def test_w8a16(gpu, threads, M, K, N):
    d = inputs.config0_w8a16(0, M=M, K=K, N=N)
    y = art(intent.weight_only_int8_matmul).run(dev(d["x"]), dev(d["w"]), dev(d["scales"]))
    assert_close_rms(host(y), oracle.w8a16(d["x"], d["w"], d["scales"], threads), what="w8a16")


# ---- W8A8 / int8 --------------------------------------------------------------------

def test_w8a8_config3(gpu, threads):
    d = inputs.config3_w8a8(0)
    A, SA, W, SW = dev(d["a"]), dev(d["a_scales"]), dev(d["w"]), dev(d["w_scales"])
    out = art(intent.w8a8_scaled_matmul).run(A, SA, W, SW)
    bits = host(out.view(torch.int16)).view(np.uint16)
    rows = np.r_[0:16, 2048:2056, 4088:4096]
    ref = oracle.w8a8(d["a"][rows], d["a_scales"][rows], d["w"], d["w_scales"], threads)
    assert np.array_equal(bits[rows], ref), "W8A8 bf16 rows differ from the oracle"
    # full size: int32 accumulators exactly, via float64 sums on the GPU
    bias = torch.zeros(W.shape[0], dtype=torch.int32, device="cuda")
    acc = art(intent.gemm_i8_nt).run(A, W, bias)
    exact = (A.double() @ W.double().T)
    assert torch.equal(acc.double(), exact), "int32 accumulators are not exact"
    f = exact.float() * SA[:, None]
    f = f * SW[None, :]
    assert torch.equal(out.view(torch.int16), f.to(torch.bfloat16).view(torch.int16)), "bf16 epilogue not exact"


def _f32(bits):
    return np.array(bits, np.uint32).view(np.float32)


@pytest.mark.parametrize("M,N", [(256, 256), (4096, 4096)])
def test_w8a8_special_values(gpu, threads, M, N):
    """The bf16 epilogue (hardware v_cvt_pk_bf16_f32) bit for bit against the oracle's
    round-to-nearest-even where the products are NaN (quiet and signalling payloads, both
    signs), +-inf, +-0, f32 subnormals, bf16 overflow and exact rounding ties: A has one
    non-zero column, so acc = a[m, 0] * w[n, 0] exactly. (256 x 256: the 128-row tiles;
    4096 x 4096: the 256 x 256 tiles.)"""
    K = 64
    rng = np.random.default_rng(11)
    a = np.zeros((M, K), np.int8)
    a[:, 0] = rng.integers(-128, 128, M, dtype=np.int8)
    w = rng.integers(-128, 128, (N, K), dtype=np.int8)
    sa_pool = np.concatenate([_f32([0x7fc00000, 0xffc00001, 0x7fa00001, 0xff812345, 0x7f800000, 0xff800000,
                                    0x00000000, 0x80000000, 0x00000001, 0x807fffff, 0x00400000, 0x7f7fffff,
                                    0x3f808000, 0x3f818000, 0xbf808000, 0x3f800000]),
                              rng.uniform(-2, 2, 16).astype(np.float32)])
    sw_pool = np.concatenate([_f32([0x3f800000, 0x3f808000, 0x3f7f8000, 0x40000000, 0x00800000, 0x00000002,
                                    0x7f000000, 0x7fbfffff, 0x3c008000, 0xbc018000]),
                              rng.uniform(-1, 1, 22).astype(np.float32)])
    sa = sa_pool[np.arange(M) % sa_pool.size]
    sw = sw_pool[np.arange(N) % sw_pool.size]
    out = art(intent.w8a8_scaled_matmul).run(dev(a), dev(sa), dev(w), dev(sw))
    bits = host(out.view(torch.int16)).view(np.uint16)
    rows = np.r_[0:64, M - 64:M]
    ref = oracle.w8a8(a[rows], sa[rows], w, sw, threads)
    got = bits[rows]
    # Where both scales are NaN, IEEE 754 leaves the payload of the product to the
    # implementation (v_mul_f32 returns its first source's, and which scale that is
    # is the compiler's choice): a NaN is required there, the exact bits elsewhere.
    both = np.isnan(sa[rows])[:, None] & np.isnan(sw)[None, :]
    assert np.all((got[both] & 0x7f80) == 0x7f80) and np.all((got[both] & 0x7f) != 0)
    bad = np.argwhere((got != ref) & ~both)
    assert bad.size == 0, f"{len(bad)} bf16 outputs differ, first at {bad[0]}: got {got[tuple(bad[0])]:#06x} " \
                          f"want {ref[tuple(bad[0])]:#06x}"


@pytest.mark.parametrize("M,K,N", [(100, 192, 77), (1, 64, 1), (129, 640, 257), (4000, 192, 4100), (4096, 64, 4096)])
def test_i8_gemm_bias(gpu, threads, M, K, N):
    rng = np.random.default_rng(5)
    a = rng.integers(-128, 128, (M, K), dtype=np.int8)
    w = rng.integers(-128, 128, (N, K), dtype=np.int8)
    bias = rng.integers(-2**31, 2**31 - 1, N, dtype=np.int64).astype(np.int32)
    c = art(intent.gemm_i8_nt).run(dev(a), dev(w), dev(bias))
    assert np.array_equal(host(c), oracle.i8_gemm_i32(a, w, bias, threads))


# ---- shapes off the tiled kernels: the generic kernels ---------------------------------

def _padded(arr, extra):
    """A device copy of arr whose rows are `extra` elements longer (a leading stride that is
    not a multiple of 16 bytes), sliced back to arr's shape."""
    t = dev(np.ascontiguousarray(np.pad(arr, ((0, 0), (0, extra)))))
    return t[:, :arr.shape[1]]


@pytest.mark.parametrize("M,K,N,group,kernel", [(1, 96, 70, 32, "auto"), (3, 160, 33, 16, "gemv"),
                                                (20, 96, 50, 48, "auto"), (40, 256, 64, 8, "gemm"),
                                                (2, 4096, 300, 128, "strided")])
def test_w4a16_generic_shapes(gpu, threads, M, K, N, group, kernel):
    # K not a multiple of 128, groups not multiples of 32, rows not 16-byte aligned: the generic
    # kernel, against the oracle and a float64 brute force
    x, q, s, z = w4_case(6, M, K, N, group)
    if kernel == "strided":
        X, kern = _padded(x, 3), "auto"
    else:
        X, kern = dev(x), kernel
    a = art(intent.weight_only_int4_asym_matmul, KERNEL=kern)
    y = host(a.run(X, dev(q), dev(s), dev(z)))
    assert a.observation.kernel == "w4a16_generic_kernel", a.observation.kernel
    assert_close_rms(y, oracle.w4a16(x, q, s, z, threads), what=f"generic w4 {M}x{K}x{N} g{group}")
    assert_close_rms(y, oracle.w4a16_f64(x, q, s, z), what="generic w4 vs f64")


@pytest.mark.parametrize("M,K,N", [(3, 100, 50), (40, 200, 130), (17, 72, 9)])
def test_w8a16_generic_shapes(gpu, threads, M, K, N):
    d = inputs.config0_w8a16(1, M=M, K=K, N=N)
    a = art(intent.weight_only_int8_matmul)
    y = host(a.run(dev(d["x"]), dev(d["w"]), dev(d["scales"])))
    assert a.observation.kernel == "w8a16_generic_kernel", a.observation.kernel
    assert_close_rms(y, oracle.w8a16(d["x"], d["w"], d["scales"], threads), what="generic w8a16")


@pytest.mark.parametrize("M,K,N", [(5, 200, 70), (64, 96, 33), (3, 1000, 8)])
def test_int8_generic_shapes_exact(gpu, threads, M, K, N):
    d = inputs.config3_w8a8(2, M=M, K=K, N=N)
    o = art(intent.w8a8_scaled_matmul)
    out = o.run(dev(d["a"]), dev(d["a_scales"]), dev(d["w"]), dev(d["w_scales"]))
    assert o.observation.kernel == "i8_generic_kernel<scaled>", o.observation.kernel
    bits = host(out.view(torch.int16)).view(np.uint16)
    assert np.array_equal(bits, oracle.w8a8(d["a"], d["a_scales"], d["w"], d["w_scales"], threads))
    rng = np.random.default_rng(M)
    a, w = rng.integers(-128, 128, (M, K), dtype=np.int8), rng.integers(-128, 128, (N, K), dtype=np.int8)
    bias = rng.integers(-2**31, 2**31 - 1, N, dtype=np.int64).astype(np.int32)
    g = art(intent.gemm_i8_nt)
    c = g.run(_padded(a, 5), _padded(w, 7), dev(bias))  # unaligned rows
    assert g.observation.kernel == "i8_generic_kernel<i32>", g.observation.kernel
    assert np.array_equal(host(c), oracle.i8_gemm_i32(a, w, bias, threads))


# ---- MoE routing ------------------------------------------------------------------

@pytest.mark.parametrize("T,E,k,renorm", [(512, 8, 2, True), (333, 64, 4, False), (7, 3, 3, True), (1, 256, 8, True),
                                         (100, 300, 4, True), (37, 1000, 8, False)])
def test_moe_route(gpu, T, E, k, renorm):
    rng = np.random.default_rng(T + E)
    logits = rng.standard_normal((T, E), dtype=np.float32)
    logits[::5, 1] = logits[::5, 0]  # exact ties resolve to the lower index
    ids, wts = art(intent.moe_route_topk, TOP_K=k, RENORMALIZE=renorm).run(dev(logits))
    rid, rw = oracle.moe_route(logits, k, renorm)
    assert np.array_equal(host(ids), rid)
    np.testing.assert_allclose(host(wts), rw, rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("T,k,E,B", [(512, 2, 8, 128), (4096, 2, 64, 128), (100, 3, 5, 16), (1, 1, 1, 128),
                                     (3000, 2, 512, 64), (700, 3, 1500, 16), (64, 2, 2048, 32)])
def test_moe_align(gpu, T, k, E, B):
    rng = np.random.default_rng(T * 7 + E)
    if T == 4096:
        ids = (np.arange(T * k) % E).astype(np.int32).reshape(T, k)  # the reference's moe_alignment case
    else:
        ids = rng.integers(0, E, (T, k), dtype=np.int32)
        ids[0, 0] = -1 if T > 1 else ids[0, 0]  # out-of-range ids are dropped
        if T > 2:
            ids[1, 0] = E
    outs = art(intent.moe_align_block_size, EXPERTS=E, BLOCK_SIZE=B).run(dev(ids))
    refs = oracle.moe_align(ids, E, B)
    for got, ref, name in zip(outs, refs, ("sorted", "blocks", "offsets", "total")):
        assert np.array_equal(host(got), ref), name


@pytest.mark.parametrize("B", [128, 160])
def test_moe_route_align_config4(gpu, B):
    """Routing and alignment of BASELINE config 4's own router logits (seed 0,
    T=512, E=8, top-2, renormalised): ids, sorted route ids, block map and
    offsets equal the oracle's exactly; 160 is the block size the composite
    uses at this shape."""
    logits = inputs.config4_logits(0, T=512, E=8)
    assert np.array_equal(logits, inputs.config4_moe(0, T=512, H=64, E=8, top_k=2, F=64)["logits"])
    ids, wts = art(intent.moe_route_topk, TOP_K=2, RENORMALIZE=True).run(dev(logits))
    rid, rw = oracle.moe_route(logits, 2, True)
    assert np.array_equal(host(ids), rid)
    np.testing.assert_allclose(host(wts), rw, rtol=2e-6, atol=1e-7)
    outs = art(intent.moe_align_block_size, EXPERTS=8, BLOCK_SIZE=B).run(ids)
    refs = oracle.moe_align(rid, 8, B)
    for got, ref, name in zip(outs, refs, ("sorted", "blocks", "offsets", "total")):
        assert np.array_equal(host(got), ref), name


# ---- MoE expert FFN -----------------------------------------------------------------

def moe_small(seed, T, H, E, k, F, group=128):
    return inputs.config4_moe(seed, T=T, H=H, E=E, top_k=k, F=F, group=group)


def run_ffn(d, y0, renorm=True):
    a = art(intent.moe_expert_ffn_w4, TOP_K=d["top_k"], RENORMALIZE=renorm)
    y = dev(y0)
    a(dev(d["logits"]), dev(d["x"]), dev(d["wgu"]), dev(d["sgu"]), dev(d["zgu"]), dev(d["wd"]), dev(d["sd"]),
      dev(d["zd"]), y)
    return host(y)


@pytest.mark.parametrize("T,H,E,k,F", [(64, 256, 4, 2, 512), (37, 512, 8, 2, 256), (5, 128, 3, 1, 128),
                                       (600, 256, 2, 1, 256)])
def test_moe_ffn_small(gpu, threads, T, H, E, k, F):
    d = moe_small(3, T, H, E, k, F)
    y0 = np.random.default_rng(1).standard_normal((T, H), dtype=np.float32)
    got = run_ffn(d, y0)
    ids, wts = oracle.moe_route(d["logits"], k, True)
    ref = oracle.moe_ffn_w4(d["x"], ids, wts, d["wgu"], d["sgu"], d["zgu"], d["wd"], d["sd"], d["zd"],
                            y=y0.copy(), threads=threads)
    assert_close_rms(got - y0, ref - y0, what="moe ffn delta")


@pytest.mark.parametrize("group", [32, 64])
def test_moe_ffn_group_sizes(gpu, threads, group):
    T, H, E, k, F = 70, 256, 4, 2, 384
    d = moe_small(5, T, H, E, k, F, group=group)
    got = run_ffn(d, np.zeros((T, H), np.float32))
    ids, wts = oracle.moe_route(d["logits"], k, True)
    ref = oracle.moe_ffn_w4(d["x"], ids, wts, d["wgu"], d["sgu"], d["zgu"], d["wd"], d["sd"], d["zd"], threads=threads)
    assert_close_rms(got, ref, what=f"moe ffn group {group}")


# Many routes per expert: experts of two and more 128-row blocks with light
# last blocks, at group sizes 32, 64 and 128 and with F not a whole number
# of four-group windows.
@pytest.mark.parametrize("T,H,E,k,F,group", [(400, 1024, 4, 2, 1024, 128), (300, 512, 3, 2, 512, 64),
                                             (512, 2048, 8, 2, 768, 128), (200, 512, 2, 1, 512, 32)])
def test_moe_ffn_many_routes(gpu, threads, T, H, E, k, F, group):
    d = moe_small(8, T, H, E, k, F, group=group)
    got = run_ffn(d, np.zeros((T, H), np.float32))
    ids, wts = oracle.moe_route(d["logits"], k, True)
    ref = oracle.moe_ffn_w4(d["x"], ids, wts, d["wgu"], d["sgu"], d["zgu"], d["wd"], d["sd"], d["zd"], threads=threads)
    assert_close_rms(got, ref, what=f"moe ffn many routes T {T} H {H} E {E} F {F} group {group}")


# More than 64 row blocks of 160 rows (64 experts of ~128 routes): the
# heavy-first block order of gate/up takes several wave-wide passes.
def test_moe_ffn_many_blocks(gpu, threads):
    T, H, E, k, F = 2048, 512, 64, 4, 512
    d = moe_small(10, T, H, E, k, F)
    got = run_ffn(d, np.zeros((T, H), np.float32))
    ids, wts = oracle.moe_route(d["logits"], k, True)
    ref = oracle.moe_ffn_w4(d["x"], ids, wts, d["wgu"], d["sgu"], d["zgu"], d["wd"], d["sd"], d["zd"], threads=threads)
    assert_close_rms(got, ref, what="moe ffn many blocks")


# Group sizes that are multiples of 64 load scales and zeros in windows of
# four groups; these shapes cross several windows in gate/up (H) and down (F),
# including an odd window count and three stages per group.
@pytest.mark.parametrize("group,H,F", [(64, 1024, 768), (128, 2048, 1536), (192, 3072, 2304), (128, 1536, 1024)])
def test_moe_ffn_group_windows(gpu, threads, group, H, F):
    T, E, k = 70, 4, 2
    d = moe_small(6, T, H, E, k, F, group=group)
    got = run_ffn(d, np.zeros((T, H), np.float32))
    ids, wts = oracle.moe_route(d["logits"], k, True)
    ref = oracle.moe_ffn_w4(d["x"], ids, wts, d["wgu"], d["sgu"], d["zgu"], d["wd"], d["sd"], d["zd"], threads=threads)
    assert_close_rms(got, ref, what=f"moe ffn group {group} H {H} F {F}")


@pytest.mark.parametrize("B", [16, 32])
def test_moe_stages_other_block_sizes(gpu, threads, B):
    # align -> gate/up -> down -> combine at block sizes the tiled kernels do not take (the generic
    # kernels), against the oracle's whole expert FFN
    T, H, E, k, F = 45, 256, 4, 2, 128
    d = moe_small(8, T, H, E, k, F)
    ids, wts = oracle.moe_route(d["logits"], k, True)
    sorted_ids, blocks, _, _ = art(intent.moe_align_block_size, EXPERTS=E, BLOCK_SIZE=B).run(dev(ids))
    gu = art(intent.moe_gate_up_w4, TOP_K=k, BLOCK_SIZE=B)
    act = gu.run(dev(d["x"]), sorted_ids, blocks, dev(d["wgu"]), dev(d["sgu"]), dev(d["zgu"]))
    assert gu.observation.kernel == "moe_gate_up_generic_kernel", gu.observation.kernel
    dn = art(intent.moe_down_w4, ROUTES=T * k, BLOCK_SIZE=B)
    route_out = dn.run(act, sorted_ids, blocks, dev(d["wd"]), dev(d["sd"]), dev(d["zd"]))
    assert dn.observation.kernel == "moe_down_generic_kernel", dn.observation.kernel
    y = dev(np.zeros((T, H), np.float32))
    art(intent.moe_combine).run(route_out, dev(wts), y)
    ref = oracle.moe_ffn_w4(d["x"], ids, wts, d["wgu"], d["sgu"], d["zgu"], d["wd"], d["sd"], d["zd"],
                            threads=threads)
    assert_close_rms(host(y), ref, what=f"moe stages B={B}")


@pytest.mark.parametrize("T,H,E,k,F,group", [(30, 192, 3, 2, 96, 32), (9, 96, 2, 1, 200, 8)])
def test_moe_ffn_off_tile_dims(gpu, threads, T, H, E, k, F, group):
    # H not a multiple of 128, F not a multiple of 64 / 128, small groups: the composite runs the
    # generic projections
    d = moe_small(9, T, H, E, k, F, group=group)
    got = run_ffn(d, np.zeros((T, H), np.float32))
    ids, wts = oracle.moe_route(d["logits"], k, True)
    ref = oracle.moe_ffn_w4(d["x"], ids, wts, d["wgu"], d["sgu"], d["zgu"], d["wd"], d["sd"], d["zd"], threads=threads)
    assert_close_rms(got, ref, what=f"moe ffn off-tile {T}x{H}x{F} g{group}")


def test_moe_ffn_config4(gpu, threads):
    d = inputs.config4_moe(0)
    T, H = d["x"].shape
    got = run_ffn(d, np.zeros((T, H), np.float32))
    ids, wts = oracle.moe_route(d["logits"], 2, True)
    # float64 restatement on the GPU (routing from the oracle, bit-exact above)
    X = dev(d["x"]).double()
    y = torch.zeros(T, H, dtype=torch.float64, device="cuda")
    F = d["wgu"].shape[1] // 2

    def deq(q, s, z):
        q, s, z = dev(q), dev(s), dev(z)
        nib = torch.stack((q & 15, q >> 4), dim=-1).reshape(q.shape[0], -1).double()
        g = nib.shape[1] // s.shape[1]
        return (nib - z.double().repeat_interleave(g, 1)) * s.double().repeat_interleave(g, 1)

    for e in range(d["wgu"].shape[0]):
        toks, slots = np.nonzero(ids == e)
        if toks.size == 0:
            continue
        gu = deq(d["wgu"][e], d["sgu"][e], d["zgu"][e])
        h = X[torch.from_numpy(toks).cuda()] @ gu.T
        g, u = h[:, :F], h[:, F:]
        a = (g / (1 + torch.exp(-g)) * u).half().double()
        o = a @ deq(d["wd"][e], d["sd"][e], d["zd"][e]).T
        w = torch.from_numpy(wts[toks, slots]).cuda().double()
        y.index_add_(0, torch.from_numpy(toks).cuda(), w[:, None] * o)
    assert_close_rms(got, y.cpu().numpy(), what="moe config4 vs f64")


# H = 512 at group 128 gives the tiled kernels whole four-group windows; block
# size 192 is off the tiles and runs the generic kernels. Block size 160 takes
# the 160-row tile where K is whole four-group windows (H 512 for gate/up,
# F 512 for down) and the generic kernels elsewhere (H 256, F 384).
@pytest.mark.parametrize("B,T,F,H", [(128, 48, 256, 256), (64, 48, 256, 256), (64, 100, 384, 256),
                                     (128, 300, 512, 512), (192, 48, 256, 256), (160, 300, 512, 512),
                                     (160, 200, 384, 512), (160, 48, 512, 256)])
def test_moe_stage_entries(gpu, threads, B, T, F, H):
    E, k = 4, 2
    d = moe_small(9, T, H, E, k, F)
    ids, wts = art(intent.moe_route_topk, TOP_K=k).run(dev(d["logits"]))
    sorted_ids, blocks, offsets, total = art(intent.moe_align_block_size, EXPERTS=E, BLOCK_SIZE=B).run(ids)
    act = art(intent.moe_gate_up_w4, TOP_K=k, BLOCK_SIZE=B).run(dev(d["x"]), sorted_ids, blocks, dev(d["wgu"]),
                                                               dev(d["sgu"]), dev(d["zgu"]))
    ro = art(intent.moe_down_w4, ROUTES=T * k, BLOCK_SIZE=B).run(act, sorted_ids, blocks, dev(d["wd"]), dev(d["sd"]),
                                                                 dev(d["zd"]))
    y = torch.zeros(T, H, dtype=torch.float32, device="cuda")
    art(intent.moe_combine).run(ro, wts, y)
    ref = oracle.moe_ffn_w4(d["x"], host(ids), host(wts), d["wgu"], d["sgu"], d["zgu"], d["wd"], d["sd"], d["zd"],
                            threads=threads)
    assert_close_rms(host(y), ref, what="staged moe")


# ---- torch custom op ------------------------------------------------------------------

def test_torch_op_roundtrip(gpu):
    x, q, s, z = w4_case(4, 4, 512, 256, 128)
    a = art(intent.weight_only_int4_asym_matmul)
    op = a.as_torch_op("intent_amd_test::w4a16")
    X, Q, S, Z = dev(x), dev(q), dev(s), dev(z)
    assert torch.equal(op(X, Q, S, Z), a.run(X, Q, S, Z))
    comb = art(intent.moe_combine)
    cop = comb.as_torch_op("intent_amd_test::combine")
    ro = torch.randn(8, 128, device="cuda")
    w = torch.rand(4, 2, device="cuda")
    y1 = torch.randn(4, 128, device="cuda")
    y2 = y1.clone()
    assert cop(ro, w, y1) is None
    comb.run(ro, w, y2)
    assert torch.equal(y1, y2)


# ---- committed golden fixtures ----------------------------------------------------

from pathlib import Path  # noqa: E402

GOLDEN = Path(__file__).resolve().parent / "golden"


@pytest.mark.parametrize("name", ["w4a16_m3_k256_n40_g128", "w4a16_m17_k512_n24_g64"])
@pytest.mark.parametrize("kernel", ["gemv", "gemm", "auto"])
def test_golden_w4a16(gpu, name, kernel):
    g = np.load(GOLDEN / f"{name}.npz")
    if kernel == "gemv" and g["x"].shape[0] > 16:
        pytest.skip("GEMV covers M <= 16")
    y = art(intent.weight_only_int4_asym_matmul, KERNEL=kernel).run(dev(g["x"]), dev(g["packed"]), dev(g["scales"]),
                                                                     dev(g["zeros"]))
    assert_close_rms(host(y), g["y_f64"], what=name)


def test_golden_w8a16_w8a8(gpu):
    g = np.load(GOLDEN / "w8a16_m5_k192_n33.npz")
    y = art(intent.weight_only_int8_matmul).run(dev(g["x"]), dev(g["w"]), dev(g["scales"]))
    assert_close_rms(host(y), g["y_f64"], what="w8a16 golden")
    g = np.load(GOLDEN / "w8a8_m9_k256_n20.npz")
    out = art(intent.w8a8_scaled_matmul).run(dev(g["a"]), dev(g["a_scales"]), dev(g["w"]), dev(g["w_scales"]))
    assert np.array_equal(host(out.view(torch.int16)).view(np.uint16), g["out_bf16_bits"])
    acc = art(intent.gemm_i8_nt).run(dev(g["a"]), dev(g["w"]), dev(g["bias"]))
    assert np.array_equal(host(acc), g["acc_i32"])


def test_golden_moe(gpu):
    g = np.load(GOLDEN / "moe_t24_h128_e4_f128.npz")
    ids, wts = art(intent.moe_route_topk, TOP_K=2).run(dev(g["logits"]))
    assert np.array_equal(host(ids), g["topk_ids"])
    outs = art(intent.moe_align_block_size, EXPERTS=4, BLOCK_SIZE=16).run(ids)
    for got, name in zip(outs, ("sorted_ids_b16", "blocks_b16", "offsets_b16", "total_b16")):
        assert np.array_equal(host(got), g[name]), name
    y = torch.zeros(24, 128, dtype=torch.float32, device="cuda")
    art(intent.moe_expert_ffn_w4, TOP_K=2)(dev(g["logits"]), dev(g["x"]), dev(g["wgu"]), dev(g["sgu"]),
                                           dev(g["zgu"]), dev(g["wd"]), dev(g["sd"]), dev(g["zd"]), y)
    assert_close_rms(host(y), g["y_f64"], what="moe golden")


# ---- K-quant records: bit-exact against the oracle ---------------------------------

def _bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def _kquant_x(seed, G):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((G, 256)) * rng.uniform(0.001, 1000.0, (G, 1))).astype(np.float32)
    if G >= 4:
        x[1] = 0.0                                  # all-zero block
        x[2, :] = 0.25
        x[2, 7], x[2, 9] = 3.0, -3.0                # tie: the minimum is the extreme
        x[3, 0] = -127.0                            # inverse 1: exact half-way products
        x[3, 1:6] = [0.5, 1.5, 2.5, -0.5, -1.5]
        x[3, 6:] = -0.0
    return x


@pytest.mark.parametrize("G", [1, 4, 5, 64, 333])
def test_q8k_quantize_bit_exact(gpu, G):
    x = _kquant_x(20 + G, G)
    rec = art(intent.q8_k_quantize).run(dev(x))
    assert np.array_equal(host(rec), oracle.q8k_quantize(x))


@pytest.mark.parametrize("N,G", [(1, 1), (7, 3), (100, 16), (33, 17), (5, 40), (4, 0)])
def test_q4k_q8k_dot_bit_exact(gpu, N, G):
    rng = np.random.default_rng(N * 100 + G)
    w = inputs.q4k_records(rng, (N, G))
    xq = oracle.q8k_quantize(_kquant_x(N + G, G)) if G else np.zeros((0, 292), np.uint8)
    y = art(intent.q4_k_q8_k_dot).run(dev(w), dev(xq))
    ref = oracle.q4k_gemv(w, xq) if G else np.zeros(N, np.float32)
    assert np.array_equal(_bits(host(y)), _bits(ref))


def test_quantized_projection_full_size_bit_exact(gpu, threads):
    d = inputs.kquant_projection(0, N=4096, K=4096)
    y = art(intent.quantized_projection).run(dev(d["w"]), dev(d["x"]))
    ref = oracle.q4k_gemv(d["w"], oracle.q8k_quantize(d["x"]), threads)
    assert np.array_equal(_bits(host(y)), _bits(ref))


@pytest.mark.parametrize("N,G", [(1, 1), (9, 3), (100, 16), (33, 17), (64, 64), (5, 65), (70, 100)])
def test_quantized_projection_bit_exact(gpu, N, G):
    """Both projection paths (one fused launch for G <= 64, quantize + GEMV
    above): the output and the Q8_K records written on the way."""
    from intent_amd import _native

    rng = np.random.default_rng(300 + N + G)
    w = inputs.q4k_records(rng, (N, G))
    x = _kquant_x(N * 3 + G, G)
    wd, xd = dev(w), dev(x)
    rec = torch.full((G, 292), 0xAB, dtype=torch.uint8, device="cuda")
    y = torch.full((N,), float("nan"), dtype=torch.float32, device="cuda")
    _native.call("intent_q4k_projection", wd.data_ptr(), N, G, G * 144, xd.data_ptr(), 256, rec.data_ptr(),
                 y.data_ptr(), torch.cuda.current_stream().cuda_stream)
    xq = oracle.q8k_quantize(x)
    assert np.array_equal(host(rec), xq)
    assert np.array_equal(_bits(host(y)), _bits(oracle.q4k_gemv(w, xq)))


def test_golden_kquant(gpu):
    g = np.load(GOLDEN / "q4k_n7_g3.npz")
    assert np.array_equal(host(art(intent.q8_k_quantize).run(dev(g["x"]))), g["xq"])
    y = art(intent.quantized_projection).run(dev(g["w"]), dev(g["x"]))
    assert np.array_equal(_bits(host(y)), _bits(g["y"]))


# ---- groupwise FP8 quantizers: bit-exact against the oracle ----------------------

@pytest.mark.parametrize("src", ["f32", "bf16"])
@pytest.mark.parametrize("M,N,G", [(1, 128, 1), (3, 300, 3), (17, 4096, 32), (2, 256, 4), (64, 8192, 64)])
def test_fp8_groupwise_quantize_bit_exact(gpu, src, M, N, G):
    rng = np.random.default_rng(M * 7 + N)
    x = (rng.standard_normal((M, N)) * rng.uniform(1e-6, 1e4, (M, 1))).astype(np.float32)
    x[0, :5] = [0.0, -0.0, 1e-30, -448.0, 3.0]
    x[-1, : min(N, 128)] = 0.0  # an all-zero group takes the eps floor
    if src == "bf16":
        xt = torch.from_numpy(x).to(torch.bfloat16)
        x = xt.float().numpy()  # exact widening: the oracle sees the same values
        defn = intent.bf16_groupwise_fp8_quantize
    else:
        xt = torch.from_numpy(x)
        defn = intent.f32_groupwise_fp8_quantize
    scales = torch.zeros(M, G, dtype=torch.float32, device="cuda")
    q = art(defn).run(xt.cuda(), scales)
    ref_q, ref_s = oracle.fp8_groupwise_quantize(x, groups=G, source=src)
    assert np.array_equal(host(q.view(torch.uint8)), ref_q)
    assert np.array_equal(host(scales).view(np.uint32), ref_s.view(np.uint32))


# ---- per-token int8 quantizer: bit-exact ------------------------------------------------

@pytest.mark.parametrize("src", ["f16", "bf16"])
@pytest.mark.parametrize("M,K", [(1, 8), (3, 24), (5, 2056), (64, 4096), (17, 16392), (4096, 8192), (2, 0)])
def test_i8_per_token_quantize_bit_exact(gpu, src, M, K):
    rng = np.random.default_rng(M * 13 + K)
    x = (rng.standard_normal((M, K)) * rng.uniform(1e-3, 1e3, (M, 1))).astype(np.float32)
    if K >= 16:
        x[0, :10] = [127.0, 2.5, 3.5, -2.5, -3.5, 0.5, -0.5, 1.5, 126.5, -127.0]  # ties at scale 1
        x[0, 10:] = 0.0
    if M > 2 and K:
        x[1] = 0.0  # zero row
        x[2, K // 2] = -1e-6  # lone tiny value
    tdt = torch.float16 if src == "f16" else torch.bfloat16
    xt = torch.from_numpy(x).to(tdt)
    ref_q, ref_s = oracle.i8_per_token_quantize(xt.float().numpy())  # exact widening of the same values
    defn = intent.per_token_int8_quantize if src == "f16" else intent.bf16_per_token_int8_quantize
    q, sc = art(defn).run(xt.cuda())
    assert np.array_equal(host(q), ref_q)
    assert np.array_equal(host(sc).view(np.uint32), ref_s.view(np.uint32))


def test_i8_per_token_strided_rows(gpu):
    rng = np.random.default_rng(11)
    big = torch.from_numpy(rng.standard_normal((9, 1040)).astype(np.float16))
    x = big[:, 8:1032]  # rows 2080 bytes apart, 16-byte aligned start
    qbuf = torch.full((9, 1040), 77, dtype=torch.int8, device="cuda")
    q = qbuf[:, :1024]
    sc = torch.empty(9, dtype=torch.float32, device="cuda")
    art(intent.per_token_int8_quantize).launch(big.cuda()[:, 8:1032], q, sc)
    ref_q, ref_s = oracle.i8_per_token_quantize(x.float().numpy())
    got = host(qbuf)
    assert np.array_equal(got[:, :1024], ref_q) and np.all(got[:, 1024:] == 77)
    assert np.array_equal(host(sc), ref_s)


def test_quantize_then_w8a8_chain(gpu, threads):
    """Per-token int8 quantizer feeding the W8A8 GEMM, against the oracle's chain (bit-exact bf16)."""
    rng = np.random.default_rng(21)
    M, K, N = 256, 1024, 384
    x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float16))
    w = rng.integers(-127, 128, (N, K), dtype=np.int8)
    sw = rng.uniform(0.001, 0.01, N).astype(np.float32)
    q, sa = art(intent.per_token_int8_quantize).run(x.cuda())
    out = art(intent.w8a8_scaled_matmul).run(q, sa, dev(w), dev(sw))
    rq, rs = oracle.i8_per_token_quantize(x.float().numpy())
    ref = oracle.w8a8(rq, rs, w, sw, threads)
    assert np.array_equal(host(out.view(torch.int16)).view(np.uint16), ref)


# ---- W4A8 and BitNet int2: exact int32 ----------------------------------------------

@pytest.mark.parametrize("M,K,N", [(1, 128, 1), (37, 256, 100), (300, 384, 130), (512, 2048, 1024), (4000, 256, 4100),
                                   (4100, 384, 3900)])
def test_w4a8_and_bitnet_exact(gpu, threads, M, K, N):
    rng = np.random.default_rng(M + 3 * N)
    a = rng.integers(-128, 128, (M, K), dtype=np.int8)
    p4 = rng.integers(0, 256, (N, K // 2), dtype=np.uint8)
    p2 = rng.integers(0, 256, (N, K // 4), dtype=np.uint8)
    got = art(intent.w4a8_packed_matmul).run(dev(a), dev(p4))
    assert np.array_equal(host(got), oracle.w4a8(a, p4, threads))
    got = art(intent.bitnet_int2_matmul).run(dev(a), dev(p2))
    assert np.array_equal(host(got), oracle.bitnet_int2(a, p2, threads))


def test_w4a8_full_size_exact(gpu):
    # The reference's W4A8 case: a [4096, 4096], packed [14336, 2048] -> int32 [14336, 4096]
    # (experiments/cpu/providers/mojo/contraction.py:201-206), checked on the GPU
    # against an exact float64 restatement (|products| sum below 2^53).
    rng = np.random.default_rng(99)
    a = torch.from_numpy(rng.integers(-128, 128, (4096, 4096), dtype=np.int8)).cuda()
    p = torch.from_numpy(rng.integers(0, 256, (14336, 2048), dtype=np.uint8)).cuda()
    got = art(intent.w4a8_packed_matmul).run(a, p)
    nib = torch.stack((p & 15, p >> 4), dim=-1).reshape(14336, -1).to(torch.int32)
    signed = (nib - ((nib & 8) << 1)).to(torch.float64)
    ref = (signed @ a.to(torch.float64).T)
    assert torch.equal(got.to(torch.float64), ref)


@pytest.mark.parametrize("M,N", [(64, 96), (4096, 4096)])
@pytest.mark.parametrize("K", [130944, 131072])
def test_w4a8_int32_extremes(gpu, M, N, K):
    # Up to K = 130944 the kernels stage the nibbles as 16 * value and shift the
    # accumulators right by 4; at the extreme operands (-128 x -8 every k) the
    # scaled sum 16 * 1024 * K is then just below 2^31. K = 131072 takes the
    # sign-extending decode. Small and large M, N cover both kernels.
    a = torch.full((M, K), -128, dtype=torch.int8, device="cuda")
    a[1::2] = 127
    p = torch.full((N, K // 2), 0x88, dtype=torch.uint8, device="cuda")  # -8, -8
    p[1::3] = 0x77  # 7, 7
    got = art(intent.w4a8_packed_matmul).run(a, p)  # [N, M]
    wv = torch.full((N,), -8, dtype=torch.int64, device="cuda")
    wv[1::3] = 7
    av = torch.full((M,), -128, dtype=torch.int64, device="cuda")
    av[1::2] = 127
    assert torch.equal(got.to(torch.int64), wv[:, None] * av[None, :] * K)


# ---- MX block-scaled FP8 ------------------------------------------------------------

def _mx_case(seed, M, K, N):
    rng = np.random.default_rng(seed)
    a = rng.integers(0, 256, (M, K), dtype=np.uint8)
    b = rng.integers(0, 256, (N, K), dtype=np.uint8)
    a[(a & 0x7F) == 0x7F] = 0x38  # keep NaN codes out of the data (E4M3FN 0x7F / 0xFF)
    b[(b & 0x7F) == 0x7F] = 0x38
    sa = rng.integers(120, 134, (M, K // 32), dtype=np.uint8)
    sb = rng.integers(120, 134, (N, K // 32), dtype=np.uint8)
    return a, sa, b, sb


@pytest.mark.parametrize("M,K,N,layout", [(64, 128, 64, "view"), (130, 256, 70, "view"), (512, 768, 512, "view"),
                                          (33, 384, 100, "contiguous"),
                                          # 256 x 256 DMA-fed tiles: ragged edges, odd / even / single stage counts;
                                          # 272 tiles on 256 CUs: the last 16 as 32 half-width tiles
                                          (4000, 384, 4200, "view"), (4096, 256, 4096, "contiguous"),
                                          (4096, 128, 4352, "view")])
def test_block_scaled_matmul(gpu, threads, M, K, N, layout):
    a, sa, b, sb = _mx_case(M + N, M, K, N)
    KB = K // 32
    lhs = dev(a).view(torch.float8_e4m3fn).view(M, KB, 32)
    bt = dev(b).view(torch.float8_e4m3fn)
    if layout == "view":  # the reference benchmark's layout: rhs = rhs_rows.T.view(KB, 32, N)
        rhs = bt.T.view(KB, 32, N)
        rs = dev(sb).T
    else:
        rhs = bt.T.contiguous().view(KB, 32, N)
        rs = dev(sb).T.contiguous()
    out = art(intent.block_scaled_matmul).run(lhs, dev(sa), rhs, rs)
    ref = oracle.mxfp8_gemm(a, sa, b, sb, threads)
    # The scaled MFMA sums 64 products per instruction in its own order and
    # precision (measured ~1e-4 of the largest term); the gate is the float one.
    assert_close_rms(host(out), ref, what=f"mxfp8 {M}x{K}x{N}")


# ---- per-tensor scaled FP8 GEMM, plain and split-K ----------------------------------

def _fp8_bits(seed, shape):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def _f16_close(got, ref, what):
    # f32 sums in another order may round to a neighbouring f16 (before and after
    # the scaling): allow a few f16 ulps of the output's magnitude.
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    assert np.all(np.isfinite(got)), what
    assert np.max(np.abs(got - ref)) <= 4e-3 * np.abs(ref).max(), what


@pytest.mark.parametrize("M,K,N", [(64, 128, 64), (130, 384, 70), (1, 256, 1), (4000, 512, 4200), (512, 4096, 1000)])
def test_scaled_fp8_matmul(gpu, threads, M, K, N):
    a, b = _fp8_bits(M + N, (M, K)), _fp8_bits(K + N, (K, N))
    lhs = dev(a).view(torch.float8_e4m3fn)
    rhs = dev(b).view(torch.float8_e4m3fn)
    out = art(intent.scaled_fp8_matmul).run(lhs, rhs, 0.5, 1.5)
    rows = _sample_rows(M)
    ref = oracle.scaled_fp8_gemm(a[rows], b, 0.5, 1.5, threads=threads)
    _f16_close(host(out)[rows], ref, f"scaled_fp8 {M}x{K}x{N}")


@pytest.mark.parametrize("M,IT,SP,N", [(64, 1, 4, 64), (300, 2, 3, 130), (4096, 1, 2, 4352)])
def test_scaled_fp8_splitk(gpu, threads, M, IT, SP, N):
    K = IT * SP * 256
    a, b = _fp8_bits(M, (M, K)), _fp8_bits(N, (K, N))
    out0 = (torch.randn(M, N, generator=torch.Generator().manual_seed(3)) * 8).half()
    lhs = dev(a).view(torch.float8_e4m3fn).view(M, IT, SP, 256)
    rhs = dev(b).view(torch.float8_e4m3fn).view(IT, SP, 256, N)
    out = out0.cuda()
    art(intent.scaled_fp8_splitk_matmul).run(lhs, rhs, out, 0.25, 2.0)
    rows = _sample_rows(M)
    ref = oracle.scaled_fp8_gemm(a[rows], b, 0.25, 2.0, splits=SP, out=out0.numpy()[rows], threads=threads)
    _f16_close(host(out)[rows], ref, f"splitk {M}x{K}x{N}/{SP}")


@pytest.mark.parametrize("M,K,N,ldb,splits,out_pad", [(300, 512, 4096, 4096, 1, 0), (257, 384, 144, 160, 1, 0),
                                                      (130, 1024, 272, 288, 2, 0), (64, 128, 16, 16, 1, 0),
                                                      (130, 1024, 272, 288, 2, 4), (520, 2048, 400, 400, 4, 8),
                                                      (600, 1536, 160, 176, 3, 2), (1, 256, 32, 32, 1, 0)])
def test_scaled_fp8_kn_in_place(gpu, threads, M, K, N, ldb, splits, out_pad):
    """intent_scaled_fp8_gemm_kn reads b [K, N] in place, with a row stride past N and
    a last column tile that is partly outside N, into outputs with 16-byte aligned rows
    or not (out_pad 2, 4: the output tile is then loaded and stored element-wise);
    against the oracle and against the transposed-copy entry on the same inputs (bit-equal:
    same tile, same k pairing per MFMA), and the padding columns stay untouched."""
    from intent_amd import _native
    a, bfull = _fp8_bits(M + K, (M, K)), _fp8_bits(N + K, (K, ldb))
    b = np.ascontiguousarray(bfull[:, :N])
    out0 = (torch.randn(M, N, generator=torch.Generator().manual_seed(5)) * 4).half()
    ld = N + out_pad
    ad, bd = dev(a), dev(bfull)
    outs = []
    for kn in (True, False):
        full = torch.full((M, ld), -3.0, dtype=torch.float16)
        full[:, :N] = out0
        out = full.cuda()
        if kn:
            _native.call("intent_scaled_fp8_gemm_kn", ad.data_ptr(), M, K, K, bd.data_ptr(), N, ldb, 0.5, 1.5,
                         splits, int(splits > 1), out.data_ptr(), ld, 0)
        else:
            bt = dev(np.ascontiguousarray(b.T))
            _native.call("intent_scaled_fp8_gemm", ad.data_ptr(), M, K, K, bt.data_ptr(), N, K, 0.5, 1.5, splits,
                         int(splits > 1), out.data_ptr(), ld, 0)
        torch.cuda.synchronize()
        got = host(out)
        assert np.all(got[:, N:] == -3.0)
        outs.append(np.ascontiguousarray(got[:, :N]))
    assert np.array_equal(outs[0].view(np.uint16), outs[1].view(np.uint16)), f"kn vs rows {M}x{K}x{N}"
    rows = _sample_rows(M)
    ref = oracle.scaled_fp8_gemm(a[rows], b, 0.5, 1.5, splits=splits,
                                 out=out0.numpy()[rows] if splits > 1 else None, threads=threads)
    _f16_close(outs[0][rows], ref, f"scaled_fp8_kn {M}x{K}x{N}/{splits}")


@pytest.mark.parametrize("R,C,sld,dld", [(256, 384, 384, 256), (128, 128, 144, 160), (4096, 1024, 1024, 4096),
                                         (100, 70, 80, 112), (300, 128, 128, 304)])
def test_fp8_transpose(gpu, R, C, sld, dld):
    """intent_fp8_transpose (whole 128 x 128 tiles, and the general path) against numpy;
    bytes of dst outside [C, R] stay untouched."""
    from intent_amd import _native
    src = np.random.default_rng(R * C).integers(0, 256, (R, sld), dtype=np.uint8)
    dst = torch.full((C, dld), 0xA5, dtype=torch.uint8, device="cuda")
    sd = dev(src)
    _native.call("intent_fp8_transpose", sd.data_ptr(), R, C, sld, dst.data_ptr(), dld, 0)
    torch.cuda.synchronize()
    got = host(dst)
    assert np.array_equal(got[:, :R], src[:, :C].T)
    assert np.all(got[:, R:] == 0xA5)


def test_scaled_fp8_kn_rejects_ragged_n(gpu):
    from intent_amd import _native
    a = torch.zeros((64, 128), dtype=torch.uint8, device="cuda")
    b = torch.zeros((128, 40), dtype=torch.uint8, device="cuda")
    out = torch.zeros((64, 40), dtype=torch.float16, device="cuda")
    with pytest.raises(Exception, match="multiple of 16"):
        _native.call("intent_scaled_fp8_gemm_kn", a.data_ptr(), 64, 128, 128, b.data_ptr(), 40, 48, 1.0, 1.0, 1, 0,
                     out.data_ptr(), 40, 0)


def test_scaled_fp8_splitk_reference_size(gpu):
    # The reference's split-K case (experiments/gpu/providers/triton/contraction.py:174-186:
    # 4096 x 4096 x 14336, IT 4, SP 4, scales 1), checked against its CPU formula
    # (cpu_runtime.py:133-139) evaluated with torch on the GPU in f32.
    M, N, IT, SP = 4096, 14336, 4, 4
    g = torch.Generator(device="cuda").manual_seed(7)
    lhs = torch.randn((M, IT * SP * 256), device="cuda", generator=g).to(torch.float8_e4m3fn)
    rhs = torch.randn((IT * SP * 256, N), device="cuda", generator=g).to(torch.float8_e4m3fn)
    out = torch.zeros((M, N), device="cuda", dtype=torch.float16)
    art(intent.scaled_fp8_splitk_matmul).run(lhs.view(M, IT, SP, 256), rhs.view(IT, SP, 256, N), out, 1.0, 1.0)
    ref = torch.zeros_like(out)
    l4, r4 = lhs.view(M, IT, SP, 256), rhs.view(IT, SP, 256, N)
    for s in range(SP):
        ref.add_((l4[:, :, s, :].float().flatten(1) @ r4[:, s, :, :].float().flatten(0, 1)).half())
    err = (out.double() - ref.double()).abs().max().item()
    assert torch.isfinite(out).all() and err <= 4e-3 * ref.double().abs().max().item()


# ---- DeepGEMM-style FP8 with f32 block scales ----------------------------------------

def _bf16_bits_to_f64(bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).double().numpy()


@pytest.mark.parametrize("M,KB,N", [(64, 1, 128), (300, 3, 200), (1, 2, 1), (4000, 4, 4200)])
def test_deepgemm_fp8(gpu, threads, M, KB, N):
    a, b = _fp8_bits(M + 1, (M, KB * 128)), _fp8_bits(N + 2, (N, KB * 128))
    g = torch.Generator().manual_seed(M + N)
    NB = (N + 127) // 128
    sa = (torch.rand(M, KB, generator=g) + 0.25).numpy()
    sb = (torch.rand(NB, KB, generator=g) + 0.25).numpy()
    lhs = dev(a).view(torch.float8_e4m3fn).view(M, KB, 128)
    rhs = dev(b).view(torch.float8_e4m3fn).view(N, KB, 128)
    out = art(intent.deepgemm_fp8_2xacc).run(lhs, rhs, dev(sa), dev(sb))
    rows = _sample_rows(M)
    ref = _bf16_bits_to_f64(oracle.deepgemm_fp8(a[rows], sa[rows], b, sb, threads))
    got = host(out.view(torch.int16)).view(np.uint16)[rows]
    # bf16 output: one rounding of ~2^-8 relative on either side
    assert np.max(np.abs(_bf16_bits_to_f64(got) - ref)) <= 1e-2 * np.abs(ref).max()


def test_deepgemm_fp8_reference_inputs(gpu):
    # The reference's case and input construction (experiments/cpu/providers/mojo/
    # contraction.py:227-236: per-block absmax scaling to 448, M = N = K = 4096),
    # checked against its CPU formula (cpu_runtime.py:127-131) evaluated on the GPU.
    g = torch.Generator(device="cuda").manual_seed(5)
    lv = torch.randn((4096, 4096), device="cuda", generator=g).bfloat16().view(4096, 32, 128)
    lmax = lv.abs().float().amax(dim=2).clamp_min(1e-4)
    lhs = (lv * (448.0 / lmax[:, :, None])).to(torch.float8_e4m3fn)
    rv = torch.randn((4096, 4096), device="cuda", generator=g).bfloat16().view(32, 128, 32, 128)
    rmax = rv.abs().float().amax(dim=(1, 3), keepdim=True).clamp_min(1e-4)
    rhs = (rv * (448.0 / rmax)).to(torch.float8_e4m3fn).view(4096, 32, 128)
    ls, rs = lmax / 448.0, (rmax / 448.0).view(32, 32)
    out = art(intent.deepgemm_fp8_2xacc).run(lhs, rhs, ls, rs.contiguous())
    left = (lhs.float() * ls[:, :, None]).flatten(1)
    right = (rhs.float() * rs.repeat_interleave(128, dim=0)[:, :, None]).flatten(1)
    ref = (left @ right.T)
    err = (out.double() - ref.double()).abs().max().item()
    assert torch.isfinite(out.float()).all() and err <= 1e-2 * ref.abs().max().item()


# ---- FP8 x FP8 -> FP8 ----------------------------------------------------------------

@pytest.mark.parametrize("fmt", ["e4m3fn", "e5m2"])
@pytest.mark.parametrize("M,K,N", [(64, 128, 64), (300, 384, 130), (4096, 1024, 4352)])
def test_fp8_out_matmul(gpu, threads, fmt, M, K, N):
    tdt = torch.float8_e4m3fn if fmt == "e4m3fn" else torch.float8_e5m2
    g = torch.Generator().manual_seed(M + N)
    a = (torch.randn(M, K, generator=g) * 0.25).to(tdt)
    b = (torch.randn(N, K, generator=g) * 0.25).to(tdt)
    defn = intent.fp8_e4m3_matmul if fmt == "e4m3fn" else intent.fp8_e5m2_matmul
    out = art(defn).run(a.cuda(), b.cuda())
    rows = _sample_rows(M)
    ref = oracle.fp8_gemm(a.view(torch.uint8).numpy()[rows], b.view(torch.uint8).numpy(), fmt, threads)
    got = host(out.view(torch.uint8))[rows]
    # identical codes except where the two f32 sums (different order) straddle a
    # rounding boundary: then the neighbouring code
    assert np.mean(got == ref) >= 0.99
    dg = torch.from_numpy(got).view(tdt).double()
    dr = torch.from_numpy(ref).view(tdt).double()
    step = 2.0 ** -2 if fmt == "e5m2" else 2.0 ** -3
    assert torch.all((dg - dr).abs() <= step * dr.abs() + 2.0 ** -9)


# ---- FP4 (E2M1) weights x bf16 activations --------------------------------------------

@pytest.mark.parametrize("M,K,N", [(64, 128, 64), (300, 384, 130), (17, 256, 40), (4096, 4096, 4096)])
def test_dequant_bf16_fp4_matmul(gpu, threads, M, K, N):
    g = torch.Generator().manual_seed(M + K)
    x = (torch.randn(M, K, generator=g) * 0.125).bfloat16()   # the reference's input scale
    packed = torch.randint(0, 256, (N, K // 2), generator=g, dtype=torch.uint8)
    out = art(intent.dequant_bf16_fp4_matmul).run(x.cuda(), packed.cuda())
    rows = np.r_[0:min(M, 8), max(0, M - 8):M]  # every element: test_fp4_whole_matrix_and_strided_output
    ref = oracle.fp4_bf16_matmul(x.view(torch.int16).numpy().view(np.uint16)[rows], packed.numpy(), threads)
    got = host(out.view(torch.int16)).view(np.uint16)[rows]
    r64 = torch.from_numpy(ref.view(np.int16)).view(torch.bfloat16).double().numpy()
    g64 = torch.from_numpy(got.view(np.int16)).view(torch.bfloat16).double().numpy()
    assert np.max(np.abs(g64 - r64)) <= 1e-2 * np.abs(r64).max()


def _fp4_decode_torch(packed):
    """E2M1 weights as f32 by the reference's recipe (cpu_runtime.py:117-124), on packed's device."""
    word = (packed[:, 0::2].int() << 8) | packed[:, 1::2].int()
    bits = torch.stack((word & 0x81C0, (word << 3) & 0x81C0, (word << 6) & 0x81C0,
                        ((word << 1) & 0x8000) | ((word >> 3) & 0x0180) | ((word >> 7) & 0x0040)),
                       dim=-1).flatten(1).to(torch.int16)
    return (bits.view(torch.bfloat16).float() * (2.0 ** 126)).bfloat16().float()


@pytest.mark.parametrize("M,K,N,y_pad", [(1000, 512, 520, 0), (700, 256, 300, 3), (4096, 1024, 1032, 8)])
def test_fp4_whole_matrix_and_strided_output(gpu, M, K, N, y_pad):
    """Every output element of intent_fp4_bf16_matmul (middle row and column tiles included)
    against an f32 product of the decoded weights, on a contiguous or padded (odd stride:
    element stores) output whose padding columns must stay untouched."""
    from intent_amd import _native

    g = torch.Generator().manual_seed(M + N + y_pad)
    x = (torch.randn(M, K, generator=g) * 0.125).bfloat16()
    packed = torch.randint(0, 256, (N, K // 2), generator=g, dtype=torch.uint8)
    dec = _fp4_decode_torch(packed)
    for r in (0, N - 1):  # the recipe is the oracle's decode
        assert np.array_equal(dec[r].numpy(), oracle.fp4_decode_row(packed[r].numpy()))
    xd, pd = x.cuda(), packed.cuda()
    ld = N + y_pad
    y = torch.full((M, ld), -7.0, dtype=torch.bfloat16, device="cuda")
    _native.call("intent_fp4_bf16_matmul", xd.data_ptr(), M, K, K, pd.data_ptr(), N, K // 2, y.data_ptr(), ld, 0)
    torch.cuda.synchronize()
    ref = xd.float() @ dec.cuda().t()
    err = (y[:, :N].float() - ref).abs().max().item()
    assert err <= 1e-2 * ref.abs().max().item(), err
    if y_pad:
        assert torch.all(y[:, N:] == -7.0)


# ---- the reference's own weight_only_int4_matmul layout --------------------------------

@pytest.mark.parametrize("M,K,N", [(512, 2048, 4096), (1, 2048, 4096), (3, 256, 100), (40, 128, 33),
                                   (1, 4096, 4096), (2, 8192, 260), (4, 64, 4), (5, 4160, 1028), (16, 4096, 512)])
def test_weight_only_int4_matmul_reference_layout(gpu, threads, M, K, N):
    # (512, 2048, 4096) is the reference's own example size (weight_only_int4.py:6-8)
    rng = np.random.default_rng(M + N)
    x = rng.standard_normal((M, K)).astype(np.float16)
    packed = rng.integers(-2**31, 2**31, (K // 8, N), dtype=np.int64).astype(np.int32)
    scales = rng.uniform(0.005, 0.02, (K // 64, N)).astype(np.float16)
    y = art(intent.weight_only_int4_matmul).run(dev(x), dev(packed), dev(scales))
    rows = _sample_rows(M)
    ref = oracle.w4_sym(x[rows], packed, scales, threads)
    assert_close_rms(host(y)[rows], ref.astype(np.float32), what=f"w4 sym {M}x{K}x{N}")


@pytest.mark.parametrize("M,K,N", [(1, 4096, 4096), (3, 1024, 64), (5, 8192, 132), (17, 64, 20), (300, 1024, 390),
                                   (2048, 4096, 1100)])
def test_weight_only_int4_matmul_in_place_strided(gpu, threads, M, K, N):
    """The in-place entries (intent_w4a16_sym_gemv up to M = 5, intent_w4a16_sym_gemm above
    M = 16) on strided x, packed words and scales, against the oracle; and the entry the
    operator picked for these shapes."""
    rng = np.random.default_rng(K + N)
    x = rng.standard_normal((M, K + 8)).astype(np.float16)
    packed = rng.integers(-2**31, 2**31, (K // 8, N + 4), dtype=np.int64).astype(np.int32)
    scales = rng.uniform(0.005, 0.02, (K // 64, N + 8)).astype(np.float16)
    a = art(intent.weight_only_int4_matmul)
    y = a.run(dev(x)[:, :K], dev(packed)[:, :N], dev(scales)[:, :N])
    assert a.observation.entry == ("intent_w4a16_sym_gemv" if M <= 5 else "intent_w4a16_sym_gemm")
    rows = np.r_[0:min(M, 16), max(0, M - 16):M]
    ref = oracle.w4_sym(np.ascontiguousarray(x[rows, :K]), np.ascontiguousarray(packed[:, :N]),
                        np.ascontiguousarray(scales[:, :N]), threads)
    assert_close_rms(host(y)[rows], ref.astype(np.float32), what=f"w4 sym in place {M}x{K}x{N}")


# ---- quantized_gemm -------------------------------------------------------------------

@pytest.mark.parametrize("M,K,N", [(64, 128, 64), (300, 384, 130), (1, 64, 1), (200, 256, 260), (4096, 4096, 14336),
                                   (300, 384, 136), (513, 640, 264)])
def test_quantized_gemm(gpu, threads, M, K, N):
    # the reference's input construction (experiments/cpu/providers/mojo/contraction.py:177-186)
    g = torch.Generator().manual_seed(M + N)
    a = torch.randn((M, K), generator=g).half() / (K ** 0.5)
    b = torch.randn((K, N), generator=g).half()
    bias = torch.randn((N,), generator=g) * 0.25
    residual = (torch.randn((M, N), generator=g) * 0.25).half()
    scale = torch.linspace(1.0 / 48.0, 1.0 / 24.0, N)
    out = art(intent.quantized_gemm).run(a.cuda(), b.cuda(), bias.cuda(), residual.cuda(), scale.cuda())
    rows = _sample_rows(M)
    ref = oracle.quantized_gemm(a.numpy()[rows], b.numpy(), bias.numpy(), residual.numpy()[rows], scale.numpy(),
                                threads)
    got = host(out)[rows]
    # the reference's own gate is IntegerTolerance(max_abs=2) (contraction.py:183-186)
    assert np.max(np.abs(got.astype(np.int32) - ref.astype(np.int32))) <= 2
    assert np.mean(got == ref) >= 0.99


@pytest.mark.parametrize("res_pad,out_pad", [(3, 5), (8, 8), (0, 0)])
def test_quantized_gemm_kn_strided(gpu, threads, res_pad, out_pad):
    """intent_quantized_gemm_kn (b [K, N] in place, int8 epilogue staged through LDS) with
    residual and output row strides that break the 16-/8-byte paths (odd pads) or keep
    them, over several row and column tiles with a partial last column tile; every sampled
    row against the oracle, padding columns untouched."""
    from intent_amd import _native
    M, K, N = 1000, 512, 520
    g = torch.Generator().manual_seed(N + res_pad)
    a = torch.randn((M, K), generator=g).half() / (K ** 0.5)
    b = torch.randn((K, N), generator=g).half()
    bias = torch.randn((N,), generator=g) * 0.25
    residual = (torch.randn((M, N), generator=g) * 0.25).half()
    scale = torch.linspace(1.0 / 48.0, 1.0 / 24.0, N)
    rfull = torch.zeros((M, N + res_pad), dtype=torch.float16)
    rfull[:, :N] = residual
    ofull = torch.full((M, N + out_pad), 77, dtype=torch.int8)
    ad, bd, biasd, rd, sd, od = a.cuda(), b.cuda(), bias.cuda(), rfull.cuda(), scale.cuda(), ofull.cuda()
    _native.call("intent_quantized_gemm_kn", ad.data_ptr(), M, K, K, bd.data_ptr(), N, N, biasd.data_ptr(),
                 rd.data_ptr(), N + res_pad, sd.data_ptr(), od.data_ptr(), N + out_pad, 0)
    torch.cuda.synchronize()
    got_full = host(od)
    assert np.all(got_full[:, N:] == 77)
    rows = _sample_rows(M)
    ref = oracle.quantized_gemm(a.numpy()[rows], b.numpy(), bias.numpy(), residual.numpy()[rows], scale.numpy(),
                                threads)
    got = got_full[rows, :N]
    assert np.max(np.abs(got.astype(np.int32) - ref.astype(np.int32))) <= 2
    assert np.mean(got == ref) >= 0.99


@pytest.mark.parametrize("M,K,N", [(100, 192, 77), (129, 640, 257), (4000, 192, 4100),
                                   (300, 1024, 4096), (257, 384, 144), (64, 128, 16)])
def test_gemm_i8_reference_layout(gpu, threads, M, K, N):
    # gemm.py:29-39 with b as [K, N], exact int32 against the oracle
    rng = np.random.default_rng(M + K)
    a = rng.integers(-128, 128, (M, K), dtype=np.int8)
    b = rng.integers(-128, 128, (K, N), dtype=np.int8)
    bias = rng.integers(-2**31, 2**31 - 1, N, dtype=np.int64).astype(np.int32)
    c = art(intent.gemm_i8).run(dev(a), dev(b), dev(bias))
    rows = _sample_rows(M)
    assert np.array_equal(host(c)[rows], oracle.i8_gemm_i32(a[rows], np.ascontiguousarray(b.T), bias, threads))


@pytest.mark.parametrize("M,K,N,ldb", [(512, 2048, 1024, 1024), (257, 384, 144, 176)])
def test_gemm_i8_kn_in_place_whole_matrix(gpu, M, K, N, ldb):
    """The in-place [K, N] entry against the [N, K] entry on the transposed operand,
    every element (both exact int32); b with a row stride past N."""
    from intent_amd import _native
    rng = np.random.default_rng(M * K)
    a = rng.integers(-128, 128, (M, K), dtype=np.int8)
    bfull = rng.integers(-128, 128, (K, ldb), dtype=np.int8)
    bias = rng.integers(-2**31, 2**31 - 1, N, dtype=np.int64).astype(np.int32)
    ad, bd, biasd = dev(a), dev(bfull), dev(bias)
    bt = dev(np.ascontiguousarray(bfull[:, :N].T))
    c_kn = torch.full((M, N), 7, dtype=torch.int32, device="cuda")
    c_nt = torch.zeros((M, N), dtype=torch.int32, device="cuda")
    _native.call("intent_i8_gemm_i32_kn", ad.data_ptr(), M, K, K, bd.data_ptr(), N, ldb, biasd.data_ptr(),
                 c_kn.data_ptr(), N, 0)
    _native.call("intent_i8_gemm_i32", ad.data_ptr(), M, K, K, bt.data_ptr(), N, K, biasd.data_ptr(), c_nt.data_ptr(),
                 N, 0)
    torch.cuda.synchronize()
    assert torch.equal(c_kn, c_nt)


# ---- f16 / bf16 grouped GEMMs (ragged, routed) -------------------------------------------

def _bits16(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("N", [300, 296])
def test_ragged_grouped_gemm(gpu, threads, dt, N):
    # N = 296: weights read in place as [G, K, N]; N = 300: the transposed-copy fallback
    tdt = torch.float16 if dt == "f16" else torch.bfloat16
    g = torch.Generator().manual_seed(61)
    R, K = 1000, 256
    offsets = torch.tensor([0, 100, 100, 650, 1000], dtype=torch.int32)  # group 1 is empty
    x = torch.randn(R, K, generator=g).to(tdt)
    w = (torch.randn(4, K, N, generator=g) / 16).to(tdt)
    defn = intent.ragged_grouped_gemm if dt == "f16" else intent.ragged_grouped_gemm_bf16
    y = art(defn).run(x.cuda(), offsets.cuda(), w.cuda())
    assert art(defn).observation.entry == ("intent_grouped_gemm_kn" if N % 8 == 0 else "intent_grouped_gemm")
    ref = oracle.grouped_gemm(_bits16(x), dt == "bf16", offsets.numpy(), _bits16(w), R, threads=threads)
    got = _bits16(y.cpu())
    r64 = torch.from_numpy(ref.view(np.int16)).view(tdt).double().numpy()
    g64 = torch.from_numpy(got.view(np.int16)).view(tdt).double().numpy()
    assert np.max(np.abs(g64 - r64)) <= 1e-2 * np.abs(r64).max()


def test_ragged_grouped_gemm_reference_size(gpu):
    # grouped_gemm.py:6-9: 8192 rows, K = N = 4096, 8 groups (ragged offsets here)
    g = torch.Generator(device="cuda").manual_seed(62)
    R, K, N, G = 8192, 4096, 4096, 8
    cuts = torch.sort(torch.randint(0, R, (G - 1,), device="cuda", generator=g)).values
    offsets = torch.cat([torch.zeros(1, device="cuda"), cuts, torch.full((1,), R, device="cuda")]).int()
    x = torch.randn(R, K, device="cuda", generator=g).half()
    w = (torch.randn(G, K, N, device="cuda", generator=g) / 64).half()
    y = art(intent.ragged_grouped_gemm).run(x, offsets, w)
    ref = torch.empty(R, N, device="cuda")
    o = offsets.tolist()
    for e in range(G):
        ref[o[e]:o[e + 1]] = x[o[e]:o[e + 1]].float() @ w[e].float()
    assert (y.double() - ref.double()).abs().max().item() <= 1e-2 * ref.abs().max().item()


# ---- the reference's f16 MoE expert FFN (moe.py:12-53) ------------------------------------

def _ffn_run(d, y0):
    dv = {k: torch.from_numpy(np.ascontiguousarray(v)).cuda() for k, v in d.items() if k != "y"}
    y = torch.from_numpy(y0.copy()).cuda()
    art(intent.moe_expert_ffn).run(dv["x"], dv["route_offsets"], dv["member_routes"], dv["route_token"],
                                   dv["route_weights"], dv["w1"], dv["w2"], y)
    return host(y)


@pytest.mark.parametrize("T,D,E,k,F,kind", [(64, 256, 4, 2, 384, "random"), (37, 128, 3, 1, 192, "random"),
                                            (16, 128, 8, 2, 128, "reference"), (300, 512, 8, 2, 1024, "random")])
def test_moe_expert_ffn(gpu, threads, T, D, E, k, F, kind):
    d = inputs.moe_ffn_f16(T + D, T=T, D=D, E=E, top_k=k, F=F, kind=kind)
    y0 = np.random.default_rng(T).standard_normal((T, D)).astype(np.float32)
    got = _ffn_run(d, y0)
    ref = oracle.moe_expert_ffn(d["x"], d["route_offsets"], d["member_routes"], d["route_token"], d["route_weights"],
                                d["w1"], d["w2"], y=y0, threads=threads)
    assert_close_rms(got - y0, ref - y0, what=f"moe_expert_ffn {T}x{D}x{F}")
    again = _ffn_run(d, y0)
    assert np.array_equal(got, again), "the combine must be deterministic"


@pytest.mark.parametrize("T,k", [(300, 2), (4096, 2), (8192, 1), (9000, 1), (5000, 2)])
def test_moe_expert_ffn_member_list(gpu, T, k):
    # The combine's per-token member list, read back from the workspace: for each token its
    # members (positions in member_routes) in ascending order. T, R <= 8192 build it in LDS,
    # larger ones in global memory (9000 x 1 and 5000 x 2 routes).
    D, F, E = 64, 64, 4
    d = inputs.moe_routes(T, k, E, "random", T)
    R, NR = len(d["member_routes"]), len(d["route_token"])
    dv = {key: torch.from_numpy(np.ascontiguousarray(v)).cuda() for key, v in d.items()}
    x = torch.zeros(T, D, dtype=torch.float16, device="cuda")
    w1 = torch.zeros(E, D, F, dtype=torch.float16, device="cuda")
    w2 = torch.zeros(E, F, D, dtype=torch.float16, device="cuda")
    y = torch.zeros(T, D, device="cuda")
    lib = _native.library()
    nbytes = int(lib.intent_moe_expert_ffn_workspace_size(T, R, D, F))
    ws = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
    _native.call("intent_moe_expert_ffn", x.data_ptr(), T, D, D, dv["route_offsets"].data_ptr(), E,
                 dv["member_routes"].data_ptr(), R, dv["route_token"].data_ptr(), dv["route_weights"].data_ptr(), NR,
                 w1.data_ptr(), w2.data_ptr(), F, y.data_ptr(), D, ws.data_ptr(), nbytes,
                 torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    r256 = lambda v: (v + 255) // 256 * 256
    o_start = r256(r256(r256(R * F * 2) + R * D * 4) + T * 4)
    o_list = r256(o_start + (T + 1) * 4)
    w = ws.cpu().numpy()
    start = w[o_start:o_start + (T + 1) * 4].view(np.int32)
    lst = w[o_list:o_list + R * 4].view(np.int32)
    offs = d["route_offsets"]
    tok = d["route_token"][d["member_routes"]]
    members = np.arange(offs[0], offs[-1])
    order = members[np.argsort(tok[members], kind="stable")]
    counts = np.bincount(tok[members], minlength=T)
    assert np.array_equal(start, np.r_[0, np.cumsum(counts)])
    assert np.array_equal(lst[:len(order)], order)


@pytest.mark.parametrize("T", [512, 4096])
def test_moe_expert_ffn_reference_size(gpu, threads, T):
    # moe.py:6-10 (T = 4096, D = 4096, F = 14336, E = 8, top-2) and the config-4 token count,
    # routes by support.py:113-130; 8 tokens checked against the oracle
    D, F, E, K = 4096, 14336, 8, 2
    d = inputs.moe_routes(T, K, E, "reference")
    g = torch.Generator(device="cuda").manual_seed(T)
    x = torch.randn(T, D, device="cuda", generator=g).half()
    w1 = (torch.randn(E, D, F, device="cuda", generator=g) / D ** 0.5).half()
    w2 = (torch.randn(E, F, D, device="cuda", generator=g) / F ** 0.5).half()
    y = torch.zeros(T, D, device="cuda")
    dv = {k: torch.from_numpy(v).cuda() for k, v in d.items()}
    art(intent.moe_expert_ffn).run(x, dv["route_offsets"], dv["member_routes"], dv["route_token"],
                                   dv["route_weights"], w1, w2, y)
    toks = np.r_[0:4, T - 4:T]
    ref = oracle.moe_expert_ffn(x.cpu().numpy(), d["route_offsets"], d["member_routes"], d["route_token"],
                                d["route_weights"], w1.cpu().numpy(), w2.cpu().numpy(), tokens=toks,
                                threads=threads)
    assert_close_rms(host(y)[toks], ref[toks], what=f"moe_expert_ffn T={T}")


def test_routed_expert_projection_bf16(gpu, threads):
    g = torch.Generator().manual_seed(63)
    T, TOP_K, E, K, N = 300, 2, 4, 256, 200
    experts = torch.randint(0, E, (T * TOP_K,), generator=g)
    member_routes = torch.sort(experts, stable=True).indices.int()   # routes grouped by expert
    offsets = torch.zeros(E + 1, dtype=torch.int32)
    offsets[1:] = torch.cumsum(torch.bincount(experts, minlength=E), 0).int()
    x = torch.randn(T, K, generator=g).bfloat16()
    w = (torch.randn(E, N, K, generator=g) / 16).bfloat16()
    out = art(intent.routed_expert_projection_bf16).run(x.cuda(), offsets.cuda(), member_routes.cuda(), w.cuda())
    ref = oracle.grouped_gemm(_bits16(x), True, offsets.numpy(), _bits16(w), T * TOP_K, routes=member_routes.numpy(),
                              top_k=TOP_K, threads=threads)
    got = _bits16(out.cpu().view(T * TOP_K, N))
    r64 = torch.from_numpy(ref.view(np.int16)).view(torch.bfloat16).double().numpy()
    g64 = torch.from_numpy(got.view(np.int16)).view(torch.bfloat16).double().numpy()
    assert np.max(np.abs(g64 - r64)) <= 1e-2 * np.abs(r64).max()


# ---- plain float GEMMs (gemm.py) ----------------------------------------------------------

@pytest.mark.parametrize("kind", ["f16", "f16_relu", "bf16"])
@pytest.mark.parametrize("M,K,N,bpad", [(64, 128, 64, 0), (300, 384, 130, 0), (4096, 4096, 4096, 0),
                                        (300, 384, 136, 0), (77, 192, 520, 8), (257, 128, 264, 3)])
def test_float_gemm(gpu, threads, kind, M, K, N, bpad):
    # N % 8 == 0 with aligned rows: b [K, N] feeds the kernel directly (transpose reads in LDS);
    # N = 130 or a row stride of N + 3: the transposed-copy fallback. Rows 0..7 and the last 8
    # against the C oracle, the whole matrix against a float64 product on the GPU.
    tdt = torch.bfloat16 if kind == "bf16" else torch.float16
    g = torch.Generator().manual_seed(M + K + N)
    a = torch.randn(M, K, generator=g).to(tdt) / (K ** 0.5)
    b = torch.randn(K, N, generator=g).to(tdt)
    bdev = torch.zeros(K, N + bpad, dtype=tdt, device="cuda")
    bdev[:, :N] = b.cuda()
    bdev = bdev[:, :N]
    if kind == "bf16":
        art_ = art(intent.bf16_gemm)
    else:
        art_ = art(intent.gemm, ACTIVATION=1 if kind == "f16_relu" else 0)
    c = art_.run(a.cuda(), bdev)
    direct = N % 8 == 0 and bpad % 8 == 0
    assert art_.observation.entry == ("intent_f16_gemm_kn" if direct else "intent_f16_gemm")
    rows = _sample_rows(M)
    ref = oracle.float_gemm(_bits16(a)[rows], _bits16(b), kind == "bf16", kind == "f16_relu", threads)
    r64 = torch.from_numpy(ref.view(np.int16)).view(tdt).double().numpy()
    g64 = torch.from_numpy(_bits16(c.cpu())[rows].view(np.int16)).view(tdt).double().numpy()
    assert np.max(np.abs(g64 - r64)) <= 1e-2 * np.abs(r64).max()
    full = a.cuda().double() @ b.cuda().double()
    if kind == "f16_relu":
        full = full.clamp_min(0.0)
    assert (c.double() - full).abs().max().item() <= 1e-2 * full.abs().max().item()


@pytest.mark.parametrize("epi", [0, 1, 2])
@pytest.mark.parametrize("c_pad", [3, 8])
def test_float_gemm_kn_strided_output(gpu, epi, c_pad):
    """intent_f16_gemm_kn (output staged through LDS, 8 columns per lane) into an output with
    row stride N + 3 (element stores) or N + 8, over several row and column tiles and a
    partial last column tile: every element against a float64 product, padding untouched."""
    from intent_amd import _native
    M, K, N = 600, 256, 520
    tdt = torch.bfloat16 if epi == 2 else torch.float16
    g = torch.Generator().manual_seed(epi * 10 + c_pad)
    a = (torch.randn(M, K, generator=g) / (K ** 0.5)).to(tdt).cuda()
    b = torch.randn(K, N, generator=g).to(tdt).cuda()
    c = torch.full((M, N + c_pad), -5.0, dtype=tdt, device="cuda")
    _native.call("intent_f16_gemm_kn", a.data_ptr(), M, K, K, b.data_ptr(), N, N, epi, c.data_ptr(), N + c_pad, 0)
    torch.cuda.synchronize()
    assert torch.all(c[:, N:] == -5.0)
    full = a.double() @ b.double()
    if epi == 1:
        full = full.clamp_min(0.0)
    assert (c[:, :N].double() - full).abs().max().item() <= 1e-2 * full.abs().max().item()


# ---- NVFP4 quantizer --------------------------------------------------------------------

@pytest.mark.parametrize("M,N,gsv", [(256, 128, 1.25), (300, 80, 1.25), (1, 16, 1.25), (8192, 4096, 1.25),
                                     (256, 128, 300.0)])
def test_nvfp4_quantize_bit_exact(gpu, M, N, gsv):
    # (8192, 4096) is the reference's registry case (experiments/cpu/registry.py:11); gs = 300
    # drives many group scales past E4M3FN's range (NaN scale bytes, zero codes)
    g = torch.Generator().manual_seed(M + N)
    x = (torch.randn(M, N, generator=g) * 3).bfloat16()
    gs = torch.tensor([gsv])
    MT, NT = (M + 127) // 128, (N // 16 + 3) // 4
    packed0 = np.full((M, N // 2), 0xAA, np.uint8)
    scales0 = np.full((MT, NT, 32, 4, 4), 0x55, np.uint8)   # entries no group writes must keep this
    packed, scales = dev(packed0), dev(scales0)
    art(intent.nvfp4_quantize).run(x.cuda(), gs.cuda(), packed, scales)
    rp, rs = oracle.nvfp4_quantize(_bits16(x), gsv, packed0, scales0)
    assert np.array_equal(host(packed), rp)
    assert np.array_equal(host(scales), rs)
    if gsv > 100:
        assert (rs == 0x7f).any()


def test_nvfp4_rejects_wider_scale_blocks(gpu):
    M, N = 256, 128
    x = torch.zeros(M, N, dtype=torch.bfloat16, device="cuda")
    packed = torch.zeros(M, N // 2, dtype=torch.uint8, device="cuda")
    scales = torch.zeros(2, 3, 32, 4, 4, dtype=torch.uint8, device="cuda")   # NT 3 where N needs 2
    with pytest.raises(ValueError):
        art(intent.nvfp4_quantize).run(x, torch.tensor([1.0], device="cuda"), packed, scales)


# ---- empty K -------------------------------------------------------------------------
# A contraction over an empty K is zero-initialised and sums nothing
# (doc/dsl/core.en.md:213, Contractions.cpp:12-41): every entry writes
# epilogue(0) to its whole output - zeros, the bias, the in-place output
# unchanged, or quantized_gemm's epilogue of a zero accumulator. Outputs are
# given as buffers filled with a non-zero pattern so a skipped write shows.

def _filled(shape, dtype, value=7):
    return torch.full(shape, value, dtype=torch.int8 if dtype == torch.int8 else dtype, device="cuda") \
        if dtype not in (torch.float8_e4m3fn, torch.float8_e5m2) else \
        torch.full(shape, 0x38, dtype=torch.uint8, device="cuda").view(dtype)


def _empty(shape, dtype):
    return torch.empty(shape, dtype=dtype, device="cuda")


M0, N0 = 37, 70


def _k0_cases():
    f16, bf16, i8, u8, i32, f32 = torch.float16, torch.bfloat16, torch.int8, torch.uint8, torch.int32, torch.float32
    f8 = torch.float8_e4m3fn
    bias = torch.arange(N0, dtype=i32, device="cuda") - 20
    zeros = lambda shape, dt: torch.zeros(shape, dtype=dt, device="cuda")  # noqa: E731
    cases = {
        "w4a16_gemv": (intent.weight_only_int4_asym_matmul, {"KERNEL": "gemv"},
                       (_empty((4, 0), f16), _empty((N0, 0), u8), _empty((N0, 0), f16), _empty((N0, 0), u8)),
                       (_filled((4, N0), f16),), zeros((4, N0), f16)),
        "w4a16_gemm": (intent.weight_only_int4_asym_matmul, {"KERNEL": "gemm"},
                       (_empty((M0, 0), f16), _empty((N0, 0), u8), _empty((N0, 0), f16), _empty((N0, 0), u8)),
                       (_filled((M0, N0), f16),), zeros((M0, N0), f16)),
        "w8a16": (intent.weight_only_int8_matmul, {},
                  (_empty((M0, 0), f16), _empty((N0, 0), i8), torch.ones(N0, dtype=f16, device="cuda")),
                  (_filled((M0, N0), f16),), zeros((M0, N0), f16)),
        "w8a8": (intent.w8a8_scaled_matmul, {},
                 (_empty((M0, 0), i8), torch.ones(M0, dtype=f32, device="cuda"), _empty((N0, 0), i8),
                  torch.ones(N0, dtype=f32, device="cuda")),
                 (_filled((M0, N0), bf16),), zeros((M0, N0), bf16)),
        "gemm_i8_nt": (intent.gemm_i8_nt, {}, (_empty((M0, 0), i8), _empty((N0, 0), i8), bias),
                       (_filled((M0, N0), i32),), bias[None, :].expand(M0, N0)),
        "gemm_i8": (intent.gemm_i8, {}, (_empty((M0, 0), i8), _empty((0, N0), i8), bias),
                    (_filled((M0, N0), i32),), bias[None, :].expand(M0, N0)),
        "w4a8": (intent.w4a8_packed_matmul, {}, (_empty((M0, 0), i8), _empty((N0, 0), u8)),
                 (_filled((N0, M0), i32),), zeros((N0, M0), i32)),
        "bitnet": (intent.bitnet_int2_matmul, {}, (_empty((M0, 0), i8), _empty((N0, 0), u8)),
                   (_filled((M0, N0), i32),), zeros((M0, N0), i32)),
        "block_scaled": (intent.block_scaled_matmul, {},
                         (_empty((M0, 0, 32), f8), _empty((M0, 0), u8), _empty((0, 32, N0), f8), _empty((0, N0), u8)),
                         (_filled((M0, N0), f32),), zeros((M0, N0), f32)),
        "scaled_fp8": (intent.scaled_fp8_matmul, {}, (_empty((M0, 0), f8), _empty((0, N0), f8), 0.5, 2.0),
                       (_filled((M0, N0), f16),), zeros((M0, N0), f16)),
        "deepgemm_fp8": (intent.deepgemm_fp8_2xacc, {},
                         (_empty((M0, 0, 128), f8), _empty((N0, 0, 128), f8), _empty((M0, 0), f32),
                          _empty(((N0 + 127) // 128, 0), f32)),
                         (_filled((M0, N0), bf16),), zeros((M0, N0), bf16)),
        "fp8_e4m3": (intent.fp8_e4m3_matmul, {}, (_empty((M0, 0), f8), _empty((N0, 0), f8)),
                     (_filled((M0, N0), f8),), zeros((M0, N0), f8)),
        "fp4_bf16": (intent.dequant_bf16_fp4_matmul, {}, (_empty((M0, 0), bf16), _empty((N0, 0), u8)),
                     (_filled((M0, N0), bf16),), zeros((M0, N0), bf16)),
        "w4_sym": (intent.weight_only_int4_matmul, {}, (_empty((M0, 0), f16), _empty((0, N0), i32),
                                                        _empty((0, N0), f16)),
                   (_filled((M0, N0), f16),), zeros((M0, N0), f16)),
        "gemm": (intent.gemm, {}, (_empty((M0, 0), f16), _empty((0, N0), f16)), (_filled((M0, N0), f16),),
                 zeros((M0, N0), f16)),
        "bf16_gemm": (intent.bf16_gemm, {}, (_empty((M0, 0), bf16), _empty((0, N0), bf16)),
                      (_filled((M0, N0), bf16),), zeros((M0, N0), bf16)),
        "ragged_grouped": (intent.ragged_grouped_gemm, {},
                           (_empty((M0, 0), f16), torch.tensor([0, 10, 10, M0], dtype=i32, device="cuda"),
                            _empty((3, 0, N0), f16)),
                           (_filled((M0, N0), f16),), zeros((M0, N0), f16)),
    }
    return cases


@pytest.mark.parametrize("name", ["w4a16_gemv", "w4a16_gemm", "w8a16", "w8a8", "gemm_i8_nt", "gemm_i8", "w4a8",
                                  "bitnet", "block_scaled", "scaled_fp8", "deepgemm_fp8", "fp8_e4m3", "fp4_bf16",
                                  "w4_sym", "gemm", "bf16_gemm", "ragged_grouped"])
def test_empty_k(gpu, name):
    defn, cx, ins, outs, expected = _k0_cases()[name]
    art(defn, **cx).prepare(*ins, outputs=outs).launch()
    got = outs[0]
    torch.cuda.synchronize()
    if got.dtype in (torch.float8_e4m3fn, torch.float8_e5m2):
        assert torch.equal(got.view(torch.uint8), expected.view(torch.uint8)), name
    else:
        assert torch.equal(got, expected), name


def test_empty_k_quantized_gemm(gpu, threads):
    # epilogue(0) = trunc(clamp((relu(0 + bias) + residual) / scale)), not zero
    M, N = 9, 40
    g = torch.Generator().manual_seed(3)
    bias = torch.randn((N,), generator=g) * 4
    residual = (torch.randn((M, N), generator=g) * 4).half()
    scale = torch.linspace(1.0 / 48.0, 1.0 / 24.0, N)
    a, b = np.zeros((M, 0), np.float16), np.zeros((0, N), np.float16)
    out = torch.full((M, N), 99, dtype=torch.int8, device="cuda")
    art(intent.quantized_gemm).prepare(dev(a), dev(b), bias.cuda(), residual.cuda(), scale.cuda(),
                                       outputs=(out,)).launch()
    ref = oracle.quantized_gemm(a, b, bias.numpy(), residual.numpy(), scale.numpy(), threads)
    assert np.array_equal(host(out), ref)


def test_empty_k_more(gpu):
    # split-K FP8 with no iterations: out = f16(out + p) per split with p = +0, so the
    # output is unchanged except that -0 becomes +0
    M, N, SP = 6, 40, 3
    out0 = (torch.randn(M, N, generator=torch.Generator().manual_seed(1)) * 8).half()
    out0[0, 0] = -0.0
    out = out0.cuda()
    f8 = torch.float8_e4m3fn
    art(intent.scaled_fp8_splitk_matmul).run(_empty((M, 0, SP, 256), f8), _empty((0, SP, 256, N), f8), out, 0.5, 2.0)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu().view(torch.int16), (out0 + 0.0).view(torch.int16))
    # a non-finite scale makes p = f16(0 * inf) = NaN, which the sum carries
    out = out0.cuda()
    art(intent.scaled_fp8_splitk_matmul).run(_empty((M, 0, SP, 256), f8), _empty((0, SP, 256, N), f8), out,
                                             float("inf"), 2.0)
    assert torch.isnan(out).all()
    # routed bf16 projection over K = 0: every routed row is zero
    T, TOP_K, E, Nr = 20, 2, 3, 24
    experts = torch.arange(T * TOP_K) % E
    member = torch.sort(experts, stable=True).indices.int().cuda()
    offs = torch.zeros(E + 1, dtype=torch.int32)
    offs[1:] = torch.cumsum(torch.bincount(experts, minlength=E), 0).int()
    y = torch.full((T, TOP_K, Nr), 3.0, dtype=torch.bfloat16, device="cuda")
    art(intent.routed_expert_projection_bf16).prepare(_empty((T, 0), torch.bfloat16), offs.cuda(), member,
                                                      _empty((E, Nr, 0), torch.bfloat16), outputs=(y,)).launch()
    torch.cuda.synchronize()
    assert torch.equal(y, torch.zeros_like(y))
    # Q4_K x Q8_K over zero blocks: +0 per row
    w = _empty((9, 0, 144), torch.uint8)
    q = _empty((0, 292), torch.uint8)
    r = torch.full((9,), 5.0, device="cuda")
    art(intent.q4_k_q8_k_dot).prepare(w, q, outputs=(r,)).launch()
    torch.cuda.synchronize()
    assert torch.equal(r, torch.zeros_like(r))
