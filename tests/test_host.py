"""Host-side logic of the operator surface, on CPU: public interface schema,
compile() stage errors, binder checks, output inference, torch op schema,
input generators and the bench's single-GPU guard."""
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

import intent_amd as intent
import oracle
from intent_amd import inputs
from intent_amd.artifact import CompiledArtifact
from intent_amd.interface import ViewKind
from intent_amd.runtime import HIPRuntime

ROOT = Path(__file__).resolve().parent.parent


def runtime_for(defn, **constexprs):
    return HIPRuntime(defn, 0, defn.resolve_constexprs(constexprs or None), "gfx950")


def test_interface_schema():
    iface = intent.weight_only_int4_asym_matmul.interface()
    names = [p.name for p in iface.parameters]
    assert names == ["activation", "packed_weight", "scales", "zeros", "output"]
    act, packed, scales, zeros, out = iface.parameters
    assert act.dimensions[0] == out.dimensions[0]  # M shared
    assert packed.dimensions[0] == scales.dimensions[0] == out.dimensions[1]  # N shared
    assert out.access is ViewKind.OUT and [p.name for p in iface.outputs] == ["output"]
    assert act.strides == (None, 1)
    ffn = intent.moe_expert_ffn_w4.interface()
    assert [p.name for p in ffn.mutable_inputs] == ["y"] and not ffn.outputs
    assert len(ffn.inputs) == 9


def test_explicit_arguments_order():
    iface = intent.moe_align_block_size.interface()
    merged = iface.explicit_arguments(("ids",), ("s", "b", "o", "t"))
    assert merged == ("ids", "s", "b", "o", "t")
    with pytest.raises(TypeError):
        iface.explicit_arguments((), ("s", "b", "o", "t"))


def test_compile_stage_errors():
    with pytest.raises(intent.CompilationStageError) as info:
        intent.compile(object(), target=intent.MI355XTarget())
    assert info.value.stage == "frontend_kir"
    with pytest.raises(intent.CompilationStageError) as info:
        intent.compile(intent.moe_route_topk, target=intent.MI355XTarget(), constexprs={"NOPE": 1})
    assert info.value.stage == "frontend_kir"
    with pytest.raises(intent.CompilationStageError) as info:
        intent.compile(intent.moe_align_block_size, target=intent.MI355XTarget())  # EXPERTS required
    assert info.value.stage == "frontend_kir"
    if not torch.cuda.is_available():
        with pytest.raises(intent.CompilationStageError) as info:
            intent.compile(intent.weight_only_int4_asym_matmul, target=intent.MI355XTarget())
        assert info.value.stage == "target_resolution"


def test_definitions_are_not_callable_and_kernel_decorator():
    with pytest.raises(intent.LanguageUseError):
        intent.weight_only_int8_matmul(1, 2, 3)
    with pytest.raises(NotImplementedError):
        intent.kernel(lambda: None)


def test_binder_shapes_and_dtypes():
    rt = runtime_for(intent.weight_only_int4_asym_matmul)
    x = torch.zeros(3, 256, dtype=torch.float16)
    q = torch.zeros(40, 128, dtype=torch.uint8)
    s = torch.zeros(40, 2, dtype=torch.float16)
    z = torch.zeros(40, 2, dtype=torch.uint8)
    y = rt.infer_outputs((x, q, s, z))
    assert y.shape == (3, 40) and y.dtype == torch.float16
    with pytest.raises(TypeError, match="dtype"):
        rt.infer_outputs((x.float(), q, s, z))
    with pytest.raises(ValueError, match="K/2"):
        rt.infer_outputs((x, q[:, :100], s, z))
    with pytest.raises(ValueError, match="relation"):
        rt.infer_outputs((x, q, s[:30], z))
    with pytest.raises(TypeError, match="input arguments"):
        rt.infer_outputs((x, q, s))
    # concrete binding checks the device
    with pytest.raises(ValueError, match="bound to cuda:0"):
        rt.run(x, q, s, z)


def test_binder_derived_output_shapes():
    rt = runtime_for(intent.moe_align_block_size, EXPERTS=8, BLOCK_SIZE=128)
    outs = rt.infer_outputs((torch.zeros(512, 2, dtype=torch.int32),))
    assert [tuple(o.shape) for o in outs] == [(1024 + 8 * 127,), (16,), (9,), (1,)]
    rt = runtime_for(intent.moe_route_topk, TOP_K=3)
    ids, w = rt.infer_outputs((torch.zeros(7, 8),))
    assert ids.shape == (7, 3) and ids.dtype == torch.int32 and w.dtype == torch.float32


def test_ffn_check_relations():
    rt = runtime_for(intent.moe_expert_ffn_w4)
    T, H, E, F = 4, 256, 2, 128
    args = [torch.zeros(T, E), torch.zeros(T, H, dtype=torch.float16),
            torch.zeros(E, 2 * F, H // 2, dtype=torch.uint8), torch.zeros(E, 2 * F, 2, dtype=torch.float16),
            torch.zeros(E, 2 * F, 2, dtype=torch.uint8), torch.zeros(E, H, F // 2, dtype=torch.uint8),
            torch.zeros(E, H, 1, dtype=torch.float16), torch.zeros(E, H, 1, dtype=torch.uint8),
            torch.zeros(T, H)]
    assert rt.infer_outputs(tuple(args)) is None
    bad = list(args)
    bad[6] = torch.zeros(E, H, 2, dtype=torch.float16)
    bad[7] = torch.zeros(E, H, 2, dtype=torch.uint8)
    with pytest.raises(ValueError, match="group size"):
        rt.infer_outputs(tuple(bad))


def test_torch_op_schema():
    rt = runtime_for(intent.moe_combine)
    art = CompiledArtifact("", "", 0, rt)
    op = art.as_torch_op("intent_amd_cpu_test::combine")
    schema = str(op._opoverload._schema)
    assert "(Tensor route_out, Tensor topk_weights, Tensor(a2!) y) -> ()" in schema
    rt4 = runtime_for(intent.weight_only_int4_asym_matmul)
    op4 = CompiledArtifact("", "", 0, rt4).as_torch_op("intent_amd_cpu_test::w4")
    assert str(op4._opoverload._schema).endswith("-> Tensor")
    with pytest.raises(ValueError):
        CompiledArtifact("", "", 0, rt4).as_torch_op("bad name")
    # the fake kernel infers outputs from shapes alone
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        y = op4(torch.empty(3, 256, dtype=torch.float16), torch.empty(8, 128, dtype=torch.uint8),
                torch.empty(8, 2, dtype=torch.float16), torch.empty(8, 2, dtype=torch.uint8))
    assert tuple(y.shape) == (3, 8) and y.dtype == torch.float16
    # an in-place view may not share storage with another input
    with FakeTensorMode(), pytest.raises(NotImplementedError, match="shares storage"):
        ro = torch.zeros(8, 16)
        op(ro, torch.zeros(4, 2), ro[:4])


def test_compile_options():
    o = intent.CompileOptions()
    assert (o.numerics, o.online_reduction, o.optimization_remarks) == ("source", True, False)
    assert o == intent.CompileOptions("source", True, False) and hash(o) == hash(intent.CompileOptions())
    with pytest.raises(ValueError):
        intent.CompileOptions(numerics="fast")
    with pytest.raises(TypeError):
        intent.CompileOptions(online_reduction=1)
    with pytest.raises(AttributeError):
        o.numerics = "relaxed_normalization"


def test_inputs_generators():
    d = inputs.config1_w4a16_decode(0, M=2, K=256, N=8)
    assert d["x"].dtype == np.float16 and d["packed"].shape == (8, 128)
    assert d["scales"].shape == (8, 2) and d["zeros"].max() <= 15
    again = inputs.config1_w4a16_decode(0, M=2, K=256, N=8)
    assert all(np.array_equal(d[k], again[k]) for k in d)
    nib = np.random.default_rng(0).integers(0, 16, (3, 64), dtype=np.uint8)
    assert np.array_equal(oracle.unpack_nibbles(inputs.pack_nibbles(nib)), nib)
    w = inputs.w4a16_work(1, 4096, 4096)
    assert w.bytes == 8_798_208 and w.flops == 33_554_432
    assert inputs.w8a8_work(4096, 8192, 8192).flops == 549_755_813_888


def test_bench_refuses_multi_gpu():
    proc = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                          timeout=120)
    assert proc.returncode == 2 and "exactly one GPU" in proc.stdout
