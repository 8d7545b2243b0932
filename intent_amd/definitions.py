"""Fixed kernel definitions of the quantized-contraction hot path.

Each definition plays the role of an ``@intent.kernel`` function of the
reference (python/intent/api/definitions.py:76): an author-ordered parameter
list with In / Out / InOut views over symbolic extents. Instead of being
lowered by a compiler, each one is bound to a hand-written gfx950 entry of
``libintent_amd.so``. Reference kernels each definition replaces are cited on
the definition.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Callable

from . import _native
from .errors import LanguageUseError
from .interface import PublicInterface, ScalarParameter, ViewKind, ViewParameter, dtype

IN, OUT, INOUT = ViewKind.IN, ViewKind.OUT, ViewKind.INOUT

Dim = Any  # str symbol | int | Callable[[dict], int]


@dataclass(frozen=True)
class Param:
    name: str
    dtype: str
    dims: tuple
    access: ViewKind = IN
    leading_stride: bool = False  # 2-D views may carry a leading stride; others must be contiguous
    free_strides: bool = False    # any strides; the definition's launch adapts the layout


@dataclass(frozen=True)
class Scalar:
    name: str
    dtype: str


@dataclass
class KernelDefinition:
    name: str
    params: tuple
    launch: Callable[..., str]
    constexprs: dict = field(default_factory=dict)
    check: Callable[[dict], None] | None = None
    workspace: Callable[[dict], int] | None = None
    reference: str = ""
    doc: str = ""

    @property
    def __name__(self) -> str:  # the reference uses definition.__name__ as the entry name
        return self.name

    def __call__(self, *args, **kwargs):
        raise LanguageUseError(f"kernel {self.name} must be compiled before runtime invocation")

    def __repr__(self) -> str:
        return f"<intent_amd kernel {self.name}>"

    def resolve_constexprs(self, overrides: dict | None) -> dict:
        values = dict(self.constexprs)
        for key, value in (overrides or {}).items():
            if key not in values:
                raise ValueError(f"{self.name} has no constexpr {key!r}; known: {sorted(values)}")
            values[key] = value
        missing = [k for k, v in values.items() if v is None]
        if missing:
            raise ValueError(f"{self.name} requires constexprs {missing}")
        return values

    def interface(self) -> PublicInterface:
        identities: dict[str, int] = {}
        parameters = []
        for position, p in enumerate(self.params):
            if isinstance(p, Scalar):
                parameters.append(ScalarParameter(position, p.name, dtype(p.dtype)))
                continue
            shape, dims = [], []
            for d in p.dims:
                if isinstance(d, int):
                    shape.append(d)
                    dims.append(0)
                elif isinstance(d, str):
                    shape.append(-1)
                    dims.append(identities.setdefault(d, len(identities) + 1))
                else:
                    shape.append(-1)
                    dims.append(0)
            rank = len(p.dims)
            strides = (None,) * rank if p.free_strides else tuple([None] * (rank - 1) + [1]) if p.leading_stride else tuple(
                None if i < rank - 1 else 1 for i in range(rank))
            parameters.append(ViewParameter(position, p.name, dtype(p.dtype), tuple(shape), tuple(dims), strides,
                                            p.access))
        return PublicInterface(tuple(parameters))


def _ptr(t) -> int:
    return t.data_ptr()


def _ld(t) -> int:
    return t.stride(0) if t.dim() >= 2 else t.shape[0]


# ---- W4A16 ------------------------------------------------------------------------

def _w4_check(env: dict) -> None:
    if env["P"] * 2 != env["K"]:
        raise ValueError(f"packed_weight.shape[1] ({env['P']}) must be K/2 ({env['K']}/2)")
    if env["K"] == 0 and env["G"] == 0:  # empty K: no groups, y = 0
        env["GROUP"] = 128
    elif env["G"] <= 0 or env["K"] % env["G"]:
        raise ValueError(f"K ({env['K']}) must be a multiple of the number of groups ({env['G']})")
    else:
        env["GROUP"] = env["K"] // env["G"]
    if env["KERNEL"] not in ("auto", "gemv", "gemm"):
        raise ValueError("KERNEL must be 'auto', 'gemv' or 'gemm'")


def _w4_launch(v: dict, env: dict, stream: int, workspace) -> str:
    x, q, s, z, y = v["activation"], v["packed_weight"], v["scales"], v["zeros"], v["output"]
    if s.stride(0) != z.stride(0):
        raise ValueError("scales and zeros must share a row stride")
    kernel = env["KERNEL"]
    if kernel == "auto":
        kernel = "gemv" if env["M"] <= 16 else "gemm"
    entry = {"gemv": "intent_w4a16_gemv", "gemm": "intent_w4a16_gemm"}[kernel]
    _native.call(entry, _ptr(x), env["M"], env["K"], _ld(x), _ptr(q), env["N"], _ld(q), _ptr(s), _ptr(z),
                 s.stride(0), env["GROUP"], _ptr(y), _ld(y), stream)
    return entry


weight_only_int4_asym_matmul = KernelDefinition(
    name="weight_only_int4_asym_matmul",
    params=(
        Param("activation", "f16", ("M", "K"), leading_stride=True),
        Param("packed_weight", "u8", ("N", "P"), leading_stride=True),
        Param("scales", "f16", ("N", "G"), leading_stride=True),
        Param("zeros", "u8", ("N", "G"), leading_stride=True),
        Param("output", "f16", ("M", "N"), OUT, leading_stride=True),
    ),
    launch=_w4_launch,
    constexprs={"KERNEL": "auto"},
    check=_w4_check,
    reference="examples/kernels/contraction/weight_only_int4.py:18-51",
    doc="y = f16(x @ ((q - z) * s).T), asymmetric uint4 group quant, packed [N, K/2]",
)


# ---- W8A16 ------------------------------------------------------------------------

def _w8a16_launch(v: dict, env: dict, stream: int, workspace) -> str:
    x, w, s, y = v["activation"], v["weight"], v["scales"], v["output"]
    _native.call("intent_w8a16_matmul", _ptr(x), env["M"], env["K"], _ld(x), _ptr(w), env["N"], _ld(w), _ptr(s),
                 _ptr(y), _ld(y), stream)
    return "intent_w8a16_matmul"


weight_only_int8_matmul = KernelDefinition(
    name="weight_only_int8_matmul",
    params=(
        Param("activation", "f16", ("M", "K"), leading_stride=True),
        Param("weight", "i8", ("N", "K"), leading_stride=True),
        Param("scales", "f16", ("N",)),
        Param("output", "f16", ("M", "N"), OUT, leading_stride=True),
    ),
    launch=_w8a16_launch,
    reference="doc/dsl/core.en.md:246 (I.cast(W_i8, f16) -> I.matmul(acc f32) -> scale)",
    doc="y = f16(scale[n] * (x @ w.T)), per-channel int8 weights",
)


# ---- W8A8 -------------------------------------------------------------------------

def _w8a8_launch(v: dict, env: dict, stream: int, workspace) -> str:
    a, sa, w, sw, out = v["activation"], v["activation_scales"], v["weight"], v["weight_scales"], v["output"]
    _native.call("intent_w8a8_gemm", _ptr(a), env["M"], env["K"], _ld(a), _ptr(sa), _ptr(w), env["N"], _ld(w),
                 _ptr(sw), _ptr(out), _ld(out), stream)
    return "intent_w8a8_gemm"


w8a8_scaled_matmul = KernelDefinition(
    name="w8a8_scaled_matmul",
    params=(
        Param("activation", "i8", ("M", "K"), leading_stride=True),
        Param("activation_scales", "f32", ("M",)),
        Param("weight", "i8", ("N", "K"), leading_stride=True),
        Param("weight_scales", "f32", ("N",)),
        Param("output", "bf16", ("M", "N"), OUT, leading_stride=True),
    ),
    launch=_w8a8_launch,
    reference="lib/Conversion/KIRToCPU/Contractions.cpp:30-35 + examples/kernels/contraction/gemm.py:83-106",
    doc="out = bf16(f32(int32 acc) * sa[m] * sw[n])",
)


def _gemm_i8_launch(v: dict, env: dict, stream: int, workspace) -> str:
    a, b, bias, c = v["a"], v["b"], v["bias"], v["c"]
    _native.call("intent_i8_gemm_i32", _ptr(a), env["M"], env["K"], _ld(a), _ptr(b), env["N"], _ld(b), _ptr(bias),
                 _ptr(c), _ld(c), stream)
    return "intent_i8_gemm_i32"


gemm_i8_nt = KernelDefinition(
    name="gemm_i8_nt",
    params=(
        Param("a", "i8", ("M", "K"), leading_stride=True),
        Param("b", "i8", ("N", "K"), leading_stride=True),
        Param("bias", "i32", ("N",)),
        Param("c", "i32", ("M", "N"), OUT, leading_stride=True),
    ),
    launch=_gemm_i8_launch,
    reference="examples/kernels/contraction/gemm.py:29-39 (gemm_i8, weight given as [N, K])",
    doc="c = a @ b.T + bias in int32 (modulo 2^32)",
)


def _gemm_i8_kn_direct(env: dict, a, b) -> bool:
    """b [K, N] feeds the kernel in place when K is a positive multiple of 128, N and
    both row strides multiples of 16 bytes, and both operands 16-byte aligned."""
    return (env["K"] > 0 and env["K"] % 128 == 0 and env["N"] % 16 == 0 and a.stride(0) % 16 == 0
            and b.stride(0) % 16 == 0 and a.data_ptr() % 16 == 0 and b.data_ptr() % 16 == 0)


def _gemm_i8_kn_workspace(env: dict) -> int:
    # the transposed copy of b is needed only off the in-place shapes
    if env["K"] > 0 and env["K"] % 128 == 0 and env["N"] % 16 == 0:
        return 0
    return env["N"] * (-(-env["K"] // 16) * 16)


def _gemm_i8_kn_launch(v: dict, env: dict, stream: int, workspace) -> str:
    a, b, bias, c = v["a"], v["b"], v["bias"], v["c"]
    M, K, N = env["M"], env["K"], env["N"]
    if _gemm_i8_kn_direct(env, a, b):
        _native.call("intent_i8_gemm_i32_kn", _ptr(a), M, K, _ld(a), _ptr(b), N, b.stride(0), _ptr(bias), _ptr(c),
                     _ld(c), stream)
        return "intent_i8_gemm_i32_kn"
    Kp = -(-K // 16) * 16
    if workspace is None or workspace.numel() < N * Kp:
        import torch

        workspace = torch.empty(N * Kp, dtype=torch.uint8, device=b.device)
        workspace.record_stream(torch.cuda.ExternalStream(stream, device=b.device))
    bt = workspace.data_ptr()  # b [K, N] -> [N, K] rows
    _native.call("intent_fp8_transpose", _ptr(b), K, N, b.stride(0), bt, Kp, stream)
    _native.call("intent_i8_gemm_i32", _ptr(a), M, K, _ld(a), bt, N, -(-K // 16) * 16, _ptr(bias), _ptr(c), _ld(c),
                 stream)
    return "intent_i8_gemm_i32"


gemm_i8 = KernelDefinition(
    name="gemm_i8",
    params=(
        Param("a", "i8", ("M", "K"), leading_stride=True),
        Param("b", "i8", ("K", "N"), leading_stride=True),
        Param("bias", "i32", ("N",)),
        Param("c", "i32", ("M", "N"), OUT, leading_stride=True),
    ),
    launch=_gemm_i8_kn_launch,
    workspace=_gemm_i8_kn_workspace,
    reference="examples/kernels/contraction/gemm.py:29-39",
    doc="c = a @ b + bias in int32 (modulo 2^32); b [K, N] read in place (K % 128 == 0, N % 16 == 0), "
        "else transposed into the workspace first",
)


# ---- MoE --------------------------------------------------------------------------

def _route_launch(v: dict, env: dict, stream: int, workspace) -> str:
    _native.call("intent_moe_route", _ptr(v["logits"]), env["T"], env["E"], env["TOP_K"], int(bool(env["RENORMALIZE"])),
                 _ptr(v["topk_ids"]), _ptr(v["topk_weights"]), stream)
    return "intent_moe_route"


moe_route_topk = KernelDefinition(
    name="moe_route_topk",
    params=(
        Param("logits", "f32", ("T", "E")),
        Param("topk_ids", "i32", ("T", lambda env: env["TOP_K"]), OUT),
        Param("topk_weights", "f32", ("T", lambda env: env["TOP_K"]), OUT),
    ),
    launch=_route_launch,
    constexprs={"TOP_K": 2, "RENORMALIZE": True},
    reference="experiments/_common/support.py:113-130 (the producer of topk_ids)",
    doc="top-k experts by logit (ties -> lower index) and their softmax weights",
)


def align_sizes(routes: int, experts: int, block: int) -> tuple[int, int]:
    capacity = routes + experts * (block - 1)
    return capacity, (capacity + block - 1) // block


def _align_launch(v: dict, env: dict, stream: int, workspace) -> str:
    cap, nb = align_sizes(env["T"] * env["K"], env["EXPERTS"], env["BLOCK_SIZE"])
    _native.call("intent_moe_align", _ptr(v["topk_ids"]), env["T"], env["K"], env["EXPERTS"], env["BLOCK_SIZE"],
                 _ptr(v["sorted_route_ids"]), cap, _ptr(v["expert_blocks"]), nb, _ptr(v["expert_offsets"]),
                 _ptr(v["total_padded"]), stream)
    return "intent_moe_align"


moe_align_block_size = KernelDefinition(
    name="moe_align_block_size",
    params=(
        Param("topk_ids", "i32", ("T", "K")),
        Param("sorted_route_ids", "i32",
              (lambda env: align_sizes(env["T"] * env["K"], env["EXPERTS"], env["BLOCK_SIZE"])[0],), OUT),
        Param("expert_blocks", "i32",
              (lambda env: align_sizes(env["T"] * env["K"], env["EXPERTS"], env["BLOCK_SIZE"])[1],), OUT),
        Param("expert_offsets", "i32", (lambda env: env["EXPERTS"] + 1,), OUT),
        Param("total_padded", "i32", (1,), OUT),
    ),
    launch=_align_launch,
    constexprs={"EXPERTS": None, "BLOCK_SIZE": 128},
    reference="examples/kernels/routing/moe_align.py:14-86 + examples/programs/composition.py:134-174",
    doc="count / block-padded prefix / stable scatter / block->expert map",
)


def _ffn_check(env: dict) -> None:
    H, F2 = env["H"], env["F2"]
    if env["HP"] * 2 != H:
        raise ValueError("w_gate_up.shape[2] must be H/2")
    if F2 % 2:
        raise ValueError("w_gate_up.shape[1] must be 2*F")
    F = F2 // 2
    env["F"] = F
    if env["FP"] * 2 != F:
        raise ValueError("w_down.shape[2] must be F/2")
    if H % env["G1"] or F % env["G2"] or H // env["G1"] != F // env["G2"]:
        raise ValueError("gate/up and down weights must share one group size")
    env["GROUP"] = H // env["G1"]
    if env["TOP_K"] > env["E"]:
        raise ValueError("TOP_K exceeds the number of experts")


def _ffn_workspace(env: dict) -> int:
    lib = _native.library()
    return int(lib.intent_moe_workspace_size(env["T"], env["TOP_K"], env["E"], env["H"], env["F"], 0))


def _ffn_launch(v: dict, env: dict, stream: int, workspace) -> str:
    _native.call("intent_moe_expert_ffn_w4", _ptr(v["router_logits"]), _ptr(v["x"]), env["T"], env["H"], env["E"],
                 env["TOP_K"], int(bool(env["RENORMALIZE"])), _ptr(v["w_gate_up"]), _ptr(v["gate_up_scales"]),
                 _ptr(v["gate_up_zeros"]), _ptr(v["w_down"]), _ptr(v["down_scales"]), _ptr(v["down_zeros"]),
                 env["F"], env["GROUP"], _ptr(v["y"]), workspace.data_ptr(), workspace.numel(), None, None, stream)
    return "intent_moe_expert_ffn_w4"


moe_expert_ffn_w4 = KernelDefinition(
    name="moe_expert_ffn_w4",
    params=(
        Param("router_logits", "f32", ("T", "E")),
        Param("x", "f16", ("T", "H")),
        Param("w_gate_up", "u8", ("E", "F2", "HP")),
        Param("gate_up_scales", "f16", ("E", "F2", "G1")),
        Param("gate_up_zeros", "u8", ("E", "F2", "G1")),
        Param("w_down", "u8", ("E", "H", "FP")),
        Param("down_scales", "f16", ("E", "H", "G2")),
        Param("down_zeros", "u8", ("E", "H", "G2")),
        Param("y", "f32", ("T", "H"), INOUT),
    ),
    launch=_ffn_launch,
    constexprs={"TOP_K": 2, "RENORMALIZE": True},
    check=_ffn_check,
    workspace=_ffn_workspace,
    reference="examples/kernels/ragged/moe.py:12-53 (+ routing/moe_align.py, programs/composition.py:134-174)",
    doc="y += sum_slots w * (silu(x Wg) * (x Wu)) Wd over the top-k experts, W4 experts",
)


# ---- the reference's f16 MoE expert FFN (moe.py:12-53) -----------------------------

def _f16ffn_check(env: dict) -> None:
    if env["E_PLUS_1"] != env["E"] + 1:
        raise ValueError(f"route_offsets has {env['E_PLUS_1']} entries; {env['E'] + 1} experts need E + 1")
    if env["D"] % 64 or env["F"] % 64:
        raise NotImplementedError(f"D ({env['D']}) and F ({env['F']}) must be multiples of 64")


def _f16ffn_workspace(env: dict) -> int:
    lib = _native.library()
    return int(lib.intent_moe_expert_ffn_workspace_size(env["T"], env["R"], env["D"], env["F"]))


def _f16ffn_launch(v: dict, env: dict, stream: int, workspace) -> str:
    _native.call("intent_moe_expert_ffn", _ptr(v["x"]), env["T"], env["D"], _ld(v["x"]), _ptr(v["route_offsets"]),
                 env["E"], _ptr(v["member_routes"]), env["R"], _ptr(v["route_token"]), _ptr(v["route_weights"]),
                 env["NR"], _ptr(v["w1"]), _ptr(v["w2"]), env["F"], _ptr(v["y"]), _ld(v["y"]), workspace.data_ptr(),
                 workspace.numel(), stream)
    return "intent_moe_expert_ffn"


moe_expert_ffn = KernelDefinition(
    name="moe_expert_ffn",
    params=(
        Param("x", "f16", ("T", "D"), leading_stride=True),
        Param("route_offsets", "i32", ("E_PLUS_1",)),
        Param("member_routes", "i32", ("R",)),
        Param("route_token", "i32", ("NR",)),
        Param("route_weights", "f32", ("NR",)),
        Param("w1", "f16", ("E", "D", "F")),
        Param("w2", "f16", ("E", "F", "D")),
        Param("y", "f32", ("T", "D"), INOUT, leading_stride=True),
    ),
    launch=_f16ffn_launch,
    check=_f16ffn_check,
    workspace=_f16ffn_workspace,
    reference="examples/kernels/ragged/moe.py:12-53",
    doc="y[token] += route_weight * (f16(relu(x[token] @ w1[e])) @ w2[e]) over the ragged routes of each expert e",
)


def _gate_up_check(env: dict) -> None:
    if env["HP"] * 2 != env["H"] or env["F2"] % 2 or env["H"] % env["G1"]:
        raise ValueError("inconsistent gate/up weight shapes")
    env["F"] = env["F2"] // 2
    env["GROUP"] = env["H"] // env["G1"]


def _gate_up_launch(v: dict, env: dict, stream: int, workspace) -> str:
    x, act = v["x"], v["act"]
    _native.call("intent_moe_gate_up_w4", _ptr(x), env["T"], env["H"], _ld(x), _ptr(v["sorted_route_ids"]),
                 _ptr(v["expert_blocks"]), env["NB"], env["BLOCK_SIZE"], env["TOP_K"], _ptr(v["w_gate_up"]),
                 _ptr(v["gate_up_scales"]), _ptr(v["gate_up_zeros"]), env["E"], env["F"], env["GROUP"], _ptr(act),
                 _ld(act), stream)
    return "intent_moe_gate_up_w4"


moe_gate_up_w4 = KernelDefinition(
    name="moe_gate_up_w4",
    params=(
        Param("x", "f16", ("T", "H"), leading_stride=True),
        Param("sorted_route_ids", "i32", ("CAP",)),
        Param("expert_blocks", "i32", ("NB",)),
        Param("w_gate_up", "u8", ("E", "F2", "HP")),
        Param("gate_up_scales", "f16", ("E", "F2", "G1")),
        Param("gate_up_zeros", "u8", ("E", "F2", "G1")),
        Param("act", "f16", (lambda env: env["NB"] * env["BLOCK_SIZE"], lambda env: env["F"]), OUT),
    ),
    launch=_gate_up_launch,
    constexprs={"TOP_K": 2, "BLOCK_SIZE": 128},
    check=_gate_up_check,
    reference="examples/kernels/ragged/moe.py:28-45",
    doc="act[p] = f16(silu(x[t] Wg[e]) * (x[t] Wu[e])) over aligned padded rows",
)


def _down_check(env: dict) -> None:
    if env["FP"] * 2 != env["F"] or env["F"] % env["G2"]:
        raise ValueError("inconsistent down weight shapes")
    env["GROUP"] = env["F"] // env["G2"]


def _down_launch(v: dict, env: dict, stream: int, workspace) -> str:
    act, out = v["act"], v["route_out"]
    _native.call("intent_moe_down_w4", _ptr(act), _ld(act), _ptr(v["sorted_route_ids"]), _ptr(v["expert_blocks"]),
                 env["NB"], env["BLOCK_SIZE"], env["ROUTES"], _ptr(v["w_down"]), _ptr(v["down_scales"]),
                 _ptr(v["down_zeros"]), env["E"], env["H"], env["F"], env["GROUP"], _ptr(out), _ld(out), stream)
    return "intent_moe_down_w4"


moe_down_w4 = KernelDefinition(
    name="moe_down_w4",
    params=(
        Param("act", "f16", ("PR", "F"), leading_stride=True),
        Param("sorted_route_ids", "i32", ("CAP",)),
        Param("expert_blocks", "i32", ("NB",)),
        Param("w_down", "u8", ("E", "H", "FP")),
        Param("down_scales", "f16", ("E", "H", "G2")),
        Param("down_zeros", "u8", ("E", "H", "G2")),
        Param("route_out", "f32", (lambda env: env["ROUTES"], "H"), OUT, leading_stride=True),
    ),
    launch=_down_launch,
    constexprs={"ROUTES": None, "BLOCK_SIZE": 128},
    check=_down_check,
    reference="examples/kernels/ragged/moe.py:46-53",
    doc="route_out[r] = act[p] Wd[e] (fp32) for every aligned row p holding route r",
)


def _combine_check(env: dict) -> None:
    if env["R"] != env["T"] * env["K"]:
        raise ValueError("route_out rows must equal T * top_k")


def _combine_launch(v: dict, env: dict, stream: int, workspace) -> str:
    ro, y = v["route_out"], v["y"]
    _native.call("intent_moe_combine", _ptr(ro), _ld(ro), _ptr(v["topk_weights"]), env["T"], env["K"], _ptr(y),
                 env["H"], _ld(y), stream)
    return "intent_moe_combine"


moe_combine = KernelDefinition(
    name="moe_combine",
    params=(
        Param("route_out", "f32", ("R", "H"), leading_stride=True),
        Param("topk_weights", "f32", ("T", "K")),
        Param("y", "f32", ("T", "H"), INOUT, leading_stride=True),
    ),
    launch=_combine_launch,
    check=_combine_check,
    reference="examples/kernels/ragged/moe.py:48-53 (scatter_reduce add, fixed slot order)",
    doc="y[t] += w[t,0] * route_out[t*k] + ... slot by slot",
)


# ---- GGUF K-quant records --------------------------------------------------------

Q4K_RECORD = 144
Q8K_RECORD = 292


def _q8k_launch(v: dict, env: dict, stream: int, workspace) -> str:
    x, r = v["values"], v["records"]
    _native.call("intent_q8k_quantize", _ptr(x), env["G"], _ld(x), _ptr(r), _ld(r), stream)
    return "intent_q8k_quantize"


q8_k_quantize = KernelDefinition(
    name="q8_k_quantize",
    params=(
        Param("values", "f32", ("G", 256), leading_stride=True),
        Param("records", "u8", ("G", Q8K_RECORD), OUT, leading_stride=True),
    ),
    launch=_q8k_launch,
    reference="doc/dsl/quantized-operations.en.md:5-10,62-70 (I.quantize(values, format=I.quant.q8_k))",
    doc="f32 [G,256] -> Q8_K records u8 [G,292] (ds, i8 q, i16 bsum)",
)


def _qdot_launch(v: dict, env: dict, stream: int, workspace) -> str:
    w, xq, y = v["weights"], v["records"], v["output"]
    _native.call("intent_q4k_q8k_gemv", _ptr(w), env["N"], env["G"], w.stride(0), _ptr(xq), _ptr(y), stream)
    return "intent_q4k_q8k_gemv"


q4_k_q8_k_dot = KernelDefinition(
    name="q4_k_q8_k_dot",
    params=(
        Param("weights", "u8", ("N", "G", Q4K_RECORD)),
        Param("records", "u8", ("G", Q8K_RECORD)),
        Param("output", "f32", ("N",), OUT),
    ),
    launch=_qdot_launch,
    reference="doc/dsl/quantized-operations.en.md:38-58 (I.quantized_dot, lhs q4_k, rhs q8_k, acc f32) per row",
    doc="output[n] = quantized_dot(weights[n], records), records added in increasing order from +0",
)


def _qproj_workspace(env: dict) -> int:
    return env["G"] * Q8K_RECORD


def _qproj_launch(v: dict, env: dict, stream: int, workspace) -> str:
    w, x, y = v["weights"], v["activation"], v["output"]
    _native.call("intent_q4k_projection", _ptr(w), env["N"], env["G"], w.stride(0), _ptr(x), _ld(x),
                 workspace.data_ptr(), _ptr(y), stream)
    return "intent_q4k_projection"


quantized_projection = KernelDefinition(
    name="quantized_projection",
    params=(
        Param("weights", "u8", ("N", "G", Q4K_RECORD)),
        Param("activation", "f32", ("G", 256), leading_stride=True),
        Param("output", "f32", ("N",), OUT),
    ),
    launch=_qproj_launch,
    workspace=_qproj_workspace,
    reference="examples/kernels/quantization/quantized_projection.py:5-19",
    doc="output[n] = quantized_dot(weights[n], quantize(activation, q8_k)), Q4_K x Q8_K",
)


# ---- groupwise FP8 activation quantizers -----------------------------------------

def _fp8q_check(env: dict) -> None:
    if env["G"] * 128 < env["N"]:
        raise ValueError(f"scales.shape[1] ({env['G']}) groups of 128 do not cover N ({env['N']})")


def _fp8q_launch(bf16: bool):
    def launch(v: dict, env: dict, stream: int, workspace) -> str:
        x, q, sc = v["x"], v["quantized"], v["scales"]
        _native.call("intent_fp8_groupwise_quantize", _ptr(x), int(bf16), env["M"], env["N"], _ld(x), _ptr(q), _ld(q),
                     _ptr(sc), env["G"], _ld(sc), stream)
        return "intent_fp8_groupwise_quantize"
    return launch


def _fp8q_definition(name: str, src: str, lines: str) -> KernelDefinition:
    return KernelDefinition(
        name=name,
        params=(
            Param("x", src, ("M", "N"), leading_stride=True),
            Param("quantized", "f8e4m3fn", ("M", "N"), OUT, leading_stride=True),
            Param("scales", "f32", ("M", "G"), INOUT, leading_stride=True),
        ),
        launch=_fp8q_launch(src == "bf16"),
        check=_fp8q_check,
        reference=f"examples/kernels/quantization/fp8.py:{lines}",
        doc="scale = max(absmax of 128 columns, eps) / 448; quantized = e4m3fn(clamp(x / scale, +-448))",
    )


bf16_groupwise_fp8_quantize = _fp8q_definition("bf16_groupwise_fp8_quantize", "bf16", "11-39")
f32_groupwise_fp8_quantize = _fp8q_definition("f32_groupwise_fp8_quantize", "f32", "42-69")


# ---- per-token int8 activation quantizer (feeds w8a8_scaled_matmul) -------------------

def _i8q_launch(bf16: bool):
    def launch(v: dict, env: dict, stream: int, workspace) -> str:
        x, q, sc = v["x"], v["quantized"], v["scales"]
        _native.call("intent_i8_per_token_quantize", _ptr(x), int(bf16), env["M"], env["K"], _ld(x), _ptr(q),
                     _ld(q), _ptr(sc), stream)
        return "intent_i8_per_token_quantize"
    return launch


def _i8q_definition(name: str, src: str) -> KernelDefinition:
    return KernelDefinition(
        name=name,
        params=(
            Param("x", src, ("M", "K"), leading_stride=True),
            Param("quantized", "i8", ("M", "K"), OUT, leading_stride=True),
            Param("scales", "f32", ("M",), OUT),
        ),
        launch=_i8q_launch(src == "bf16"),
        reference="lib/Conversion/KIRToGPU/Quantization.cpp:191-203 (clamp, then round half to even)",
        doc="scale = absmax(row) / 127; quantized = rne(clamp(x * (127 / absmax), -128, 127)); zero row -> 0",
    )


per_token_int8_quantize = _i8q_definition("per_token_int8_quantize", "f16")
bf16_per_token_int8_quantize = _i8q_definition("bf16_per_token_int8_quantize", "bf16")


# ---- low-bit weight x int8 activation (exact int32) ---------------------------------

def _lowbit_check(per_byte: int):
    def check(env: dict) -> None:
        if env["P"] * per_byte != env["K"]:
            raise ValueError(f"packed_weight.shape[1] ({env['P']}) must be K/{per_byte} ({env['K']}/{per_byte})")
    return check


def _w4a8_launch(v: dict, env: dict, stream: int, workspace) -> str:
    a, w, out = v["activation"], v["packed_weight"], v["output"]
    _native.call("intent_w4a8_gemm", _ptr(a), env["M"], env["K"], _ld(a), _ptr(w), env["N"], _ld(w), _ptr(out),
                 _ld(out), stream)
    return "intent_w4a8_gemm"


w4a8_packed_matmul = KernelDefinition(
    name="w4a8_packed_matmul",
    params=(
        Param("activation", "i8", ("M", "K"), leading_stride=True),
        Param("packed_weight", "u8", ("N", "P"), leading_stride=True),
        Param("output", "i32", ("N", "M"), OUT, leading_stride=True),
    ),
    launch=_w4a8_launch,
    check=_lowbit_check(2),
    reference="examples/kernels/contraction/weight_only_int4.py:54-91",
    doc="output[n, m] = sum_k sext4(packed nibble k of row n) * activation[m, k], int32",
)


def _bitnet_launch(v: dict, env: dict, stream: int, workspace) -> str:
    a, w, out = v["activation"], v["packed_weight"], v["output"]
    _native.call("intent_bitnet_int2_gemm", _ptr(a), env["M"], env["K"], _ld(a), _ptr(w), env["N"], _ld(w),
                 _ptr(out), _ld(out), stream)
    return "intent_bitnet_int2_gemm"


bitnet_int2_matmul = KernelDefinition(
    name="bitnet_int2_matmul",
    params=(
        Param("activation", "i8", ("M", "K"), leading_stride=True),
        Param("packed_weight", "u8", ("N", "P"), leading_stride=True),
        Param("output", "i32", ("M", "N"), OUT, leading_stride=True),
    ),
    launch=_bitnet_launch,
    check=_lowbit_check(4),
    reference="examples/kernels/contraction/weight_only_int4.py:94-124",
    doc="output[m, n] = sum_k activation[m, k] * int2 value k of row n (interleaved packing), int32",
)


# ---- MX block-scaled FP8 --------------------------------------------------------

def _mx_launch(v: dict, env: dict, stream: int, workspace) -> str:
    import torch

    lhs, ls, rhs, rs, out = v["lhs"], v["lhs_scale"], v["rhs"], v["rhs_scale"], v["output"]
    M, KB, N = env["M"], env["KB"], env["N"]
    # The kernel reads rows with K contiguous. The reference's benchmark passes
    # rhs as such a view of [N, K] (strides (32, 1, K)); other layouts are
    # re-laid out once here.
    if not (rhs.stride(1) == 1 and (KB == 1 or rhs.stride(0) == 32)):
        rhs = rhs.permute(2, 0, 1).contiguous().permute(1, 2, 0)
    if not (N == 1 or rs.stride(0) == 1) or rs.stride(1) % 4:
        rs = rs.t().contiguous().t()
    b_ld = rhs.stride(2) if N > 1 else KB * 32
    sb_ld = rs.stride(1) if N > 1 else KB
    _native.call("intent_mxfp8_gemm", _ptr(lhs.view(torch.uint8)), M, KB * 32, KB * 32, _ptr(ls), KB,
                 _ptr(rhs.view(torch.uint8)), N, b_ld, _ptr(rs), sb_ld, _ptr(out), _ld(out), stream)
    return "intent_mxfp8_gemm"


def _mx_check(env: dict) -> None:
    if env["KB"] % 4:
        raise NotImplementedError(f"the number of 32-element blocks ({env['KB']}) must be a multiple of 4 (K % 128)")


block_scaled_matmul = KernelDefinition(
    name="block_scaled_matmul",
    params=(
        Param("lhs", "f8e4m3fn", ("M", "KB", 32)),
        Param("lhs_scale", "u8", ("M", "KB")),
        Param("rhs", "f8e4m3fn", ("KB", 32, "N"), free_strides=True),
        Param("rhs_scale", "u8", ("KB", "N"), free_strides=True),
        Param("output", "f32", ("M", "N"), OUT, leading_stride=True),
    ),
    launch=_mx_launch,
    check=_mx_check,
    reference="examples/kernels/contraction/block_scaled.py:11-39 (I.scaled_matmul, e4m3 x e4m3, E8M0, group 32)",
    doc="output = sum over k of (lhs * 2^(lhs_scale-127)) * (rhs * 2^(rhs_scale-127)), f32",
)


# ---- per-tensor scaled FP8 GEMM and its split-K form ---------------------------

def _fp8_kn_shape(env: dict) -> bool:
    return env["N"] % 16 == 0


def _fp8_kn_direct(env: dict, lhs, rhs_kn) -> bool:
    """rhs [K, N] feeds the kernel in place (no transposed copy) when N and its row stride
    are multiples of 16 bytes and both operands are 16-byte aligned. The in-place kernel
    (producer waves transpose the bytes on their way to LDS) is faster than the copy plus
    the row-form kernel at every M measured on MI355X (N=14336, K=4096: M=256 28 vs 58 us,
    M=4096 234 vs 283 us, split-K SP 4 276 vs 293 us)."""
    return (_fp8_kn_shape(env) and rhs_kn.stride(0) % 16 == 0 and rhs_kn.data_ptr() % 16 == 0
            and lhs.data_ptr() % 16 == 0)


def _fp8_rhs_rows(rhs_kn, K: int, N: int, workspace, stream: int):
    """The [K, N] right operand transposed into [N, K] rows (the fallback when it cannot
    be read in place): in the workspace, or in a scratch buffer whose memory the caching
    allocator holds back until the launch stream has passed it."""
    if workspace is None or workspace.numel() < K * N:
        import torch

        workspace = torch.empty(K * N, dtype=torch.uint8, device=rhs_kn.device)
        workspace.record_stream(torch.cuda.ExternalStream(stream, device=rhs_kn.device))
    _native.call("intent_fp8_transpose", _ptr(rhs_kn), K, N, rhs_kn.stride(0), workspace.data_ptr(), K, stream)
    return workspace.data_ptr()


def _sfp8_workspace(env: dict) -> int:
    # the transposed copy of rhs is not needed on the in-place shapes
    return 0 if _fp8_kn_shape(env) else env["K"] * env["N"]


def _sfp8_gemm(lhs, rhs_kn, env: dict, M: int, K: int, N: int, lhs_ld: int, splits: int, accumulate: int, out,
               stream: int, workspace) -> str:
    scales = (float(env["lhs_scale"]), float(env["rhs_scale"]))
    if _fp8_kn_direct(env, lhs, rhs_kn):
        _native.call("intent_scaled_fp8_gemm_kn", _ptr(lhs), M, K, lhs_ld, _ptr(rhs_kn), N, rhs_kn.stride(0), *scales,
                     splits, accumulate, _ptr(out), _ld(out), stream)
        return "intent_scaled_fp8_gemm_kn"
    bt = _fp8_rhs_rows(rhs_kn, K, N, workspace, stream)
    _native.call("intent_scaled_fp8_gemm", _ptr(lhs), M, K, lhs_ld, bt, N, K, *scales, splits, accumulate, _ptr(out),
                 _ld(out), stream)
    return "intent_scaled_fp8_gemm"


def _sfp8_launch(v: dict, env: dict, stream: int, workspace) -> str:
    lhs, rhs, out = v["lhs"], v["rhs"], v["output"]
    return _sfp8_gemm(lhs, rhs, env, env["M"], env["K"], env["N"], _ld(lhs), 1, 0, out, stream, workspace)


def _sfp8_check(env: dict) -> None:
    if env["K"] % 128:
        raise NotImplementedError(f"K ({env['K']}) must be a multiple of 128")


scaled_fp8_matmul = KernelDefinition(
    name="scaled_fp8_matmul",
    params=(
        Param("lhs", "f8e4m3fn", ("M", "K"), leading_stride=True),
        Param("rhs", "f8e4m3fn", ("K", "N"), leading_stride=True),
        Param("output", "f16", ("M", "N"), OUT, leading_stride=True),
        Scalar("lhs_scale", "f32"),
        Scalar("rhs_scale", "f32"),
    ),
    launch=_sfp8_launch,
    check=_sfp8_check,
    workspace=_sfp8_workspace,
    reference="examples/kernels/contraction/block_scaled.py:42-63",
    doc="output = f16((lhs @ rhs (f32) * lhs_scale) * rhs_scale), E4M3FN operands",
)


def _sfp8_splitk_workspace(env: dict) -> int:
    return 0 if _fp8_kn_shape(env) else env["IT"] * env["SP"] * 256 * env["N"]


def _sfp8_splitk_launch(v: dict, env: dict, stream: int, workspace) -> str:
    lhs, rhs, out = v["lhs"], v["rhs"], v["output"]
    M, N, SP = env["M"], env["N"], env["SP"]
    K = env["IT"] * SP * 256
    return _sfp8_gemm(lhs, rhs.view(K, N), env, M, K, N, K, SP, 1, out, stream, workspace)


scaled_fp8_splitk_matmul = KernelDefinition(
    name="scaled_fp8_splitk_matmul",
    params=(
        Param("lhs", "f8e4m3fn", ("M", "IT", "SP", 256)),
        Param("rhs", "f8e4m3fn", ("IT", "SP", 256, "N")),
        Param("output", "f16", ("M", "N"), INOUT, leading_stride=True),
        Scalar("lhs_scale", "f32"),
        Scalar("rhs_scale", "f32"),
    ),
    launch=_sfp8_splitk_launch,
    workspace=_sfp8_splitk_workspace,
    reference="examples/kernels/contraction/block_scaled.py:66-98",
    doc="for each split s in order: output = f16(output + f16((partial_s * lhs_scale) * rhs_scale))",
)


# ---- DeepGEMM-style FP8 with f32 block scales ------------------------------------

def _deepgemm_check(env: dict) -> None:
    if env["NB"] * 128 < env["N"]:
        raise ValueError(f"rhs_scale has {env['NB']} row blocks; N = {env['N']} needs {(env['N'] + 127) // 128}")


def _deepgemm_launch(v: dict, env: dict, stream: int, workspace) -> str:
    lhs, rhs, ls, rs, out = v["lhs"], v["rhs"], v["lhs_scale"], v["rhs_scale"], v["output"]
    M, KB, N = env["M"], env["KB"], env["N"]
    _native.call("intent_deepgemm_fp8", _ptr(lhs), M, KB * 128, KB * 128, _ptr(ls), KB, _ptr(rhs), N, KB * 128,
                 _ptr(rs), KB, _ptr(out), _ld(out), stream)
    return "intent_deepgemm_fp8"


deepgemm_fp8_2xacc = KernelDefinition(
    name="deepgemm_fp8_2xacc",
    params=(
        Param("lhs", "f8e4m3fn", ("M", "KB", 128)),
        Param("rhs", "f8e4m3fn", ("N", "KB", 128)),
        Param("lhs_scale", "f32", ("M", "KB")),
        Param("rhs_scale", "f32", ("NB", "KB")),
        Param("output", "bf16", ("M", "N"), OUT, leading_stride=True),
    ),
    launch=_deepgemm_launch,
    check=_deepgemm_check,
    reference="examples/kernels/contraction/block_scaled.py:101-122",
    doc="output = bf16(sum over k-blocks of (lhs . rhs) * lhs_scale[m, kb] * rhs_scale[n // 128, kb])",
)


# ---- FP8 x FP8 -> FP8 ------------------------------------------------------------

def _fp8_out_launch(fmt: int):
    def launch(v: dict, env: dict, stream: int, workspace) -> str:
        lhs, rhs, out = v["lhs"], v["rhs_transposed"], v["output"]
        _native.call("intent_fp8_gemm", _ptr(lhs), env["M"], env["K"], _ld(lhs), _ptr(rhs), env["N"], _ld(rhs), fmt,
                     _ptr(out), _ld(out), stream)
        return "intent_fp8_gemm"
    return launch


def _fp8_out_definition(name: str, dt: str, fmt: int, lines: str) -> KernelDefinition:
    return KernelDefinition(
        name=name,
        params=(
            Param("lhs", dt, ("M", "K"), leading_stride=True),
            Param("rhs_transposed", dt, ("N", "K"), leading_stride=True),
            Param("output", dt, ("M", "N"), OUT, leading_stride=True),
        ),
        launch=_fp8_out_launch(fmt),
        check=_sfp8_check,
        reference=f"examples/kernels/contraction/weight_only_int4.py:{lines}",
        doc=f"output = {dt}(lhs @ rhs_transposed^T, f32 accumulation), nearest even",
    )


fp8_e4m3_matmul = _fp8_out_definition("fp8_e4m3_matmul", "f8e4m3fn", 0, "178-195")
fp8_e5m2_matmul = _fp8_out_definition("fp8_e5m2_matmul", "f8e5m2", 1, "198-215")


# ---- FP4 (E2M1) weights x bf16 activations ---------------------------------------

def _fp4_launch(v: dict, env: dict, stream: int, workspace) -> str:
    x, w, y = v["activation"], v["packed_weight"], v["output"]
    _native.call("intent_fp4_bf16_matmul", _ptr(x), env["M"], env["K"], _ld(x), _ptr(w), env["N"], _ld(w), _ptr(y),
                 _ld(y), stream)
    return "intent_fp4_bf16_matmul"


def _fp4_check(env: dict) -> None:
    if env["P"] * 2 != env["K"]:
        raise ValueError(f"packed_weight.shape[1] ({env['P']}) must be K / 2 ({env['K'] // 2})")
    if env["K"] % 64:
        raise NotImplementedError(f"K ({env['K']}) must be a multiple of 64")


dequant_bf16_fp4_matmul = KernelDefinition(
    name="dequant_bf16_fp4_matmul",
    params=(
        Param("activation", "bf16", ("M", "K"), leading_stride=True),
        Param("packed_weight", "u8", ("N", "P"), leading_stride=True),
        Param("output", "bf16", ("M", "N"), OUT, leading_stride=True),
    ),
    launch=_fp4_launch,
    check=_fp4_check,
    reference="examples/kernels/contraction/weight_only_int4.py:127-175",
    doc="output = bf16(activation @ e2m1(packed_weight)^T), f32 accumulation",
)


# ---- the reference's own weight_only_int4_matmul layout ---------------------------

W4_SYM_GROUP = 64  # weight_only_int4.py:9 (GROUP_SIZE)


def _w4sym_layout(env: dict) -> tuple:
    N, K, G = env["N"], env["K"], env["G"]
    q = 0
    s = -(-(N * K // 2) // 256) * 256
    z = s + -(-(N * G * 2) // 256) * 256
    return q, s, z, z + N * G


def _w4sym_workspace(env: dict) -> int:
    # the repacked copy is not needed on the in-place shapes (alignment permitting)
    if (env["M"] <= 5 and env["K"] <= 8192 and env["N"] % 4 == 0) or env["M"] > 16:
        return 0
    return _w4sym_layout(env)[3]


def _w4sym_check(env: dict) -> None:
    if env["P"] * 8 != env["K"]:
        raise ValueError(f"packed_weight.shape[0] ({env['P']}) must be K / 8 ({env['K'] // 8})")
    if env["G"] * W4_SYM_GROUP != env["K"]:
        raise ValueError(f"scales.shape[0] ({env['G']}) must be K / {W4_SYM_GROUP} ({env['K'] // W4_SYM_GROUP})")
    if env["K"] % 64:
        raise NotImplementedError(f"K ({env['K']}) must be a multiple of 64")


def _w4sym_in_place(v: dict, env: dict) -> bool:
    """Decode shapes the in-place kernel (intent_w4a16_sym_gemv) takes."""
    x, packed, scales = v["activation"], v["packed_weight"], v["scales"]
    return (env["M"] <= 5 and env["K"] <= 8192 and env["N"] % 4 == 0 and x.data_ptr() % 16 == 0
            and x.stride(0) % 8 == 0 and packed.data_ptr() % 16 == 0 and packed.stride(0) % 4 == 0
            and scales.data_ptr() % 8 == 0 and scales.stride(0) % 4 == 0)


def _w4sym_launch(v: dict, env: dict, stream: int, workspace) -> str:
    x, packed, scales, y = v["activation"], v["packed_weight"], v["scales"], v["output"]
    M, K, N, G = env["M"], env["K"], env["N"], env["G"]
    if _w4sym_in_place(v, env):
        _native.call("intent_w4a16_sym_gemv", _ptr(x), M, K, x.stride(0), _ptr(packed), N, packed.stride(0),
                     _ptr(scales), scales.stride(0), _ptr(y), _ld(y), stream)
        return "intent_w4a16_sym_gemv"
    if M > 16 and x.data_ptr() % 16 == 0 and x.stride(0) % 8 == 0 and packed.data_ptr() % 4 == 0:
        _native.call("intent_w4a16_sym_gemm", _ptr(x), M, K, x.stride(0), _ptr(packed), N, packed.stride(0),
                     _ptr(scales), scales.stride(0), _ptr(y), _ld(y), stream)
        return "intent_w4a16_sym_gemm"
    if workspace is None or workspace.numel() < _w4sym_layout(env)[3]:
        import torch

        workspace = torch.empty(_w4sym_layout(env)[3], dtype=torch.uint8, device=x.device)
        workspace.record_stream(torch.cuda.ExternalStream(stream, device=x.device))
    oq, os_, oz, _ = _w4sym_layout(env)
    base = workspace.data_ptr()
    _native.call("intent_w4_sym_repack", _ptr(packed), env["P"], N, packed.stride(0), _ptr(scales), G,
                 scales.stride(0), base + oq, K // 2, base + os_, base + oz, G, stream)
    entry = "intent_w4a16_gemv" if M <= 16 else "intent_w4a16_gemm"
    _native.call(entry, _ptr(x), M, K, _ld(x), base + oq, N, K // 2, base + os_, base + oz, G, W4_SYM_GROUP, _ptr(y),
                 _ld(y), stream)
    return entry


weight_only_int4_matmul = KernelDefinition(
    name="weight_only_int4_matmul",
    params=(
        Param("activation", "f16", ("M", "K"), leading_stride=True),
        Param("packed_weight", "i32", ("P", "N"), leading_stride=True),
        Param("scales", "f16", ("G", "N"), leading_stride=True),
        Param("output", "f16", ("M", "N"), OUT, leading_stride=True),
    ),
    launch=_w4sym_launch,
    check=_w4sym_check,
    workspace=_w4sym_workspace,
    reference="examples/kernels/contraction/weight_only_int4.py:18-51",
    doc="the reference's symmetric signed-nibble W4 (int32 [K/8, N], f16 scales [K/64, N]): read in place up to "
        "M = 5 and above M = 16, repacked for the W4A16 GEMV in between",
)


# ---- quantized_gemm: f16 GEMM with the fused int8 epilogue -------------------------

def _qgemm_workspace(env: dict) -> int:
    # the transposed copy of b is needed only when N is not a multiple of 8
    return 0 if env["N"] % 8 == 0 else env["K"] * env["N"] * 2


def _qgemm_check(env: dict) -> None:
    if env["K"] % 64:
        raise NotImplementedError(f"K ({env['K']}) must be a multiple of 64")


def _kn_direct(env: dict, *mats) -> bool:
    """b [K, N] feeds the kernels directly (no transposed copy) when N and every
    row stride are multiples of 8 elements and the operands 16-byte aligned."""
    return env["N"] % 8 == 0 and all(t.stride(0) % 8 == 0 and t.data_ptr() % 16 == 0 for t in mats)


def _transposed(b, K: int, N: int, workspace, stream: int) -> int:
    """[K, N] -> [N, K] copy of b in the workspace (the fallback of the [K, N] entries:
    N a multiple of 8 with an unaligned operand gets a scratch copy whose memory the
    caching allocator holds back until the launch stream has passed it)."""
    if workspace is None or workspace.numel() < K * N * 2:
        import torch

        workspace = torch.empty(K * N * 2, dtype=torch.uint8, device=b.device)
        workspace.record_stream(torch.cuda.ExternalStream(stream, device=b.device))
    _native.call("intent_f16_transpose", _ptr(b), K, N, b.stride(0), workspace.data_ptr(), K, stream)
    return workspace.data_ptr()


def _qgemm_launch(v: dict, env: dict, stream: int, workspace) -> str:
    a, b, out = v["a"], v["b"], v["output"]
    M, K, N = env["M"], env["K"], env["N"]
    if _kn_direct(env, a, b):
        _native.call("intent_quantized_gemm_kn", _ptr(a), M, K, _ld(a), _ptr(b), N, b.stride(0), _ptr(v["bias"]),
                     _ptr(v["residual"]), _ld(v["residual"]), _ptr(v["output_scale"]), _ptr(out), _ld(out), stream)
        return "intent_quantized_gemm_kn"
    bt = _transposed(b, K, N, workspace, stream)
    _native.call("intent_quantized_gemm", _ptr(a), M, K, _ld(a), bt, N, K, _ptr(v["bias"]), _ptr(v["residual"]),
                 _ld(v["residual"]), _ptr(v["output_scale"]), _ptr(out), _ld(out), stream)
    return "intent_quantized_gemm"


quantized_gemm = KernelDefinition(
    name="quantized_gemm",
    params=(
        Param("a", "f16", ("M", "K"), leading_stride=True),
        Param("b", "f16", ("K", "N"), leading_stride=True),
        Param("bias", "f32", ("N",)),
        Param("residual", "f16", ("M", "N"), leading_stride=True),
        Param("output_scale", "f32", ("N",)),
        Param("output", "i8", ("M", "N"), OUT, leading_stride=True),
    ),
    launch=_qgemm_launch,
    check=_qgemm_check,
    workspace=_qgemm_workspace,
    reference="examples/kernels/contraction/gemm.py:83-106",
    doc="output = i8(clamp((relu(a @ b + bias) + residual) / output_scale, -128, 127))",
)


# ---- f16 / bf16 grouped GEMMs (the reference's ragged kernels) ------------------

def _ragged_workspace(env: dict) -> int:
    # the transposed copy of the weights is needed only when N is not a multiple of 8
    return 0 if env["N"] % 8 == 0 else env["G"] * env["N"] * env["K"] * 2


def _ragged_check(env: dict) -> None:
    if env["G_PLUS_1"] != env["G"] + 1:
        raise ValueError(f"group_offsets has {env['G_PLUS_1']} entries; {env['G'] + 1} groups need G + 1")
    if env["K"] % 64:
        raise NotImplementedError(f"K ({env['K']}) must be a multiple of 64")


def _ragged_launch(bf16: bool):
    def launch(v: dict, env: dict, stream: int, workspace) -> str:
        x, offs, w, y = v["x"], v["group_offsets"], v["weight"], v["y"]
        G, K, N = env["G"], env["K"], env["N"]
        if _kn_direct(env, x) and w.data_ptr() % 16 == 0:
            # [G, K, N] weights in place (grouped_kn.hip)
            _native.call("intent_grouped_gemm_kn", _ptr(x), env["R"], K, _ld(x), _ptr(offs), G, _ptr(w), N,
                         w.stride(1), w.stride(0), int(bf16), _ptr(y), _ld(y), stream)
            return "intent_grouped_gemm_kn"
        if workspace is None or workspace.numel() < G * N * K * 2:
            import torch

            workspace = torch.empty(G * N * K * 2, dtype=torch.uint8, device=w.device)
            workspace.record_stream(torch.cuda.ExternalStream(stream, device=w.device))
        wt = workspace.data_ptr()  # [G, K, N] -> [G, N, K]
        _native.call("intent_f16_transpose_batched", _ptr(w), G, K, N, w.stride(1), w.stride(0), wt, K, N * K, stream)
        _native.call("intent_grouped_gemm", _ptr(x), env["R"], K, _ld(x), _ptr(offs), G, None, 1, wt, N, K, N * K,
                     int(bf16), _ptr(y), _ld(y), stream)
        return "intent_grouped_gemm"
    return launch


def _ragged_definition(name: str, dt: str, lines: str) -> KernelDefinition:
    return KernelDefinition(
        name=name,
        params=(
            Param("x", dt, ("R", "K"), leading_stride=True),
            Param("group_offsets", "i32", ("G_PLUS_1",)),
            Param("weight", dt, ("G", "K", "N")),
            Param("y", dt, ("R", "N"), OUT, leading_stride=True),
        ),
        launch=_ragged_launch(dt == "bf16"),
        check=_ragged_check,
        workspace=_ragged_workspace,
        reference=f"examples/kernels/ragged/grouped_gemm.py:{lines}",
        doc="y[rows of g] = x[rows of g] @ weight[g], rows of g = group_offsets[g] .. group_offsets[g+1]",
    )


ragged_grouped_gemm = _ragged_definition("ragged_grouped_gemm", "f16", "11-38")
ragged_grouped_gemm_bf16 = _ragged_definition("ragged_grouped_gemm_bf16", "bf16", "41-70")


def _routed_check(env: dict) -> None:
    if env["E_PLUS_1"] != env["E"] + 1:
        raise ValueError(f"expert_offsets has {env['E_PLUS_1']} entries; {env['E'] + 1} experts need E + 1")
    if env["K"] % 64:
        raise NotImplementedError(f"K ({env['K']}) must be a multiple of 64")


def _routed_launch(v: dict, env: dict, stream: int, workspace) -> str:
    x, offs, routes, w, out = v["x"], v["expert_offsets"], v["member_routes"], v["weight"], v["output"]
    E, K, N = env["E"], env["K"], env["N"]
    _native.call("intent_grouped_gemm", _ptr(x), env["R"], K, _ld(x), _ptr(offs), E, _ptr(routes), env["TOP_K"],
                 _ptr(w), N, K, N * K, 1, _ptr(out), N, stream)
    return "intent_grouped_gemm"


routed_expert_projection_bf16 = KernelDefinition(
    name="routed_expert_projection_bf16",
    params=(
        Param("x", "bf16", ("T", "K"), leading_stride=True),
        Param("expert_offsets", "i32", ("E_PLUS_1",)),
        Param("member_routes", "i32", ("R",)),
        Param("weight", "bf16", ("E", "N", "K")),
        Param("output", "bf16", ("T", "TOP_K", "N"), OUT),
    ),
    launch=_routed_launch,
    constexprs={"TOP_K": 2},
    check=_routed_check,
    reference="examples/kernels/ragged/grouped_gemm.py:101-138",
    doc="output[r // TOP_K, r % TOP_K] = x[r // TOP_K] @ weight[e].T for the routes r of expert e",
)


# ---- plain float GEMMs (gemm.py) -------------------------------------------------

def _fgemm_launch(kind: str):
    def launch(v: dict, env: dict, stream: int, workspace) -> str:
        a, b, c = v["a"], v["b"], v["c"]
        M, K, N = env["M"], env["K"], env["N"]
        epi = 2 if kind == "bf16" else (1 if int(env.get("ACTIVATION", 0)) == 1 else 0)
        if _kn_direct(env, a, b):
            _native.call("intent_f16_gemm_kn", _ptr(a), M, K, _ld(a), _ptr(b), N, b.stride(0), epi, _ptr(c), _ld(c),
                         stream)
            return "intent_f16_gemm_kn"
        bt = _transposed(b, K, N, workspace, stream)
        _native.call("intent_f16_gemm", _ptr(a), M, K, _ld(a), bt, N, K, epi, _ptr(c), _ld(c), stream)
        return "intent_f16_gemm"
    return launch


def _fgemm_definition(name: str, dt: str, lines: str, constexprs: dict) -> KernelDefinition:
    return KernelDefinition(
        name=name,
        params=(
            Param("a", dt, ("M", "K"), leading_stride=True),
            Param("b", dt, ("K", "N"), leading_stride=True),
            Param("c", dt, ("M", "N"), OUT, leading_stride=True),
        ),
        launch=_fgemm_launch(dt),
        constexprs=constexprs,
        check=_qgemm_check,
        workspace=_qgemm_workspace,
        reference=f"examples/kernels/contraction/gemm.py:{lines}",
        doc=f"c = {dt}(a @ b) with f32 accumulation" + (" (ACTIVATION 1 = RELU: max(acc, 0))" if constexprs else ""),
    )


gemm = _fgemm_definition("gemm", "f16", "42-61", {"ACTIVATION": 0})
bf16_gemm = _fgemm_definition("bf16_gemm", "bf16", "64-80", {})


# ---- NVFP4 activation quantizer ---------------------------------------------------

def _nvfp4_check(env: dict) -> None:
    if env["N"] % 16 or env["P"] * 2 != env["N"]:
        raise ValueError(f"N ({env['N']}) must be a multiple of 16 and packed.shape[1] ({env['P']}) N / 2")
    # The CPU formula copies into scales of exactly this block shape (cpu_runtime.py:1338-1339);
    # the kernel's block stride follows from N, so a wider tensor is refused rather than misindexed.
    want = ((env["M"] + 127) // 128, (env["N"] + 63) // 64)
    if (env["MT"], env["NT"]) != want:
        raise ValueError(f"scales blocks ({env['MT']}, {env['NT']}) must be {want} for M = {env['M']}, N = {env['N']}")


def _nvfp4_launch(v: dict, env: dict, stream: int, workspace) -> str:
    x, gs, packed, scales = v["x"], v["global_scale"], v["packed"], v["scales"]
    _native.call("intent_nvfp4_quantize", _ptr(x), env["M"], env["N"], _ld(x), _ptr(gs), _ptr(packed), _ld(packed),
                 _ptr(scales), stream)
    return "intent_nvfp4_quantize"


nvfp4_quantize = KernelDefinition(
    name="nvfp4_quantize",
    params=(
        Param("x", "bf16", ("M", "N"), leading_stride=True),
        Param("global_scale", "f32", (1,)),
        Param("packed", "u8", ("M", "P"), INOUT, leading_stride=True),
        Param("scales", "u8", ("MT", "NT", 32, 4, 4), INOUT),
    ),
    launch=_nvfp4_launch,
    check=_nvfp4_check,
    reference="examples/kernels/quantization/nvfp4.py",
    doc="E2M1 values two per byte and E4M3 scales per 16 in the reference's swizzled 128 x 4 blocks",
)


ALL_DEFINITIONS = (
    weight_only_int4_matmul, weight_only_int4_asym_matmul, weight_only_int8_matmul, w8a8_scaled_matmul, gemm_i8_nt,
    gemm_i8,
    moe_route_topk, moe_align_block_size, moe_expert_ffn_w4, moe_gate_up_w4, moe_down_w4, moe_combine, moe_expert_ffn,
    q8_k_quantize, q4_k_q8_k_dot, quantized_projection, bf16_groupwise_fp8_quantize, f32_groupwise_fp8_quantize,
    w4a8_packed_matmul, bitnet_int2_matmul, block_scaled_matmul, scaled_fp8_matmul, scaled_fp8_splitk_matmul,
    deepgemm_fp8_2xacc, fp8_e4m3_matmul, fp8_e5m2_matmul, dequant_bf16_fp4_matmul, quantized_gemm,
    ragged_grouped_gemm, ragged_grouped_gemm_bf16, routed_expert_projection_bf16, gemm, bf16_gemm,
    nvfp4_quantize, per_token_int8_quantize, bf16_per_token_int8_quantize,
)
