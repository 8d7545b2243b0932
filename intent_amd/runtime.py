"""HIP runtime behind a compiled artifact: binding, output allocation, launch.

Semantics follow the reference's GPU provider runtime
(python/intent/runtime/artifact.py:130-176, runtime/invocation.py:56-159,
runtime/gpu/program.py:68-124): the binder checks dtypes, ranks, shared
extents and strides against the public interface; ``run`` allocates declared
Out buffers with torch on the artifact's device; launches are asynchronous on
torch's current stream; ``infer_outputs`` builds outputs from shapes alone so
that torch fake tensors never touch data.
"""
from __future__ import annotations

from dataclasses import dataclass, field

from . import _native
from .definitions import KernelDefinition, Param, Scalar
from .interface import DTYPES, PublicInterface, ViewKind, torch_dtype


@dataclass(frozen=True)
class NativeObservation:
    """Facts of the latest launch, read without compiling or launching."""

    entry: str
    definition: str
    arch: str
    library: str
    constexprs: dict = field(default_factory=dict)
    kernel: str = ""  # the kernel variant the entry dispatched to


@dataclass(frozen=True)
class ConfigurationAssessment:
    entry: str
    eligible: bool
    reason: str


@dataclass
class Binding:
    views: dict
    env: dict
    outputs: tuple
    workspace: object = None


class HIPRuntime:
    def __init__(self, definition: KernelDefinition, device: int, constexprs: dict, arch: str):
        self.definition = definition
        self.device = device
        self.constexprs = constexprs
        self.arch = arch
        self._interface = definition.interface()
        self._workspace = None
        self.observation: NativeObservation | None = None

    @property
    def interface(self) -> PublicInterface:
        return self._interface

    # ---- binding ------------------------------------------------------------
    def _bind(self, arguments: tuple, explicit_outputs: tuple | None, abstract: bool = False) -> Binding:
        import torch

        d = self.definition
        params = d.params
        inputs = [p for p in params if isinstance(p, Scalar) or p.access is not ViewKind.OUT]
        outputs = [p for p in params if isinstance(p, Param) and p.access is ViewKind.OUT]
        if len(arguments) != len(inputs):
            raise TypeError(f"{d.name}: expected {len(inputs)} input arguments, got {len(arguments)}")
        env = dict(self.constexprs)
        views: dict = {}

        def observe(p: Param, t, supplied_by_caller: bool) -> None:
            if not isinstance(t, torch.Tensor):
                raise TypeError(f"{d.name}: {p.name} must be a torch.Tensor, got {type(t).__name__}")
            want = torch_dtype(DTYPES[p.dtype])
            if t.dtype != want:
                raise TypeError(f"{d.name}: {p.name} must have dtype {want}, got {t.dtype}")
            if t.dim() != len(p.dims):
                raise ValueError(f"{d.name}: {p.name} must have rank {len(p.dims)}, got {t.dim()}")
            for axis, dim in enumerate(p.dims):
                extent = int(t.shape[axis])
                if isinstance(dim, int):
                    if extent != dim:
                        raise ValueError(f"{d.name}: {p.name}.shape[{axis}] must be {dim}, got {extent}")
                elif isinstance(dim, str):
                    known = env.setdefault(dim, extent)
                    if known != extent:
                        raise ValueError(f"{d.name}: {p.name}.shape[{axis}] violates the declared interface "
                                         f"relation ({dim}={known}, got {extent})")
                else:
                    expected = int(dim(env))
                    if extent != expected:
                        raise ValueError(f"{d.name}: {p.name}.shape[{axis}] must be {expected}, got {extent}")
            if not abstract:
                self._check_layout(p, t)

        for p, value in zip(inputs, arguments):
            if isinstance(p, Scalar):
                env[p.name] = value
                continue
            observe(p, value, True)
            views[p.name] = value
        if d.check is not None:
            d.check(env)
        if explicit_outputs is None:
            outs = []
            device = next((v.device for v in views.values()), None)
            for p in outputs:
                shape = tuple(self._extent(p, dim, env) for dim in p.dims)
                t = torch.empty(shape, dtype=torch_dtype(DTYPES[p.dtype]), device=device)
                views[p.name] = t
                outs.append(t)
            outs = tuple(outs)
        else:
            if len(explicit_outputs) != len(outputs):
                raise TypeError(f"{d.name}: expected {len(outputs)} explicit output buffers, "
                                f"got {len(explicit_outputs)}")
            for p, t in zip(outputs, explicit_outputs):
                observe(p, t, True)
                views[p.name] = t
            outs = tuple(explicit_outputs)
        if not abstract:
            self._check_aliases(views)
        return Binding(views, env, outs)

    @staticmethod
    def _extent(p: Param, dim, env: dict) -> int:
        if isinstance(dim, int):
            return dim
        if isinstance(dim, str):
            if dim not in env:
                raise NotImplementedError(f"{p.name}: extent {dim} is not supplied by the inputs; "
                                          "provide explicit output buffers")
            return int(env[dim])
        return int(dim(env))

    def _check_layout(self, p: Param, t) -> None:
        import torch

        expected = torch.device("cuda", self.device)
        if t.device != expected:
            raise ValueError(f"compiled artifact is bound to {expected}, but {p.name} is on {t.device}")
        if t.numel() == 0 or p.free_strides:
            return
        if p.leading_stride and t.dim() == 2:
            if t.stride(1) != 1 and t.shape[1] > 1:
                raise ValueError(f"{p.name}.strides[1] violates the declared interface relation (must be 1)")
            if t.stride(0) < t.shape[1] and t.shape[0] > 1:
                raise ValueError(f"{p.name}.strides[0] is smaller than the row")
        elif not t.is_contiguous():
            raise ValueError(f"{p.name} must be contiguous")

    def _check_aliases(self, views: dict) -> None:
        """Writable views may not overlap any other view (noalias contract)."""
        writable = {p.name for p in self.definition.params if isinstance(p, Param) and p.access is not ViewKind.IN}
        spans = {}
        for name, t in views.items():
            if t.numel() == 0:
                continue
            start = t.data_ptr()
            last = sum((extent - 1) * stride for extent, stride in zip(t.shape, t.stride()))
            spans[name] = (start, start + (last + 1) * t.element_size())
        names = list(spans)
        for i, a in enumerate(names):
            for b in names[i + 1:]:
                if a not in writable and b not in writable:
                    continue
                (s0, e0), (s1, e1) = spans[a], spans[b]
                if s0 < e1 and s1 < e0:
                    raise ValueError(f"{self.definition.name}: {a} and {b} overlap; writable views must not alias")

    def _workspace_for(self, env: dict):
        import torch

        if self.definition.workspace is None:
            return None
        need = self.definition.workspace(env)
        if self._workspace is None or self._workspace.numel() < need:
            self._workspace = torch.empty(max(need, 16), dtype=torch.uint8, device=torch.device("cuda", self.device))
        return self._workspace

    def _launch(self, binding: Binding) -> None:
        import torch

        stream = torch.cuda.current_stream(self.device).cuda_stream
        entry = self.definition.launch(binding.views, binding.env, stream, binding.workspace)
        self.observation = NativeObservation(entry, self.definition.name, self.arch, str(_native.LIBRARY_PATH),
                                             dict(self.constexprs), _native.last_kernel())

    # ---- provider surface -------------------------------------------------------
    def run(self, *arguments):
        binding = self._bind(arguments, None)
        binding.workspace = self._workspace_for(binding.env)
        self._launch(binding)
        return _result(binding.outputs)

    def launch(self, *arguments):
        interface = self._interface
        n_in = len(interface.inputs)
        if len(arguments) != len(interface.parameters):
            raise TypeError(f"{self.definition.name}: expected {len(interface.parameters)} runtime arguments, "
                            f"got {len(arguments)}")
        ins = tuple(a for a, p in zip(arguments, interface.parameters) if not getattr(p, "output", False))
        outs = tuple(a for a, p in zip(arguments, interface.parameters) if getattr(p, "output", False))
        assert len(ins) == n_in
        binding = self._bind(ins, outs)
        binding.workspace = self._workspace_for(binding.env)
        self._launch(binding)
        return None

    def prepare_call(self, arguments: tuple, *, outputs: tuple | None = None) -> "HIPPreparedCall":
        binding = self._bind(tuple(arguments), outputs)
        binding.workspace = self._workspace_for(binding.env)
        return HIPPreparedCall(self, binding)

    def infer_outputs(self, arguments: tuple):
        binding = self._bind(tuple(arguments), None, abstract=True)
        return _result(binding.outputs)

    def tuning_configurations(self, *arguments):
        return ()


def _result(outputs: tuple):
    if not outputs:
        return None
    return outputs[0] if len(outputs) == 1 else outputs


class HIPPreparedCall:
    """Invocation-owned arguments and outputs; launch() runs on torch's current stream."""

    def __init__(self, runtime: HIPRuntime, binding: Binding):
        self._runtime = runtime
        self._binding = binding

    def compile(self) -> None:
        _native.library()  # the code objects are prebuilt; this validates the library and ABI

    def launch(self) -> None:
        self._runtime._launch(self._binding)

    def result(self):
        return _result(self._binding.outputs)

    @property
    def observation(self) -> NativeObservation | None:
        return self._runtime.observation

    def inspect_configurations(self) -> tuple[ConfigurationAssessment, ...]:
        d = self._runtime.definition
        env = self._binding.env
        if d.name == "weight_only_int4_asym_matmul":
            m = env["M"]
            choice = env["KERNEL"]
            return (
                ConfigurationAssessment("intent_w4a16_gemv", m <= 16 and choice in ("auto", "gemv"),
                                        "decode GEMV covers M <= 16"),
                ConfigurationAssessment("intent_w4a16_gemm", (m > 16 and choice == "auto") or choice == "gemm",
                                        "MFMA tile GEMM for M > 16"),
            )
        return (ConfigurationAssessment(d.name, True, "single fixed kernel"),)
