"""``compile(definition, *, target, ...)`` — the reference's entry point, MI355X-native.

Signature of python/intent/compiler/pipeline.py:19-34. There is no DSL
lowering and no subprocess: the definition names a fixed hot-path operator,
target resolution checks for a gfx950 device and the prebuilt
``libintent_amd.so``, and the result is a ``CompiledArtifact`` over the HIP
runtime. Failures raise ``CompilationStageError`` tagged with the stage
("frontend_kir" for an unknown definition, "target_resolution" for the
device/library check), as the reference does.
"""
from __future__ import annotations

from dataclasses import dataclass
from pathlib import Path
from typing import Literal

from . import _native
from .artifact import CompiledArtifact
from .definitions import KernelDefinition
from .errors import CompilationStageError
from .runtime import HIPRuntime


@dataclass(frozen=True, slots=True)
class CompileOptions:
    """Numerical policy (python/intent/compiler/options.py:7-57). The HIP kernels
    implement the "source" contract; the other fields are accepted and recorded."""

    numerics: Literal["source", "relaxed_normalization"] = "source"
    online_reduction: bool = True
    optimization_remarks: bool = False

    def __post_init__(self) -> None:
        if self.numerics not in ("source", "relaxed_normalization"):
            raise ValueError("numerics must be 'source' or 'relaxed_normalization'")
        if type(self.online_reduction) is not bool or type(self.optimization_remarks) is not bool:
            raise TypeError("online_reduction and optimization_remarks must be booleans")


@dataclass(frozen=True)
class MI355XTarget:
    """gfx950 (MI355X) device target; ``device`` is the torch/HIP device index."""

    device: int = 0
    arch: str = "gfx950"

    def resolve(self) -> "MI355XTarget":
        import torch

        if not torch.cuda.is_available():
            raise RuntimeError("no HIP device is visible; the MI355X target needs a gfx950 GPU")
        if self.device >= torch.cuda.device_count():
            raise RuntimeError(f"HIP device {self.device} does not exist")
        found = _native.device_arch(self.device).split(":")[0]
        if found != self.arch:
            raise RuntimeError(f"device {self.device} is {found}, not {self.arch}")
        return self


def compile(definition: KernelDefinition, *, target: MI355XTarget, compiler: str | Path | None = None,
            constexprs: dict | None = None, tuning_config: str | Path | None = None,
            options: CompileOptions | None = None) -> CompiledArtifact:
    if not isinstance(definition, KernelDefinition):
        raise CompilationStageError(
            "frontend_kir", f"{definition!r} is not one of the quantized-contraction definitions of intent_amd; "
                            "general DSL kernels are not compiled by this build")
    if options is not None and not isinstance(options, CompileOptions):
        raise TypeError("options must be an intent_amd.CompileOptions or None")
    try:
        values = definition.resolve_constexprs(constexprs)
    except ValueError as error:
        raise CompilationStageError("frontend_kir", str(error)) from error
    try:
        _native.library()
        resolved = target.resolve()
    except Exception as error:
        raise CompilationStageError("target_resolution", str(error)) from error
    runtime = HIPRuntime(definition, resolved.device, values, resolved.arch)
    source = (f"// {definition.name}: hand-written {resolved.arch} HIP kernels in libintent_amd.so\n"
              f"// replaces {definition.reference}\n// {definition.doc}\n")
    return CompiledArtifact(source, "", resolved.device, runtime, device_type="cuda",
                            cache_directory=_native.LIBRARY_PATH.parent)
