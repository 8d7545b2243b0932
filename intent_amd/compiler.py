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


NUMERICS_POLICIES = ("source", "relaxed_normalization")


class CompileOptions:
    """Numerical policy accepted by ``compile`` (fields of python/intent/compiler/options.py:8-35).

    The HIP kernels implement the ``"source"`` contract (f32 accumulation, no
    TF32, no flush-to-zero); the other settings are validated and recorded so
    that calls written for the reference keep working. Instances are immutable
    and compare by value.
    """

    __slots__ = ("numerics", "online_reduction", "optimization_remarks")

    def __init__(self, numerics: Literal["source", "relaxed_normalization"] = "source",
                 online_reduction: bool = True, optimization_remarks: bool = False) -> None:
        if numerics not in NUMERICS_POLICIES:
            raise ValueError(f"numerics={numerics!r} is not one of {NUMERICS_POLICIES}")
        for label, flag in (("online_reduction", online_reduction), ("optimization_remarks", optimization_remarks)):
            if not isinstance(flag, bool):
                raise TypeError(f"{label} takes a bool, got {type(flag).__name__}")
        object.__setattr__(self, "numerics", numerics)
        object.__setattr__(self, "online_reduction", online_reduction)
        object.__setattr__(self, "optimization_remarks", optimization_remarks)

    def __setattr__(self, name, value):
        raise AttributeError("CompileOptions is immutable")

    def _key(self) -> tuple:
        return (self.numerics, self.online_reduction, self.optimization_remarks)

    def __eq__(self, other) -> bool:
        return isinstance(other, CompileOptions) and self._key() == other._key()

    def __hash__(self) -> int:
        return hash(self._key())

    def __repr__(self) -> str:
        return ("CompileOptions(numerics={!r}, online_reduction={!r}, optimization_remarks={!r})"
                .format(*self._key()))


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
