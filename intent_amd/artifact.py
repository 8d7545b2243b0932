"""``CompiledArtifact``: what ``intent_amd.compile`` hands back to the caller.

Public contract kept from the reference (python/intent/runtime/artifact.py:
98-237):
* ``run(*inputs)`` allocates the declared Out buffers and returns None, the
  single Out, or a tuple of them in declaration order; InOut views are
  updated in place;
* ``launch(*all)`` (also the artifact's ``__call__``) takes every argument,
  explicit Out buffers included, and returns None;
* ``prepare(*inputs, outputs=None)`` binds once and returns a prepared call
  with ``compile`` / ``launch`` / ``result`` / ``observation``;
* ``as_torch_op(name)`` registers a PyTorch custom operator;
* ``interface``, ``observation``, ``ir``, ``source``, ``mlir``, ``device``,
  ``device_type`` and ``cache_directory`` describe the artifact;
* a tensor on another device than the artifact's raises ``ValueError``
  before anything launches, and every call runs with the artifact's device
  current (torch's "cuda" device type names the HIP device on ROCm).
"""
from __future__ import annotations

import functools
from pathlib import Path
from typing import Any

from .interface import PublicInterface


def _on_artifact_device(method):
    """Wrap a method taking user arguments: check their devices, then run with the artifact's device current."""

    @functools.wraps(method)
    def wrapper(self, *arguments, **keywords):
        import torch

        home = torch.device(self.device_type, self.device)
        stray = next(((i, a.device) for i, a in enumerate(arguments)
                      if isinstance(a, torch.Tensor) and a.device != home), None)
        if stray is not None:
            raise ValueError(f"argument {stray[0]} lives on {stray[1]}; this artifact is bound to {home}")
        if torch.cuda.current_device() == self.device:
            return method(self, *arguments, **keywords)
        with torch.cuda.device(self.device):
            return method(self, *arguments, **keywords)

    return wrapper


class CompiledArtifact:
    """A bound hot-path operator: the HIP runtime behind it plus descriptive metadata."""

    __slots__ = ("source", "mlir", "device", "runtime", "device_type", "cache_directory", "backend_ir")

    def __init__(self, source: str, mlir: str, device: int, runtime: Any, *, device_type: str = "cuda",
                 cache_directory: Path | None = None) -> None:
        self.source = source
        self.mlir = mlir
        self.device = device
        self.runtime = runtime
        self.device_type = device_type
        self.cache_directory = cache_directory
        self.backend_ir: dict = {}

    def __repr__(self) -> str:
        name = getattr(getattr(self.runtime, "definition", None), "name", "?")
        return f"CompiledArtifact({name} on {self.device_type}:{self.device})"

    # ---- description ---------------------------------------------------------------
    @property
    def interface(self) -> PublicInterface:
        return self.runtime.interface

    @property
    def observation(self):
        """What the most recent launch ran (entry, definition, arch, library), or None before any."""
        return getattr(self.runtime, "observation", None)

    @property
    def ir(self) -> dict:
        # No intermediate representation is produced: the kernels are prebuilt HIP.
        return dict(self.backend_ir, intent=self.mlir)

    @property
    def entry(self):
        return self.launch

    # ---- invocation ----------------------------------------------------------------
    @_on_artifact_device
    def run(self, *inputs: Any) -> object:
        return self.runtime.run(*inputs)

    @_on_artifact_device
    def launch(self, *arguments: Any) -> None:
        self.runtime.launch(*arguments)

    def __call__(self, *arguments: Any) -> None:
        self.launch(*arguments)

    @_on_artifact_device
    def prepare(self, *inputs: Any, outputs: tuple | None = None):
        return self.runtime.prepare_call(inputs, outputs=outputs)

    @_on_artifact_device
    def tuning_configurations(self, *inputs: Any) -> tuple:
        return self.runtime.tuning_configurations(*inputs)

    def inspect_configurations(self, *inputs: Any, outputs: tuple | None = None) -> tuple:
        return self.prepare(*inputs, outputs=outputs).inspect_configurations()

    def as_torch_op(self, name: str):
        from .torch_op import register_operator

        return register_operator(self, name)
