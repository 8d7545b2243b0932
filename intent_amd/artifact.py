"""``CompiledArtifact``: the operator surface returned by ``intent_amd.compile``.

Same public behaviour as the reference's artifact
(python/intent/runtime/artifact.py:98-237): ``run`` allocates declared Out
buffers and returns None / the single Out / a tuple in declaration order;
``launch`` (also ``__call__``) takes every argument including explicit Out
buffers; ``prepare`` binds once for repeated launches; ``as_torch_op``
registers a PyTorch custom op. Every tensor argument must live on the
artifact's device and the call runs with that device current.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from pathlib import Path
from typing import Any, Callable

from .interface import PublicInterface


@dataclass(slots=True)
class CompiledArtifact:
    source: str
    mlir: str
    device: int
    runtime: Any = field(repr=False)
    device_type: str = field(default="cuda", kw_only=True)
    cache_directory: Path | None = field(default=None, kw_only=True)
    backend_ir: dict = field(default_factory=dict, init=False)

    @property
    def observation(self):
        """Latest native invocation snapshot, or None before the first launch."""
        return getattr(self.runtime, "observation", None)

    @property
    def entry(self) -> Callable[..., None]:
        return self.__call__

    @property
    def ir(self) -> dict:
        return {"intent": self.mlir, **self.backend_ir}

    @property
    def interface(self) -> PublicInterface:
        return self.runtime.interface

    def run(self, *arguments: Any) -> object:
        return self._invoke(self.runtime.run, arguments)

    def prepare(self, *arguments: Any, outputs: tuple | None = None):
        return self._invoke(lambda *args: self.runtime.prepare_call(args, outputs=outputs), arguments)

    def as_torch_op(self, name: str):
        from .torch_op import register_operator

        return register_operator(self, name)

    def tuning_configurations(self, *arguments: Any) -> tuple:
        return self._invoke(self.runtime.tuning_configurations, arguments)

    def inspect_configurations(self, *arguments: Any, outputs: tuple | None = None) -> tuple:
        return self.prepare(*arguments, outputs=outputs).inspect_configurations()

    def launch(self, *arguments: Any) -> None:
        self._invoke(self.runtime.launch, arguments)

    __call__ = launch

    def _invoke(self, function: Callable[..., object], arguments: tuple) -> object:
        import torch

        expected = torch.device(self.device_type, self.device)
        for index, argument in enumerate(arguments):
            if isinstance(argument, torch.Tensor) and argument.device != expected:
                raise ValueError(f"compiled artifact is bound to {expected}, but tensor argument "
                                 f"{index} is on {argument.device}")
        if torch.cuda.current_device() == self.device:
            return function(*arguments)
        with torch.cuda.device(self.device):
            return function(*arguments)
