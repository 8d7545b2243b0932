"""Typed public parameters of a compiled definition.

Same concepts and field meanings as the reference's public interface
(python/intent/runtime/interface.py:16-47,100-185; ViewKind values from
python/intent/language/annotations.py:77-80): author-ordered views and
scalars, symbolic extents as -1 with a dimension identity shared by axes that
must agree, element strides (None = unconstrained, 1 = unit), access In / Out /
InOut. Only the pieces this operator family needs are restated.
"""
from __future__ import annotations

from dataclasses import dataclass
from enum import IntEnum


class ViewKind(IntEnum):
    IN = 0
    OUT = 1
    INOUT = 2


@dataclass(frozen=True, slots=True)
class DType:
    name: str
    bits: int
    category: str  # "float", "bfloat", "signed", "unsigned", "bool"

    @property
    def bytes(self) -> int:
        return self.bits // 8

    def __str__(self) -> str:
        return self.name


DTYPES = {
    "f16": DType("f16", 16, "float"),
    "bf16": DType("bf16", 16, "bfloat"),
    "f32": DType("f32", 32, "float"),
    "i8": DType("i8", 8, "signed"),
    "u8": DType("u8", 8, "unsigned"),
    "i32": DType("i32", 32, "signed"),
    "i64": DType("i64", 64, "signed"),
    "bool": DType("bool", 8, "bool"),
    "f8e4m3fn": DType("f8e4m3fn", 8, "float"),
    "f8e5m2": DType("f8e5m2", 8, "float"),
}


def dtype(name: str) -> DType:
    try:
        return DTYPES[name]
    except KeyError:
        raise ValueError(f"unsupported dtype {name!r}") from None


def torch_dtype(element: DType):
    import torch

    return {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32, "i8": torch.int8,
            "u8": torch.uint8, "i32": torch.int32, "i64": torch.int64, "bool": torch.bool,
            "f8e4m3fn": torch.float8_e4m3fn, "f8e5m2": torch.float8_e5m2}[element.name]


@dataclass(frozen=True, slots=True)
class ScalarParameter:
    position: int
    name: str
    dtype: DType


@dataclass(frozen=True, slots=True)
class ViewParameter:
    position: int
    name: str
    dtype: DType
    shape: tuple[int, ...]
    dimensions: tuple[int, ...]
    strides: tuple[int | None, ...]
    access: ViewKind
    alias: str = ""
    noalias: bool = False

    @property
    def writable(self) -> bool:
        return self.access is not ViewKind.IN

    @property
    def output(self) -> bool:
        return self.access is ViewKind.OUT


@dataclass(frozen=True, slots=True)
class PublicInterface:
    parameters: tuple[ScalarParameter | ViewParameter, ...]

    @property
    def views(self) -> tuple[ViewParameter, ...]:
        return tuple(p for p in self.parameters if isinstance(p, ViewParameter))

    @property
    def inputs(self) -> tuple[ScalarParameter | ViewParameter, ...]:
        return tuple(p for p in self.parameters if not isinstance(p, ViewParameter) or not p.output)

    @property
    def outputs(self) -> tuple[ViewParameter, ...]:
        """Declared Out buffers; an InOut remains a supplied input."""
        return tuple(v for v in self.views if v.output)

    @property
    def mutable_inputs(self) -> tuple[ViewParameter, ...]:
        return tuple(v for v in self.views if v.access is ViewKind.INOUT)

    def explicit_arguments(self, arguments: tuple, outputs: tuple) -> tuple:
        """Merge inputs and explicit Out buffers into declaration order."""
        if len(arguments) != len(self.inputs):
            raise TypeError(f"expected {len(self.inputs)} input arguments, got {len(arguments)}")
        if len(outputs) != len(self.outputs):
            raise TypeError(f"expected {len(self.outputs)} explicit output buffers, got {len(outputs)}")
        supplied, allocated = iter(arguments), iter(outputs)
        return tuple(next(allocated) if isinstance(p, ViewParameter) and p.output else next(supplied)
                     for p in self.parameters)
