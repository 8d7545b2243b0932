"""Expose a compiled artifact as a PyTorch custom operator.

Contract kept from the reference (python/intent/runtime/torch.py:27-93):
* every input appears in the schema in author order; an InOut view is written
  ``Tensor(aN!)`` (N = its input position) and declared mutated; Out views are
  the returned tensors (``()`` when there are none);
* integer scalars are ``SymInt``, floating ones ``float``, booleans ``bool``;
* the fake kernel derives outputs from shapes through the runtime's binder and
  never launches device code;
* a writable view that shares storage with another input raises
  ``NotImplementedError`` (functionalization may clone it on its own);
* a name that is not ``namespace::operator`` raises ``ValueError``.

Here the schema arguments carry the interface's own parameter names, so a
traced graph reads like the operator's signature.
"""
from __future__ import annotations

from dataclasses import dataclass

from .interface import PublicInterface, ScalarParameter, ViewParameter

# Schema spelling of a scalar parameter, keyed by the dtype category.
SCALAR_TYPES = {"bool": "bool", "signed": "SymInt", "unsigned": "SymInt", "float": "float", "bfloat": "float"}


@dataclass(frozen=True)
class OperatorSchema:
    """Schema text plus what the kernel wrapper needs to enforce it."""

    text: str
    names: tuple[str, ...]
    mutated: tuple[str, ...]
    writable_positions: tuple[int, ...]
    tensor_positions: tuple[int, ...]

    @classmethod
    def from_interface(cls, interface: PublicInterface) -> "OperatorSchema":
        fields, names, mutated, writable, tensors = [], [], [], [], []
        for position, p in enumerate(interface.inputs):
            if isinstance(p, ViewParameter):
                tensors.append(position)
                if p.writable:
                    writable.append(position)
                    mutated.append(p.name)
                    token = f"Tensor(a{position}!)"
                else:
                    token = "Tensor"
            elif isinstance(p, ScalarParameter) and p.dtype.category in SCALAR_TYPES:
                token = SCALAR_TYPES[p.dtype.category]
            else:
                raise NotImplementedError(f"no PyTorch schema type for parameter {p.name} ({p.dtype})")
            fields.append(f"{token} {p.name}")
            names.append(p.name)
        if not tensors:
            raise NotImplementedError("a PyTorch operator needs at least one tensor input to pick its device")
        results = ["Tensor"] * len(interface.outputs)
        returns = results[0] if len(results) == 1 else f"({', '.join(results)})"
        return cls(f"({', '.join(fields)}) -> {returns}", tuple(names), tuple(mutated), tuple(writable),
                   tuple(tensors))

    def positional(self, args: tuple, kwargs: dict) -> tuple:
        """Arguments in schema order, whether the dispatcher passed them by position or by name."""
        if not kwargs:
            return args
        values = list(args) + [None] * (len(self.names) - len(args))
        for name, value in kwargs.items():
            values[self.names.index(name)] = value
        return tuple(values)

    def reject_shared_storage(self, args: tuple) -> None:
        import torch

        for w in self.writable_positions:
            for other in self.tensor_positions:
                if other != w and torch._C._is_alias_of(args[w], args[other]):
                    raise NotImplementedError(
                        f"{self.names[w]} is written in place but shares storage with {self.names[other]}; "
                        "a PyTorch operator needs separate storage here (call the artifact directly instead)")


def _checked_namespace(name: str) -> str:
    parts = name.split("::")
    if len(parts) == 2 and all(part.isidentifier() for part in parts):
        return name
    raise ValueError(f"operator name {name!r} must have the form 'namespace::operator'")


def register_operator(artifact, name: str):
    import torch

    qualified = _checked_namespace(name)
    schema = OperatorSchema.from_interface(artifact.interface)

    def real(*args, **kwargs):
        bound = schema.positional(args, kwargs)
        schema.reject_shared_storage(bound)
        return artifact.run(*bound)

    def fake(*args, **kwargs):
        bound = schema.positional(args, kwargs)
        schema.reject_shared_storage(bound)
        return artifact.runtime.infer_outputs(bound)

    op = torch.library.custom_op(qualified, real, mutates_args=schema.mutated,
                                 device_types=artifact.device_type, schema=schema.text)
    op.register_fake(fake)
    return op
