"""PyTorch custom-op registration for compiled artifacts.

Behaviour of the reference's registration (python/intent/runtime/torch.py:
27-93): the schema lists every input in author order, InOut views become
``Tensor(aN!)`` and are declared in ``mutates_args``; Out views are returned;
the fake implementation infers outputs from shapes without running device
code; a mutable input sharing storage with another input is rejected.
"""
from __future__ import annotations

from inspect import Parameter, Signature

from .interface import ScalarParameter, ViewParameter


def register_operator(artifact, name: str):
    import torch

    interface = artifact.interface
    inputs = interface.inputs
    views = tuple((index, p) for index, p in enumerate(inputs) if isinstance(p, ViewParameter))
    if not views:
        raise NotImplementedError("PyTorch registration requires an input tensor to determine device dispatch")
    pieces = name.split("::")
    if len(pieces) != 2 or not all(piece.isidentifier() for piece in pieces):
        raise ValueError("operator name must be 'your_namespace::your_operator'")
    mutable_names = tuple(f"arg{index}" for index, p in views if p.writable)
    writable_pairs = tuple((i, j, a.name, b.name) for n, (i, a) in enumerate(views) for j, b in views[n + 1:]
                           if a.writable or b.writable)
    parameters = []
    for index, p in enumerate(inputs):
        if isinstance(p, ViewParameter):
            kind = f"Tensor(a{index}!)" if p.writable else "Tensor"
        elif isinstance(p, ScalarParameter):
            if p.dtype.category == "bool":
                kind = "bool"
            elif p.dtype.category in ("signed", "unsigned"):
                kind = "SymInt"
            else:
                kind = "float"
        parameters.append(f"{kind} arg{len(parameters)}")
    outs = interface.outputs
    if not outs:
        returns = "()"
    elif len(outs) == 1:
        returns = "Tensor"
    else:
        returns = "(" + ", ".join("Tensor" for _ in outs) + ")"
    schema = f"({', '.join(parameters)}) -> {returns}"
    signature = Signature(Parameter(f"arg{i}", Parameter.POSITIONAL_OR_KEYWORD) for i in range(len(parameters)))

    def wrap(invoke):
        def operator(*arguments, **keywords):
            arguments = signature.bind(*arguments, **keywords).args
            for left, right, left_name, right_name in writable_pairs:
                if torch._C._is_alias_of(arguments[left], arguments[right]):
                    raise NotImplementedError(
                        f"PyTorch mutable calls require independent input storage: {left_name} and "
                        f"{right_name} share storage; use ordinary artifact calls for this binding")
            return invoke(*arguments)

        return operator

    operator = torch.library.custom_op(name, wrap(artifact.run), mutates_args=mutable_names,
                                       device_types=artifact.device_type, schema=schema)
    operator.register_fake(wrap(lambda *arguments: artifact.runtime.infer_outputs(arguments)))
    return operator
