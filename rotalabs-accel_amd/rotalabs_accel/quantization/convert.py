"""Whole-model conversion: every ``nn.Linear`` of a module tree replaced by
its int8 counterpart -- the ``quantize_model`` recipe of the reference's GEMM
guide (docs/api/kernels/gemm.md:87-107), as a function.
"""
from __future__ import annotations

from typing import Callable, Iterable, Optional, Type

import torch

from rotalabs_accel.quantization.symmetric import QuantizedLinear


def quantize_model(model: torch.nn.Module, linear_cls: Optional[Type[torch.nn.Module]] = None,
                   skip: Iterable[str] = (),
                   predicate: Optional[Callable[[str, torch.nn.Linear], bool]] = None) -> torch.nn.Module:
    """Replace, in place, each ``nn.Linear`` child (recursively) by
    ``linear_cls.from_linear(child)`` and return ``model``.

    linear_cls: ``QuantizedLinear`` (default, as the recipe) or ``Int8Linear``
        -- any class with a ``from_linear`` constructor.
    skip: qualified names (``"lm_head"``, ``"layers.0.mlp.down"``) left as is.
    predicate: optional filter ``(qualified_name, linear) -> bool``.
    Both int8 modules run the W8A16 GEMM on GPU tensors and keep their
    state_dict layout (weight_int8, per-channel scale, bias).
    """
    cls = linear_cls or QuantizedLinear
    skip = set(skip)

    def walk(module: torch.nn.Module, prefix: str) -> None:
        for name, child in module.named_children():
            qual = f"{prefix}.{name}" if prefix else name
            if isinstance(child, torch.nn.Linear) and not isinstance(child, cls):
                if qual in skip or (predicate is not None and not predicate(qual, child)):
                    continue
                setattr(module, name, cls.from_linear(child))
            else:
                walk(child, qual)

    walk(model, "")
    return model
