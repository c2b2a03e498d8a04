"""Layer base class (reference: python/graph_executor_v2/layers/base.py:7-200), reduced to
what the GEMM layer uses: lazy build on first call, train / eval, forward and
backward hooks, capture-safe hooks, and parameter / gradient access.  Parameters
are device arrays (see graph_executor_v2.ops.common)."""
from __future__ import annotations

from typing import Any, Iterable, List, Optional, Tuple


class Layer:
    def __init__(self, *, name: Optional[str] = None, build_on_call: bool = True) -> None:
        self.name: Optional[str] = name
        self.built: bool = False
        self.training: bool = True
        self.build_on_call: bool = bool(build_on_call)
        self.input_shape: Optional[Tuple[int, ...]] = None
        self.output_shape: Optional[Tuple[Optional[int], ...]] = None

    # ---------- lifecycle (base.py:33-55) ----------
    def build(self, input_shape: Tuple[int, ...]) -> None:
        self.input_shape = tuple(int(x) if x is not None else None for x in input_shape)
        try:
            self.output_shape = self.compute_output_shape(input_shape)
        except NotImplementedError:
            self.output_shape = tuple(input_shape)
        self.built = True

    def compute_output_shape(self, input_shape: Tuple[int, ...]) -> Tuple[Optional[int], ...]:
        if input_shape is None:
            raise ValueError("input_shape must not be None")
        return tuple(int(x) if x is not None else None for x in input_shape)

    # ---------- forward / backward (base.py:57-79) ----------
    def call(self, x):
        raise NotImplementedError(f"{self.__class__.__name__}.call is not implemented")

    def backward(self, grad_output):
        raise NotImplementedError(f"{self.__class__.__name__}.backward is not implemented")

    def __call__(self, x):
        if (not self.built) and self.build_on_call:
            if not hasattr(x, "shape"):
                raise ValueError("__call__ received an input without 'shape'")
            self.build(tuple(int(s) for s in x.shape))
        return self.call(x)

    # ---------- capture-safe hooks (base.py:81-91) ----------
    def forward_into(self, x, out, **_kw: Any) -> None:
        raise NotImplementedError(f"{self.__class__.__name__}.forward_into is not implemented")

    def backward_into(self, grad_output, **_kw: Any) -> None:
        raise NotImplementedError(f"{self.__class__.__name__}.backward_into is not implemented")

    # ---------- params / grads ----------
    def param_triples(self) -> Iterable[Tuple[Any, Optional[Any], str]]:
        return iter(())

    def parameters(self) -> List[Any]:
        return [p for (p, _g, _n) in self.param_triples()]

    def grads(self) -> List[Optional[Any]]:
        return [g for (_p, g, _n) in self.param_triples()]

    def zero_grad(self) -> None:
        for (_p, g, _n) in self.param_triples():
            if g is not None:
                g.fill(0)

    # ---------- training mode (base.py:152-158) ----------
    def train(self, mode: bool = True) -> "Layer":
        self.training = bool(mode)
        return self

    def eval(self) -> "Layer":
        self.training = False
        return self
