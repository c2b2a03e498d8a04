"""Layers on the GEMM operator path (reference: python/graph_executor_v2/layers).

Only ``Dense`` (layers/dense_gemm.py) and the ``Layer`` base it needs are part
of this build.
"""
from .base import Layer
from .dense_gemm import Dense

__all__ = ["Layer", "Dense"]
