"""HIP graph capture for the capture-safe layer paths (forward_into / backward_into)."""
from .capture import Graph, GraphExec, capture_stream

__all__ = ["Graph", "GraphExec", "capture_stream"]
