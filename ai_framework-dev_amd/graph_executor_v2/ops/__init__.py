"""Operator modules (reference: python/graph_executor_v2/ops/__init__.py).

The native extensions ``_ops_common`` and ``_ops_gemm`` are imported lazily by
the glue modules; importing this package never loads a GPU library.
"""
