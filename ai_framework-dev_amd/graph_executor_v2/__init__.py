"""graph_executor_v2 (MI355X build): the GEMM + bias + activation operator.

Only the operator path of the reference package is provided here: the
``ops`` subpackage with the native ``_ops_common`` / ``_ops_gemm`` modules and
the ``ops.gemm`` glue (reference: graph_executor_v2/python/graph_executor_v2).
"""
