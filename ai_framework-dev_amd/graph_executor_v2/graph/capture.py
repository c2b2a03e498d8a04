"""Stream capture into HIP graphs, in the shape the reference's training-step
recorder uses with CuPy (python/graph_executor_v2/graph/graph_exec.py:119-136):

    with capture_stream(stream) as cap:
        layer.forward_into(x, out, z, stream=stream.ptr)
        layer.backward_into(gy, gA, gW, gB, work_dZ=dz, stream=stream.ptr)
    gexec = cap.graph.instantiate()
    gexec.launch(stream)

The calls inside the block are recorded, not run, and allocate nothing: the
*_into paths take every buffer from the caller (the dZ buffer is the
operator's dY' workspace), and an operator call that lacks a workspace it
would use eagerly takes its scratch-free kernels while the stream captures.
No eager warm-up call is needed.
"""
from __future__ import annotations

import ctypes
from contextlib import contextmanager
from typing import Iterator, Optional

from ..ops import capi


def _stream_ptr(stream) -> int:
    p = getattr(stream, "ptr", stream)
    if not p:
        raise ValueError("capture needs a created stream (capi.Stream), not the null stream")
    return int(p)


class GraphExec:
    """An instantiated graph: launch it on a stream any number of times."""

    def __init__(self, ptr: int):
        self.ptr = ptr

    def launch(self, stream) -> None:
        capi.check(capi.lib().gev2_graph_launch(self.ptr, _stream_ptr(stream)), "graph_launch")

    def close(self) -> None:
        if self.ptr:
            capi.lib().gev2_graph_destroy(self.ptr)
            self.ptr = 0

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Graph:
    """The captured graph; the C ABI instantiates it when the capture ends."""

    def __init__(self, exec_ptr: int):
        self._exec: Optional[GraphExec] = GraphExec(exec_ptr)

    def instantiate(self) -> GraphExec:
        if self._exec is None:
            raise RuntimeError("graph already instantiated")
        g, self._exec = self._exec, None
        return g


class _Capture:
    graph: Optional[Graph] = None


@contextmanager
def capture_stream(stream) -> Iterator[_Capture]:
    s = _stream_ptr(stream)
    L = capi.lib()
    capi.check(L.gev2_graph_begin(s), "graph_begin")
    cap = _Capture()
    try:
        yield cap
    except BaseException:
        p = ctypes.c_void_p()
        if L.gev2_graph_end(s, ctypes.byref(p)) == 0 and p.value:
            L.gev2_graph_destroy(p.value)
        raise
    p = ctypes.c_void_p()
    capi.check(L.gev2_graph_end(s, ctypes.byref(p)), "graph_end")
    cap.graph = Graph(int(p.value))
