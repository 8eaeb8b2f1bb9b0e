"""hipGraph capture / replay through libd2sd.so (d2sd_graph_* in include/d2sd.h).

Replaces the torch.cuda.CUDAGraph wrapper of model/cascade_graph.py:67-71, 107:
the graph is captured and owned by the C++ side.  Work issued inside
`capture()` must not allocate device memory (every d2sd launch is
allocation-free when given its outputs and workspace).
"""
from __future__ import annotations

import ctypes as C
from contextlib import contextmanager
from typing import Optional

import torch

from ._lib import check, lib


_CAPTURING: list = []


def capturing() -> bool:
    """Whether a HipGraph (or a torch graph on the current stream) is capturing."""
    return bool(_CAPTURING) or torch.cuda.is_current_stream_capturing()


def keep_alive(*objs) -> None:
    """Called by d2sd ops with the device buffers a launch reads or writes:
    while a HipGraph is capturing, it holds references to them for as long as
    the graph exists, so a captured launch never sees freed memory (e.g. after
    the op's owner re-plans into new buffers)."""
    if _CAPTURING:
        _CAPTURING[-1]._keep.extend(o for o in objs if o is not None)


class HipGraph:
    def __init__(self) -> None:
        self._exec: Optional[C.c_void_p] = None
        self.stream: Optional[torch.cuda.Stream] = None
        self._keep: list = []

    @contextmanager
    def capture(self, stream: Optional[torch.cuda.Stream] = None):
        if self._exec is not None:
            raise RuntimeError("HipGraph already captured")
        self.stream = stream if stream is not None else torch.cuda.Stream()
        torch.cuda.synchronize()
        with torch.cuda.stream(self.stream):
            check(lib.d2sd_graph_begin_capture(C.c_void_p(self.stream.cuda_stream)), "graph begin capture")
            exec_ = C.c_void_p()
            _CAPTURING.append(self)
            try:
                yield self
            finally:
                _CAPTURING.pop()
                rc = lib.d2sd_graph_end_capture(C.c_void_p(self.stream.cuda_stream), C.byref(exec_))
            check(rc, "graph end capture")
            self._exec = exec_
        torch.cuda.synchronize()

    def replay(self, stream: Optional[torch.cuda.Stream] = None) -> None:
        if self._exec is None:
            raise RuntimeError("HipGraph.replay before capture")
        s = stream if stream is not None else torch.cuda.current_stream()
        check(lib.d2sd_graph_launch(self._exec, C.c_void_p(s.cuda_stream)), "graph launch")

    def reset(self) -> None:
        if self._exec is not None:
            check(lib.d2sd_graph_destroy(self._exec), "graph destroy")
            self._exec = None
        self._keep = []

    def __del__(self) -> None:
        try:
            if self._exec is not None:
                lib.d2sd_graph_destroy(self._exec)
                self._exec = None
        except Exception:
            pass
