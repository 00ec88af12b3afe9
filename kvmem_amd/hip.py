"""The few HIP runtime calls that callers of the recall library need beside
it: events for timing and stream capture into graphs.  Plumbing only; the
recall work itself goes through the C ABI in _capi."""
from __future__ import annotations

import ctypes as C
from typing import Optional

_CAPTURE_MODE_RELAXED = 2   # hipStreamCaptureModeRelaxed
_EVENT_RECORD_EXTERNAL = 1  # hipEventRecordExternal


class HipError(RuntimeError):
    pass


class Hip:
    def __init__(self):
        self.lib = C.CDLL("libamdhip64.so")
        L = self.lib
        vp = C.c_void_p
        L.hipEventCreate.argtypes = [C.POINTER(vp)]
        L.hipEventDestroy.argtypes = [vp]
        L.hipEventRecord.argtypes = [vp, vp]
        L.hipEventRecordWithFlags.argtypes = [vp, vp, C.c_uint]
        L.hipEventSynchronize.argtypes = [vp]
        L.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), vp, vp]
        L.hipStreamWaitEvent.argtypes = [vp, vp, C.c_uint]
        L.hipStreamSynchronize.argtypes = [vp]
        L.hipStreamBeginCapture.argtypes = [vp, C.c_int]
        L.hipStreamEndCapture.argtypes = [vp, C.POINTER(vp)]
        L.hipGraphInstantiate.argtypes = [C.POINTER(vp), vp, vp, vp, C.c_size_t]
        L.hipGraphLaunch.argtypes = [vp, vp]
        L.hipGraphExecDestroy.argtypes = [vp]
        L.hipGraphDestroy.argtypes = [vp]
        L.hipMemcpy.argtypes = [vp, vp, C.c_size_t, C.c_int]
        L.hipDeviceSynchronize.argtypes = []
        L.hipGetErrorString.argtypes = [C.c_int]
        L.hipGetErrorString.restype = C.c_char_p

    def ok(self, e: int, what: str) -> None:
        if e != 0:
            raise HipError(f"{what}: {self.lib.hipGetErrorString(e).decode()} ({e})")

    # ---- events --------------------------------------------------------------
    def event(self) -> int:
        e = C.c_void_p()
        self.ok(self.lib.hipEventCreate(C.byref(e)), "hipEventCreate")
        return e.value

    def destroy_event(self, ev: int) -> None:
        self.ok(self.lib.hipEventDestroy(ev), "hipEventDestroy")

    def record(self, ev: int, stream: int, external: bool = False) -> None:
        """Record `ev` on `stream`; `external` makes it an event node of a
        graph being captured (so replays record it too)."""
        if external:
            self.ok(self.lib.hipEventRecordWithFlags(ev, stream, _EVENT_RECORD_EXTERNAL), "hipEventRecordWithFlags")
        else:
            self.ok(self.lib.hipEventRecord(ev, stream), "hipEventRecord")

    def wait(self, stream: int, ev: int) -> None:
        self.ok(self.lib.hipStreamWaitEvent(stream, ev, 0), "hipStreamWaitEvent")

    def elapsed_ms(self, a: int, b: int) -> float:
        ms = C.c_float()
        self.ok(self.lib.hipEventElapsedTime(C.byref(ms), a, b), "hipEventElapsedTime")
        return ms.value

    def stream_sync(self, stream: int) -> None:
        self.ok(self.lib.hipStreamSynchronize(stream), "hipStreamSynchronize")

    def sync(self) -> None:
        self.ok(self.lib.hipDeviceSynchronize(), "hipDeviceSynchronize")

    def d2h(self, dst: int, src: int, n: int) -> None:
        self.ok(self.lib.hipMemcpy(dst, src, n, 2), "hipMemcpy D2H")

    # ---- graphs --------------------------------------------------------------
    def begin_capture(self, stream: int) -> None:
        self.ok(self.lib.hipStreamBeginCapture(stream, _CAPTURE_MODE_RELAXED), "hipStreamBeginCapture")

    def end_capture(self, stream: int) -> int:
        g = C.c_void_p()
        self.ok(self.lib.hipStreamEndCapture(stream, C.byref(g)), "hipStreamEndCapture")
        return g.value

    def instantiate(self, graph: int) -> int:
        ex = C.c_void_p()
        self.ok(self.lib.hipGraphInstantiate(C.byref(ex), graph, None, None, 0), "hipGraphInstantiate")
        return ex.value

    def launch(self, graph_exec: int, stream: int) -> None:
        self.ok(self.lib.hipGraphLaunch(graph_exec, stream), "hipGraphLaunch")

    def destroy_graph(self, graph: Optional[int], graph_exec: Optional[int] = None) -> None:
        if graph_exec:
            self.ok(self.lib.hipGraphExecDestroy(graph_exec), "hipGraphExecDestroy")
        if graph:
            self.ok(self.lib.hipGraphDestroy(graph), "hipGraphDestroy")


class Graph:
    """A capture of work enqueued on `stream` (and on streams forked from it
    through events, which must be joined back before `end`)."""

    def __init__(self, hip: Hip, stream: int):
        self.hip, self.stream = hip, stream
        self.graph = self.exec = None

    def begin(self) -> "Graph":
        self.hip.begin_capture(self.stream)
        return self

    def end(self) -> "Graph":
        self.graph = self.hip.end_capture(self.stream)
        self.exec = self.hip.instantiate(self.graph)
        return self

    def abort(self) -> None:
        """End a capture that failed part-way and drop what it recorded."""
        try:
            g = self.hip.end_capture(self.stream)
        except HipError:
            g = None
        if g:
            self.hip.destroy_graph(g)

    def replay(self, stream: Optional[int] = None) -> None:
        self.hip.launch(self.exec, self.stream if stream is None else stream)

    def close(self) -> None:
        self.hip.destroy_graph(self.graph, self.exec)
        self.graph = self.exec = None


_HIP: Optional[Hip] = None


def runtime() -> Hip:
    global _HIP
    if _HIP is None:
        _HIP = Hip()
    return _HIP
