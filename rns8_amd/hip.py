"""Minimal ctypes access to the HIP runtime (device memory and copies).

Used by tests and the benchmark to move data to and from device buffers whose
raw addresses come from the rns8 library (for example the residue planes of a
matrix). Loads the same libamdhip64 the rns8 library links against.
"""
from __future__ import annotations

import ctypes as C

_lib = None
H2D, D2H, D2D = 1, 2, 3


def runtime() -> C.CDLL:
    global _lib
    if _lib is None:
        _lib = C.CDLL("libamdhip64.so")
        _lib.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
        _lib.hipFree.argtypes = [C.c_void_p]
        _lib.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        _lib.hipMemset.argtypes = [C.c_void_p, C.c_int, C.c_size_t]
        _lib.hipDeviceSynchronize.argtypes = []
        _lib.hipGetDeviceCount.argtypes = [C.POINTER(C.c_int)]
    return _lib


def _check(err: int, what: str) -> None:
    if err != 0:
        raise RuntimeError(f"{what} failed with hipError {err}")


def device_count() -> int:
    n = C.c_int(0)
    if runtime().hipGetDeviceCount(C.byref(n)) != 0:
        return 0
    return n.value


def malloc(nbytes: int) -> int:
    p = C.c_void_p()
    _check(runtime().hipMalloc(C.byref(p), max(16, nbytes)), "hipMalloc")
    return p.value


def free(ptr: int) -> None:
    if ptr:
        _check(runtime().hipFree(C.c_void_p(ptr)), "hipFree")


def memset(ptr: int, value: int, nbytes: int) -> None:
    _check(runtime().hipMemset(C.c_void_p(ptr), value, nbytes), "hipMemset")


def to_device(dst: int, array) -> None:
    _check(runtime().hipMemcpy(C.c_void_p(dst), array.ctypes.data_as(C.c_void_p), array.nbytes, H2D), "hipMemcpy H2D")


def from_device(array, src: int) -> None:
    _check(runtime().hipMemcpy(array.ctypes.data_as(C.c_void_p), C.c_void_p(src), array.nbytes, D2H), "hipMemcpy D2H")


def synchronize() -> None:
    _check(runtime().hipDeviceSynchronize(), "hipDeviceSynchronize")


def _bind_streams():
    rt = runtime()
    if getattr(rt, "_streams_bound", False):
        return rt
    rt.hipStreamCreate.argtypes = [C.POINTER(C.c_void_p)]
    rt.hipStreamDestroy.argtypes = [C.c_void_p]
    rt.hipStreamSynchronize.argtypes = [C.c_void_p]
    rt.hipEventCreate.argtypes = [C.POINTER(C.c_void_p)]
    rt.hipEventDestroy.argtypes = [C.c_void_p]
    rt.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]
    rt.hipEventSynchronize.argtypes = [C.c_void_p]
    rt.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
    rt.hipMemcpyAsync.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int, C.c_void_p]
    rt._streams_bound = True
    return rt


def stream_create() -> int:
    s = C.c_void_p()
    _check(_bind_streams().hipStreamCreate(C.byref(s)), "hipStreamCreate")
    return s.value


def stream_destroy(s: int) -> None:
    _check(_bind_streams().hipStreamDestroy(C.c_void_p(s)), "hipStreamDestroy")


def stream_synchronize(s: int) -> None:
    _check(_bind_streams().hipStreamSynchronize(C.c_void_p(s)), "hipStreamSynchronize")


def event_create() -> int:
    e = C.c_void_p()
    _check(_bind_streams().hipEventCreate(C.byref(e)), "hipEventCreate")
    return e.value


def event_destroy(e: int) -> None:
    _check(_bind_streams().hipEventDestroy(C.c_void_p(e)), "hipEventDestroy")


def event_record(e: int, stream: int) -> None:
    _check(_bind_streams().hipEventRecord(C.c_void_p(e), C.c_void_p(stream)), "hipEventRecord")


def event_elapsed_ms(start: int, stop: int) -> float:
    ms = C.c_float(0.0)
    _check(_bind_streams().hipEventSynchronize(C.c_void_p(stop)), "hipEventSynchronize")
    _check(_bind_streams().hipEventElapsedTime(C.byref(ms), C.c_void_p(start), C.c_void_p(stop)),
           "hipEventElapsedTime")
    return float(ms.value)


# ---- graphs (stream capture) ------------------------------------------------------

CAPTURE_MODE_GLOBAL = 0  # hipStreamCaptureModeGlobal: unsafe calls from any thread fail the capture


def _bind_graphs():
    rt = _bind_streams()
    if getattr(rt, "_graphs_bound", False):
        return rt
    rt.hipStreamBeginCapture.argtypes = [C.c_void_p, C.c_int]
    rt.hipStreamEndCapture.argtypes = [C.c_void_p, C.POINTER(C.c_void_p)]
    rt.hipGraphInstantiate.argtypes = [C.POINTER(C.c_void_p), C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t]
    rt.hipGraphLaunch.argtypes = [C.c_void_p, C.c_void_p]
    rt.hipGraphExecDestroy.argtypes = [C.c_void_p]
    rt.hipGraphDestroy.argtypes = [C.c_void_p]
    rt._graphs_bound = True
    return rt


def capture_begin(stream: int) -> None:
    _check(_bind_graphs().hipStreamBeginCapture(C.c_void_p(stream), CAPTURE_MODE_GLOBAL), "hipStreamBeginCapture")


def capture_end(stream: int) -> tuple[int, int]:
    """Ends the capture; returns (graph, executable graph)."""
    rt = _bind_graphs()
    g = C.c_void_p()
    _check(rt.hipStreamEndCapture(C.c_void_p(stream), C.byref(g)), "hipStreamEndCapture")
    ex = C.c_void_p()
    _check(rt.hipGraphInstantiate(C.byref(ex), g, None, None, 0), "hipGraphInstantiate")
    return g.value, ex.value


def graph_launch(exec_graph: int, stream: int) -> None:
    _check(_bind_graphs().hipGraphLaunch(C.c_void_p(exec_graph), C.c_void_p(stream)), "hipGraphLaunch")


def graph_destroy(graph: int, exec_graph: int) -> None:
    rt = _bind_graphs()
    _check(rt.hipGraphExecDestroy(C.c_void_p(exec_graph)), "hipGraphExecDestroy")
    _check(rt.hipGraphDestroy(C.c_void_p(graph)), "hipGraphDestroy")
