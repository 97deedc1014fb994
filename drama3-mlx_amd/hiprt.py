"""Minimal ctypes access to the HIP runtime the sampler library links
(device memory, copies, streams, events) for the Python tests and the bench.
The library is loaded first so both share one libamdhip64.so.7."""
import ctypes

import numpy as np

_hip = None


def hip():
    global _hip
    if _hip is None:
        import d3s  # loads libd3sampler.so, which pulls in libamdhip64.so.7
        d3s.lib()
        H = ctypes.CDLL("libamdhip64.so.7")
        vp, sz, i32 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int
        H.hipMalloc.argtypes = [ctypes.POINTER(vp), sz]
        H.hipFree.argtypes = [vp]
        H.hipMemcpy.argtypes = [vp, vp, sz, i32]
        H.hipMemcpyAsync.argtypes = [vp, vp, sz, i32, vp]
        H.hipMemset.argtypes = [vp, i32, sz]
        H.hipDeviceSynchronize.argtypes = []
        H.hipGetDeviceCount.argtypes = [ctypes.POINTER(i32)]
        H.hipStreamCreate.argtypes = [ctypes.POINTER(vp)]
        H.hipStreamDestroy.argtypes = [vp]
        H.hipStreamSynchronize.argtypes = [vp]
        H.hipStreamWaitEvent.argtypes = [vp, vp, ctypes.c_uint]
        H.hipEventCreate.argtypes = [ctypes.POINTER(vp)]
        H.hipEventDestroy.argtypes = [vp]
        H.hipEventRecord.argtypes = [vp, vp]
        H.hipEventSynchronize.argtypes = [vp]
        H.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), vp, vp]
        H.hipGetErrorString.argtypes = [i32]
        H.hipGetErrorString.restype = ctypes.c_char_p
        H.hipStreamBeginCapture.argtypes = [vp, i32]
        H.hipStreamEndCapture.argtypes = [vp, ctypes.POINTER(vp)]
        H.hipGraphInstantiate.argtypes = [ctypes.POINTER(vp), vp, vp, ctypes.c_char_p, sz]
        H.hipGraphLaunch.argtypes = [vp, vp]
        H.hipGraphExecDestroy.argtypes = [vp]
        H.hipGraphDestroy.argtypes = [vp]
        H.hipGraphGetNodes.argtypes = [vp, ctypes.POINTER(vp), ctypes.POINTER(sz)]
        H.hipGraphNodeGetType.argtypes = [vp, ctypes.POINTER(i32)]
        for f in ("hipMalloc", "hipFree", "hipMemcpy", "hipMemcpyAsync", "hipMemset",
                  "hipDeviceSynchronize", "hipGetDeviceCount", "hipStreamCreate",
                  "hipStreamDestroy", "hipStreamSynchronize", "hipStreamWaitEvent", "hipEventCreate", "hipEventDestroy",
                  "hipEventRecord", "hipEventSynchronize", "hipEventElapsedTime",
                  "hipStreamBeginCapture", "hipStreamEndCapture", "hipGraphInstantiate",
                  "hipGraphLaunch", "hipGraphExecDestroy", "hipGraphDestroy", "hipGraphGetNodes",
                  "hipGraphNodeGetType"):
            getattr(H, f).restype = i32
        _hip = H
    return _hip


H2D, D2H, D2D = 1, 2, 3
# hipGraphNodeType values (hip_runtime_api.h)
GRAPH_NODE_TYPES = {0: "kernel", 1: "memcpy", 2: "memset", 3: "host", 4: "graph", 5: "empty",
                    6: "wait_event", 7: "event_record", 10: "mem_alloc", 11: "mem_free"}


def check(rc, what="hip"):
    if rc != 0:
        raise RuntimeError(f"{what}: {hip().hipGetErrorString(rc).decode()} ({rc})")


def device_count():
    n = ctypes.c_int(0)
    rc = hip().hipGetDeviceCount(ctypes.byref(n))
    return n.value if rc == 0 else 0


class DeviceBuffer:
    """Device memory of `nbytes`; .ptr is the device address."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        check(hip().hipMalloc(ctypes.byref(p), max(self.nbytes, 1)), "hipMalloc")
        self.ptr = p.value

    def free(self):
        if self.ptr:
            hip().hipFree(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def upload(self, arr, offset=0):
        a = np.ascontiguousarray(arr)
        assert offset + a.nbytes <= self.nbytes
        check(hip().hipMemcpy(self.ptr + offset, a.ctypes.data, a.nbytes, H2D), "hipMemcpy H2D")
        return self

    def download(self, shape, dtype, offset=0):
        out = np.empty(shape, dtype)
        assert offset + out.nbytes <= self.nbytes
        check(hip().hipMemcpy(out.ctypes.data, self.ptr + offset, out.nbytes, D2H), "hipMemcpy D2H")
        return out

    def zero(self):
        check(hip().hipMemset(self.ptr, 0, self.nbytes), "hipMemset")
        return self


def to_device(arr):
    a = np.ascontiguousarray(arr)
    return DeviceBuffer(a.nbytes).upload(a)


def synchronize():
    check(hip().hipDeviceSynchronize(), "hipDeviceSynchronize")


class Stream:
    def __init__(self):
        s = ctypes.c_void_p()
        check(hip().hipStreamCreate(ctypes.byref(s)), "hipStreamCreate")
        self.ptr = s.value

    def synchronize(self):
        check(hip().hipStreamSynchronize(self.ptr), "hipStreamSynchronize")

    def wait(self, event):
        """later work on this stream waits for `event` (no host wait)"""
        check(hip().hipStreamWaitEvent(self.ptr, event.ptr, 0), "hipStreamWaitEvent")

    def destroy(self):
        if self.ptr:
            hip().hipStreamDestroy(self.ptr)
            self.ptr = None


class Event:
    def __init__(self):
        e = ctypes.c_void_p()
        check(hip().hipEventCreate(ctypes.byref(e)), "hipEventCreate")
        self.ptr = e.value

    def record(self, stream=None):
        check(hip().hipEventRecord(self.ptr, stream.ptr if stream else None), "hipEventRecord")

    def synchronize(self):
        check(hip().hipEventSynchronize(self.ptr), "hipEventSynchronize")

    def elapsed_ms(self, end):
        ms = ctypes.c_float()
        check(hip().hipEventElapsedTime(ctypes.byref(ms), self.ptr, end.ptr), "hipEventElapsedTime")
        return ms.value

    def destroy(self):
        if self.ptr:
            hip().hipEventDestroy(self.ptr)
            self.ptr = None


def graph_node_types(graph):
    """The type name of every node of a captured hipGraph_t (by
    hipGraphGetNodes / hipGraphNodeGetType), in the order HIP lists them."""
    H = hip()
    n = ctypes.c_size_t(0)
    check(H.hipGraphGetNodes(graph, None, ctypes.byref(n)), "hipGraphGetNodes")
    nodes = (ctypes.c_void_p * max(n.value, 1))()
    check(H.hipGraphGetNodes(graph, nodes, ctypes.byref(n)), "hipGraphGetNodes")
    out = []
    for i in range(n.value):
        t = ctypes.c_int(-1)
        check(H.hipGraphNodeGetType(nodes[i], ctypes.byref(t)), "hipGraphNodeGetType")
        out.append(GRAPH_NODE_TYPES.get(t.value, f"type{t.value}"))
    return out
