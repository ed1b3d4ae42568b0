"""HIP event timing on the library's own stream (the stream every jas_* kernel launches on
when called with a NULL stream), through the HIP runtime that libjasmine_hip.so links."""
import ctypes as C

from .capi import lib

_hip = None


def hip():
    global _hip
    if _hip is None:
        _hip = C.CDLL("libamdhip64.so", mode=C.RTLD_GLOBAL)
        _hip.hipEventCreate.argtypes = [C.POINTER(C.c_void_p)]
        _hip.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]
        _hip.hipEventSynchronize.argtypes = [C.c_void_p]
        _hip.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
        _hip.hipEventDestroy.argtypes = [C.c_void_p]
    return _hip


def _ok(rc, what):
    if rc != 0:
        raise RuntimeError(f"{what} failed with hipError {rc}")


class EventTimer:
    """t = EventTimer(); t.start(); <launches>; ms = t.stop()  -- GPU time between the two
    event records on `stream` (default: the library stream)."""

    def __init__(self, stream=None):
        h = hip()
        self.stream = stream if stream is not None else lib.jas_default_stream()
        self.a, self.b = C.c_void_p(), C.c_void_p()
        _ok(h.hipEventCreate(C.byref(self.a)), "hipEventCreate")
        _ok(h.hipEventCreate(C.byref(self.b)), "hipEventCreate")

    def start(self):
        _ok(hip().hipEventRecord(self.a, self.stream), "hipEventRecord")

    def stop(self):
        h = hip()
        _ok(h.hipEventRecord(self.b, self.stream), "hipEventRecord")
        _ok(h.hipEventSynchronize(self.b), "hipEventSynchronize")
        ms = C.c_float()
        _ok(h.hipEventElapsedTime(C.byref(ms), self.a, self.b), "hipEventElapsedTime")
        return ms.value

    def __del__(self):
        if _hip is not None:
            for e in (self.a, self.b):
                if e:
                    _hip.hipEventDestroy(e)


_gate_buf = None


def busy_gate(stream=None, elems=1 << 28):
    """Enqueue about a millisecond of device work (a seeded normal fill of `elems` floats)
    so that launches enqueued right after it queue up behind it and then run back to back:
    the events that follow measure device time, not the host's launch rate."""
    global _gate_buf
    if _gate_buf is None:
        p = C.c_void_p()
        _ok(lib.jas_malloc(C.byref(p), elems * 4), "jas_malloc")
        _gate_buf = p
    _ok(lib.jas_fill_normal(_gate_buf, elems, 0, 0, C.c_float(0.0), C.c_float(1.0),
                            stream if stream is not None else None), "jas_fill_normal")


def time_launches(fn, reps, warmup=2, stream=None, gate=True):
    """Average GPU milliseconds per call of fn() (each call enqueues the launches to time).
    With `gate`, the timed launches are queued behind busy_gate(), so short kernels are timed
    back to back instead of at the host's launch rate."""
    for _ in range(warmup):
        fn()
    t = EventTimer(stream)
    if gate:
        busy_gate(stream)
    t.start()
    for _ in range(reps):
        fn()
    return t.stop() / reps
