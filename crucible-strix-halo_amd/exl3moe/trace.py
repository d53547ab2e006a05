"""HIP events for the library's stage trace (cx_moe_plan_set_trace), via libamdhip64."""
from __future__ import annotations

import ctypes

from . import check, lib

_hip = None


def hip() -> ctypes.CDLL:
    global _hip
    if _hip is None:
        _hip = ctypes.CDLL("libamdhip64.so")
        _hip.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        _hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
        _hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        _hip.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        _hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    return _hip


class EventTimer:
    """Per-call device times of calls issued on one stream (default: the null stream):
    an event is recorded before each call and after the last."""

    def __init__(self, calls: int, stream=None):
        self.n = calls + 1
        self.stream = stream
        self.events = []
        for _ in range(self.n):
            h = ctypes.c_void_p()
            if hip().hipEventCreate(ctypes.byref(h)) != 0:
                raise RuntimeError("hipEventCreate failed")
            self.events.append(h.value)
        self.i = 0

    def mark(self):
        if hip().hipEventRecord(self.events[self.i], self.stream) != 0:
            raise RuntimeError("hipEventRecord failed")
        self.i += 1

    def ms(self) -> list[float]:
        hip().hipEventSynchronize(self.events[self.i - 1])
        t = ctypes.c_float()
        out = []
        for a, b in zip(self.events[:self.i - 1], self.events[1:self.i]):
            if hip().hipEventElapsedTime(ctypes.byref(t), a, b) != 0:
                raise RuntimeError("hipEventElapsedTime failed")
            out.append(t.value)
        return out

    def close(self):
        for e in self.events:
            hip().hipEventDestroy(e)
        self.events = []


class StageTrace:
    """A ring of hipEvents the plan records between its stages (8 marks per call)."""

    MARKS = 8
    STAGES = ["route", "group", "input", "gate_up", "mid", "down", "combine"]

    def __init__(self, plan, calls: int):
        self.plan = plan
        self.calls = calls
        n = calls * self.MARKS
        self.events = (ctypes.c_void_p * n)()
        for i in range(n):
            h = ctypes.c_void_p()
            rc = hip().hipEventCreate(ctypes.byref(h))
            self.events[i] = h.value
            if rc != 0:
                raise RuntimeError(f"hipEventCreate failed ({rc})")
        check("cx_moe_plan_set_trace", lib().cx_moe_plan_set_trace(plan.handle, self.events, n))

    def stage_ms(self, calls: int | None = None) -> list[list[float]]:
        """Per call, the duration of each stage in ms, for the first `calls` traced calls
        (default: all the ring holds).  Call after the traced calls finished."""
        out = []
        t = ctypes.c_float()
        for c in range(self.calls if calls is None else calls):
            base = c * self.MARKS
            hip().hipEventSynchronize(self.events[base + self.MARKS - 1])
            row = []
            for s in range(self.MARKS - 1):
                rc = hip().hipEventElapsedTime(ctypes.byref(t), self.events[base + s], self.events[base + s + 1])
                if rc != 0:
                    raise RuntimeError(f"hipEventElapsedTime failed ({rc})")
                row.append(t.value)
            out.append(row)
        return out

    def close(self):
        if self.plan is not None and getattr(self.plan, "handle", None):
            lib().cx_moe_plan_set_trace(self.plan.handle, None, 0)
        for i in range(len(self.events)):
            if self.events[i]:
                hip().hipEventDestroy(self.events[i])
        self.plan = None
