"""Kernel dispatch helper -- mirror of src/dispatch.js:17-48.

run(kernel, buffers, grid, group, params) binds device buffers by slot
index, inline bytes at params['index'], and dispatches grid = TOTAL threads
(Metal dispatchThreads semantics, which the bridge keeps) then waits, or
records the GPU time when profiling is on.
"""
from . import device

GROUP_1D = 256
_profiling = False
_records = {}


def enable_profiling(on=True):
    global _profiling
    _profiling = bool(on)
    if on:
        _records.clear()


def is_profiling_enabled():
    return _profiling


def record_kernel(name, ms):
    r = _records.setdefault(name, {"count": 0, "totalMs": 0.0})
    r["count"] += 1
    r["totalMs"] += ms


def report():
    return {k: dict(v) for k, v in _records.items()}


def run(kernel, buffers, grid, group=None, params=None):
    pso = device.pipeline(kernel)
    enc = device.begin()
    device.set_pipeline(enc, pso)
    for b in buffers:
        device.set_buffer(enc, b["buffer"], b["index"])
    if params is not None:
        device.set_bytes(enc, params["data"], params["index"])
    gx = grid.get("x", 1) or 1
    gy = grid.get("y", 1) or 1
    gz = grid.get("z", 1) or 1
    group = group or {}
    bx = group.get("x") or min(gx, GROUP_1D)
    by = group.get("y") or 1
    bz = group.get("z") or 1
    device.dispatch(enc, gx, gy, gz, bx, by, bz)
    if _profiling:
        t = device.end_timed(enc)
        record_kernel(kernel, t["gpuMs"])
    else:
        device.end_sync(enc)
