"""HIP context and device buffers over the C ABI (include/orca_hip.h)."""
from __future__ import annotations

import ctypes
import json

import numpy as np

from . import _lib


class Context:
    """One HIP device, its stream and its caching allocator
    (orca_hip_ctx_create).  Plays the role of the process-global backend
    behind global_backend_gpu() (orca-python/src/lib.rs:23-33)."""

    # Dropped buffers are released in batches of this many (orca_hip_free_many): one call
    # instead of one per storage.  The allocator reuses a block once it is released.
    RELEASE_BATCH = 64

    def __init__(self, device: int = 0):
        h = ctypes.c_void_p()
        _lib.call("orca_hip_ctx_create", device, ctypes.byref(h))
        self.handle = h
        self.device = device
        self._dropped = []  # device pointers of dropped buffers not yet released
        self.on_side = False  # launches go to the second stream (use_side_stream)

    def release(self, ptr: int) -> None:
        """Releases a buffer's block (batched; see RELEASE_BATCH)."""
        dropped = self._dropped
        dropped.append(ptr)
        if len(dropped) >= self.RELEASE_BATCH:
            self.release_dropped()

    def release_dropped(self) -> None:
        dropped, self._dropped = self._dropped, []
        if dropped and self.handle:
            _lib.call("orca_hip_free_many", self.handle, (ctypes.c_void_p * len(dropped))(*dropped), len(dropped))

    def close(self) -> None:
        if self.handle:
            self.release_dropped()
            _lib.call("orca_hip_ctx_destroy", self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ---- memory ----
    def alloc(self, nbytes: int) -> "Buffer":
        p = ctypes.c_void_p()
        _lib.call("orca_hip_alloc", self.handle, nbytes, ctypes.byref(p))
        return Buffer(self, p.value, nbytes)

    def upload(self, arr: np.ndarray) -> "Buffer":
        arr = np.ascontiguousarray(arr)
        buf = self.alloc(max(arr.nbytes, 4))
        if arr.nbytes:
            _lib.call("orca_hip_h2d", self.handle, buf.ptr, arr.ctypes.data_as(ctypes.c_void_p), arr.nbytes)
        return buf

    def fill(self, buf: "Buffer", value: float, count: int) -> None:
        _lib.call("orca_hip_fill", self.handle, buf.ptr, value, count)

    def d2d(self, dst: "Buffer", src: "Buffer", nbytes: int) -> None:
        _lib.call("orca_hip_d2d", self.handle, dst.ptr, src.ptr, nbytes)

    def sync(self) -> None:
        self.release_dropped()
        _lib.call("orca_hip_sync", self.handle)

    # ---- the second stream (orca_hip_use_side_stream) and events that order the two ----
    def use_side_stream(self, blocks_per_cu: int) -> None:
        """Later launches go to the second stream (blocks_per_cu != 0: an optimizer pass there
        takes at most that many blocks per CU if > 0, its full grid if < 0) or back (0)."""
        _lib.call("orca_hip_use_side_stream", self.handle, int(blocks_per_cu))
        self.on_side = blocks_per_cu != 0

    def event_record(self) -> int:
        """An event marking the current stream's work so far (orca_hip_event_record)."""
        ev = ctypes.c_void_p()
        _lib.call("orca_hip_event_record", self.handle, ctypes.byref(ev))
        return ev.value

    def event_wait(self, ev: int) -> None:
        """The current stream waits for `ev` (no host wait)."""
        _lib.call("orca_hip_event_wait", self.handle, ev)

    def event_release(self, ev: int) -> None:
        """Hands an event back for reuse (waits already enqueued are unaffected)."""
        _lib.call("orca_hip_event_release", self.handle, ev)

    def set_ew_jit(self, mode: int) -> None:
        """How fused elementwise programs run (orca_hip_ew_set_jit): 0 interpreted, 1 compiled
        at a structure's second use (the default), 2 at its first."""
        _lib.call("orca_hip_ew_set_jit", self.handle, int(mode))

    def ew_jit_stats(self) -> dict:
        """Interpreted and compiled launches, structures compiled, failed compiles."""
        v = [ctypes.c_uint64() for _ in range(4)]
        _lib.call("orca_hip_ew_jit_stats", self.handle, *[ctypes.byref(x) for x in v])
        return dict(zip(("interpreted", "compiled_launches", "compiles", "failures"), (x.value for x in v)))

    def sync_count(self) -> int:
        """Host waits on this context's work so far (orca_hip_sync_count)."""
        n = ctypes.c_uint64()
        _lib.call("orca_hip_sync_count", self.handle, ctypes.byref(n))
        return n.value

    def mem_stats(self) -> dict:
        self.release_dropped()
        live, cached, mallocs = ctypes.c_size_t(), ctypes.c_size_t(), ctypes.c_size_t()
        _lib.call("orca_hip_mem_stats", self.handle, ctypes.byref(live), ctypes.byref(cached), ctypes.byref(mallocs))
        return dict(live=live.value, cached=cached.value, device_allocs=mallocs.value)

    def empty_cache(self) -> None:
        self.release_dropped()
        _lib.call("orca_hip_empty_cache", self.handle)

    # ---- timing ----
    def prof_enable(self, on: bool = True) -> None:
        _lib.call("orca_hip_prof_enable", self.handle, 1 if on else 0)

    def prof_reset(self) -> None:
        _lib.call("orca_hip_prof_reset", self.handle)

    def prof_report(self) -> dict:
        buf = ctypes.create_string_buffer(1 << 16)
        _lib.call("orca_hip_prof_report", self.handle, buf, len(buf))
        return json.loads(buf.value.decode())

    def timer_start(self) -> None:
        _lib.call("orca_hip_timer_start", self.handle)

    def timer_stop(self) -> float:
        ms = ctypes.c_float()
        _lib.call("orca_hip_timer_stop", self.handle, ctypes.byref(ms))
        return ms.value


class Buffer:
    """A device allocation owned by a Context; released on garbage collection."""

    def __init__(self, ctx: Context, ptr: int, nbytes: int):
        self.ctx = ctx
        self.ptr = ptr
        self.nbytes = nbytes

    def free(self) -> None:
        """Releases the block now."""
        if self.ptr and self.ctx.handle:
            _lib.call("orca_hip_free", self.ctx.handle, self.ptr)
        self.ptr = None

    def __del__(self):
        # a dropped buffer's block is released with the context's next batch
        try:
            if self.ptr and self.ctx.handle:
                self.ctx.release(self.ptr)
            self.ptr = None
        except Exception:
            pass

    def download(self, dtype=np.float32, count: int | None = None) -> np.ndarray:
        dtype = np.dtype(dtype)
        if count is None:
            count = self.nbytes // dtype.itemsize
        out = np.empty(count, dtype)
        if out.nbytes:
            _lib.call("orca_hip_d2h", self.ctx.handle, out.ctypes.data_as(ctypes.c_void_p), self.ptr, out.nbytes)
        return out

    def upload(self, arr: np.ndarray) -> None:
        arr = np.ascontiguousarray(arr)
        if arr.nbytes > self.nbytes:
            raise ValueError("upload larger than the buffer")
        if arr.nbytes:
            _lib.call("orca_hip_h2d", self.ctx.handle, self.ptr, arr.ctypes.data_as(ctypes.c_void_p), arr.nbytes)
