"""Host->device uploads of small int32 metadata through a persistent pinned ring.

Allocating fresh pinned memory for every upload (torch's `pin_memory()`) costs far more than the
copy itself when the previous buffers are still in flight. Here each device owns a ring of pinned
slots; an upload copies into the next slot, enqueues an asynchronous copy on the current stream
and records the slot's event, and a slot is reused only after its event has completed (normally
long before the ring wraps).

The copy and the event go straight to the HIP runtime that torch has loaded (hipMemcpyAsync,
hipEventRecord on raw pointers, one event per slot created once): through torch tensor views,
`copy_` and a new event per upload, the per-step metadata upload of the serving loop cost about
16 us of host time.
"""
from __future__ import annotations

import ctypes
import os
import weakref

import numpy as np
import torch

from src.kernels.hip_paged_attention import _stream_ptr

_SLOT_BYTES = 256 * 1024
_SLOTS = 32
_H2D = 1  # hipMemcpyHostToDevice
_EVENT_DISABLE_TIMING = 0x2


class _Hip:
    """The entry points of torch's HIP runtime (torch/lib/libamdhip64.so) that the ring uses."""

    def __init__(self):
        path = os.path.join(os.path.dirname(torch.__file__), "lib", "libamdhip64.so")
        # a torch built against the system ROCm has no bundled copy: the runtime it loaded is
        # found by its soname
        lib = ctypes.CDLL(path if os.path.exists(path) else "libamdhip64.so")
        vp = ctypes.c_void_p
        for name, args in (("hipMemcpyAsync", [vp, vp, ctypes.c_size_t, ctypes.c_int, vp]),
                           ("hipEventCreateWithFlags", [ctypes.POINTER(vp), ctypes.c_uint]),
                           ("hipEventRecord", [vp, vp]),
                           ("hipEventSynchronize", [vp]),
                           ("hipEventDestroy", [vp]),
                           ("hipHostMalloc", [ctypes.POINTER(vp), ctypes.c_size_t, ctypes.c_uint]),
                           ("hipHostFree", [vp]),
                           ("hipHostGetDevicePointer", [ctypes.POINTER(vp), vp, ctypes.c_uint])):
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = ctypes.c_int
        self.memcpy_async = lib.hipMemcpyAsync
        self.event_create = lib.hipEventCreateWithFlags
        self.event_record = lib.hipEventRecord
        self.event_sync = lib.hipEventSynchronize
        self.event_destroy = lib.hipEventDestroy
        self.host_malloc = lib.hipHostMalloc
        self.host_free = lib.hipHostFree
        self.host_device_pointer = lib.hipHostGetDevicePointer


_hip: _Hip | None = None


def _runtime() -> _Hip:
    global _hip
    if _hip is None:
        _hip = _Hip()
    return _hip


def _check(status: int, what: str) -> None:
    if status != 0:
        raise RuntimeError(f"{what} failed with HIP error {status}")


class _PinnedRing:
    def __init__(self, device: torch.device):
        _runtime()
        self.device = device
        self.host = torch.empty(_SLOTS * _SLOT_BYTES, dtype=torch.uint8, pin_memory=True)
        self.host_np = self.host.numpy()
        self.host_ptr = self.host.data_ptr()
        with torch.cuda.device(device):
            self.events = []
            for _ in range(_SLOTS):
                ev = ctypes.c_void_p()
                _check(_hip.event_create(ctypes.byref(ev), _EVENT_DISABLE_TIMING), "hipEventCreateWithFlags")
                self.events.append(ev)
        self.pending = [False] * _SLOTS
        self.next = 0

    def upload_into(self, arr: np.ndarray, dst: torch.Tensor) -> None:
        """Asynchronous copy of the contiguous array arr into the leading bytes of the contiguous
        device tensor dst on the current stream, through the next pinned slot (arrays larger
        than a slot through torch's own pinned copy, which tracks that buffer's lifetime)."""
        nbytes = arr.nbytes
        if nbytes > _SLOT_BYTES:
            src = torch.from_numpy(arr.view(np.uint8).reshape(-1)).pin_memory()
            dst.view(-1).view(torch.uint8)[:nbytes].copy_(src, non_blocking=True)
            return
        stream = _stream_ptr(self.device)
        i = self.next
        self.next = (i + 1) % _SLOTS
        ev = self.events[i]
        if self.pending[i]:
            _check(_hip.event_sync(ev), "hipEventSynchronize")
        off = i * _SLOT_BYTES
        self.host_np[off:off + nbytes] = arr.view(np.uint8).reshape(-1)
        _check(_hip.memcpy_async(dst.data_ptr(), self.host_ptr + off, nbytes, _H2D, stream), "hipMemcpyAsync")
        _check(_hip.event_record(ev, stream), "hipEventRecord")
        self.pending[i] = True


_rings: dict[int, _PinnedRing] = {}


def _ring(device: torch.device) -> _PinnedRing:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    ring = _rings.get(idx)
    if ring is None:
        ring = _rings[idx] = _PinnedRing(torch.device("cuda", idx))
    return ring


def upload(arr: np.ndarray, device: torch.device) -> torch.Tensor:
    """Asynchronously copy a contiguous numpy array to `device`; returns a flat device tensor of
    the same dtype, valid in stream order on the current stream."""
    arr = np.ascontiguousarray(arr)
    out = torch.empty(arr.size, dtype=torch.from_numpy(arr[:0]).dtype, device=device)
    if arr.nbytes:
        _ring(out.device).upload_into(arr, out)
    return out


def upload_into(arr: np.ndarray, dst: torch.Tensor) -> None:
    """Asynchronously copy a contiguous numpy array into the leading bytes of the contiguous
    device tensor dst (on the current stream), without an intermediate device buffer."""
    arr = np.ascontiguousarray(arr)
    if not dst.is_contiguous() or dst.numel() * dst.element_size() < arr.nbytes:
        raise ValueError("upload_into: destination must be contiguous and large enough")
    if arr.nbytes:
        _ring(dst.device).upload_into(arr, dst)


_HOST_MAPPED_COHERENT = 0x2 | 0x40000000  # hipHostMallocMapped | hipHostMallocCoherent


def _free_mapped(host_ptr: int, event) -> tuple[int, int, int]:
    """Wait for the last launch recorded on `event`, then free the pinned words and the event;
    returns the three HIP statuses. Holds no reference to the MappedHostWords it frees."""
    return (_hip.event_sync(event), _hip.host_free(ctypes.c_void_p(host_ptr)), _hip.event_destroy(event))


class MappedHostWords:
    """int32 words of pinned host memory that kernels read (and write) directly: allocated with
    hipHostMalloc as mapped, coherent memory, so a kernel sees the host's latest stores without a
    copy call and without stale cache lines. The host must not rewrite words a launch reads until
    that launch has run: mark(stream) after enqueueing such a launch, wait() before the next
    rewrite (an event; free when the launch has already finished). close() frees it, once no
    launch that reads it can run again (the graphs captured with its device address are gone).
    An object dropped without close() is freed the same way when it is collected (its owner, a
    captured step, drops the graph with it); at interpreter exit the process releases it."""

    def __init__(self, words: int, device: torch.device):
        hip = _runtime()
        with torch.cuda.device(device):
            ptr = ctypes.c_void_p()
            _check(hip.host_malloc(ctypes.byref(ptr), 4 * words, _HOST_MAPPED_COHERENT), "hipHostMalloc")
            dptr = ctypes.c_void_p()
            _check(hip.host_device_pointer(ctypes.byref(dptr), ptr, 0), "hipHostGetDevicePointer")
            ev = ctypes.c_void_p()
            _check(hip.event_create(ctypes.byref(ev), _EVENT_DISABLE_TIMING), "hipEventCreateWithFlags")
        self.words = np.ctypeslib.as_array((ctypes.c_int32 * words).from_address(ptr.value))
        self.words[:] = 0
        self.host_ptr = ptr.value
        self.device_ptr = dptr.value
        self.event = ev
        self.pending = False
        self._finalizer = weakref.finalize(self, _free_mapped, ptr.value, ev)
        self._finalizer.atexit = False

    def device_addr(self, word: int = 0) -> int:
        return self.device_ptr + 4 * word

    def wait(self) -> None:
        if self.pending:
            _check(_hip.event_sync(self.event), "hipEventSynchronize")
            self.pending = False

    def mark(self, stream: int) -> None:
        _check(_hip.event_record(self.event, stream), "hipEventRecord")
        self.pending = True

    def close(self) -> None:
        """Wait for the last marked launch, then free the memory and the event (idempotent)."""
        if self.host_ptr is None:
            return
        self.words = None
        self.pending = False
        sync, free, destroy = self._finalizer()
        self.host_ptr = self.device_ptr = self.event = None
        _check(sync, "hipEventSynchronize")
        _check(free, "hipHostFree")
        _check(destroy, "hipEventDestroy")
