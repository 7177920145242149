"""The steps on either side of the codec that a serving stack needs.

hit_bitmap: the PoisonShield per-page fallback (research/paper/main.tex:173).
  A page that fails AAD, MAC or freshness checks on ingress is not written to
  hot memory and its slot reads False in the serving engine's hit bitmap, so
  the engine recomputes that prefix instead of failing the worker.  The
  per-page ingress policy (``ZTCP_PER_PAGE``) already zeroes failing pages
  and keeps verified ones; this turns its verdicts into the bitmap.

WireRing: the egress wire step.  The reference only models it
  (research/benchmarks/bench_cold_page_pipeline.py:1089-1162: blob bytes over
  a 100GbE link after the codec).  Here a batch of blobs leaves HBM into a
  ring of pinned host slots on a copy stream of its own, ordered after the
  egress launch by an event, so the next batch's egress overlaps the copy.

Both are the library's (include/ztcp.h: ztcp_hit_bitmap, ztcp_wire_ring_*);
this module binds them to torch tensors.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import torch

from . import _native as N


def _stream(device: torch.device) -> C.c_void_p:
    return C.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _raise(rc: int, what: str) -> None:
    if rc != N.OK:
        raise RuntimeError(f"{what}: {N.strerror(rc)} (code {rc})")


def hit_bitmap(page_status: torch.Tensor, packed: bool = False) -> torch.Tensor:
    """True for every page whose ingress verdict is 0 (verified and written).

    ``page_status`` is a 1-D int32 device tensor of per-page verdicts, as the
    per-page ingress writes it; the bitmap is made on the device by the
    library (ztcp_hit_bitmap) on the current stream.  ``packed`` returns
    uint8 bytes instead, page i in bit i % 8 of byte i // 8 (least
    significant bit first), trailing bits 0."""
    if page_status.dtype != torch.int32 or page_status.dim() != 1:
        raise ValueError("page_status must be a 1-D int32 tensor of per-page verdicts")
    if not page_status.is_cuda:
        raise ValueError("page_status must be a device tensor (the bitmap is made on the GPU)")
    st = page_status.contiguous()
    n = st.numel()
    out = torch.empty((n + 7) // 8 if packed else n, dtype=torch.uint8 if packed else torch.bool,
                      device=st.device)
    with torch.cuda.device(st.device):
        rc = N.lib().ztcp_hit_bitmap(C.c_void_p(st.data_ptr()), n, C.c_void_p(out.data_ptr()),
                                     1 if packed else 0, _stream(st.device))
    _raise(rc, "ztcp_hit_bitmap")
    return out


class _RingHandle:
    """Owns a native ring (ztcp_wire_ring_*): destroyed when the last of its
    holders is gone -- the WireRing and every host view that ``wait``
    returned, since those views are the ring's pinned slot memory."""

    def __init__(self, ptr: C.c_void_p, destroy=None):
        self.ptr = ptr
        self._destroy = destroy if destroy is not None else (lambda p: N.lib().ztcp_wire_ring_destroy(p))

    def __del__(self):
        if self.ptr:
            ptr, self.ptr = self.ptr, None
            try:
                self._destroy(ptr)
            except Exception:  # noqa: BLE001  (interpreter shutdown)
                pass


def _host_view(address: int, nbytes: int, owner) -> torch.Tensor:
    """A uint8 host tensor over ``nbytes`` at ``address`` that keeps ``owner``
    (the memory's holder) alive for as long as the tensor or any view of it
    exists: tensor -> numpy array -> memoryview -> ctypes array -> owner."""
    if nbytes == 0:
        return torch.empty(0, dtype=torch.uint8)
    buf = (C.c_uint8 * nbytes).from_address(address)
    buf._owner = owner
    return torch.from_numpy(np.ctypeslib.as_array(buf))


class WireRing:
    """A ring of ``n_slots`` pinned host buffers of ``slot_bytes`` each, with a
    copy stream of its own (the library's ztcp_wire_ring).

    ``push(blobs)`` copies a contiguous device tensor of blobs into the next
    slot after the work already queued on the caller's current stream (the
    egress launch that wrote the blobs) and returns the slot index.
    ``wait(slot)`` blocks until that copy has landed and returns the slot's
    bytes as a host tensor (a view of the pinned slot).  A slot is reused
    ``n_slots`` pushes later, after its previous copy has landed, so the bytes
    ``wait`` returned stay those of that push until then.  The views keep the
    ring's memory alive: ``close()`` (or dropping the ring) frees it only once
    no view that ``wait`` returned is left."""

    def __init__(self, slot_bytes: int, n_slots: int = 2, device: torch.device | int | None = None):
        if slot_bytes <= 0 or n_slots <= 0:
            raise ValueError("slot_bytes and n_slots must be positive")
        if not torch.cuda.is_available():
            raise RuntimeError("WireRing needs a GPU (pinned host memory and a copy stream)")
        self.slot_bytes = slot_bytes
        self.device = torch.device("cuda", torch.cuda.current_device() if device is None else
                                   torch.device(device).index or 0)
        ring = C.c_void_p()
        with torch.cuda.device(self.device):
            rc = N.lib().ztcp_wire_ring_create(slot_bytes, n_slots, C.byref(ring))
        _raise(rc, "ztcp_wire_ring_create")
        self._h: _RingHandle | None = _RingHandle(ring)
        self._held: dict[int, torch.Tensor] = {}  # slot -> device blobs still being copied

    def _ptr(self) -> C.c_void_p:
        if self._h is None:
            raise RuntimeError("WireRing is closed")
        return self._h.ptr

    def push(self, blobs: torch.Tensor) -> int:
        if blobs.device != self.device or blobs.dtype != torch.uint8 or not blobs.is_contiguous():
            raise ValueError("blobs must be a contiguous uint8 tensor on the ring's device")
        n = blobs.numel()
        if n > self.slot_bytes:
            raise ValueError(f"{n} blob bytes exceed the slot size {self.slot_bytes}")
        slot = C.c_int32(-1)
        with torch.cuda.device(self.device):
            rc = N.lib().ztcp_wire_ring_push(self._ptr(), C.c_void_p(blobs.data_ptr()), n,
                                             _stream(self.device), C.byref(slot))
        _raise(rc, "ztcp_wire_ring_push")
        self._held[slot.value] = blobs  # the copy reads it on the ring's stream
        return slot.value

    def wait(self, slot: int) -> torch.Tensor:
        host, n = C.c_void_p(), C.c_size_t()
        rc = N.lib().ztcp_wire_ring_wait(self._ptr(), slot, C.byref(host), C.byref(n))
        if rc == N.EINVAL:
            raise ValueError(f"slot {slot} holds no copy")
        _raise(rc, "ztcp_wire_ring_wait")
        self._held.pop(slot, None)
        return _host_view(host.value or 0, n.value, self._h)

    def close(self) -> None:
        """Releases the ring; its memory is freed once no view from ``wait``
        is left (at once if there is none).  The copies in flight complete
        first (ztcp_wire_ring_destroy)."""
        self._h = None
        self._held.clear()

    def __del__(self):
        self._h = None
