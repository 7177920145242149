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
"""
from __future__ import annotations

import torch



def hit_bitmap(page_status: torch.Tensor, packed: bool = False) -> torch.Tensor:
    """True for every page whose ingress verdict is 0 (verified and written).

    ``page_status`` holds one int32 verdict per page, as the per-page ingress
    writes it.  ``packed`` returns uint8 bytes instead, page i in bit i % 8
    of byte i // 8 (least significant bit first), trailing bits 0."""
    if page_status.dtype != torch.int32 or page_status.dim() != 1:
        raise ValueError("page_status must be a 1-D int32 tensor of per-page verdicts")
    hits = page_status == 0
    if not packed:
        return hits
    n = hits.numel()
    pad = (-n) % 8
    bits = torch.cat([hits, hits.new_zeros(pad)]).view(-1, 8).to(torch.uint8)
    weights = torch.tensor([1, 2, 4, 8, 16, 32, 64, 128], dtype=torch.uint8, device=bits.device)
    return (bits * weights).sum(dim=1, dtype=torch.uint8)


class WireRing:
    """A ring of ``n_slots`` pinned host buffers of ``slot_bytes`` each.

    ``push(blobs)`` copies a contiguous device tensor of blobs into the next
    slot on the ring's own copy stream (default priority), after the work
    already queued on the caller's current stream (the egress launch that
    wrote the blobs), and returns the slot index.  ``wait(slot)`` blocks until
    that copy has landed and returns the slot's bytes as a host tensor.  A
    slot is reused after ``n_slots`` further pushes; its previous copy is
    waited for first, so the bytes ``wait`` returned stay valid until then."""

    def __init__(self, slot_bytes: int, n_slots: int = 2, device: torch.device | int | None = None):
        if slot_bytes <= 0 or n_slots <= 0:
            raise ValueError("slot_bytes and n_slots must be positive")
        if not torch.cuda.is_available():
            raise RuntimeError("WireRing needs a GPU (pinned host memory and a copy stream)")
        self.slot_bytes = slot_bytes
        self.device = torch.device("cuda", torch.cuda.current_device() if device is None else
                                   torch.device(device).index or 0)
        self.slots = [torch.empty(slot_bytes, dtype=torch.uint8, pin_memory=True) for _ in range(n_slots)]
        self.sizes = [0] * n_slots
        self.done: list[torch.cuda.Event | None] = [None] * n_slots
        self.stream = torch.cuda.Stream(device=self.device)
        self.next = 0

    def push(self, blobs: torch.Tensor) -> int:
        if blobs.device != self.device or blobs.dtype != torch.uint8 or not blobs.is_contiguous():
            raise ValueError("blobs must be a contiguous uint8 tensor on the ring's device")
        n = blobs.numel()
        if n > self.slot_bytes:
            raise ValueError(f"{n} blob bytes exceed the slot size {self.slot_bytes}")
        i = self.next
        self.next = (i + 1) % len(self.slots)
        if self.done[i] is not None:
            self.done[i].synchronize()
        ready = torch.cuda.Event()
        ready.record(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(self.stream):
            self.stream.wait_event(ready)
            self.slots[i][:n].copy_(blobs.view(-1), non_blocking=True)
            blobs.record_stream(self.stream)
            ev = torch.cuda.Event()
            ev.record(self.stream)
        self.done[i] = ev
        self.sizes[i] = n
        return i

    def wait(self, slot: int) -> torch.Tensor:
        if self.done[slot] is None:
            raise ValueError(f"slot {slot} holds no copy")
        self.done[slot].synchronize()
        return self.slots[slot][:self.sizes[slot]]
