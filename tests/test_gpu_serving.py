"""GPU tests of the serving-side steps (include/ztcp.h: ztcp_hit_bitmap,
ztcp_wire_ring_*): the hit bitmap against numpy's bit packing, and the wire
ring's ordering after the producer's stream, slot reuse and argument errors.
The full-size round trip of both (a 1 GiB prefix's verdicts and blobs) is in
tests/test_gpu_fullsize.py."""
from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n", [1, 7, 8, 9, 63, 64, 65, 1000, 100003])
def test_hit_bitmap_matches_numpy(hip, n):
    import vlx_tee_amd.serving as SV
    rng = np.random.default_rng(n)
    st = rng.choice(np.array([0, 0, 0, 1, 2, 3, 4], dtype=np.int32), size=n)
    t = torch.from_numpy(st).cuda()
    print(f"case hit_bitmap n={n}", flush=True)
    hits = SV.hit_bitmap(t)
    assert hits.dtype == torch.bool and np.array_equal(hits.cpu().numpy(), st == 0)
    packed = SV.hit_bitmap(t, packed=True).cpu().numpy()
    assert np.array_equal(packed, np.packbits(st == 0, bitorder="little"))


def test_hit_bitmap_empty(hip):
    import vlx_tee_amd.serving as SV
    t = torch.zeros(0, dtype=torch.int32, device="cuda")
    assert SV.hit_bitmap(t).numel() == 0 and SV.hit_bitmap(t, packed=True).numel() == 0


def test_wire_ring_orders_after_the_producer_and_reuses_slots(hip):
    """Each push is issued right after the kernels that write its source, with
    no synchronization: the ring's copy stream must wait for them.  Three
    slots, seven pushes: a slot's bytes are those of its latest push."""
    import vlx_tee_amd.serving as SV
    n = 3 << 20
    ring = SV.WireRing(n, n_slots=3)
    src = [torch.empty(n, dtype=torch.uint8, device="cuda") for _ in range(7)]
    print("case wire ring: 7 pushes of 3 MiB into 3 slots", flush=True)
    got = {}
    for i, s in enumerate(src):
        # a slow producer: many small kernels, the last one writing the value
        for j in range(20):
            s.fill_((i * 31 + j) & 0xFF)
        s.fill_(i + 1)
        slot = ring.push(s)
        assert slot == i % 3
        if i >= 4:  # slot (i - 4) % 3 was last written by push i - 3 ... i - 1
            back = (i - 2) % 3
            got[i - 2] = ring.wait(back).clone()
    for i in (4, 5, 6):
        got[i] = ring.wait(i % 3).clone()
    for i, t in got.items():
        assert t.numel() == n and bool((t == i + 1).all()), f"push {i}: slot bytes are not its source's"
    ring.close()


def test_wire_ring_partial_and_errors(hip):
    import vlx_tee_amd.serving as SV
    ring = SV.WireRing(4096, n_slots=2)
    a = torch.arange(1000, dtype=torch.int64, device="cuda").to(torch.uint8)
    slot = ring.push(a)
    out = ring.wait(slot)
    assert out.numel() == 1000 and torch.equal(out, a.cpu())
    with pytest.raises(ValueError, match="exceed the slot size"):
        ring.push(torch.zeros(4097, dtype=torch.uint8, device="cuda"))
    with pytest.raises(ValueError, match="holds no copy"):
        ring.wait(1)
    with pytest.raises(ValueError, match="contiguous uint8"):
        ring.push(torch.zeros(10, dtype=torch.int32, device="cuda"))
    empty = ring.push(torch.zeros(0, dtype=torch.uint8, device="cuda"))
    assert ring.wait(empty).numel() == 0
    ring.close()


def test_wire_ring_view_outlives_the_ring(hip):
    """A view that wait() returned stays readable after the ring is closed and
    dropped: the pinned slots are freed only with the last view."""
    import gc

    import vlx_tee_amd.serving as SV
    ring = SV.WireRing(1 << 16, n_slots=2)
    a = (torch.arange(1 << 16, device="cuda") * 7).to(torch.uint8)
    view = ring.wait(ring.push(a))[100:1100]
    ring.close()
    del ring
    gc.collect()
    assert torch.equal(view, a[100:1100].cpu())
    with pytest.raises(RuntimeError, match="closed"):
        r2 = SV.WireRing(64, n_slots=1)
        r2.close()
        r2.push(torch.zeros(8, dtype=torch.uint8, device="cuda"))
