"""Transaction logic of the session-bound codec class that runs before or
instead of a kernel (no GPU): the reference's ordering of nonce burn,
argument checks, output zeroing and session errors (nfc:148-606)."""
from __future__ import annotations

import numpy as np
import pytest
import torch


@pytest.fixture(scope="module")
def C(pkg):
    import vlx_tee_amd.codec as C

    return C


@pytest.fixture()
def codec(C):
    from vlx_tee_amd.spec import ColdPageGeometry

    ring = C.EphemeralSessionKeyRing(b"p" * 32)
    return C.NativeCppFusedColdPageCodec(ColdPageGeometry(num_tokens=16, num_kv_heads=2), ring)


def _aad(seq):
    from vlx_tee_amd.spec import ColdPageAAD

    return ColdPageAAD(1, 2, 3, 0, seq)


def test_host_tensors_are_refused_after_the_nonce_burn(C, codec):
    k = torch.ones((1, 16, 2, 128), dtype=torch.float16)
    th = torch.tensor([5], dtype=torch.int64)
    nbytes = codec.geometry.cold_blob_bytes(2, 1)
    out = torch.full((1, nbytes), 9, dtype=torch.uint8)
    with pytest.raises(RuntimeError, match="HIP"):
        codec.encode_cold_pages_peak_into(k, k.clone(), th, out, "t", "s", _aad(7))
    assert not out.any()  # zeroed on failure after the preflight
    with pytest.raises(C.NonceReuseError):  # the nonce stayed burned
        codec.encode_cold_pages_peak_into(k, k.clone(), th, out, "t", "s", _aad(7))


def test_argument_errors_in_reference_order(C, codec):
    k = torch.ones((2, 16, 2, 128), dtype=torch.float16)
    with pytest.raises(RuntimeError, match="non-empty torch.Tensor"):
        codec.encode_cold_pages_batch_tensor(k, k, torch.empty(0, dtype=torch.int64), "t", "s", _aad(1))
    # wrong token-hash dtype: the preflight burns the nonces first, then the check fails
    with pytest.raises(RuntimeError, match="1D contiguous int64"):
        codec.encode_cold_pages_batch_tensor(k, k, torch.tensor([1, 2], dtype=torch.int32), "t", "s", _aad(1))
    with pytest.raises(C.NonceReuseError):
        codec.encode_cold_pages_batch_tensor(k, k, torch.tensor([1, 2]), "t", "s", _aad(2))
    with pytest.raises(RuntimeError, match="does not match batch geometry"):
        codec.encode_cold_pages_batch_tensor(k[:1], k, torch.tensor([1, 2]), "t", "s", _aad(10))


def test_ingress_needs_a_live_session(C, codec):
    blobs = torch.zeros((1, 100), dtype=torch.uint8)
    th = torch.tensor([1])
    k = torch.ones((1, 16, 2, 128), dtype=torch.float16)
    with pytest.raises(C.SessionShreddedError, match=r"Session \(t, s\) key is missing"):
        codec.decode_cold_pages_peak_into(blobs, th, k, k.clone(), "t", "s", "m", 0)
    assert k.all()  # nothing touched before the session check
    codec.keyring.derive_or_get("t", "s")
    with pytest.raises(RuntimeError, match="with batch=1"):
        codec.decode_cold_pages_peak_into(blobs[0], th, k, k.clone(), "t", "s", "m", 0)
    with pytest.raises(RuntimeError, match="must not alias"):
        codec.decode_cold_pages_peak_into(blobs, th, k, k, "t", "s", "m", 0)


def test_reference_names_are_exported(C):
    assert C.NativeCppFusedColdPageCodec is C.NativeHipFusedColdPageCodec
    for name in ("encode_cold_page_tensor", "decode_cold_page_tensor", "decode_cold_pages_batch_tensor",
                 "decode_cold_pages_peak_into", "encode_cold_pages_batch_tensor", "encode_cold_pages_peak_into"):
        assert callable(getattr(C.NativeCppFusedColdPageCodec, name))
    assert issubclass(C.StalePageReplayError, C.KVIntegrityError)
    assert issubclass(C.CrossTenantContaminationError, C.KVIntegrityError)
    assert issubclass(C.NonceReuseError, ValueError)
    assert issubclass(C.SessionShreddedError, RuntimeError)


def test_hit_bitmap_rejects_bad_verdict_tensors(pkg):
    """The bitmap is made on the GPU from int32 verdicts; anything else is an
    argument error before any device call (the packing itself is checked
    against numpy in tests/test_gpu_serving.py)."""
    import vlx_tee_amd.serving as SV
    with pytest.raises(ValueError, match="1-D int32"):
        SV.hit_bitmap(torch.zeros(4, dtype=torch.int64))
    with pytest.raises(ValueError, match="1-D int32"):
        SV.hit_bitmap(torch.zeros((2, 2), dtype=torch.int32))
    with pytest.raises(ValueError, match="device tensor"):
        SV.hit_bitmap(torch.zeros(4, dtype=torch.int32))


def test_wire_ring_views_keep_the_slot_memory_alive(pkg):
    """A host view that WireRing.wait returned is the ring's pinned slot
    memory: the ring is destroyed only after the ring object and every such
    view are gone (modelled here with host memory and a recording destroy)."""
    import ctypes as C
    import gc

    import vlx_tee_amd.serving as SV

    freed = []
    mem = (C.c_uint8 * 64)(*range(64))
    h = SV._RingHandle(C.c_void_p(1), destroy=freed.append)
    view = SV._host_view(C.addressof(mem), 64, h)[8:24]
    del h  # the ring object lets go (close / garbage collection)
    gc.collect()
    assert not freed, "the ring was freed while a view of its slot was alive"
    assert view.tolist() == list(range(8, 24))
    del view
    gc.collect()
    assert len(freed) == 1
