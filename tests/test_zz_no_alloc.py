"""The no-allocation ingress entry point against the allocating one, on the GPU.

ztcp_ingress_peak_into_noalloc keeps its call state, and the generic
kernels' per-page status array, in a fixed device array instead of allocated
memory.  Each case runs two calls in a row through the C ABI, the second with
a smaller batch, and checks return codes, per-page statuses and decoded
outputs against ztcp_ingress_peak_into on the same inputs: fused kernels
(clean and tampered, all-or-nothing and per-page), the generic kernels with
no status array from the caller (the case that uses the scratch status
array), and the batch-size limit.
"""
import ctypes as C

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _case(hip, shape, preset, rope_mode, n, seed, tamper=()):
    import vlx_tee_amd._native as N
    import vlx_tee_amd.workloads as W

    T, H, D, R = shape
    keys = W.session_keys()
    g = torch.Generator(device="cuda").manual_seed(seed)
    k = torch.randn((n, T, H, D), generator=g, device="cuda").to(torch.bfloat16)
    v = torch.randn((n, T, H, D), generator=g, device="cuda").to(torch.bfloat16)
    geo = N.geometry(T, H, D, R, N.HOT_BF16, False)
    exp = N.lib().ztcp_payload_bytes(C.byref(geo), preset, rope_mode)
    blobs = torch.empty((n, 48 + exp), dtype=torch.uint8, device="cuda")
    th = torch.arange(n, dtype=torch.int64, device="cuda") * 7 + seed
    hip.fused_encode_cold_pages_peak_into(k, v, th, blobs, preset, rope_mode, R, exp, W.TENANT_HASH, W.MODEL_HASH,
                                          3, 0, 100, keys["k0"], keys["k1"], keys["mk0"], keys["mk1"], keys["k2"],
                                          keys["k3"])
    for pg, byte in tamper:
        blobs[pg, byte] ^= 0x04
    torch.cuda.synchronize()
    return N, W, keys, geo, blobs, th, k.shape


def _run(N, W, keys, geo, blobs, th, shape, entry, flags, with_status):
    ko = torch.full(shape, 3.0, dtype=torch.bfloat16, device="cuda")
    vo = torch.full(shape, 3.0, dtype=torch.bfloat16, device="cuda")
    st = torch.full((shape[0],), -1, dtype=torch.int32, device="cuda") if with_status else None
    rc = getattr(N.lib(), entry)(blobs.data_ptr(), blobs.size(1), th.data_ptr(), ko.data_ptr(), vo.data_ptr(),
                                 shape[0], C.byref(geo), W.TENANT_HASH, W.MODEL_HASH, 3, C.byref(N.keys(**keys)),
                                 None if st is None else st.data_ptr(), flags,
                                 C.c_void_p(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    return rc, (None if st is None else st.cpu().numpy()), ko, vo


CASES = [
    # (name, shape T,H,D,R, preset, rope_mode, first batch, second batch, tamper, per_page, with_status)
    ("fused-clean", (16, 4, 128, 64), 1, 1, 512, 200, (), False, False),
    ("fused-tampered-all", (16, 8, 128, 64), 2, 1, 300, 77, ((5, 900),), False, True),
    ("fused-tampered-per-page", (16, 8, 128, 64), 2, 1, 300, 77, ((0, 3000), (40, 40)), True, True),
    ("generic-no-status", (3, 1, 48, 16), 1, 1, 1000, 333, ((7, 60),), False, False),
    ("generic-per-page", (3, 1, 48, 16), 3, 0, 700, 129, ((2, 70), (5, 20)), True, True),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_noalloc_matches_allocating_entry_point(hip, case):
    name, shape, preset, rm, n1, n2, tamper, per_page, with_status = case
    for n in (n1, n2):  # two calls in a row, the second smaller
        print(f"case {name}: {n} pages", flush=True)
        N, W, keys, geo, blobs, th, sh = _case(hip, shape, preset, rm, n, seed=n,
                                               tamper=[t for t in tamper if t[0] < n])
        flags = N.PER_PAGE if per_page else 0
        a = _run(N, W, keys, geo, blobs, th, sh, "ztcp_ingress_peak_into", flags, with_status)
        b = _run(N, W, keys, geo, blobs, th, sh, "ztcp_ingress_peak_into_noalloc", flags, with_status)
        assert a[0] == b[0]
        assert a[0] == (0 if not tamper else 3)
        if with_status:
            assert np.array_equal(a[1], b[1])
        assert torch.equal(a[2], b[2]) and torch.equal(a[3], b[3])
        if not tamper:
            assert a[2].abs().sum() > 0  # decoded, not zeroed
        elif not per_page:
            assert not b[2].any() and not b[3].any()


def test_noalloc_rejects_batches_beyond_its_scratch(hip):
    import vlx_tee_amd._native as N
    import vlx_tee_amd.workloads as W

    buf = torch.zeros(1 << 20, dtype=torch.uint8, device="cuda")
    geo = N.geometry(16, 4, 128, 64, N.HOT_BF16, False)
    rc = N.lib().ztcp_ingress_peak_into_noalloc(buf.data_ptr(), 12336, buf.data_ptr(), buf.data_ptr(), buf.data_ptr(),
                                                N.NOALLOC_MAX_PAGES + 1, C.byref(geo), W.TENANT_HASH, W.MODEL_HASH, 0,
                                                C.byref(N.keys(1, 2, 3, 4)), None, 0,
                                                C.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == N.ESCRATCH
    assert "ZTCP_NOALLOC_MAX_PAGES" in N.last_error()


def _noalloc(N, W, keys, geo, blobs, th, ko, vo, st, flags, stream):
    return N.lib().ztcp_ingress_peak_into_noalloc(
        blobs.data_ptr(), blobs.size(1), th.data_ptr(), ko.data_ptr(), vo.data_ptr(), ko.size(0), C.byref(geo),
        W.TENANT_HASH, W.MODEL_HASH, 3, C.byref(N.keys(**keys)), None if st is None else st.data_ptr(), flags,
        C.c_void_p(stream.cuda_stream))


def test_noalloc_allocates_no_device_memory(hip):
    """Device memory in use (hipMemGetInfo) is the same before and after
    no-allocation calls of both kernel paths, once every tensor of the test
    exists and the kernels' code is loaded."""
    print("case no-alloc: device memory across calls", flush=True)
    cases = [_case(hip, (16, 8, 128, 64), 2, 1, 300, 5, tamper=((3, 200),)),
             _case(hip, (3, 1, 48, 16), 1, 1, 900, 6, tamper=((1, 60),))]
    outs = [(torch.empty(c[6], dtype=torch.bfloat16, device="cuda"), torch.empty(c[6], dtype=torch.bfloat16,
                                                                                   device="cuda")) for c in cases]
    stream = torch.cuda.current_stream()
    for (N, W, keys, geo, blobs, th, _), (ko, vo) in zip(cases, outs):  # warm: code objects loaded
        assert _noalloc(N, W, keys, geo, blobs, th, ko, vo, None, 0, stream) == 3
    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info()
    for rep in range(3):
        for (N, W, keys, geo, blobs, th, _), (ko, vo) in zip(cases, outs):
            assert _noalloc(N, W, keys, geo, blobs, th, ko, vo, None, N.PER_PAGE if rep else 0, stream) == 3
    torch.cuda.synchronize()
    free1, _ = torch.cuda.mem_get_info()
    assert free1 == free0, (free0, free1)


def test_noalloc_asynchronous_call_replays_from_a_graph(hip):
    """Only a ZTCP_ASYNC call can be captured: a synchronous one on a stream
    under capture is refused with ZTCP_EINVAL, and a captured asynchronous call
    replays correctly several times, with eager work on the same buffers and
    synchronizations between the replays."""
    N, W, keys, geo, blobs, th, sh = _case(hip, (16, 4, 128, 64), 1, 1, 256, 11)
    want = _run(N, W, keys, geo, blobs, th, sh, "ztcp_ingress_peak_into", 0, True)
    assert want[0] == 0
    ko = torch.empty(sh, dtype=torch.bfloat16, device="cuda")
    vo = torch.empty(sh, dtype=torch.bfloat16, device="cuda")
    st = torch.full((sh[0],), -1, dtype=torch.int32, device="cuda")
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):  # warm outside the capture
        assert _noalloc(N, W, keys, geo, blobs, th, ko, vo, st, N.ASYNC, s) == 0
    torch.cuda.synchronize()
    print("case no-alloc: graph capture of an asynchronous call", flush=True)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        assert _noalloc(N, W, keys, geo, blobs, th, ko, vo, st, 0, s) == N.EINVAL
        assert "ZTCP_ASYNC" in N.last_error()
        assert _noalloc(N, W, keys, geo, blobs, th, ko, vo, st, N.ASYNC, s) == 0
    for rep in range(3):
        ko.fill_(5.0)
        vo.fill_(5.0)
        st.fill_(-1)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert (st.cpu().numpy() == 0).all(), rep
        assert torch.equal(ko, want[2]) and torch.equal(vo, want[3]), rep
