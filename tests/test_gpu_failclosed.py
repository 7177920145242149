"""Per-call ingress verdicts and fail-closed bounded waits, on the GPU.

* Two ingress calls in flight on one device at once (two streams, and two
  host threads) keep their own verdicts: a tampered all-or-nothing batch still
  raises and is zeroed while a clean batch decodes, whatever the interleaving
  of their kernels (the reference keeps its status codes per call,
  cpp:2056-2057 and cpp:2307, and zeroes in the same call, cpp:2481-2495),
  also when asynchronous calls in flight hold every other call slot.
* A bounded wait that gives up (forced from the host: the wait limit set to
  zero polls, so each kernel's own wait expires and the kernel ends normally)
  fails closed: ingress returns ZTCP_EDEVICE and zeroes every output, per page
  the status is ZTCP_ERR_DEVICE; egress writes blobs no ingress accepts.
* Egress rejects the extension presets unless the call asks for them, with
  the reference's message (cpp:1947-1948); argument errors carry the
  reference's TORCH_CHECK text.
"""
import ctypes as C
import threading

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

N_PAGES = 2048


@pytest.fixture(scope="module")
def env(hip, pkg):
    import vlx_tee_amd._native as N
    import vlx_tee_amd.workloads as W

    w = W.WORKLOADS["c1_int4_gqa256"]  # 16 tok x 4 heads x 128, INT4_SYM + PRESERVE_FP8
    dev = torch.device("cuda")
    keys = W.session_keys()
    k, v = W.generate(w, dev, torch.bfloat16, n_pages=N_PAGES)
    th = torch.arange(N_PAGES, dtype=torch.int64, device=dev)
    blobs = torch.empty((N_PAGES, w.blob_bytes), dtype=torch.uint8, device=dev)
    hip.fused_encode_cold_pages_peak_into(k, v, th, blobs, w.preset, w.rope_mode, w.rope_dim,
                                          w.payload_bytes, W.TENANT_HASH, W.MODEL_HASH, 0, 0, 0,
                                          keys["k0"], keys["k1"], keys["mk0"], keys["mk1"], keys["k2"],
                                          keys["k3"])
    ko = torch.empty_like(k)
    vo = torch.empty_like(v)
    hip.fused_decode_cold_pages_peak_into(blobs, th, ko, vo, w.rope_dim, False, W.TENANT_HASH,
                                          W.MODEL_HASH, 0, keys["k0"], keys["k1"], keys["mk0"],
                                          keys["mk1"], keys["k2"], keys["k3"])
    torch.cuda.synchronize()
    tampered = blobs.clone()
    tampered[0, 100] ^= 0x10          # payload byte of page 0: MAC failure (status 3)
    tampered[N_PAGES - 1, 5000] ^= 1  # and of the last page
    return dict(N=N, W=W, w=w, keys=keys, k=k, v=v, th=th, blobs=blobs, tampered=tampered,
                ref_k=ko, ref_v=vo)


def _ingress_async(e, blobs, ko, vo, status, stream, flags=0):
    N, w, keys = e["N"], e["w"], e["keys"]
    g = N.geometry(w.num_tokens, w.num_heads, w.head_dim, w.rope_dim, N.HOT_BF16, False)
    return N.lib().ztcp_ingress_peak_into(
        blobs.data_ptr(), blobs.size(1), e["th"].data_ptr(), ko.data_ptr(), vo.data_ptr(), blobs.size(0),
        C.byref(g), e["W"].TENANT_HASH, e["W"].MODEL_HASH, 0, C.byref(N.keys(**keys)), status.data_ptr(),
        N.ASYNC | flags, C.c_void_p(stream.cuda_stream))


@pytest.mark.parametrize("delay", [0, 20_000, 200_000, 1_000_000])
def test_two_streams_keep_their_own_verdicts(env, delay):
    """The tampered call's kernels are enqueued first; the clean call's reset
    lands before, during or after them (a spin kernel delays its stream)."""
    print(f"case two streams, delay {delay}", flush=True)
    e = env
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    ka, va = torch.full_like(e["k"], 3.0), torch.full_like(e["v"], 3.0)
    kb, vb = torch.full_like(e["k"], 3.0), torch.full_like(e["v"], 3.0)
    sta = torch.full((N_PAGES,), -1, dtype=torch.int32, device="cuda")
    stb = torch.full_like(sta, -1)
    torch.cuda.synchronize()
    assert _ingress_async(e, e["tampered"], ka, va, sta, sa) == 0
    with torch.cuda.stream(sb):
        if delay:
            torch.cuda._sleep(delay)
    assert _ingress_async(e, e["blobs"], kb, vb, stb, sb) == 0
    torch.cuda.synchronize()
    st_a = sta.cpu().numpy()
    assert st_a[0] == 3 and st_a[-1] == 3 and (st_a[1:-1] == 0).all()
    assert not ka.any() and not va.any(), "all-or-nothing: the tampered batch's outputs are zeroed"
    assert (stb.cpu().numpy() == 0).all()
    assert torch.equal(kb, e["ref_k"]) and torch.equal(vb, e["ref_v"])


def test_two_threads_synchronous_calls(env, hip):
    """Synchronous calls from two host threads on two streams (ctypes releases
    the GIL): each returns its own verdict."""
    e = env
    W, keys = e["W"], e["keys"]
    results = {}

    def run(name, blobs, stream, barrier, ko, vo):
        barrier.wait()
        try:
            with torch.cuda.stream(stream):
                hip.fused_decode_cold_pages_peak_into(blobs, e["th"], ko, vo, e["w"].rope_dim, False,
                                                      W.TENANT_HASH, W.MODEL_HASH, 0, keys["k0"], keys["k1"],
                                                      keys["mk0"], keys["mk1"], keys["k2"], keys["k3"])
            results[name] = ("ok", ko, vo)
        except RuntimeError as ex:
            results[name] = (str(ex), ko, vo)

    for rep in range(6):
        print(f"case two threads, repeat {rep}", flush=True)
        results.clear()
        barrier = threading.Barrier(2)
        outs = [(torch.full_like(e["k"], 3.0), torch.full_like(e["v"], 3.0)) for _ in range(2)]
        torch.cuda.synchronize()
        ta = threading.Thread(target=run, args=("a", e["tampered"], torch.cuda.Stream(), barrier, *outs[0]))
        tb = threading.Thread(target=run, args=("b", e["blobs"], torch.cuda.Stream(), barrier, *outs[1]))
        ta.start(); tb.start(); ta.join(); tb.join()
        torch.cuda.synchronize()
        msg, ka, va = results["a"]
        assert msg.startswith("KV_INTEGRITY_ERROR: Cold-page MAC verification failed"), msg
        assert not ka.any() and not va.any()
        msg, kb, vb = results["b"]
        assert msg == "ok"
        assert torch.equal(kb, e["ref_k"]) and torch.equal(vb, e["ref_v"])


def test_synchronous_calls_with_every_other_slot_pending(env, hip):
    """63 asynchronous calls held in flight behind a sleeping kernel take all
    but one of the device's 64 call slots; two synchronous calls from two
    threads then share the last one in turn (the second waits), and each
    still returns its own verdict: a slot held by a call in progress is never
    handed to another call."""
    e = env
    W, keys = e["W"], e["keys"]
    s0 = torch.cuda.Stream()
    n = 64
    ko, vo = torch.empty_like(e["k"][:n]), torch.empty_like(e["v"][:n])
    st = torch.empty((n,), dtype=torch.int32, device="cuda")
    results = {}

    def run(name, blobs, stream, barrier, ko_, vo_):
        barrier.wait()
        try:
            with torch.cuda.stream(stream):
                hip.fused_decode_cold_pages_peak_into(blobs, e["th"], ko_, vo_, e["w"].rope_dim, False,
                                                      W.TENANT_HASH, W.MODEL_HASH, 0, keys["k0"], keys["k1"],
                                                      keys["mk0"], keys["mk1"], keys["k2"], keys["k3"])
            results[name] = ("ok", ko_, vo_)
        except RuntimeError as ex:
            results[name] = (str(ex), ko_, vo_)

    for rep in range(3):
        print(f"case 63 pending slots, repeat {rep}", flush=True)
        results.clear()
        torch.cuda.synchronize()
        with torch.cuda.stream(s0):
            torch.cuda._sleep(50_000_000)
        for _ in range(63):
            assert _ingress_async(e, e["blobs"][:n], ko, vo, st, s0) == 0
        barrier = threading.Barrier(2)
        outs = [(torch.full_like(e["k"], 3.0), torch.full_like(e["v"], 3.0)) for _ in range(2)]
        ta = threading.Thread(target=run, args=("a", e["tampered"], torch.cuda.Stream(), barrier, *outs[0]))
        tb = threading.Thread(target=run, args=("b", e["blobs"], torch.cuda.Stream(), barrier, *outs[1]))
        ta.start(); tb.start(); ta.join(); tb.join()
        torch.cuda.synchronize()
        msg, ka, va = results["a"]
        assert msg.startswith("KV_INTEGRITY_ERROR: Cold-page MAC verification failed"), msg
        assert not ka.any() and not va.any()
        msg, kb, vb = results["b"]
        assert msg == "ok"
        assert torch.equal(kb, e["ref_k"]) and torch.equal(vb, e["ref_v"])
        assert (st.cpu().numpy() == 0).all()


def test_expired_wait_fails_ingress_closed(env, hip):
    """Every wait that is not already satisfied gives up at once.  A workgroup
    whose waits all happened to be satisfied at their first poll decodes
    normally; every page of any other workgroup fails with ZTCP_ERR_DEVICE and
    is zeroed, and the call reports ZTCP_EDEVICE."""
    e = env
    N, W, keys = e["N"], e["W"], e["keys"]
    assert hip.device_diag() == 0
    prev = hip.debug_spin_limit(0)
    try:
        for per_page in (False, True):
            print(f"case expired ingress wait, per_page={per_page}", flush=True)
            ko, vo = torch.full_like(e["k"], 3.0), torch.full_like(e["v"], 3.0)
            st = torch.full((N_PAGES,), -1, dtype=torch.int32, device="cuda")
            g = N.geometry(e["w"].num_tokens, e["w"].num_heads, e["w"].head_dim, e["w"].rope_dim, N.HOT_BF16,
                           False)
            rc = N.lib().ztcp_ingress_peak_into(
                e["blobs"].data_ptr(), e["blobs"].size(1), e["th"].data_ptr(), ko.data_ptr(), vo.data_ptr(),
                N_PAGES, C.byref(g), W.TENANT_HASH, W.MODEL_HASH, 0, C.byref(N.keys(**keys)), st.data_ptr(),
                N.PER_PAGE if per_page else 0, C.c_void_p(torch.cuda.current_stream().cuda_stream))
            assert rc == N.EDEVICE
            s_ = st.cpu().numpy()
            assert np.isin(s_, (0, N.ERR_DEVICE)).all() and (s_ == N.ERR_DEVICE).any()
            if per_page:
                bad = torch.from_numpy(s_ != 0).cuda()
                assert not ko[bad].any() and not vo[bad].any()
                assert torch.equal(ko[~bad], e["ref_k"][~bad]) and torch.equal(vo[~bad], e["ref_v"][~bad])
            else:
                assert not ko.any() and not vo.any()
        ko, vo = torch.full_like(e["k"], 3.0), torch.full_like(e["v"], 3.0)
        with pytest.raises(RuntimeError, match="^KV_INTEGRITY_ERROR: device-side bounded wait expired"):
            hip.fused_decode_cold_pages_peak_into(e["blobs"], e["th"], ko, vo, e["w"].rope_dim, False,
                                                  W.TENANT_HASH, W.MODEL_HASH, 0, keys["k0"], keys["k1"],
                                                  keys["mk0"], keys["mk1"], keys["k2"], keys["k3"])
        assert not ko.any() and not vo.any()
    finally:
        hip.debug_spin_limit(prev)
    assert hip.device_diag() & 2  # the ingress bit, read and cleared
    assert hip.device_diag() == 0
    # with the default limit the same batch decodes again
    ko, vo = torch.empty_like(e["k"]), torch.empty_like(e["v"])
    hip.fused_decode_cold_pages_peak_into(e["blobs"], e["th"], ko, vo, e["w"].rope_dim, False, W.TENANT_HASH,
                                          W.MODEL_HASH, 0, keys["k0"], keys["k1"], keys["mk0"], keys["mk1"],
                                          keys["k2"], keys["k3"])
    assert torch.equal(ko, e["ref_k"]) and torch.equal(vo, e["ref_v"])


@pytest.mark.parametrize("n", [N_PAGES, 256], ids=["row-pipeline", "small-batch"])
def test_expired_wait_fails_egress_closed(env, hip, n):
    """Egress whose waits give up fails closed.  Synchronous (the reference's
    form): the call raises KV_INTEGRITY_ERROR with every blob zeroed, before
    any caller could commit the batch (nfc:597-600 zeroes out_blobs on any
    failure).  Asynchronous: the call returns once enqueued, and the blobs of
    the affected workgroups carry a zero header magic, which every ingress
    rejects with status 1 (cpp:2313-2316).  2,048 pages run the row-pipeline
    kernel, 256 pages (one per workgroup) the small-batch kernel."""
    e = dict(env)
    for key in ("k", "v", "th", "blobs"):
        e[key] = env[key][:n]
    N, W, keys, w = e["N"], e["W"], e["keys"], e["w"]
    print(f"case expired egress wait, {n} pages, synchronous", flush=True)
    blobs = torch.full_like(e["blobs"], 0xA5)
    prev = hip.debug_spin_limit(0)
    try:
        with pytest.raises(RuntimeError, match="^KV_INTEGRITY_ERROR: device-side bounded wait expired"):
            hip.fused_encode_cold_pages_peak_into(e["k"], e["v"], e["th"], blobs, w.preset, w.rope_mode,
                                                  w.rope_dim, w.payload_bytes, W.TENANT_HASH, W.MODEL_HASH, 0, 0,
                                                  0, keys["k0"], keys["k1"], keys["mk0"], keys["mk1"], keys["k2"],
                                                  keys["k3"])
        assert not blobs.any(), "every blob of the failed call is zeroed"
        print("case expired egress wait, asynchronous", flush=True)
        blobs.fill_(0xA5)
        g = N.geometry(w.num_tokens, w.num_heads, w.head_dim, w.rope_dim, N.HOT_BF16, False)
        aad = N.Aad(W.TENANT_HASH, W.MODEL_HASH, 0, 0)
        rc = N.lib().ztcp_egress_peak_into_ext(
            e["k"].data_ptr(), e["v"].data_ptr(), e["th"].data_ptr(), blobs.data_ptr(), n, C.byref(g),
            w.preset, w.rope_mode, w.payload_bytes, C.byref(aad), 0, C.byref(N.keys(**keys)), N.ASYNC,
            C.c_void_p(torch.cuda.current_stream().cuda_stream))
        assert rc == N.OK
        torch.cuda.synchronize()
    finally:
        hip.debug_spin_limit(prev)
    assert hip.device_diag() & 1
    assert not blobs[:, :16].any()
    ko, vo = torch.empty_like(e["k"]), torch.empty_like(e["v"])
    st = torch.full((n,), -1, dtype=torch.int32, device="cuda")
    with pytest.raises(RuntimeError, match="^KV_INTEGRITY_ERROR: Invalid cold-page header"):
        hip.fused_decode_cold_pages_peak_into(blobs, e["th"], ko, vo, w.rope_dim, False, W.TENANT_HASH,
                                              W.MODEL_HASH, 0, keys["k0"], keys["k1"], keys["mk0"], keys["mk1"],
                                              keys["k2"], keys["k3"], page_status=st, per_page=True)
    assert (st.cpu().numpy() == 1).all()
    assert hip.device_diag() == 0
    # the default limit encodes the same pages again, synchronously
    hip.fused_encode_cold_pages_peak_into(e["k"], e["v"], e["th"], blobs, w.preset, w.rope_mode, w.rope_dim,
                                          w.payload_bytes, W.TENANT_HASH, W.MODEL_HASH, 0, 0, 0, keys["k0"],
                                          keys["k1"], keys["mk0"], keys["mk1"], keys["k2"], keys["k3"])
    assert torch.equal(blobs, e["blobs"])


@pytest.mark.parametrize("limit", [16, 32])
def test_one_expired_wait_ends_the_workgroup_promptly(env, hip, limit):
    """With a small nonzero wait limit the MAC / verify wave's first wait (the
    first row takes tens of microseconds) expires in every workgroup; every
    later wait of the workgroup then returns at its next poll, so each launch
    still ends in about a normal launch time plus one bound, and fails
    closed.  (If each later wait spun out its own bound, the hundreds of
    waits per wave would take milliseconds.)"""
    e = env
    N, W, keys, w = e["N"], e["W"], e["keys"], e["w"]
    print(f"case wait limit {limit}: egress + ingress launch times", flush=True)
    g = N.geometry(w.num_tokens, w.num_heads, w.head_dim, w.rope_dim, N.HOT_BF16, False)
    aad = N.Aad(W.TENANT_HASH, W.MODEL_HASH, 0, 0)
    blobs = torch.empty_like(e["blobs"])
    ko, vo = torch.empty_like(e["k"]), torch.empty_like(e["v"])
    st = torch.full((N_PAGES,), -1, dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream()
    s = C.c_void_p(stream.cuda_stream)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
    prev = hip.debug_spin_limit(limit)
    try:
        torch.cuda.synchronize()
        ev[0].record(stream)
        rc = N.lib().ztcp_egress_peak_into_ext(
            e["k"].data_ptr(), e["v"].data_ptr(), e["th"].data_ptr(), blobs.data_ptr(), N_PAGES, C.byref(g),
            w.preset, w.rope_mode, w.payload_bytes, C.byref(aad), 0, C.byref(N.keys(**keys)), N.ASYNC, s)
        assert rc == N.OK
        ev[1].record(stream)
        rc = N.lib().ztcp_ingress_peak_into(
            e["blobs"].data_ptr(), e["blobs"].size(1), e["th"].data_ptr(), ko.data_ptr(), vo.data_ptr(), N_PAGES,
            C.byref(g), W.TENANT_HASH, W.MODEL_HASH, 0, C.byref(N.keys(**keys)), st.data_ptr(),
            N.ASYNC | N.PER_PAGE, s)
        assert rc == N.OK
        ev[2].record(stream)
        torch.cuda.synchronize()
    finally:
        hip.debug_spin_limit(prev)
    t_e, t_i = ev[0].elapsed_time(ev[1]), ev[1].elapsed_time(ev[2])
    print(f"limit {limit}: egress {t_e:.3f} ms, ingress {t_i:.3f} ms", flush=True)
    assert hip.device_diag() == 3  # both kernels' bits
    assert not blobs[:, :16].any()
    s_ = st.cpu().numpy()
    assert (s_ == N.ERR_DEVICE).all()
    assert not ko.any() and not vo.any()
    assert t_e < 2.0 and t_i < 2.0, (t_e, t_i)


def test_egress_extension_presets_need_the_flag(env, hip, O):
    e = env
    N, W, keys, w = e["N"], e["W"], e["keys"], e["w"]
    k, v, th = e["k"][:4], e["v"][:4], e["th"][:4]
    g = N.geometry(w.num_tokens, w.num_heads, w.head_dim, w.rope_dim, N.HOT_BF16, False)
    exp = O.payload_bytes(4, 3, w.num_tokens * w.num_heads, w.head_dim, w.rope_dim, True)
    out = torch.zeros((4, 48 + exp), dtype=torch.uint8, device="cuda")
    aad = N.Aad(W.TENANT_HASH, W.MODEL_HASH, 0, 0)
    s = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = N.lib().ztcp_egress_peak_into(k.data_ptr(), v.data_ptr(), th.data_ptr(), out.data_ptr(), 4, C.byref(g), 4,
                                       1, exp, C.byref(aad), 0, C.byref(N.keys(**keys)), s)
    assert rc == N.EINVAL and N.last_error() == "Invalid preset (must be 1..3)"
    rc = N.lib().ztcp_egress_peak_into(k.data_ptr(), v.data_ptr(), th.data_ptr(), out.data_ptr(), 4, C.byref(g), 1,
                                       3, exp, C.byref(aad), 0, C.byref(N.keys(**keys)), s)
    assert rc == N.EINVAL and N.last_error() == "Invalid rope_mode (must be 0..2)"
    with pytest.raises(RuntimeError, match=r"Invalid preset \(must be 1\.\.3\)"):
        hip.fused_encode_cold_pages_peak_into(k, v, th, out, 4, 3, w.rope_dim, exp, W.TENANT_HASH, W.MODEL_HASH,
                                              0, 0, 0, keys["k0"], keys["k1"], keys["mk0"], keys["mk1"],
                                              keys["k2"], keys["k3"])
    rc = N.lib().ztcp_egress_peak_into_ext(k.data_ptr(), v.data_ptr(), th.data_ptr(), out.data_ptr(), 4,
                                           C.byref(g), 4, 3, exp, C.byref(aad), 0, C.byref(N.keys(**keys)),
                                           N.EXT_LAYOUTS, s)
    assert rc == N.OK and N.last_error() == ""
    torch.cuda.synchronize()
    kb = k.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    vb = v.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    want = O.egress_batch(kb, vb, th.cpu().numpy(), dtype=O.BF16, preset=4, rope_mode=3, rope_dim=w.rope_dim,
                          expected_payload_bytes=exp, tenant_id_hash=W.TENANT_HASH, model_id_hash=W.MODEL_HASH,
                          layer_id=0, head_group_id=0, base_sequence_nonce=0, **keys)
    assert np.array_equal(out.cpu().numpy(), want)


def test_argument_errors_carry_the_reference_messages(env, hip):
    """Each EINVAL / EOVERLAP cause reports the reference's TORCH_CHECK text
    (cpp:1934-1957, cpp:2277-2294)."""
    e = env
    N, W, keys, w = e["N"], e["W"], e["keys"], e["w"]
    s = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    k, v, th = e["k"][:2], e["v"][:2], e["th"][:2]
    out = torch.zeros((2, w.blob_bytes), dtype=torch.uint8, device="cuda")
    aad = N.Aad(W.TENANT_HASH, W.MODEL_HASH, 0, 0)
    K = C.byref(N.keys(**keys))

    def eg(g, preset=1, rm=1, exp=w.payload_bytes, blobs=out, n=2):
        rc = N.lib().ztcp_egress_peak_into(k.data_ptr(), v.data_ptr(), th.data_ptr(), blobs.data_ptr(), n,
                                           C.byref(g), preset, rm, exp, C.byref(aad), 0, K, s)
        return rc, N.last_error()  # this thread's message for this call

    good = N.geometry(16, 4, 128, 64, N.HOT_BF16, False)
    cases = [
        (eg(N.geometry(16, 4, 120, 64, N.HOT_BF16, False)), N.EINVAL, "Invalid k_pages dimensions"),
        (eg(good, n=0), N.EINVAL, "Invalid k_pages dimensions"),
        (eg(N.geometry(16, 4, 128, 72, N.HOT_BF16, False)), N.EINVAL, "Invalid rope_dim"),
        (eg(good, exp=w.payload_bytes - 4), N.EINVAL, "expected_payload_bytes smaller than required payload"),
        (eg(good, blobs=k.view(torch.uint8)), N.EOVERLAP, "out_blobs must not alias or overlap input tensors"),
    ]
    for (rc, got), want_rc, msg in cases:
        assert rc == want_rc and got == msg, (rc, got, msg)
    ko = torch.empty_like(k)

    def ig(blob_bytes=w.blob_bytes, out_v=e["v"][2:4], out_k=ko, blobs=out):
        rc = N.lib().ztcp_ingress_peak_into(blobs.data_ptr(), blob_bytes, th.data_ptr(), out_k.data_ptr(),
                                            None if out_v is None else out_v.data_ptr(), 2, C.byref(good),
                                            W.TENANT_HASH, W.MODEL_HASH, 0, K, None, 0, s)
        return rc, N.last_error()

    # an output that overlaps the blobs by 16 bytes, inside one buffer large
    # enough for both
    kn = ko.numel() * 2
    both = torch.zeros(out.numel() + kn, dtype=torch.uint8, device="cuda")
    both[:out.numel()] = out.view(-1)
    cases = [
        (ig(blob_bytes=48), N.EINVAL, "cold_blob too small"),
        (ig(out_v=None), N.EINVAL, "out_v_pages is required for non-MLA geometry"),
        (ig(out_v=ko), N.EOVERLAP, "out_k_pages and out_v_pages must not alias or overlap in memory"),
        (ig(out_k=both[out.numel() - 16:out.numel() - 16 + kn], blobs=both[:out.numel()]), N.EOVERLAP,
         "out_k_pages must not alias or overlap input tensors"),
    ]
    for (rc, got), want_rc, msg in cases:
        assert rc == want_rc and got == msg, (rc, got, msg)
    # two errors at once: the reference's check order decides which is reported
    # (egress: overlap before preset, cpp:1940 / cpp:1952; ingress: the out_k
    # overlap before the missing out_v, cpp:2283 / cpp:2288)
    assert eg(good, preset=9, blobs=k.view(torch.uint8)) == (
        N.EOVERLAP, "out_blobs must not alias or overlap input tensors")
    assert ig(out_v=None, out_k=both[out.numel() - 16:out.numel() - 16 + kn], blobs=both[:out.numel()]) == (
        N.EOVERLAP, "out_k_pages must not alias or overlap input tensors")
    with pytest.raises(RuntimeError, match="^expected_payload_bytes smaller than required payload$"):
        hip.fused_encode_cold_pages_peak_into(k, v, th, torch.zeros((2, w.blob_bytes - 4), dtype=torch.uint8,
                                                                    device="cuda"),
                                              w.preset, w.rope_mode, w.rope_dim, w.payload_bytes - 4,
                                              W.TENANT_HASH, W.MODEL_HASH, 0, 0, 0, keys["k0"], keys["k1"],
                                              keys["mk0"], keys["mk1"], keys["k2"], keys["k3"])
