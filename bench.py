"""Benchmark: fused cold-page egress + ingress of a 1 GiB BF16 KV prefix on one MI355X.

A step is one egress pass (quantize -> ChaCha20 -> SipHash-2-4-128) and one
ingress pass (verify -> decrypt -> dequantize) over the whole prefix, with
pages resident in HBM and outputs preallocated: 4096 tokens x 64 layers =
16384 pages of 16 tokens x 8 KV heads x head_dim 128, K and V in BF16
(1 GiB hot), encoded through the descriptor API in one launch per direction.

  value     = 2 x hot bytes x steps / (egress + ingress time)   [GB/s]
  roofline  = the slower direction's kernel: algorithmic bytes (hot + wire:
              one read of the input, one write of the output) per launch / its
              average launch time (HIP events on its stream), against
              MI355X's 8 TB/s HBM peak
  cpu_baseline = the reference's own C++ codec (oracle/_ref, compiled from the
              reference sources) on this host's cores, FP16 (its only dtype),
              on a bounded sample of the same pages

Before the W warmup steps, each workload runs untimed egress + ingress pairs
for --settle-seconds (0.3 s; half that for the extra workloads), so that the
timed steps see the chip's clock under load rather than its climb from idle;
the line reports the number of those pairs and the first pair's times from
idle ("settle").

Usage: python bench.py [--gpus 1] [--steps 10] [--warmup 3] [--workload NAME]
"""
from __future__ import annotations

import argparse
import importlib.util
import json
import os
import statistics
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
METRIC = "hot-byte GB/s egress+ingress, 1 GiB BF16 prefix, 1 GPU; % of HBM roofline"
HBM_PEAK_GBPS = 8000.0


def _package():
    name = "vlx_tee_amd"
    if name in sys.modules:
        return sys.modules[name]
    root = REPO / "vlx-tee_amd"
    spec = importlib.util.spec_from_file_location(name, root / "__init__.py",
                                                  submodule_search_locations=[str(root)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def _log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# Phase-timer slots (TimerSlot in vlx-tee_amd/csrc/ztcp_rows.h).
_TM = dict(mac_rows_begin=0, mac_first_row=1, mac_rows_end=2, mac_end=3, wg_end=4, prod_first_row=5,
           prod_last=6, prod_busy=7, mac_wait=8, mac_miss=16, ring_wait=24, stage_wait=25, free_wait=26,
           storer_wait=27, feed_wait=28, storer_end=29, feed_end=30, prod_waves=31, rows=32, prod_setup=33,
           prod_loaded=34,
           abs_start=40, abs_end=41, real_start=42, real_end=43)


def summarize_phase_timers(rec) -> dict:
    """Per-workgroup means of the phase-timer records of one launch (shader
    clocks from the wave's leaving the first barrier), the shader clock rate
    (s_memtime against the 100 MHz s_memrealtime) and the launch's spread."""
    import numpy as np

    r = rec.astype(np.float64)
    col = lambda name, i=0: r[:, _TM[name] + i]  # noqa: E731
    real = (col("real_end") - col("real_start")) / 1e8
    ghz = float(np.mean((col("abs_end") - col("abs_start")) / np.maximum(real, 1e-12)) / 1e9)
    waves = np.maximum(col("prod_waves"), 1)
    m = lambda x: round(float(np.mean(x)), 1)  # noqa: E731
    return dict(
        workgroups=int(r.shape[0]), shader_ghz=round(ghz, 3),
        start_spread_us=round(float((col("real_start").max() - col("real_start").min()) / 100), 2),
        launch_span_us=round(float((col("real_end").max() - col("real_start").min()) / 100), 2),
        wg_clocks=m(col("wg_end")), wg_clocks_max=round(float(col("wg_end").max()), 1),
        # workgroup 0 also writes the row trace, which slows it down
        wg_clocks_max_untraced=round(float(col("wg_end")[1:].max()), 1) if r.shape[0] > 1 else None,
        wg_clocks_p90=round(float(np.percentile(col("wg_end"), 90)), 1),
        mac=dict(rows_begin=m(col("mac_rows_begin")), first_row=m(col("mac_first_row")),
                 rows_end=m(col("mac_rows_end")), end=m(col("mac_end")),
                 wait_total=m(sum(col("mac_wait", i) for i in range(8))),
                 wait_by_64_rows=[m(col("mac_wait", i)) for i in range(8)],
                 rows_not_ready_by_64_rows=[m(col("mac_miss", i)) for i in range(8)]),
        workers=dict(waves=m(col("prod_waves")), rows=m(col("rows")), setup=m(col("prod_setup")),
                     first_data=m(col("prod_loaded")), first_row=m(col("prod_first_row")),
                     last=m(col("prod_last")), busy_per_wave=m(col("prod_busy") / waves),
                     ring_wait_per_wave=m(col("ring_wait") / waves),
                     stage_wait_per_wave=m(col("stage_wait") / waves),
                     free_wait_per_wave=m(col("free_wait") / waves)),
        storer=dict(wait=m(col("storer_wait")), end=m(col("storer_end"))),
        feeder=dict(wait=m(col("feed_wait")), end=m(col("feed_end"))),
    )


def run_gpu(wname: str, steps: int, warmup: int, settle_s: float, timers: bool = False) -> dict:
    import numpy as np
    import torch

    _package().load_native()
    import vlx_tee_amd.pages as P
    from vlx_tee_amd.workloads import (MODEL_HASH, TENANT_HASH, WORKLOADS, generate, page_metadata,
                                       session_keys, tamper_plan)

    w = WORKLOADS[wname]
    dev = torch.device("cuda:0")
    keys = session_keys()
    _log(f"{wname}: generating {w.n_pages} pages on {dev}")
    k, v = generate(w, dev, torch.bfloat16)
    th, seq, layers = page_metadata(w)
    blobs = torch.empty((w.n_pages, w.blob_bytes), dtype=torch.uint8, device=dev)
    ko = torch.empty_like(k)
    vo = None if v is None else torch.empty_like(v)
    status = torch.full((w.n_pages,), -1, dtype=torch.int32, device=dev)
    d_out = P.build_descriptors(k, v, blobs, th, seq, layers)
    # tamper workloads: ingress reads a copy of the blobs with one bit flipped
    # in a seeded 1% of pages, under the per-page policy (failing pages zeroed)
    t_pages, t_bits = tamper_plan(w, w.blob_bytes)
    blobs_in = blobs.clone() if len(t_pages) else blobs
    d_in = P.build_descriptors(ko, vo, blobs_in, th, seq, layers)
    geo = dict(num_tokens=w.num_tokens, num_heads=w.num_heads, head_dim=w.head_dim,
               rope_dim=w.rope_dim, dtype=torch.bfloat16, is_mla_single_buffer=w.mla)

    def egress():
        P.egress(d_out, w.n_pages, preset=w.preset, rope_mode=w.rope_mode,
                 expected_payload_bytes=w.payload_bytes, tenant_id_hash=TENANT_HASH,
                 model_id_hash=MODEL_HASH, ext_layouts=w.extension, asynchronous=True, **geo, **keys)

    def ingress():
        P.ingress(d_in, w.n_pages, w.blob_bytes, expected_tenant_hash=TENANT_HASH,
                  expected_model_hash=MODEL_HASH, page_status=status, asynchronous=True,
                  per_page=bool(len(t_pages)), ext_layouts=w.extension, **geo, **keys)

    want_status = np.zeros(w.n_pages, dtype=np.int32)
    egress()
    torch.cuda.synchronize()
    if len(t_pages):
        blobs_in.copy_(blobs)
        idx = torch.from_numpy(t_pages).to(dev)
        cols = torch.from_numpy(t_bits // 8).to(dev)
        blobs_in[idx, cols] = blobs_in[idx, cols] ^ torch.from_numpy((1 << (t_bits % 8)).astype(np.uint8)).to(dev)
        want_status[t_pages] = -1  # any rejection verdict
    # self-consistency: a second encode reproduces the blobs bit for bit
    ref_blobs = blobs.clone()
    egress()
    torch.cuda.synchronize()
    if not torch.equal(ref_blobs, blobs):
        raise SystemExit("bench: egress is not deterministic")
    del ref_blobs

    # Settle: the chip leaves its idle clock over the first ~10 ms of load, and
    # pairs timed from idle run about 10 % slower than under sustained load (a
    # serving loop's state).  The same egress + ingress pairs run for at least
    # `settle_s` before the warmup steps; the result reports how many, and the
    # first pair's times from idle.
    stream = torch.cuda.current_stream()
    f0, f1, f2 = (torch.cuda.Event(enable_timing=True) for _ in range(3))
    torch.cuda.synchronize()
    ts = time.perf_counter()
    f0.record(stream)
    egress()
    f1.record(stream)
    ingress()
    f2.record(stream)
    settle_pairs = 1
    while time.perf_counter() - ts < settle_s:
        for _ in range(10):
            egress()
            ingress()
        settle_pairs += 10
        torch.cuda.synchronize()
    settle = dict(pairs=settle_pairs, s=round(time.perf_counter() - ts, 3),
                  first_pair_from_idle_ms=dict(egress=round(f0.elapsed_time(f1), 4),
                                               ingress=round(f1.elapsed_time(f2), 4)))
    for _ in range(warmup):
        egress()
        ingress()
    torch.cuda.synchronize()

    def check_status(when):
        st = status.cpu().numpy()
        bad = (st != 0) != (want_status != 0)
        if bad.any():
            raise SystemExit(f"bench: {int(bad.sum())} pages with the wrong verdict {when}")

    check_status("after warmup")
    import vlx_tee_amd.native_hip_codec as H

    diag = H.device_diag()

    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True),
           torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for e0, e1, e2 in ev:
        e0.record(stream)
        egress()
        e1.record(stream)
        ingress()
        e2.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    te = [a.elapsed_time(b) for a, b, _ in ev]
    ti = [b.elapsed_time(c) for _, b, c in ev]
    check_status("in the timed region")
    phase = None
    if timers:  # the records of the last step's two launches
        import vlx_tee_amd._native as N
        rows = w.payload_bytes // 64
        phase = dict(egress=summarize_phase_timers(N.phase_timers(0)),
                     ingress=summarize_phase_timers(N.phase_timers(1)))
        for d, name in ((0, "egress"), (1, "ingress")):
            arrive, absorb, group_wait, _ = N.phase_trace(d)
            phase[name]["trace_wg0"] = dict(arrive=arrive[:rows].tolist(), absorb=absorb[:rows].tolist(),
                                            group_wait=group_wait[:rows].tolist())
    hot = w.n_pages * w.hot_bytes_per_page
    wire = w.n_pages * w.blob_bytes
    me, mi = statistics.mean(te), statistics.mean(ti)
    res = dict(
        workload=wname, pages=w.n_pages, hot_bytes=hot, wire_bytes=wire,
        egress_ms=me, ingress_ms=mi, egress_ms_median=statistics.median(te),
        ingress_ms_median=statistics.median(ti), wall_s=wall,
        egress_hot_gbps=hot / me / 1e6, egress_wire_gbps=wire / me / 1e6,
        ingress_hot_gbps=hot / mi / 1e6, ingress_wire_gbps=wire / mi / 1e6,
        roundtrip_hot_gbps=2 * hot / (me + mi) / 1e6,
        egress_hbm_frac=(hot + wire) / me / 1e6 / HBM_PEAK_GBPS,
        ingress_hbm_frac=(hot + wire) / mi / 1e6 / HBM_PEAK_GBPS,
        tampered_pages_rejected=f"{len(t_pages)}/{len(t_pages)}" if len(t_pages) else None,
        settle=settle,
        device_diag=diag,
    )
    if phase is not None:
        res["phase_timers"] = phase
    del k, v, blobs, blobs_in, ko, vo
    torch.cuda.empty_cache()
    return res


def run_small(wname: str, steps: int) -> dict:
    """Egress and ingress of a small batch (the reference's peak-256 case,
    research/benchmarks/bench_cold_page_pipeline.py:924-930), each direction
    timed apart: pages in HBM, blobs and outputs preallocated.  Timed twice:
    launches back to back, with the 8 MiB of hot pages resident in the
    caches ("warm", the mean per launch), and each launch after the caches
    were flushed by writing a 1 GiB buffer ("flushed", HIP events around the
    launch alone)."""
    import torch

    _package().load_native()
    import vlx_tee_amd.pages as P
    from vlx_tee_amd.workloads import MODEL_HASH, TENANT_HASH, WORKLOADS, generate, page_metadata, session_keys

    w = WORKLOADS[wname]
    dev = torch.device("cuda:0")
    keys = session_keys()
    k, v = generate(w, dev, torch.bfloat16)
    th, seq, layers = page_metadata(w)
    blobs = torch.empty((w.n_pages, w.blob_bytes), dtype=torch.uint8, device=dev)
    ko, vo = torch.empty_like(k), torch.empty_like(v)
    status = torch.full((w.n_pages,), -1, dtype=torch.int32, device=dev)
    d = P.build_descriptors(k, v, blobs, th, seq, layers)
    d_in = P.build_descriptors(ko, vo, blobs, th, seq, layers)
    geo = dict(num_tokens=w.num_tokens, num_heads=w.num_heads, head_dim=w.head_dim,
               rope_dim=w.rope_dim, dtype=torch.bfloat16, is_mla_single_buffer=w.mla)

    def egress():
        P.egress(d, w.n_pages, preset=w.preset, rope_mode=w.rope_mode,
                 expected_payload_bytes=w.payload_bytes, tenant_id_hash=TENANT_HASH,
                 model_id_hash=MODEL_HASH, ext_layouts=w.extension, asynchronous=True, **geo, **keys)

    def ingress():
        P.ingress(d_in, w.n_pages, w.blob_bytes, expected_tenant_hash=TENANT_HASH,
                  expected_model_hash=MODEL_HASH, page_status=status, asynchronous=True,
                  ext_layouts=w.extension, **geo, **keys)

    egress()
    torch.cuda.synchronize()
    ref = blobs.clone()
    flush = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream()
    # warm: `steps` launches back to back between one pair of events (the
    # launches are queued while the GPU works, so no host gap is timed);
    # flushed: each launch queued behind a 1 GiB fill, between its own events
    times = {(f, c): [] for f in ("egress", "ingress") for c in ("warm", "flushed")}
    for name, fn in (("egress", egress), ("ingress", ingress)):
        for _ in range(3):
            fn()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        flush.fill_(0)  # keeps the GPU busy while the launches below are queued
        a.record(stream)
        for _ in range(steps):
            fn()
        b.record(stream)
        torch.cuda.synchronize()
        times[(name, "warm")].append(a.elapsed_time(b) / steps)
        for i in range(3 + steps):
            flush.fill_(i & 0xFF)
            c, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            c.record(stream)
            fn()
            e.record(stream)
            torch.cuda.synchronize()
            if i >= 3:
                times[(name, "flushed")].append(c.elapsed_time(e))
    if not torch.equal(ref, blobs):
        raise SystemExit(f"bench: {wname} egress is not deterministic")
    if not bool((status == 0).all()):
        raise SystemExit(f"bench: {wname} pages failed verification")
    hot = w.n_pages * w.hot_bytes_per_page
    wire = w.n_pages * w.blob_bytes
    res = dict(workload=wname, pages=w.n_pages, hot_bytes=hot, wire_bytes=wire, direction="egress and ingress")
    for (name, cache), t in times.items():
        m = statistics.mean(t)
        res[f"{name}_ms_{cache}"] = m
        res[f"{name}_hot_gbps_{cache}"] = hot / m / 1e6
    res["note"] = ("one page per workgroup (256 workgroups on 256 CUs), small-batch kernels: each launch lasts "
                   "about one page's SipHash chain, 1541 words in sequence")
    del k, v, blobs, flush, ref, ko, vo
    torch.cuda.empty_cache()
    return res


def run_wire_ring(wname: str, parts: int = 4, reps: int = 3) -> dict:
    """The egress wire step (serving.WireRing): the prefix's blobs leave HBM
    through two pinned host slots, one part of the pages per push.
    "copy": the blobs are already encoded; the time from the first push to the
    last landed copy.  "pipelined": egress of part i + 1 overlaps the copy of
    part i on the ring's own stream; the time from the first egress launch to
    the last landed copy.  Both are host wall clock over PCIe, so they are
    reported beside, never as, the HBM-resident figures."""
    import torch

    _package().load_native()
    import vlx_tee_amd.pages as P
    import vlx_tee_amd.serving as SV
    from vlx_tee_amd.workloads import MODEL_HASH, TENANT_HASH, WORKLOADS, generate, page_metadata, session_keys

    w = WORKLOADS[wname]
    dev = torch.device("cuda:0")
    keys = session_keys()
    k, v = generate(w, dev, torch.bfloat16)
    th, seq, layers = page_metadata(w)
    blobs = torch.empty((w.n_pages, w.blob_bytes), dtype=torch.uint8, device=dev)
    d = P.build_descriptors(k, v, blobs, th, seq, layers)
    geo = dict(num_tokens=w.num_tokens, num_heads=w.num_heads, head_dim=w.head_dim,
               rope_dim=w.rope_dim, dtype=torch.bfloat16, is_mla_single_buffer=w.mla)
    q = w.n_pages // parts

    def egress(i):
        P.egress(d[i * q:(i + 1) * q], q, preset=w.preset, rope_mode=w.rope_mode,
                 expected_payload_bytes=w.payload_bytes, tenant_id_hash=TENANT_HASH,
                 model_id_hash=MODEL_HASH, ext_layouts=w.extension, asynchronous=True, **geo, **keys)

    ring = SV.WireRing(q * w.blob_bytes, n_slots=2)
    copy_s, pipe_s = [], []
    for rep in range(1 + reps):
        for i in range(parts):
            egress(i)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(parts):
            ring.push(blobs[i * q:(i + 1) * q])
        ring.wait((parts - 1) % 2)
        ring.wait((parts - 2) % 2)
        t1 = time.perf_counter()
        for i in range(parts):
            egress(i)
            ring.push(blobs[i * q:(i + 1) * q])
        ring.wait((parts - 1) % 2)
        ring.wait((parts - 2) % 2)
        t2 = time.perf_counter()
        if rep:
            copy_s.append(t1 - t0)
            pipe_s.append(t2 - t1)
    wire = w.n_pages * w.blob_bytes
    mc, mp = statistics.mean(copy_s), statistics.mean(pipe_s)
    res = dict(workload=wname, parts=parts, slot_bytes=q * w.blob_bytes, wire_bytes=wire,
               copy_s=mc, pipelined_s=mp, copy_wire_gbps=wire / mc / 1e9,
               pipelined_wire_gbps=wire / mp / 1e9, pipelined_hot_gbps=w.n_pages * w.hot_bytes_per_page / mp / 1e9,
               note="device-to-host over PCIe into pinned slots, host wall clock; not an HBM figure")
    del k, v, blobs, ring
    torch.cuda.empty_cache()
    return res


def cpu_baseline(wname: str, budget_s: float) -> dict | None:
    """The reference's C++ codec on this host (FP16), on a bounded page sample."""
    import numpy as np
    import torch

    sys.path.insert(0, str(REPO))
    from oracle import oracle as O
    from vlx_tee_amd.workloads import MODEL_HASH, TENANT_HASH, WORKLOADS, generate, session_keys

    w = WORKLOADS[wname]
    keys = session_keys()
    ref = O.ref_module()
    threads = os.cpu_count() or 1

    def run(n):
        k, v = generate(w, "cpu", torch.float16, n_pages=n)
        th = torch.arange(n, dtype=torch.int64)
        if ref is not None:
            t0 = time.perf_counter()
            blobs = ref.fused_encode_cold_pages_batch_cpu(
                k, v, th, w.preset, w.rope_mode, w.rope_dim, w.payload_bytes, TENANT_HASH,
                MODEL_HASH, 0, 0, 0, keys["k0"], keys["k1"], keys["mk0"], keys["mk1"],
                keys["k2"], keys["k3"])
            t1 = time.perf_counter()
            ref.fused_decode_cold_pages_batch_cpu(
                blobs, th, w.num_tokens, w.num_heads, w.head_dim, w.rope_dim, w.mla, TENANT_HASH,
                MODEL_HASH, 0, keys["k0"], keys["k1"], keys["mk0"], keys["mk1"], keys["k2"], keys["k3"])
            t2 = time.perf_counter()
        else:
            kb = k.view(torch.int16).numpy().view(np.uint16)
            vb = None if v is None else v.view(torch.int16).numpy().view(np.uint16)
            t0 = time.perf_counter()
            blobs = O.egress_batch(kb, vb, th.numpy(), dtype=O.FP16, preset=w.preset,
                                   rope_mode=w.rope_mode, rope_dim=w.rope_dim,
                                   tenant_id_hash=TENANT_HASH, model_id_hash=MODEL_HASH, layer_id=0,
                                   head_group_id=0, base_sequence_nonce=0, threads=threads, **keys)
            t1 = time.perf_counter()
            O.ingress_batch(blobs, th.numpy(), num_tokens=w.num_tokens, num_heads=w.num_heads,
                            head_dim=w.head_dim, rope_dim=w.rope_dim, is_mla_single_buffer=w.mla,
                            dtype=O.FP16, expected_tenant_hash=TENANT_HASH,
                            expected_model_hash=MODEL_HASH, expected_layer_id=0, threads=1, **keys)
            t2 = time.perf_counter()
        return t1 - t0, t2 - t1

    def egress_1thread(n):
        """Egress one page per call: the reference's batch encoder runs
        min(batch, hardware threads) std::threads (cpp:1858-1861), so one."""
        k, v = generate(w, "cpu", torch.float16, n_pages=n)
        th = torch.arange(n, dtype=torch.int64)
        t0 = time.perf_counter()
        for i in range(n):
            if ref is not None:
                ref.fused_encode_cold_pages_batch_cpu(
                    k[i:i + 1], None if v is None else v[i:i + 1], th[i:i + 1], w.preset, w.rope_mode,
                    w.rope_dim, w.payload_bytes, TENANT_HASH, MODEL_HASH, 0, 0, i, keys["k0"], keys["k1"],
                    keys["mk0"], keys["mk1"], keys["k2"], keys["k3"])
            else:
                kb = k[i:i + 1].view(torch.int16).numpy().view(np.uint16)
                vb = None if v is None else v[i:i + 1].view(torch.int16).numpy().view(np.uint16)
                O.egress_batch(kb, vb, th[i:i + 1].numpy(), dtype=O.FP16, preset=w.preset,
                               rope_mode=w.rope_mode, rope_dim=w.rope_dim, tenant_id_hash=TENANT_HASH,
                               model_id_hash=MODEL_HASH, layer_id=0, head_group_id=0,
                               base_sequence_nonce=i, threads=1, **keys)
        return time.perf_counter() - t0

    te, ti = run(64)
    te1 = egress_1thread(16) * 4  # per 64 pages
    per_page = (te + ti + te1) / 64
    n = int(max(64, min(w.n_pages, budget_s / max(per_page, 1e-9))))
    te, ti = run(n)
    te1 = egress_1thread(n)
    hot = n * w.hot_bytes_per_page
    egress_threads = min(n, threads)
    try:
        model = next(l.split(":", 1)[1].strip() for l in open("/proc/cpuinfo") if l.startswith("model name"))
    except Exception:  # noqa: BLE001
        model = "unknown"
    return dict(
        value=2 * hot / (te1 + ti) / 1e9, unit="GB/s", cores=1,
        kind="reference" if ref is not None else "port",
        sample=(f"{n} pages of {wname} (FP16: the reference's only hot dtype) on one thread: egress "
                f"one page per fused_encode_cold_pages_batch_cpu call (one std::thread, cpp:1858-1861), "
                f"ingress through fused_decode_cold_pages_batch_cpu (serial on Linux, cpp:2215-2229); "
                f"host {threads} logical CPUs, {model}"),
        egress_hot_gbps=hot / te1 / 1e9, ingress_hot_gbps=hot / ti / 1e9,
        egress_s=te1, ingress_s=ti,
        threaded=dict(
            value=2 * hot / (te + ti) / 1e9, egress_threads=egress_threads, ingress_threads=1,
            egress_hot_gbps=hot / te / 1e9,
            note=("the reference's own threading: egress through fused_encode_cold_pages_batch_cpu on "
                  f"{egress_threads} std::threads, ingress serial"),
        ),
    )


def calibrate_copy(nbytes: int, reps: int) -> dict:
    """A plain copy kernel of known size (bitwise_not over int32: reads and writes
    nbytes each) whose FETCH_SIZE / WRITE_SIZE counters scale the codec's."""
    import torch

    dev = torch.device("cuda:0")
    src = torch.randint(-2**31, 2**31 - 1, (nbytes // 4,), dtype=torch.int32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(reps):
        torch.bitwise_not(src, out=dst)
    torch.cuda.synchronize()
    return dict(calibration="bitwise_not int32 copy", bytes_read=nbytes, bytes_written=nbytes, reps=reps)


def _rounded(d: dict) -> dict:
    return {k: (round(v, 4) if isinstance(v, float) else (_rounded(v) if isinstance(v, dict) else v))
            for k, v in d.items()}


def _describe(wname: str) -> str:
    """One line naming the workload's page shape, kinds and input distribution."""
    _package()
    from vlx_tee_amd.spec import QuantPreset, RoPEMode
    from vlx_tee_amd.workloads import WORKLOADS
    w = WORKLOADS[wname]
    if w.mla:
        shape = (f"{w.n_pages} MLA pages of {w.num_tokens} tok x {w.head_dim} "
                 f"({w.rope_dim} RoPE + {w.head_dim - w.rope_dim} latent), BF16")
        dist = f"latent N(0,{w.sigma:g}), RoPE N(0,{w.rope_sigma:g})"
    else:
        shape = (f"{w.n_pages} pages of {w.num_tokens} tok x {w.num_heads} KV heads x head_dim "
                 f"{w.head_dim}, K+V BF16")
        dist = f"N(0,{w.sigma:g}) with RoPE dims x{w.rope_scale:g}"
    if w.outlier_frac:
        dist += f", {w.outlier_frac:.0%} of channels x{w.outlier_scale:g}"
    hot = w.n_pages * w.hot_bytes_per_page
    layers = w.n_pages // w.pages_per_layer
    out = (f"{wname}: {w.pages_per_layer * w.num_tokens} tok x {layers} layers = {shape} ({hot / 2**30:.3g} GiB hot), {QuantPreset(w.preset).name} + "
           f"{RoPEMode(w.rope_mode).name}, {dist}")
    if w.tamper_frac:
        out += f", ingress over a copy with one bit flipped in {w.tamper_frac:.0%} of the pages"
    return out + ", one descriptor-batch launch per direction"


def _traffic(kernel: str, workload: str):
    """HBM bytes per launch from the committed rocprofv3 PMC summary, if any."""
    f = REPO / "profiles" / "hbm_traffic.json"
    if not f.is_file():
        return None
    try:
        return json.loads(f.read_text()).get(f"{kernel}/{workload}", {}).get("bytes_per_launch")
    except Exception:  # noqa: BLE001
        return None


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="c2_k8v4_prefix1g")
    ap.add_argument("--also", default=("c2_int4_prefix1g,c3_fp8only_tamper,c4_mla_int4,c2_k8v4asym_prefix1g,"
                                       "c3_e4m3_tamper,c4_mla_int4g32"),
                    help="comma list of extra workloads")
    ap.add_argument("--small", default="c1_int4_gqa256",
                    help="comma list of small workloads, egress and ingress timed apart (warm and cache-flushed)")
    ap.add_argument("--cpu-seconds", type=float, default=8.0)
    ap.add_argument("--settle-seconds", type=float, default=0.3,
                    help="untimed egress + ingress pairs before the warmup steps (clock leaves idle)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-wire", action="store_true", help="skip the wire-ring (device-to-host) measurement")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="BYTES",
                    help="only run a plain copy kernel of BYTES (counter calibration)")
    ap.add_argument("--phase-timers", action="store_true",
                    help=("only print the per-phase clock breakdown of the workloads' fused kernels, "
                          "from the timer build (libztcp_hip_timers.so); never a bench line"))
    a = ap.parse_args()
    if a.calibrate_copy:
        print(json.dumps(calibrate_copy(a.calibrate_copy, max(1, a.steps))))
        return
    if a.phase_timers:
        _package()
        import vlx_tee_amd._native as N
        N.use_timer_library()
        out = {}
        for wn in [a.workload] + [x for x in a.also.split(",") if x and x != a.workload]:
            r = run_gpu(wn, a.steps, a.warmup, a.settle_seconds, timers=True)
            out[wn] = dict(egress_ms=round(r["egress_ms"], 4), ingress_ms=round(r["ingress_ms"], 4),
                           phase_timers=r["phase_timers"])
            _log(f"{wn}: egress {out[wn]['egress_ms']} ms, ingress {out[wn]['ingress_ms']} ms")
        print(json.dumps(dict(phase_timers=out, build="libztcp_hip_timers.so")))
        return
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the cold-page codec has no cross-GPU step "
              "(pages shard independently); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    main_res = run_gpu(a.workload, a.steps, a.warmup, a.settle_seconds)
    extras = {}
    for wn in [x for x in a.also.split(",") if x and x != a.workload]:
        extras[wn] = run_gpu(wn, max(3, a.steps // 2), 2, a.settle_seconds / 2)
    for wn in [x for x in a.small.split(",") if x]:
        extras[wn] = run_small(wn, max(5, a.steps))
    wire_ring = None if a.no_wire else run_wire_ring(a.workload)
    cpu = None if a.no_cpu else cpu_baseline(a.workload, a.cpu_seconds)

    r = main_res
    # the roofline is that of the slower (dominant) direction's kernel; the
    # ingress time also covers its two small bookkeeping kernels
    dominant = "egress" if r["egress_ms"] >= r["ingress_ms"] else "ingress"
    kernel = f"{dominant}_fused_kernel"
    achieved = (r["hot_bytes"] + r["wire_bytes"]) / r[f"{dominant}_ms"] / 1e6
    out = {
        "metric": METRIC,
        "value": round(r["roundtrip_hot_gbps"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(r["egress_ms"] + r["ingress_ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u32",
        "data": "synthetic",
        "config": {
            "workload": _describe(a.workload),
            "pages": r["pages"], "hot_bytes": r["hot_bytes"], "wire_bytes": r["wire_bytes"],
        },
        "roofline": {
            "bound": "hbm", "kernel": kernel,
            "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": _traffic(kernel, a.workload),
        },
        "cpu_baseline": None if cpu is None else _rounded(cpu),
        "egress": {k: round(r[k], 4) for k in ("egress_ms", "egress_hot_gbps", "egress_wire_gbps", "egress_hbm_frac")},
        "ingress": {k: round(r[k], 4) for k in ("ingress_ms", "ingress_hot_gbps", "ingress_wire_gbps", "ingress_hbm_frac")},
        "extra_workloads": {n: {k: (round(v, 4) if isinstance(v, float) else v) for k, v in x.items()}
                            for n, x in extras.items()},
        "wire_ring": None if wire_ring is None else _rounded(wire_ring),
        "settle": r["settle"],
        "device_diag": r["device_diag"],
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
