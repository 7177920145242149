"""Payload sizing and the C ABI surface (no GPU needed).

Sizes are pinned by the ten blob sizes the reference publishes
(research/benchmarks/RESULTS_LOG.md:41-54) and by the compiled reference's
required_payload_bytes_for_flags behaviour via the oracle.
"""
import ctypes as C
import re
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent

PUBLISHED = {  # (tokens, heads, head_dim, rope, mla) -> [(preset, rope_mode, blob bytes)]
    (64, 8, 128, 64, False): [(1, 0, 81968), (1, 1, 98352), (1, 2, 127024), (2, 1, 114736),
                              (3, 1, 147504)],
    (128, 1, 576, 64, True): [(1, 0, 46128), (1, 1, 50224), (1, 2, 57392), (2, 1, 82992),
                              (3, 1, 82992)],
}
CONFIG_BLOBS = {  # the benchmark workloads' blob sizes
    "c0_int4_gqa64": 12336, "c1_int4_gqa256": 12336, "c2_k8v4_prefix1g": 28720,
    "c2_int4_prefix1g": 24624, "c3_fp8only_tamper": 36912, "c4_mla_int4": 25136,
    # extension kinds: asym8 K + e4m3 RoPE + int4/32 V; e4m3 everywhere; MLA int4/32 + e4m3 RoPE
    "c2_k8v4asym_prefix1g": 27184, "c3_e4m3_tamper": 36912, "c4_mla_int4g32": 23088,
}


@pytest.mark.parametrize("geo", list(PUBLISHED))
def test_published_blob_sizes(pkg, O, geo):
    import vlx_tee_amd._native as N
    from vlx_tee_amd.spec import ColdPageGeometry

    T, H, D, R, mla = geo
    g = N.geometry(T, H, D, R, N.HOT_FP16, mla)
    spec = ColdPageGeometry(T, H, D, R, 16, 2, mla)
    for preset, rm, blob in PUBLISHED[geo]:
        assert N.lib().ztcp_blob_bytes(C.byref(g), preset, rm) == blob
        assert spec.cold_blob_bytes(preset, rm) == blob
        assert O.payload_bytes(preset, rm, T * H, D, R, not mla) + 48 == blob


def test_workload_blob_sizes(pkg):
    from vlx_tee_amd.workloads import WORKLOADS

    for name, blob in CONFIG_BLOBS.items():
        assert WORKLOADS[name].blob_bytes == blob, name


def test_invalid_flags_sizes(pkg, O):
    import vlx_tee_amd._native as N

    g = N.geometry(16, 4, 128, 64, N.HOT_FP16, False)
    for preset, rm in [(0, 1), (7, 1), (1, 4), (1, -1)]:
        assert N.lib().ztcp_payload_bytes(C.byref(g), preset, rm) == (1 << 64) - 1
        assert O.required_payload(preset, rm, 64, 128, 64, True) == -1
    # extension kinds whose group does not divide the section width
    g = N.geometry(16, 4, 128, 16, N.HOT_FP16, False)   # K main section: 112 columns
    for preset in (4, 6):
        assert N.lib().ztcp_payload_bytes(C.byref(g), preset, 1) == (1 << 64) - 1
        assert O.required_payload(preset, 1, 64, 128, 16, True) == -1


def test_extension_sizes_agree(pkg, O):
    """Native sizing == oracle == Python spec for every extension preset / RoPE mode."""
    import vlx_tee_amd._native as N
    from vlx_tee_amd.spec import ColdPageGeometry

    for (T, H, D, R, mla) in [(16, 8, 128, 64, False), (64, 1, 576, 64, True), (4, 2, 64, 32, False),
                              (2, 2, 128, 0, False), (3, 1, 256, 128, True)]:
        g = N.geometry(T, H, D, R, N.HOT_BF16, mla)
        geo = ColdPageGeometry(T, H, D, R, is_mla_single_buffer=mla)
        for preset in range(1, 7):
            for rm in range(4):
                if preset <= 3 and rm <= 2:
                    continue
                req = O.required_payload(preset, rm, T * H, D, R, not mla)
                if req == -1:  # a group wider than its section: rejected by all three
                    assert N.lib().ztcp_required_payload_bytes(C.byref(g), preset, rm) == (1 << 64) - 1
                    with pytest.raises(ValueError):
                        geo.cold_blob_bytes(preset, rm)
                    continue
                assert N.lib().ztcp_required_payload_bytes(C.byref(g), preset, rm) == req
                assert N.lib().ztcp_blob_bytes(C.byref(g), preset, rm) == ((req + 3) & ~3) + 48
                assert geo.cold_blob_bytes(preset, rm) == ((req + 3) & ~3) + 48


def test_required_vs_padded(pkg, O):
    import vlx_tee_amd._native as N

    for (T, H, D, R, mla) in [(1, 1, 16, 16, False), (3, 1, 48, 16, True), (5, 3, 32, 0, False)]:
        g = N.geometry(T, H, D, R, N.HOT_BF16, mla)
        for preset in (1, 2, 3):
            for rm in (0, 1, 2):
                req = O.required_payload(preset, rm, T * H, D, R, not mla)
                assert N.lib().ztcp_required_payload_bytes(C.byref(g), preset, rm) == req
                assert N.lib().ztcp_payload_bytes(C.byref(g), preset, rm) == (req + 3) & ~3


@pytest.mark.parametrize("header,exports", [("ztcp.h", "EXPORTS"), ("ztcp_keyring.h", "KEYRING_EXPORTS")])
def test_library_exports_every_declared_symbol(pkg, header, exports):
    import vlx_tee_amd._native as N

    text = (REPO / "include" / header).read_text()
    declared = set(re.findall(r"^\s*(?:[\w\*\s]+?)\b(ztcp_\w+)\s*\(", text, flags=re.M))
    assert declared == set(getattr(N, exports)), declared ^ set(getattr(N, exports))
    lib = N.lib()
    for name in declared:
        assert hasattr(lib, name), name


def test_strerror_matches_reference_messages(pkg):
    import vlx_tee_amd._native as N

    assert N.strerror(1).startswith("KV_INTEGRITY_ERROR:")
    assert N.strerror(2).startswith("CROSS_TENANT_CONTAMINATION:")
    assert N.strerror(3) == "KV_INTEGRITY_ERROR: Cold-page MAC verification failed"


def test_python_mirror_rejects_host_tensors(pkg):
    import torch
    import vlx_tee_amd.native_hip_codec as H

    k = torch.zeros((1, 16, 4, 128), dtype=torch.float16)
    with pytest.raises(RuntimeError, match="contiguous HIP float16 or bfloat16"):
        H.fused_encode_cold_pages_peak_into(k, k, torch.zeros(1, dtype=torch.int64),
                                            torch.zeros((1, 12336), dtype=torch.uint8), 1, 1, 64,
                                            12288, 0, 0, 0, 0, 0, 1, 2, 3, 4)


def test_library_exports_exactly_the_declared_symbols(pkg):
    """The product library's dynamic symbol table holds the entry points of
    include/ztcp.h and include/ztcp_keyring.h and nothing else; the timer
    build adds ztcp_phase_timers_read (include/ztcp_timers.h)."""
    import shutil
    import subprocess

    import vlx_tee_amd._native as N

    if shutil.which("nm") is None:
        pytest.skip("nm (binutils) not available")

    def exported(path):
        out = subprocess.run(["nm", "-D", "--defined-only", str(path)], capture_output=True, text=True,
                             check=True).stdout
        return {line.split()[-1] for line in out.splitlines() if line.strip()}

    declared = set(N.EXPORTS) | set(N.KEYRING_EXPORTS)
    assert exported(N.LIB_PATH) == declared
    if N.TIMERS_LIB_PATH.is_file():
        assert exported(N.TIMERS_LIB_PATH) == declared | {"ztcp_phase_timers_read", "ztcp_phase_trace_read"}
