"""The C ABI from C++: vlx-tee_amd/example/ztcp_capi_example.cpp, built by
vlx-tee_amd/build.py against include/ztcp.h and libztcp_hip.so, run as a
child process on the GPU; its blobs and decoded pages are compared with the
oracle.  The program encodes through the contiguous and the descriptor entry
points (ztcp_egress_peak_into, ztcp_egress_batch), decodes, and checks a
tampered batch's verdict and zeroing itself."""
import subprocess
from pathlib import Path

import numpy as np
import pytest

REPO = Path(__file__).resolve().parents[1]
EXE = REPO / "vlx-tee_amd" / "ztcp_capi_example"

PAGES, T, H, D, R = 64, 16, 4, 128, 64
TENANT, MODEL, LAYER, HEAD_GROUP, BASE_SEQ = 0x1234ABCD, 0x0BADF00D, 7, 1, 1000
KEYS = dict(k0=0x0706050403020100, k1=0x0F0E0D0C0B0A0908, k2=0x1716151413121110, k3=0x1F1E1D1C1B1A1918,
            mk0=0x2726252423222120, mk1=0x2F2E2D2C2B2A2928)


def _pages():
    """The program's page values: a 64-bit LCG, one state per element."""
    n = 2 * PAGES * T * H * D
    out = np.empty(n, dtype=np.uint16)
    x, m = 2024, (1 << 64) - 1
    for i in range(n):
        x = (x * 6364136223846793005 + 1442695040888963407) & m
        out[i] = ((x >> 63) << 15) | ((120 + (x >> 56) % 11) << 7) | ((x >> 40) & 0x7F)
    k, v = out.reshape(2, PAGES, T, H, D)
    return k, v


def test_example_is_built_against_the_library():
    assert EXE.is_file(), "build with python vlx-tee_amd/build.py"
    ldd = subprocess.run(["ldd", str(EXE)], capture_output=True, text=True, check=True).stdout
    assert str(REPO / "vlx-tee_amd" / "libztcp_hip.so") in ldd


@pytest.mark.gpu
def test_cpp_caller_matches_the_oracle(hip, O, tmp_path):
    print("case C++ caller of the C ABI: 64 pages, INT4_SYM + PRESERVE_FP8, BF16", flush=True)
    out = tmp_path / "capi.bin"
    r = subprocess.run([str(EXE), str(out)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    print(r.stdout.strip(), flush=True)
    k, v = _pages()
    th = np.array([(0x9E3779B97F4A7C15 * (i + 1)) & ((1 << 64) - 1) for i in range(PAGES)],
                  dtype=np.uint64).view(np.int64)
    want = O.egress_batch(k, v, th, dtype=O.BF16, preset=1, rope_mode=1, rope_dim=R, tenant_id_hash=TENANT,
                          model_id_hash=MODEL, layer_id=LAYER, head_group_id=HEAD_GROUP,
                          base_sequence_nonce=BASE_SEQ, **KEYS)
    raw = np.fromfile(out, dtype=np.uint8)
    blobs = raw[:want.size].reshape(want.shape)
    assert np.array_equal(blobs, want)
    rc, st, ok, ov = O.ingress_batch(want, th, num_tokens=T, num_heads=H, head_dim=D, rope_dim=R,
                                     is_mla_single_buffer=False, dtype=O.BF16, expected_tenant_hash=TENANT,
                                     expected_model_hash=MODEL, expected_layer_id=LAYER, **KEYS)
    assert rc == 0
    dec = raw[want.size:].view(np.uint16).reshape(2, PAGES, T, H, D)
    assert np.array_equal(dec[0], ok) and np.array_equal(dec[1], ov)
