"""ctypes binding of the C-ABI library (include/ztcp.h and include/ztcp_keyring.h
-> libztcp_hip.so).

The library is loaded after ``torch`` so both share torch's HIP runtime (the
library's DT_NEEDED ``libamdhip64.so.7`` resolves to the copy torch already
mapped).  There is no fallback: a missing library raises at load time.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import torch  # noqa: F401  (must be loaded before the HIP library)

LIB_PATH = Path(__file__).resolve().parent / "libztcp_hip.so"

# Return codes (include/ztcp.h).
OK, ERR_HEADER, ERR_AAD, ERR_MAC, ERR_DEVICE = 0, 1, 2, 3, 4
EINVAL, EOVERLAP, EHIP, EDEVICE, ESCRATCH = -1, -2, -3, -4, -5
NOALLOC_MAX_PAGES = 65536
ASYNC, PER_PAGE, EXT_LAYOUTS = 0x1, 0x2, 0x4
HOT_FP16, HOT_BF16 = 0, 1

# Every symbol include/ztcp.h declares.
EXPORTS = (
    "ztcp_payload_bytes", "ztcp_required_payload_bytes", "ztcp_blob_bytes",
    "ztcp_egress_peak_into", "ztcp_egress_peak_into_ext", "ztcp_egress_batch", "ztcp_egress_batch_ext",
    "ztcp_ingress_peak_into", "ztcp_ingress_peak_into_noalloc", "ztcp_ingress_batch",
    "ztcp_chacha20_xor", "ztcp_siphash128",
    "ztcp_selftest", "ztcp_device_diag", "ztcp_debug_spin_limit", "ztcp_strerror",
    "ztcp_last_error", "ztcp_hit_bitmap", "ztcp_wire_ring_create", "ztcp_wire_ring_push",
    "ztcp_wire_ring_wait", "ztcp_wire_ring_destroy",
)

# Every symbol include/ztcp_keyring.h declares (host code, callable without a GPU).
KEYRING_EXPORTS = (
    "ztcp_keyring_create", "ztcp_keyring_destroy", "ztcp_keyring_derive_or_get",
    "ztcp_keyring_derive_with_secret_for_test", "ztcp_keyring_next_sequence_nonce",
    "ztcp_keyring_preflight_egress", "ztcp_keyring_begin_egress", "ztcp_keyring_commit_egress",
    "ztcp_keyring_release_reservation", "ztcp_reservation_last_sequence",
    "ztcp_reservation_generation", "ztcp_keyring_begin_ingress", "ztcp_keyring_verify_freshness",
    "ztcp_keyring_verify_freshness_batch", "ztcp_keyring_finish_ingress",
    "ztcp_keyring_shred_session", "ztcp_keyring_shred_tenant", "ztcp_keyring_last_error",
    "ztcp_sha256", "ztcp_hmac_sha256",
)

# Key-ring return codes (include/ztcp_keyring.h).
KR_EINVAL, KR_ESTALE, KR_ENONCE, KR_ESHREDDED, KR_ENOMEM, KR_ERANDOM = -1, -10, -11, -12, -13, -14


class Geometry(C.Structure):
    _fields_ = [("num_tokens", C.c_int64), ("num_heads", C.c_int64), ("head_dim", C.c_int64),
                ("rope_dim", C.c_int64), ("hot_dtype", C.c_int32),
                ("is_mla_single_buffer", C.c_int32)]


class Aad(C.Structure):
    _fields_ = [("tenant_id_hash", C.c_uint32), ("model_id_hash", C.c_uint32),
                ("layer_id", C.c_uint16), ("head_group_id", C.c_uint16)]


class Keys(C.Structure):
    _fields_ = [("k0", C.c_uint64), ("k1", C.c_uint64), ("k2", C.c_uint64), ("k3", C.c_uint64),
                ("mk0", C.c_uint64), ("mk1", C.c_uint64)]


class PageDesc(C.Structure):
    _fields_ = [("k", C.c_void_p), ("v", C.c_void_p), ("blob", C.c_void_p),
                ("token_hash", C.c_int64), ("sequence_nonce", C.c_uint64),
                ("layer_id", C.c_uint16), ("head_group_id", C.c_uint16),
                ("reserved", C.c_uint32)]


# The phase-timer build of the same sources (vlx-tee_amd/build.py): the same
# ABI plus ztcp_phase_timers_read (include/ztcp_timers.h).  Only a caller
# that asks for it (bench.py --phase-timers) loads it, before any other use.
TIMERS_LIB_PATH = Path(__file__).resolve().parent / "libztcp_hip_timers.so"

_lib: C.CDLL | None = None


def use_timer_library() -> None:
    """Load the phase-timer build instead of the product library; must be
    called before the library is first loaded."""
    global LIB_PATH
    if _lib is not None and LIB_PATH != TIMERS_LIB_PATH:
        raise RuntimeError("the product library is already loaded")
    LIB_PATH = TIMERS_LIB_PATH


def lib() -> C.CDLL:
    """The loaded C-ABI library (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.is_file():
        raise RuntimeError(
            f"HIP codec library missing: {LIB_PATH} (build it with python vlx-tee_amd/build.py)")
    L = C.CDLL(str(LIB_PATH))
    if LIB_PATH == TIMERS_LIB_PATH:
        L.ztcp_phase_timers_read.argtypes = [C.c_int32, C.c_void_p, C.c_int64]
        L.ztcp_phase_timers_read.restype = C.c_int64
        L.ztcp_phase_trace_read.argtypes = [C.c_int32, C.c_void_p, C.c_int64]
        L.ztcp_phase_trace_read.restype = C.c_int64
    P, G, A, K = C.c_void_p, C.POINTER(Geometry), C.POINTER(Aad), C.POINTER(Keys)
    i64, u64, u32, u16, i32 = C.c_int64, C.c_uint64, C.c_uint32, C.c_uint16, C.c_int
    for name in ("ztcp_payload_bytes", "ztcp_required_payload_bytes", "ztcp_blob_bytes"):
        f = getattr(L, name)
        f.argtypes = [G, i64, i64]
        f.restype = C.c_size_t
    L.ztcp_egress_peak_into.argtypes = [P, P, P, P, i64, G, i64, i64, i64, A, u64, K, P]
    L.ztcp_egress_peak_into.restype = i32
    L.ztcp_egress_peak_into_ext.argtypes = [P, P, P, P, i64, G, i64, i64, i64, A, u64, K, u32, P]
    L.ztcp_egress_peak_into_ext.restype = i32
    L.ztcp_egress_batch.argtypes = [P, i64, G, i64, i64, i64, u32, u32, K, P]
    L.ztcp_egress_batch.restype = i32
    L.ztcp_egress_batch_ext.argtypes = [P, i64, G, i64, i64, i64, u32, u32, K, u32, P]
    L.ztcp_egress_batch_ext.restype = i32
    L.ztcp_ingress_peak_into.argtypes = [P, i64, P, P, P, i64, G, u32, u32, u16, K, P, u32, P]
    L.ztcp_ingress_peak_into.restype = i32
    L.ztcp_ingress_peak_into_noalloc.argtypes = [P, i64, P, P, P, i64, G, u32, u32, u16, K, P, u32, P]
    L.ztcp_ingress_peak_into_noalloc.restype = i32
    L.ztcp_ingress_batch.argtypes = [P, i64, i64, G, u32, u32, K, P, u32, P]
    L.ztcp_ingress_batch.restype = i32
    L.ztcp_chacha20_xor.argtypes = [P, P, C.c_size_t, P, u32, P, P]
    L.ztcp_chacha20_xor.restype = i32
    L.ztcp_siphash128.argtypes = [P, C.c_size_t, u64, u64, P, P]
    L.ztcp_siphash128.restype = i32
    L.ztcp_selftest.argtypes = []
    L.ztcp_selftest.restype = i32
    L.ztcp_device_diag.argtypes = []
    L.ztcp_device_diag.restype = i32
    L.ztcp_debug_spin_limit.argtypes = [i64]
    L.ztcp_debug_spin_limit.restype = i64
    L.ztcp_strerror.argtypes = [i32]
    L.ztcp_strerror.restype = C.c_char_p
    L.ztcp_last_error.argtypes = []
    L.ztcp_last_error.restype = C.c_char_p
    L.ztcp_hit_bitmap.argtypes = [P, i64, P, i32, P]
    L.ztcp_hit_bitmap.restype = i32
    L.ztcp_wire_ring_create.argtypes = [C.c_size_t, i32, C.POINTER(C.c_void_p)]
    L.ztcp_wire_ring_create.restype = i32
    L.ztcp_wire_ring_push.argtypes = [P, P, C.c_size_t, P, C.POINTER(C.c_int32)]
    L.ztcp_wire_ring_push.restype = i32
    L.ztcp_wire_ring_wait.argtypes = [P, i32, C.POINTER(C.c_void_p), C.POINTER(C.c_size_t)]
    L.ztcp_wire_ring_wait.restype = i32
    L.ztcp_wire_ring_destroy.argtypes = [P]
    L.ztcp_wire_ring_destroy.restype = i32
    _bind_keyring(L)
    _lib = L
    return L


def _bind_keyring(L: C.CDLL) -> None:
    P, S, B, SZ = C.c_void_p, C.c_char_p, C.c_char_p, C.c_size_t
    u64, u32, u16, i32 = C.c_uint64, C.c_uint32, C.c_uint16, C.c_int
    PP, PU64 = C.POINTER(C.c_void_p), C.POINTER(C.c_uint64)
    sig = {
        "ztcp_keyring_create": ([B, SZ, PP], i32),
        "ztcp_keyring_destroy": ([P], None),
        "ztcp_keyring_derive_or_get": ([P, S, S, P, P, PU64], i32),
        "ztcp_keyring_derive_with_secret_for_test": ([P, S, S, B, P, P, PU64], i32),
        "ztcp_keyring_next_sequence_nonce": ([P, S, S, u64, PU64], i32),
        "ztcp_keyring_preflight_egress": ([P, S, S, u32, u16, u16, u64, P, SZ, PP], i32),
        "ztcp_keyring_begin_egress": ([P, S, S, P, P, P], i32),
        "ztcp_keyring_commit_egress": ([P, S, S, P], i32),
        "ztcp_keyring_release_reservation": ([P, S, S, P], None),
        "ztcp_reservation_last_sequence": ([P], u64),
        "ztcp_reservation_generation": ([P], u64),
        "ztcp_keyring_begin_ingress": ([P, S, S, PU64, P, P], i32),
        "ztcp_keyring_verify_freshness": ([P, S, S, u32, u16, u16, u64, u64, PU64, PU64, PU64], i32),
        "ztcp_keyring_verify_freshness_batch": ([P, S, S, P, SZ, PU64, PU64], i32),
        "ztcp_keyring_finish_ingress": ([P, S, S, u64], i32),
        "ztcp_keyring_shred_session": ([P, S, S], i32),
        "ztcp_keyring_shred_tenant": ([P, S], i32),
        "ztcp_keyring_last_error": ([], C.c_char_p),
        "ztcp_sha256": ([B, SZ, P], None),
        "ztcp_hmac_sha256": ([B, SZ, B, SZ, P], None),
    }
    for name, (args, res) in sig.items():
        f = getattr(L, name)
        f.argtypes = args
        f.restype = res


TIMER_SLOTS = 48  # include/ztcp_timers.h ZTCP_TIMER_SLOTS
TRACE_ROWS = 1024  # ZTCP_TRACE_ROWS


def phase_timers(direction: int):
    """Phase-timer records of the last fused launch of `direction` (0 egress,
    1 ingress) as a uint64 array [workgroups, TIMER_SLOTS] (timer build only)."""
    import numpy as np

    L = lib()
    if not hasattr(L, "ztcp_phase_timers_read"):
        raise RuntimeError("phase timers need the timer build (use_timer_library)")
    buf = np.zeros(4096 * TIMER_SLOTS, dtype=np.uint64)
    n = L.ztcp_phase_timers_read(direction, buf.ctypes.data, buf.size)
    if n < 0:
        raise RuntimeError(f"ztcp_phase_timers_read: {strerror(int(n))}")
    return buf[:n].reshape(-1, TIMER_SLOTS)


def phase_trace(direction: int):
    """Workgroup 0's row trace of the last fused launch of `direction`:
    uint32 arrays of TRACE_ROWS (ring arrival clocks, absorption clocks,
    at the first row of each group of four that was not ready: the clocks
    waited for its rows; a fourth array of zeros)."""
    import numpy as np

    L = lib()
    buf = np.zeros(4 * TRACE_ROWS, dtype=np.uint32)
    n = L.ztcp_phase_trace_read(direction, buf.ctypes.data, buf.size)
    if n < 0:
        raise RuntimeError(f"ztcp_phase_trace_read: {strerror(int(n))}")
    return tuple(buf[i * TRACE_ROWS:(i + 1) * TRACE_ROWS] for i in range(4))


def strerror(code: int) -> str:
    return lib().ztcp_strerror(code).decode()


def last_error() -> str:
    """Why this thread's last call returned EINVAL / EOVERLAP (the reference's message)."""
    return lib().ztcp_last_error().decode()


def geometry(num_tokens: int, num_heads: int, head_dim: int, rope_dim: int, hot_dtype: int,
             is_mla_single_buffer: bool) -> Geometry:
    return Geometry(num_tokens, num_heads, head_dim, rope_dim, hot_dtype, int(is_mla_single_buffer))


def keys(k0: int, k1: int, mk0: int, mk1: int, k2: int = 0, k3: int = 0) -> Keys:
    m = (1 << 64) - 1
    return Keys(k0 & m, k1 & m, k2 & m, k3 & m, mk0 & m, mk1 & m)
