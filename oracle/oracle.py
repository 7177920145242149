"""ctypes view of the CPU oracle (oracle/ztcp_oracle.c).

TEST INFRASTRUCTURE ONLY: tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg use this module as the CPU reference the HIP path is
compared against.  The product path never imports it.

Arrays are numpy; hot pages are passed as raw 16-bit patterns (uint16 views of
float16 / bfloat16 data).  ``dtype`` is ``FP16`` (the reference's dtype) or
``BF16`` (the extension).
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "build" / "libztcp_oracle.so"
REF_DIR = HERE / "_ref"

FP16, BF16 = 0, 1

_lib = None


class _EgressArgs(C.Structure):
    _fields_ = [
        ("k_pages", C.c_void_p), ("v_pages", C.c_void_p), ("token_hashes", C.c_void_p),
        ("out_blobs", C.c_void_p),
        ("batch", C.c_int64), ("num_tokens", C.c_int64), ("num_heads", C.c_int64),
        ("head_dim", C.c_int64), ("rope_dim", C.c_int64),
        ("dtype", C.c_int32),
        ("preset", C.c_int64), ("rope_mode", C.c_int64), ("expected_payload_bytes", C.c_int64),
        ("tenant_id_hash", C.c_uint32), ("model_id_hash", C.c_uint32),
        ("layer_id", C.c_uint16), ("head_group_id", C.c_uint16),
        ("base_sequence_nonce", C.c_uint64),
        ("k0", C.c_uint64), ("k1", C.c_uint64), ("k2", C.c_uint64), ("k3", C.c_uint64),
        ("mk0", C.c_uint64), ("mk1", C.c_uint64),
    ]


class _IngressArgs(C.Structure):
    _fields_ = [
        ("blobs", C.c_void_p), ("blob_bytes", C.c_int64), ("expected_token_hashes", C.c_void_p),
        ("out_k", C.c_void_p), ("out_v", C.c_void_p),
        ("batch", C.c_int64), ("num_tokens", C.c_int64), ("num_heads", C.c_int64),
        ("head_dim", C.c_int64), ("rope_dim", C.c_int64),
        ("dtype", C.c_int32), ("is_mla_single_buffer", C.c_int32),
        ("expected_tenant_hash", C.c_uint32), ("expected_model_hash", C.c_uint32),
        ("expected_layer_id", C.c_uint16),
        ("k0", C.c_uint64), ("k1", C.c_uint64), ("k2", C.c_uint64), ("k3", C.c_uint64),
        ("mk0", C.c_uint64), ("mk1", C.c_uint64),
    ]


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.is_file():
            raise RuntimeError(f"oracle not built ({LIB_PATH}); run: python oracle/build.py oracle")
        _lib = C.CDLL(str(LIB_PATH))
        _lib.zo_f32_to_f16.restype = C.c_uint16
        _lib.zo_f32_to_f16.argtypes = [C.c_float]
        _lib.zo_required_payload.restype = C.c_size_t
        _lib.zo_required_payload.argtypes = [C.c_int64] * 5 + [C.c_int]
        _lib.zo_payload_bytes.restype = C.c_size_t
        _lib.zo_payload_bytes.argtypes = [C.c_int64] * 5 + [C.c_int]
        _lib.zo_siphash128.argtypes = [C.c_void_p, C.c_size_t, C.c_uint64, C.c_uint64, C.c_void_p]
        _lib.zo_chacha20_xor.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p,
                                         C.c_uint32, C.c_void_p]
        _lib.zo_egress_batch.argtypes = [C.POINTER(_EgressArgs), C.c_int]
        _lib.zo_egress_batch.restype = C.c_int
        _lib.zo_ingress_batch.argtypes = [C.POINTER(_IngressArgs), C.c_void_p, C.c_int, C.c_int]
        _lib.zo_ingress_batch.restype = C.c_int
        for n in ("zo_f32_to_f16_array", "zo_f32_to_bf16_array", "zo_f16_to_f32_array"):
            getattr(_lib, n).argtypes = [C.c_void_p, C.c_void_p, C.c_size_t]
        _lib.zo_quant_groups.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_size_t, C.c_void_p,
                                         C.c_void_p]
        _lib.zo_dequant_groups.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_int,
                                           C.c_size_t, C.c_void_p]
        _lib.zo_quant_groups_ext.argtypes = [C.c_int, C.c_void_p, C.c_int, C.c_size_t, C.c_void_p,
                                             C.c_void_p]
        _lib.zo_dequant_groups_ext.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_int, C.c_size_t,
                                               C.c_void_p]
        _lib.zo_f32_to_e4m3_array.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t]
        _lib.zo_e4m3_to_f32_array.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t]
    return _lib


def _ptr(a: np.ndarray | None) -> int | None:
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def _u16(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a)
    return a.view(np.uint16)


# ---- primitives ------------------------------------------------------------

def chacha20_xor(data: bytes | np.ndarray, key32: bytes, counter: int, nonce12: bytes) -> bytes:
    src = np.frombuffer(bytes(data), dtype=np.uint8).copy()
    dst = np.empty_like(src)
    k = np.frombuffer(key32, dtype=np.uint8).copy()
    n = np.frombuffer(nonce12, dtype=np.uint8).copy()
    lib().zo_chacha20_xor(_ptr(src), _ptr(dst), src.size, _ptr(k), counter & 0xFFFFFFFF, _ptr(n))
    return dst.tobytes()


def siphash128(data: bytes | np.ndarray, mk0: int, mk1: int) -> bytes:
    src = np.frombuffer(bytes(data), dtype=np.uint8).copy()
    tag = np.empty(16, dtype=np.uint8)
    lib().zo_siphash128(_ptr(src) if src.size else None, src.size, mk0, mk1, _ptr(tag))
    return tag.tobytes()


def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().zo_f32_to_f16_array(_ptr(x), _ptr(out), x.size)
    return out


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().zo_f32_to_bf16_array(_ptr(x), _ptr(out), x.size)
    return out


def f16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().zo_f16_to_f32_array(_ptr(h), _ptr(out), h.size)
    return out


def quant_groups(src_bits: np.ndarray, dtype: int, bits: int):
    """src_bits: [n, 16] uint16 hot patterns -> (codes [n, 16|8] u8, scales [n] u16)."""
    s = np.ascontiguousarray(src_bits, dtype=np.uint16).reshape(-1, 16)
    n = s.shape[0]
    q = np.empty((n, 16 if bits == 8 else 8), dtype=np.uint8)
    sc = np.empty(n, dtype=np.uint16)
    lib().zo_quant_groups(_ptr(s), dtype, bits, n, _ptr(q), _ptr(sc))
    return q, sc


def dequant_groups(q: np.ndarray, scales: np.ndarray, dtype: int, bits: int) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.uint8)
    sc = np.ascontiguousarray(scales, dtype=np.uint16)
    n = sc.size
    out = np.empty((n, 16), dtype=np.uint16)
    lib().zo_dequant_groups(_ptr(q), _ptr(sc), dtype, bits, n, _ptr(out))
    return out


# Extension section kinds (no counterpart in the reference):
# kind -> (elements per group, code bytes per group, parameter bytes per group)
SEC_E4M3, SEC_INT4G32, SEC_ASYM8 = 3, 4, 5
EXT_KINDS = {SEC_E4M3: (16, 16, 2), SEC_INT4G32: (32, 16, 2), SEC_ASYM8: (64, 64, 4)}


def f32_to_e4m3(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint8)
    lib().zo_f32_to_e4m3_array(_ptr(x), _ptr(out), x.size)
    return out


def e4m3_to_f32(c: np.ndarray) -> np.ndarray:
    c = np.ascontiguousarray(c, dtype=np.uint8)
    out = np.empty(c.shape, dtype=np.float32)
    lib().zo_e4m3_to_f32_array(_ptr(c), _ptr(out), c.size)
    return out


def quant_groups_ext(src_bits: np.ndarray, dtype: int, kind: int):
    """src_bits: [n, ges] uint16 hot patterns -> (codes [n, cb] u8, params [n, 2] u16:
    fp16 scale bits, zero point)."""
    ges, cb, _ = EXT_KINDS[kind]
    s = np.ascontiguousarray(src_bits, dtype=np.uint16).reshape(-1, ges)
    n = s.shape[0]
    q = np.empty((n, cb), dtype=np.uint8)
    prm = np.empty((n, 2), dtype=np.uint16)
    assert lib().zo_quant_groups_ext(kind, _ptr(s), dtype, n, _ptr(q), _ptr(prm)) == 0
    return q, prm


def dequant_groups_ext(q: np.ndarray, params: np.ndarray, dtype: int, kind: int) -> np.ndarray:
    ges, cb, _ = EXT_KINDS[kind]
    q = np.ascontiguousarray(q, dtype=np.uint8).reshape(-1, cb)
    prm = np.ascontiguousarray(params, dtype=np.uint16).reshape(-1, 2)
    out = np.empty((q.shape[0], ges), dtype=np.uint16)
    assert lib().zo_dequant_groups_ext(kind, _ptr(q), _ptr(prm), dtype, q.shape[0], _ptr(out)) == 0
    return out


def required_payload(preset, rope_mode, vecs, head_dim, rope_dim, has_v) -> int:
    r = lib().zo_required_payload(preset, rope_mode, vecs, head_dim, rope_dim, int(has_v))
    return -1 if r == (1 << 64) - 1 else int(r)


def payload_bytes(preset, rope_mode, vecs, head_dim, rope_dim, has_v) -> int:
    r = lib().zo_payload_bytes(preset, rope_mode, vecs, head_dim, rope_dim, int(has_v))
    return -1 if r == (1 << 64) - 1 else int(r)


# ---- batches ---------------------------------------------------------------

def egress_batch(k: np.ndarray, v: np.ndarray | None, token_hashes: np.ndarray, *,
                 dtype: int, preset: int, rope_mode: int, rope_dim: int,
                 expected_payload_bytes: int | None = None,
                 tenant_id_hash: int, model_id_hash: int, layer_id: int,
                 head_group_id: int, base_sequence_nonce: int,
                 k0: int, k1: int, mk0: int, mk1: int, k2: int = 0, k3: int = 0,
                 threads: int = 1, out: np.ndarray | None = None) -> np.ndarray:
    """Oracle batch egress: k, v are [B, T, H, D] 16-bit hot patterns."""
    k = _u16(k)
    v = _u16(v) if v is not None else None
    B, T, H, D = k.shape
    if expected_payload_bytes is None:
        expected_payload_bytes = payload_bytes(preset, rope_mode, T * H, D, rope_dim, v is not None)
    th = np.ascontiguousarray(token_hashes, dtype=np.int64)
    blob = 32 + expected_payload_bytes + 16
    if out is None:
        out = np.empty((B, blob), dtype=np.uint8)
    a = _EgressArgs(_ptr(k), _ptr(v), _ptr(th), _ptr(out), B, T, H, D, rope_dim, dtype,
                    preset, rope_mode, expected_payload_bytes, tenant_id_hash & 0xFFFFFFFF,
                    model_id_hash & 0xFFFFFFFF, layer_id & 0xFFFF, head_group_id & 0xFFFF,
                    base_sequence_nonce & (2**64 - 1), k0, k1, k2, k3, mk0, mk1)
    rc = lib().zo_egress_batch(C.byref(a), threads)
    if rc != 0:
        raise RuntimeError("oracle egress rejected its arguments")
    return out


def ingress_batch(blobs: np.ndarray, expected_token_hashes: np.ndarray, *, num_tokens: int,
                  num_heads: int, head_dim: int, rope_dim: int, is_mla_single_buffer: bool,
                  dtype: int, expected_tenant_hash: int, expected_model_hash: int,
                  expected_layer_id: int, k0: int, k1: int, mk0: int, mk1: int,
                  k2: int = 0, k3: int = 0, all_or_nothing: bool = True, threads: int = 1,
                  out_k: np.ndarray | None = None, out_v: np.ndarray | None = None):
    """Returns (rc, status[B], k_out u16, v_out u16 | None)."""
    blobs = np.ascontiguousarray(blobs, dtype=np.uint8)
    B, L = blobs.shape
    th = np.ascontiguousarray(expected_token_hashes, dtype=np.int64)
    shape = (B, num_tokens, num_heads, head_dim)
    if out_k is None:
        out_k = np.empty(shape, dtype=np.uint16)
    if out_v is None and not is_mla_single_buffer:
        out_v = np.empty(shape, dtype=np.uint16)
    status = np.zeros(B, dtype=np.int32)
    a = _IngressArgs(_ptr(blobs), L, _ptr(th), _ptr(out_k),
                     None if is_mla_single_buffer else _ptr(out_v), B, num_tokens, num_heads,
                     head_dim, rope_dim, dtype, int(is_mla_single_buffer),
                     expected_tenant_hash & 0xFFFFFFFF, expected_model_hash & 0xFFFFFFFF,
                     expected_layer_id & 0xFFFF, k0, k1, k2, k3, mk0, mk1)
    rc = lib().zo_ingress_batch(C.byref(a), _ptr(status), int(all_or_nothing), threads)
    if rc < 0:
        raise RuntimeError("oracle ingress rejected its arguments")
    return rc, status, out_k, (None if is_mla_single_buffer else out_v)


def ref_module():
    """The reference codec compiled by oracle/build.py, or None if absent."""
    import importlib
    import sys

    if not any(REF_DIR.glob("ztcp_fused_cold_page_cpp*.so")):
        return None
    if str(REF_DIR) not in sys.path:
        sys.path.insert(0, str(REF_DIR))
    import torch  # noqa: F401  (the extension links libtorch)

    return importlib.import_module("ztcp_fused_cold_page_cpp")


def default_threads() -> int:
    return max(1, os.cpu_count() or 1)
