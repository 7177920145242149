"""Descriptor-based batch egress / ingress for paged, multi-layer KV pools.

One call covers pages of many layers: each page carries its own token hash,
sequence nonce, layer id and head-group id (``ztcp_page_desc`` in
include/ztcp.h).  This is how a whole evicted prefix (every layer) is encoded
in one launch instead of one reference call per layer
(fused_encode_cold_pages_peak_into_cpu takes a single layer_id, cpp:1915).
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import torch

from . import _native as N

DESC_BYTES = C.sizeof(N.PageDesc)
_DTYPES = {torch.float16: N.HOT_FP16, torch.bfloat16: N.HOT_BF16}


def build_descriptors(k_pages: torch.Tensor, v_pages: torch.Tensor | None, blobs: torch.Tensor,
                      token_hashes: np.ndarray, sequence_nonces: np.ndarray,
                      layer_ids: np.ndarray, head_group_ids: np.ndarray | None = None) -> torch.Tensor:
    """Descriptors for page i = (k_pages[i], v_pages[i], blobs[i], metadata[i]), on the
    pages' device.  Each page of k/v/blobs is contiguous; consecutive pages
    are k_pages.stride(0) (...) elements apart, so a pool of padded slots
    (e.g. blob slots rounded up to 128 bytes: ``buf[:, :blob_bytes]``) works."""
    n = k_pages.size(0)
    for name, t in (("k_pages", k_pages), ("v_pages", v_pages), ("blobs", blobs)):
        if t is not None and not t[0].is_contiguous():
            raise ValueError(f"build_descriptors: every page of {name} must be contiguous")
    dt = np.dtype([("k", "<u8"), ("v", "<u8"), ("blob", "<u8"), ("token_hash", "<i8"),
                   ("sequence_nonce", "<u8"), ("layer_id", "<u2"), ("head_group_id", "<u2"),
                   ("reserved", "<u4")])
    assert dt.itemsize == DESC_BYTES
    d = np.zeros(n, dtype=dt)
    idx = np.arange(n, dtype=np.uint64)
    step = lambda t: np.uint64(t.stride(0) * t.element_size())  # noqa: E731
    d["k"] = np.uint64(k_pages.data_ptr()) + idx * step(k_pages)
    if v_pages is not None:
        d["v"] = np.uint64(v_pages.data_ptr()) + idx * step(v_pages)
    d["blob"] = np.uint64(blobs.data_ptr()) + idx * step(blobs)
    d["token_hash"] = np.asarray(token_hashes, dtype=np.int64)
    d["sequence_nonce"] = np.asarray(sequence_nonces, dtype=np.uint64)
    d["layer_id"] = np.asarray(layer_ids, dtype=np.uint16)
    if head_group_ids is not None:
        d["head_group_id"] = np.asarray(head_group_ids, dtype=np.uint16)
    return torch.from_numpy(d.view(np.uint8).reshape(n, DESC_BYTES).copy()).to(k_pages.device)


def _stream() -> C.c_void_p:
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def egress(descs: torch.Tensor, n_pages: int, *, num_tokens: int, num_heads: int, head_dim: int,
           rope_dim: int, dtype: torch.dtype, is_mla_single_buffer: bool, preset: int,
           rope_mode: int, expected_payload_bytes: int, tenant_id_hash: int, model_id_hash: int,
           k0: int, k1: int, mk0: int, mk1: int, k2: int = 0, k3: int = 0,
           ext_layouts: bool = False, asynchronous: bool = False) -> None:
    """``ext_layouts`` admits the extension presets 4..6 / RoPE mode 3.
    Synchronous unless ``asynchronous``: an expired device-side wait then
    raises (every blob zeroed); asynchronously it shows as blobs no ingress
    accepts and in ``native_hip_codec.device_diag()``."""
    g = N.geometry(num_tokens, num_heads, head_dim, rope_dim, _DTYPES[dtype], is_mla_single_buffer)
    flags = (N.EXT_LAYOUTS if ext_layouts else 0) | (N.ASYNC if asynchronous else 0)
    rc = N.lib().ztcp_egress_batch_ext(descs.data_ptr(), n_pages, C.byref(g), preset, rope_mode,
                                       expected_payload_bytes, tenant_id_hash & 0xFFFFFFFF,
                                       model_id_hash & 0xFFFFFFFF,
                                       C.byref(N.keys(k0, k1, mk0, mk1, k2, k3)), flags, _stream())
    if rc in (N.EINVAL, N.EOVERLAP):
        raise RuntimeError(f"ztcp_egress_batch: {N.last_error()}")
    if rc == N.EDEVICE:
        raise RuntimeError("KV_INTEGRITY_ERROR: device-side bounded wait expired; outputs zeroed")
    if rc != N.OK:
        raise RuntimeError(f"ztcp_egress_batch: {N.strerror(rc)} ({rc})")


def ingress(descs: torch.Tensor, n_pages: int, blob_bytes: int, *, num_tokens: int,
            num_heads: int, head_dim: int, rope_dim: int, dtype: torch.dtype,
            is_mla_single_buffer: bool, expected_tenant_hash: int, expected_model_hash: int,
            k0: int, k1: int, mk0: int, mk1: int, k2: int = 0, k3: int = 0,
            page_status: torch.Tensor | None = None, per_page: bool = False,
            asynchronous: bool = False, ext_layouts: bool = False) -> int:
    """Returns the verdict of the lowest failing page (0 = all verified), or 0
    when ``asynchronous`` (verdicts then land in ``page_status``).
    ``ext_layouts`` accepts the extension presets / RoPE mode in headers."""
    g = N.geometry(num_tokens, num_heads, head_dim, rope_dim, _DTYPES[dtype], is_mla_single_buffer)
    flags = ((N.PER_PAGE if per_page else 0) | (N.ASYNC if asynchronous else 0)
             | (N.EXT_LAYOUTS if ext_layouts else 0))
    rc = N.lib().ztcp_ingress_batch(descs.data_ptr(), n_pages, blob_bytes, C.byref(g),
                                    expected_tenant_hash & 0xFFFFFFFF,
                                    expected_model_hash & 0xFFFFFFFF,
                                    C.byref(N.keys(k0, k1, mk0, mk1, k2, k3)),
                                    page_status.data_ptr() if page_status is not None else None,
                                    flags, _stream())
    if rc in (N.EINVAL, N.EOVERLAP):
        raise RuntimeError(f"ztcp_ingress_batch: {N.last_error()}")
    if rc < 0:
        raise RuntimeError(f"ztcp_ingress_batch: {N.strerror(rc)} ({rc})")
    return rc
