"""HIP drop-in for the reference's native codec module.

The reference exposes its C++ codec to Python as the pybind11 module
``ztcp_fused_cold_page_cpp`` (research/baseline_codec/csrc/
fused_cold_page_cpu.cpp:2540-2683), called only by
``NativeCppFusedColdPageCodec`` (research/baseline_codec/native_fused_codec.py).
This module exposes the same functions, with the same argument names, order,
meaning and error behaviour, on HIP tensors resident in HBM, by calling the
C-ABI library (include/ztcp.h).  Names drop the ``_cpu`` suffix.

Differences, all extensions:
  * pages may be ``torch.bfloat16`` as well as ``torch.float16`` (the wire
    format is unchanged; scales stay fp16);
  * token hashes may live on the host or the device;
  * decode entry points take optional ``page_status`` (int32 device tensor,
    per-page verdicts) and ``per_page`` (keep verified pages, zero only the
    failing ones instead of the reference's all-or-nothing zeroing).

Errors: argument problems raise ``RuntimeError`` (the reference's
TORCH_CHECKs); integrity failures raise ``RuntimeError`` whose message starts
with ``KV_INTEGRITY_ERROR:`` or ``CROSS_TENANT_CONTAMINATION:`` exactly as the
reference's (cpp:2237-2243), which native_fused_codec.py:416-422 maps to its
exception types.
"""
from __future__ import annotations

import ctypes as C

import torch

from . import _native as N

_DTYPES = {torch.float16: N.HOT_FP16, torch.bfloat16: N.HOT_BF16}

_MSG = {
    N.ERR_HEADER: "KV_INTEGRITY_ERROR: Invalid cold-page header magic, version, or flags",
    N.ERR_AAD: "CROSS_TENANT_CONTAMINATION: Cold-page AAD mismatch",
    N.ERR_MAC: "KV_INTEGRITY_ERROR: Cold-page MAC verification failed",
}


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _stream() -> C.c_void_p:
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def _hot_dtype(t: torch.Tensor, name: str) -> int:
    _check(t.is_cuda and t.is_contiguous() and t.dtype in _DTYPES,
           f"{name} must be a contiguous HIP float16 or bfloat16 tensor")
    return _DTYPES[t.dtype]


def _hashes_on(t: torch.Tensor, device: torch.device, name: str, n: int) -> torch.Tensor:
    _check(isinstance(t, torch.Tensor) and t.dtype == torch.int64 and t.is_contiguous(),
           f"{name} must be contiguous int64")
    _check(t.dim() == 1 and t.size(0) == n, f"{name} must be 1D with length equal to batch_size")
    return t if t.device == device else t.to(device)


def _raise_rc(rc: int) -> None:
    if rc == N.OK:
        return
    if rc in _MSG:
        raise RuntimeError(_MSG[rc])
    if rc in (N.EINVAL, N.EOVERLAP):  # the reference's TORCH_CHECK message for the condition
        raise RuntimeError(N.last_error())
    if rc == N.EDEVICE:  # fail closed: outputs are zeroed, the batch is rejected
        raise RuntimeError("KV_INTEGRITY_ERROR: device-side bounded wait expired; outputs zeroed")
    raise RuntimeError(f"ztcp: {N.strerror(rc)} (code {rc})")


# ---- egress -------------------------------------------------------------------

def fused_encode_cold_pages_peak_into(
    k_pages: torch.Tensor, v_pages_opt: torch.Tensor | None, page_token_hashes: torch.Tensor,
    out_blobs: torch.Tensor, preset: int, rope_mode: int, rope_dim: int,
    expected_payload_bytes: int, tenant_id_hash: int, model_id_hash: int, layer_id: int,
    head_group_id: int, base_sequence_nonce: int, k0: int, k1: int, mk0: int, mk1: int,
    k2: int = 0, k3: int = 0, *, ext_layouts: bool = False,
) -> None:
    """Batch egress into a preallocated [B, blob_bytes] uint8 tensor (cpp:1904-2004).

    Presets 1..3 and RoPE modes 0..2, as the reference; ``ext_layouts`` also
    admits this codec's extension presets 4..6 and RoPE mode 3."""
    dt = _hot_dtype(k_pages, "k_pages")
    _check(k_pages.dim() == 4, "k_pages must have shape [batch, num_tokens, num_heads, head_dim]")
    _check(out_blobs.is_cuda and out_blobs.is_contiguous() and out_blobs.dtype == torch.uint8,
           "out_blobs must be contiguous HIP uint8 tensor")
    _check(out_blobs.dim() == 2, "out_blobs must have shape [batch, total_blob_bytes]")
    B, T, H, D = k_pages.shape
    _check(B > 0 and T > 0 and H > 0 and D >= 16 and D % 16 == 0, "Invalid k_pages dimensions")
    _check(0 <= rope_dim <= D and rope_dim % 16 == 0, "Invalid rope_dim")
    _check(out_blobs.size(0) == B and out_blobs.size(1) == 48 + expected_payload_bytes,
           "out_blobs shape must be [batch_size, total_blob_bytes]")
    if v_pages_opt is not None:
        _check(_hot_dtype(v_pages_opt, "v_pages") == dt and v_pages_opt.device == k_pages.device,
               "v_pages must match k_pages dtype and device")
        _check(v_pages_opt.shape == k_pages.shape, "v_pages shape must match k_pages shape")
    # cpp:1947-1948; presets 4..6 and RoPE mode 3 are this codec's extension
    # kinds (include/ztcp.h), admitted only on request
    if ext_layouts:
        _check(1 <= preset <= 6, "Invalid preset (must be 1..6)")
        _check(0 <= rope_mode <= 3, "Invalid rope_mode (must be 0..3)")
    else:
        _check(1 <= preset <= 3, "Invalid preset (must be 1..3)")
        _check(0 <= rope_mode <= 2, "Invalid rope_mode (must be 0..2)")
    th = _hashes_on(page_token_hashes, k_pages.device, "page_token_hashes", B)
    g = N.geometry(T, H, D, rope_dim, dt, False)
    aad = N.Aad(tenant_id_hash & 0xFFFFFFFF, model_id_hash & 0xFFFFFFFF, layer_id & 0xFFFF,
                head_group_id & 0xFFFF)
    with torch.cuda.device(k_pages.device):
        rc = N.lib().ztcp_egress_peak_into_ext(
            k_pages.data_ptr(), v_pages_opt.data_ptr() if v_pages_opt is not None else None,
            th.data_ptr(), out_blobs.data_ptr(), B, C.byref(g), preset, rope_mode,
            expected_payload_bytes, C.byref(aad), base_sequence_nonce & ((1 << 64) - 1),
            C.byref(N.keys(k0, k1, mk0, mk1, k2, k3)), N.EXT_LAYOUTS if ext_layouts else 0,
            _stream())
    _raise_rc(rc)


def fused_encode_cold_pages_batch(
    k_pages: torch.Tensor, v_pages_opt: torch.Tensor | None, page_token_hashes: torch.Tensor,
    preset: int, rope_mode: int, rope_dim: int, expected_payload_bytes: int,
    tenant_id_hash: int, model_id_hash: int, layer_id: int, head_group_id: int,
    base_sequence_nonce: int, k0: int, k1: int, mk0: int, mk1: int, k2: int = 0, k3: int = 0, *,
    ext_layouts: bool = False,
) -> torch.Tensor:
    """Allocating batch egress (cpp:1775-1902): returns [B, blob_bytes] uint8."""
    _check(k_pages.dim() == 4, "k_pages must have shape [batch, num_tokens, num_heads, head_dim]")
    out = torch.empty((k_pages.size(0), 48 + expected_payload_bytes), dtype=torch.uint8,
                      device=k_pages.device)
    fused_encode_cold_pages_peak_into(
        k_pages, v_pages_opt, page_token_hashes, out, preset, rope_mode, rope_dim,
        expected_payload_bytes, tenant_id_hash, model_id_hash, layer_id, head_group_id,
        base_sequence_nonce, k0, k1, mk0, mk1, k2, k3, ext_layouts=ext_layouts)
    return out


def fused_encode_cold_page(
    k_page: torch.Tensor, v_page_opt: torch.Tensor | None, preset: int, rope_mode: int,
    rope_dim: int, expected_payload_bytes: int, tenant_id_hash: int, model_id_hash: int,
    layer_id: int, head_group_id: int, page_token_hash: int, sequence_nonce: int,
    k0: int, k1: int, mk0: int, mk1: int, k2: int = 0, k3: int = 0, *, ext_layouts: bool = False,
) -> torch.Tensor:
    """Single-page egress (cpp:1478-1555): returns a 1D uint8 blob."""
    _check(k_page.dim() == 3, "k_page must have shape [num_tokens, num_heads, head_dim]")
    th = torch.tensor([page_token_hash - (1 << 64) if page_token_hash >= (1 << 63) else page_token_hash],
                      dtype=torch.int64)
    out = fused_encode_cold_pages_batch(
        k_page.unsqueeze(0), v_page_opt.unsqueeze(0) if v_page_opt is not None else None, th,
        preset, rope_mode, rope_dim, expected_payload_bytes, tenant_id_hash, model_id_hash,
        layer_id, head_group_id, sequence_nonce, k0, k1, mk0, mk1, k2, k3, ext_layouts=ext_layouts)
    return out[0]


# ---- ingress ------------------------------------------------------------------

def fused_decode_cold_pages_peak_into(
    cold_blobs: torch.Tensor, expected_token_hashes: torch.Tensor, out_k_pages: torch.Tensor,
    out_v_pages_opt: torch.Tensor | None, rope_dim: int, is_mla_single_buffer: bool,
    expected_tenant_hash: int, expected_model_hash: int, expected_layer_id: int,
    k0: int, k1: int, mk0: int, mk1: int, k2: int = 0, k3: int = 0, *,
    page_status: torch.Tensor | None = None, per_page: bool = False, ext_layouts: bool = False,
) -> None:
    """Batch ingress into preallocated outputs (cpp:2250-2496).

    Raises the reference's integrity errors for the lowest failing page; with
    the default all-or-nothing policy both outputs are zeroed first.
    ``ext_layouts`` accepts the extension presets / RoPE mode in headers
    (otherwise they fail the flags check, as in the reference)."""
    _check(cold_blobs.is_cuda and cold_blobs.is_contiguous() and cold_blobs.dtype == torch.uint8,
           "cold_blobs must be contiguous HIP uint8")
    _check(cold_blobs.dim() == 2, "cold_blobs must have shape [batch, total_blob_bytes]")
    dt = _hot_dtype(out_k_pages, "out_k_pages")
    _check(out_k_pages.dim() == 4, "out_k_pages must have shape [batch, num_tokens, num_heads, head_dim]")
    B, T, H, D = out_k_pages.shape
    _check(B > 0 and T > 0 and H > 0 and D >= 16 and D % 16 == 0, "Invalid out_k_pages dimensions")
    _check(0 <= rope_dim <= D and rope_dim % 16 == 0, "Invalid rope_dim")
    _check(cold_blobs.size(0) == B, "cold_blobs batch size must match out_k_pages batch size")
    L = cold_blobs.size(1)
    _check(L > 48, "cold_blob too small")
    v_ptr = None
    if not is_mla_single_buffer:
        _check(out_v_pages_opt is not None, "out_v_pages is required for non-MLA geometry")
        _check(_hot_dtype(out_v_pages_opt, "out_v_pages") == dt, "out_v_pages must match out_k_pages dtype")
        _check(out_v_pages_opt.shape == out_k_pages.shape, "out_v_pages shape must match out_k_pages shape")
        v_ptr = out_v_pages_opt.data_ptr()
    th = _hashes_on(expected_token_hashes, cold_blobs.device, "expected_token_hashes", B)
    st_ptr = None
    if page_status is not None:
        _check(page_status.is_cuda and page_status.dtype == torch.int32 and page_status.numel() == B
               and page_status.is_contiguous(), "page_status must be a contiguous HIP int32 [batch]")
        st_ptr = page_status.data_ptr()
    g = N.geometry(T, H, D, rope_dim, dt, is_mla_single_buffer)
    flags = (N.PER_PAGE if per_page else 0) | (N.EXT_LAYOUTS if ext_layouts else 0)
    with torch.cuda.device(cold_blobs.device):
        rc = N.lib().ztcp_ingress_peak_into(
            cold_blobs.data_ptr(), L, th.data_ptr(), out_k_pages.data_ptr(), v_ptr, B, C.byref(g),
            expected_tenant_hash & 0xFFFFFFFF, expected_model_hash & 0xFFFFFFFF,
            expected_layer_id & 0xFFFF, C.byref(N.keys(k0, k1, mk0, mk1, k2, k3)), st_ptr, flags,
            _stream())
    _raise_rc(rc)


def fused_decode_cold_pages_batch(
    cold_blobs: torch.Tensor, expected_token_hashes: torch.Tensor, num_tokens: int,
    num_heads: int, head_dim: int, rope_dim: int, is_mla_single_buffer: bool,
    expected_tenant_hash: int, expected_model_hash: int, expected_layer_id: int,
    k0: int, k1: int, mk0: int, mk1: int, k2: int = 0, k3: int = 0, *,
    dtype: torch.dtype = torch.float16, ext_layouts: bool = False,
) -> tuple[torch.Tensor, torch.Tensor | None]:
    """Allocating batch ingress (cpp:2006-2248)."""
    _check(cold_blobs.dim() == 2, "cold_blobs must have shape [batch, total_blob_bytes]")
    shape = (cold_blobs.size(0), num_tokens, num_heads, head_dim)
    k = torch.empty(shape, dtype=dtype, device=cold_blobs.device)
    v = None if is_mla_single_buffer else torch.empty(shape, dtype=dtype, device=cold_blobs.device)
    fused_decode_cold_pages_peak_into(
        cold_blobs, expected_token_hashes, k, v, rope_dim, is_mla_single_buffer,
        expected_tenant_hash, expected_model_hash, expected_layer_id, k0, k1, mk0, mk1, k2, k3,
        ext_layouts=ext_layouts)
    return k, v


def fused_decode_cold_page(
    cold_blob: torch.Tensor, num_tokens: int, num_heads: int, head_dim: int, rope_dim: int,
    is_mla_single_buffer: bool, expected_tenant_hash: int, expected_model_hash: int,
    expected_layer_id: int, expected_token_hash: int, k0: int, k1: int, mk0: int, mk1: int,
    k2: int = 0, k3: int = 0, *, dtype: torch.dtype = torch.float16, ext_layouts: bool = False,
) -> tuple[torch.Tensor, torch.Tensor | None]:
    """Single-page ingress (cpp:1557-1773)."""
    _check(cold_blob.dim() == 1, "cold_blob must be a 1D tensor")
    _check(cold_blob.numel() > 48, "cold_blob too small")
    h = expected_token_hash & ((1 << 64) - 1)
    th = torch.tensor([h - (1 << 64) if h >= (1 << 63) else h], dtype=torch.int64)
    k, v = fused_decode_cold_pages_batch(
        cold_blob.unsqueeze(0), th, num_tokens, num_heads, head_dim, rope_dim,
        is_mla_single_buffer, expected_tenant_hash, expected_model_hash, expected_layer_id,
        k0, k1, mk0, mk1, k2, k3, dtype=dtype, ext_layouts=ext_layouts)
    return k[0], (None if v is None else v[0])


# ---- known-answer hooks ----------------------------------------------------------

def chacha20_rfc8439_xor(data_u8: torch.Tensor, key_u8: torch.Tensor, initial_counter: int,
                         nonce_u8: torch.Tensor) -> torch.Tensor:
    """RFC 8439 ChaCha20 XOR of a device buffer (cpp:2499-2524)."""
    _check(data_u8.is_cuda and data_u8.is_contiguous() and data_u8.dtype == torch.uint8,
           "data_u8 must be contiguous HIP uint8")
    key = bytes(key_u8.cpu().contiguous().numpy().tobytes())
    nonce = bytes(nonce_u8.cpu().contiguous().numpy().tobytes())
    _check(len(key) == 32, "key_u8 must be 32-byte uint8")
    _check(len(nonce) == 12, "nonce_u8 must be 12-byte uint8")
    out = torch.empty_like(data_u8)
    kb = (C.c_uint8 * 32).from_buffer_copy(key)
    nb = (C.c_uint8 * 12).from_buffer_copy(nonce)
    with torch.cuda.device(data_u8.device):
        rc = N.lib().ztcp_chacha20_xor(data_u8.data_ptr(), out.data_ptr(), data_u8.numel(), kb,
                                       initial_counter & 0xFFFFFFFF, nb, _stream())
    _raise_rc(rc)
    return out


def siphash24_128(data_u8: torch.Tensor, mk0: int, mk1: int) -> torch.Tensor:
    """SipHash-2-4-128 of a device buffer (cpp:2526-2538): 16-byte device tensor."""
    _check(data_u8.is_cuda and data_u8.is_contiguous() and data_u8.dtype == torch.uint8,
           "data_u8 must be contiguous HIP uint8")
    out = torch.empty(16, dtype=torch.uint8, device=data_u8.device)
    with torch.cuda.device(data_u8.device):
        rc = N.lib().ztcp_siphash128(data_u8.data_ptr() if data_u8.numel() else None,
                                     data_u8.numel(), mk0 & ((1 << 64) - 1), mk1 & ((1 << 64) - 1),
                                     out.data_ptr(), _stream())
    _raise_rc(rc)
    return out


def device_diag() -> int:
    """Sticky device diagnostics (0 = none); synchronizes the device."""
    return N.lib().ztcp_device_diag()


def debug_spin_limit(n: int) -> int:
    """Test hook: polls before a fused kernel's bounded wait gives up, for later
    calls (n < 0 restores the default); returns the previous value."""
    return N.lib().ztcp_debug_spin_limit(n)
