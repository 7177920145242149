"""Session-bound cold-page codec on the HIP path: drop-in for the reference's
``NativeCppFusedColdPageCodec`` (research/baseline_codec/native_fused_codec.py,
"nfc", lines 68-606).

Every method runs the reference's transaction around the fused kernels, in
the reference's order:

  egress   preflight_validate_egress (nonces burned) -> begin_egress_execution
           -> argument checks -> fused egress kernel -> commit_egress; any
           failure after the preflight zeroes the output blobs; the
           reservation is always released;
  ingress  begin_ingress -> argument checks -> fused ingress kernel (tag and
           AAD verified on the device; failures mapped to the reference's
           exception classes) -> freshness check of the decoded headers ->
           finish_ingress; any failure after the checks zeroes the outputs.

Method names, parameter names and order, return values and exceptions are the
reference's, so callers switch by import.  The parameter names keep the
reference's ``_cpu`` suffixes; the tensors are HIP tensors resident in HBM
(pages ``float16`` or ``bfloat16``, blobs ``uint8``), which is the point.  Token
hash tensors may live on the host (as the reference requires) or the device.
Allocating decodes return ``float16`` pages as the reference's do, unless the
codec was built with ``dtype=torch.bfloat16``.
"""
from __future__ import annotations

import struct

import numpy as np
import torch

from . import native_hip_codec as H
from .keyring import (  # noqa: F401  (re-exported: the reference imports them from here)
    CrossTenantContaminationError,
    EphemeralSessionKeyRing,
    KVIntegrityError,
    NonceReuseError,
    SessionShreddedError,
    StalePageReplayError,
)
from .spec import HEADER_BYTES, ColdPageAAD, ColdPageGeometry, hash32


def _map_integrity(exc: RuntimeError) -> Exception:
    """The reference's message-to-class mapping (nfc:253-259)."""
    msg = str(exc)
    if "CROSS_TENANT_CONTAMINATION" in msg:
        return CrossTenantContaminationError(msg)
    if "KV_INTEGRITY_ERROR" in msg:
        return KVIntegrityError(msg)
    return exc


def _keys(enc_key: bytes, mac_key: bytes) -> dict:
    k0, k1, k2, k3 = struct.unpack("<QQQQ", enc_key[:32])
    mk0, mk1 = struct.unpack("<QQ", mac_key[:16])
    return dict(k0=k0, k1=k1, k2=k2, k3=k3, mk0=mk0, mk1=mk1)


def _header_records(blobs: torch.Tensor) -> np.ndarray:
    """Bytes 8..32 of every header (model, layer, head group, token hash,
    sequence nonce): the key ring's freshness record layout."""
    return blobs[:, 8:HEADER_BYTES].contiguous().cpu().numpy()


class NativeHipFusedColdPageCodec:
    """Fused quantizer + ChaCha20 + SipHash-2-4-128 on the GPU, bound to a
    session key ring (nfc:68-78)."""

    def __init__(self, geometry: ColdPageGeometry, keyring: EphemeralSessionKeyRing,
                 dtype: torch.dtype = torch.float16, accept_extension_layouts: bool = False) -> None:
        """``accept_extension_layouts``: encode with, and decode pages whose
        headers carry, this codec's extension presets / RoPE mode (QuantPreset
        4..6, RoPEMode.PRESERVE_E4M3); by default egress rejects them as
        invalid arguments and ingress fails them at the flags check, as the
        reference does (cpp:1947-1948; KVIntegrityError)."""
        if dtype not in (torch.float16, torch.bfloat16):
            raise ValueError("dtype must be torch.float16 or torch.bfloat16")
        self.geometry = geometry
        self.keyring = keyring
        self.dtype = dtype
        self.accept_extension_layouts = bool(accept_extension_layouts)
        from . import _native

        self._ext = _native.lib()  # fails loudly when the HIP library is missing

    # ---- argument checks (nfc:80-146) ---------------------------------------------------

    def _validate_single_shapes(self, k_page_cpu: torch.Tensor, v_page_cpu: torch.Tensor | None) -> None:
        exp = (self.geometry.num_tokens, self.geometry.num_kv_heads, self.geometry.head_dim)
        if tuple(k_page_cpu.shape) != exp:
            raise RuntimeError(f"k_page_cpu shape {tuple(k_page_cpu.shape)} does not match geometry {exp}")
        if not self.geometry.is_mla_single_buffer:
            if v_page_cpu is None or tuple(v_page_cpu.shape) != exp:
                raise RuntimeError(
                    f"v_page_cpu shape {None if v_page_cpu is None else tuple(v_page_cpu.shape)} "
                    f"does not match geometry {exp}")

    @staticmethod
    def _validate_token_hashes_tensor(page_token_hashes_i64: torch.Tensor) -> int:
        """Checks as the reference's (nfc:99-115), the device may also be HIP;
        returns the batch size."""
        if not isinstance(page_token_hashes_i64, torch.Tensor):
            raise RuntimeError("page_token_hashes_i64 must be a torch.Tensor")
        t = page_token_hashes_i64
        if (t.device.type not in ("cpu", "cuda") or not t.is_contiguous() or t.dtype != torch.int64
                or t.dim() != 1 or t.numel() < 1):
            raise RuntimeError(
                "page_token_hashes_i64 must be a non-empty 1D contiguous int64 tensor, got "
                f"shape={tuple(t.shape)} dtype={t.dtype} device={t.device}")
        return int(t.numel())

    @staticmethod
    def _tensors_overlap(a: torch.Tensor | None, b: torch.Tensor | None) -> bool:
        if a is None or b is None or a.numel() == 0 or b.numel() == 0:
            return False
        if a.device != b.device:
            return False
        a0, b0 = a.data_ptr(), b.data_ptr()
        a1, b1 = a0 + a.numel() * a.element_size(), b0 + b.numel() * b.element_size()
        return a0 < b1 and b0 < a1

    def _validate_batch_shapes(self, k_pages_cpu: torch.Tensor, v_pages_cpu: torch.Tensor | None,
                               n_pages: int) -> None:
        exp = (n_pages, self.geometry.num_tokens, self.geometry.num_kv_heads, self.geometry.head_dim)
        if tuple(k_pages_cpu.shape) != exp:
            raise RuntimeError(
                f"k_pages_cpu shape {tuple(k_pages_cpu.shape)} does not match batch geometry {exp}")
        if not self.geometry.is_mla_single_buffer:
            if v_pages_cpu is None or tuple(v_pages_cpu.shape) != exp:
                raise RuntimeError(
                    f"v_pages_cpu shape {None if v_pages_cpu is None else tuple(v_pages_cpu.shape)} "
                    f"does not match batch geometry {exp}")

    # ---- single page (nfc:148-282) ---------------------------------------------------------

    def encode_cold_page_tensor(self, k_page_cpu: torch.Tensor, v_page_cpu: torch.Tensor | None,
                                tenant_id: str, session_id: str, aad: ColdPageAAD) -> torch.Tensor:
        """One page -> contiguous 1D uint8 blob on the page's device (nfc:148-214)."""
        staged, slots, last_seq = self.keyring.preflight_validate_egress(
            tenant_id=tenant_id, session_id=session_id, model_id_hash=aad.model_id_hash,
            layer_id=aad.layer_id, head_group_id=aad.head_group_id,
            base_sequence_nonce=aad.sequence_nonce, token_hashes=[aad.page_token_hash])
        try:
            enc_key, mac_key = self.keyring.begin_egress_execution(
                tenant_id=tenant_id, session_id=session_id, staged_nonces=staged)
            self._validate_single_shapes(k_page_cpu, v_page_cpu)
            expected_payload = self.geometry.payload_bytes(aad.preset, aad.rope_mode)
            blob = H.fused_encode_cold_page(
                k_page_cpu, v_page_cpu, int(aad.preset), int(aad.rope_mode), self.geometry.rope_dim,
                expected_payload, aad.tenant_id_hash, aad.model_id_hash, aad.layer_id,
                aad.head_group_id, aad.page_token_hash & 0xFFFFFFFFFFFFFFFF,
                aad.sequence_nonce & 0xFFFFFFFFFFFFFFFF, **_keys(enc_key, mac_key))
            try:
                self.keyring.commit_egress(tenant_id=tenant_id, session_id=session_id,
                                           staged_nonces=staged, staged_slots=slots, last_seq=last_seq)
            except BaseException:
                blob.zero_()
                raise
            return blob
        finally:
            self.keyring.release_egress_reservation(tenant_id=tenant_id, session_id=session_id,
                                                    staged_nonces=staged)

    def decode_cold_page_tensor(self, cold_blob_u8: torch.Tensor, expected_tenant_id: str, session_id: str,
                                expected_model_id: str, expected_layer_id: int, expected_token_hash: int,
                                min_sequence_nonce: int | None = None,
                                expected_sequence_nonce: int | None = None
                                ) -> tuple[torch.Tensor, torch.Tensor | None]:
        """Verify AAD + tag + freshness, decrypt and dequantize one page (nfc:216-282)."""
        gen, enc_key, mac_key = self.keyring.begin_ingress(expected_tenant_id, session_id)
        g = self.geometry
        try:
            k_out, v_out = H.fused_decode_cold_page(
                cold_blob_u8, g.num_tokens, g.num_kv_heads, g.head_dim, g.rope_dim,
                g.is_mla_single_buffer, hash32(expected_tenant_id), hash32(expected_model_id),
                expected_layer_id, expected_token_hash & 0xFFFFFFFFFFFFFFFF,
                **_keys(enc_key, mac_key), dtype=self.dtype, ext_layouts=self.accept_extension_layouts)
        except RuntimeError as exc:
            mapped = _map_integrity(exc)
            if mapped is exc:
                raise
            raise mapped from exc
        aad = ColdPageAAD.unpack_header(cold_blob_u8[:HEADER_BYTES].cpu().numpy().tobytes())
        try:
            self.keyring.verify_and_update_freshness(
                tenant_id=expected_tenant_id, session_id=session_id, model_id_hash=aad.model_id_hash,
                layer_id=aad.layer_id, head_group_id=aad.head_group_id,
                page_token_hash=aad.page_token_hash, sequence_nonce=aad.sequence_nonce,
                min_sequence_nonce=min_sequence_nonce, expected_sequence_nonce=expected_sequence_nonce,
                expected_generation=gen)
            self.keyring.finish_ingress(expected_tenant_id, session_id, gen)
        except BaseException:
            k_out.zero_()
            if v_out is not None:
                v_out.zero_()
            raise
        return k_out, v_out

    # ---- batches (nfc:284-606) --------------------------------------------------------------

    def _decode_into(self, cold_blobs_u8, expected_token_hashes_i64, out_k, out_v, expected_tenant_id,
                     session_id, expected_model_id, expected_layer_id, min_sequence_nonce, gen, keys):
        try:
            try:
                H.fused_decode_cold_pages_peak_into(
                    cold_blobs_u8, expected_token_hashes_i64, out_k, out_v, self.geometry.rope_dim,
                    self.geometry.is_mla_single_buffer, hash32(expected_tenant_id),
                    hash32(expected_model_id), expected_layer_id, **keys,
                    ext_layouts=self.accept_extension_layouts)
            except RuntimeError as exc:
                mapped = _map_integrity(exc)
                if mapped is exc:
                    raise
                raise mapped from exc
            self.keyring.verify_and_update_freshness_batch(
                tenant_id=expected_tenant_id, session_id=session_id,
                records=_header_records(cold_blobs_u8), min_sequence_nonce=min_sequence_nonce,
                expected_generation=gen)
            self.keyring.finish_ingress(expected_tenant_id, session_id, gen)
        except BaseException:
            if isinstance(out_k, torch.Tensor):
                out_k.zero_()
            if isinstance(out_v, torch.Tensor):
                out_v.zero_()
            raise

    def decode_cold_pages_batch_tensor(self, cold_blobs_u8: torch.Tensor,
                                       expected_token_hashes_i64: torch.Tensor, expected_tenant_id: str,
                                       session_id: str, expected_model_id: str, expected_layer_id: int,
                                       min_sequence_nonce: int | None = None
                                       ) -> tuple[torch.Tensor, torch.Tensor | None]:
        """[B, blob_bytes] -> ([B, T, H, D], [B, T, H, D] | None) (nfc:284-357)."""
        gen, enc_key, mac_key = self.keyring.begin_ingress(expected_tenant_id, session_id)
        n_b = self._validate_token_hashes_tensor(expected_token_hashes_i64)
        if cold_blobs_u8.dim() != 2 or cold_blobs_u8.size(0) != n_b:
            raise RuntimeError(
                "cold_blobs_u8 must be 2D [batch, blob_bytes] matching expected_token_hashes_i64 "
                f"length {n_b}, got shape={tuple(cold_blobs_u8.shape)}")
        g = self.geometry
        shape = (n_b, g.num_tokens, g.num_kv_heads, g.head_dim)
        k_out = torch.empty(shape, dtype=self.dtype, device=cold_blobs_u8.device)
        v_out = None if g.is_mla_single_buffer else torch.empty(shape, dtype=self.dtype,
                                                                 device=cold_blobs_u8.device)
        self._decode_into(cold_blobs_u8, expected_token_hashes_i64, k_out, v_out, expected_tenant_id,
                          session_id, expected_model_id, expected_layer_id, min_sequence_nonce, gen,
                          _keys(enc_key, mac_key))
        return k_out, v_out

    def decode_cold_pages_peak_into(self, cold_blobs_u8: torch.Tensor, expected_token_hashes_i64: torch.Tensor,
                                    out_k_pages_cpu: torch.Tensor, out_v_pages_cpu: torch.Tensor | None,
                                    expected_tenant_id: str, session_id: str, expected_model_id: str,
                                    expected_layer_id: int, min_sequence_nonce: int | None = None) -> None:
        """Batch ingress into preallocated pages, no allocation (nfc:359-444)."""
        gen, enc_key, mac_key = self.keyring.begin_ingress(expected_tenant_id, session_id)
        n_b = self._validate_token_hashes_tensor(expected_token_hashes_i64)
        if cold_blobs_u8.dim() != 2 or int(cold_blobs_u8.size(0)) != n_b:
            raise RuntimeError(f"cold_blobs_u8 must be 2D [batch, blob_bytes] with batch={n_b}, "
                               f"got shape={tuple(cold_blobs_u8.shape)}")
        self._validate_batch_shapes(out_k_pages_cpu, out_v_pages_cpu, n_b)
        if (self._tensors_overlap(out_k_pages_cpu, out_v_pages_cpu)
                or self._tensors_overlap(out_k_pages_cpu, cold_blobs_u8)
                or self._tensors_overlap(out_k_pages_cpu, expected_token_hashes_i64)
                or self._tensors_overlap(out_v_pages_cpu, cold_blobs_u8)
                or self._tensors_overlap(out_v_pages_cpu, expected_token_hashes_i64)):
            raise RuntimeError("Peak ingress output tensors must not alias or overlap each other or input tensors")
        self._decode_into(cold_blobs_u8, expected_token_hashes_i64, out_k_pages_cpu, out_v_pages_cpu,
                          expected_tenant_id, session_id, expected_model_id, expected_layer_id,
                          min_sequence_nonce, gen, _keys(enc_key, mac_key))

    def _preflight_batch(self, page_token_hashes_i64, tenant_id, session_id, aad_template):
        if not isinstance(page_token_hashes_i64, torch.Tensor) or page_token_hashes_i64.numel() < 1:
            raise RuntimeError("page_token_hashes_i64 must be a non-empty torch.Tensor")
        return self.keyring.preflight_validate_egress(
            tenant_id=tenant_id, session_id=session_id, model_id_hash=aad_template.model_id_hash,
            layer_id=aad_template.layer_id, head_group_id=aad_template.head_group_id,
            base_sequence_nonce=aad_template.sequence_nonce, token_hashes=page_token_hashes_i64)

    def _encode_into(self, k_pages_cpu, v_pages_cpu, page_token_hashes_i64, out_blobs_u8, tenant_id,
                     session_id, aad_template, staged) -> None:
        enc_key, mac_key = self.keyring.begin_egress_execution(
            tenant_id=tenant_id, session_id=session_id, staged_nonces=staged)
        n_b = self._validate_token_hashes_tensor(page_token_hashes_i64)
        self._validate_batch_shapes(k_pages_cpu, v_pages_cpu, n_b)
        expected_payload = self.geometry.payload_bytes(aad_template.preset, aad_template.rope_mode)
        H.fused_encode_cold_pages_peak_into(
            k_pages_cpu, v_pages_cpu, page_token_hashes_i64, out_blobs_u8, int(aad_template.preset),
            int(aad_template.rope_mode), self.geometry.rope_dim, expected_payload,
            aad_template.tenant_id_hash, aad_template.model_id_hash, aad_template.layer_id,
            aad_template.head_group_id, aad_template.sequence_nonce & 0xFFFFFFFFFFFFFFFF,
            **_keys(enc_key, mac_key), ext_layouts=self.accept_extension_layouts)

    def encode_cold_pages_batch_tensor(self, k_pages_cpu: torch.Tensor, v_pages_cpu: torch.Tensor | None,
                                       page_token_hashes_i64: torch.Tensor, tenant_id: str, session_id: str,
                                       aad_template: ColdPageAAD) -> torch.Tensor:
        """[B, T, H, D] pages -> [B, blob_bytes] blobs (nfc:446-520); page b
        carries sequence nonce ``aad_template.sequence_nonce + b``."""
        staged, slots, last_seq = self._preflight_batch(page_token_hashes_i64, tenant_id, session_id,
                                                        aad_template)
        try:
            blob_bytes = self.geometry.cold_blob_bytes(aad_template.preset, aad_template.rope_mode)
            out_blobs = torch.empty((int(page_token_hashes_i64.numel()), blob_bytes), dtype=torch.uint8,
                                    device=k_pages_cpu.device)
            self._encode_into(k_pages_cpu, v_pages_cpu, page_token_hashes_i64, out_blobs, tenant_id,
                              session_id, aad_template, staged)
            try:
                self.keyring.commit_egress(tenant_id=tenant_id, session_id=session_id,
                                           staged_nonces=staged, staged_slots=slots, last_seq=last_seq)
            except BaseException:
                out_blobs.zero_()
                raise
            return out_blobs
        finally:
            self.keyring.release_egress_reservation(tenant_id=tenant_id, session_id=session_id,
                                                    staged_nonces=staged)

    def encode_cold_pages_peak_into(self, k_pages_cpu: torch.Tensor, v_pages_cpu: torch.Tensor | None,
                                    page_token_hashes_i64: torch.Tensor, out_blobs_u8: torch.Tensor,
                                    tenant_id: str, session_id: str, aad_template: ColdPageAAD) -> None:
        """Batch egress into a preallocated (e.g. pre-registered RDMA) buffer (nfc:522-606)."""
        staged, slots, last_seq = self._preflight_batch(page_token_hashes_i64, tenant_id, session_id,
                                                        aad_template)
        try:
            if (self._tensors_overlap(out_blobs_u8, k_pages_cpu)
                    or self._tensors_overlap(out_blobs_u8, v_pages_cpu)
                    or self._tensors_overlap(out_blobs_u8, page_token_hashes_i64)):
                raise RuntimeError("out_blobs_u8 must not alias or overlap input tensors")
            try:
                self._encode_into(k_pages_cpu, v_pages_cpu, page_token_hashes_i64, out_blobs_u8,
                                  tenant_id, session_id, aad_template, staged)
                self.keyring.commit_egress(tenant_id=tenant_id, session_id=session_id,
                                           staged_nonces=staged, staged_slots=slots, last_seq=last_seq)
            except BaseException:
                if isinstance(out_blobs_u8, torch.Tensor):
                    out_blobs_u8.zero_()
                raise
        finally:
            self.keyring.release_egress_reservation(tenant_id=tenant_id, session_id=session_id,
                                                    staged_nonces=staged)


# The reference's class name, for callers that switch by import only.
NativeCppFusedColdPageCodec = NativeHipFusedColdPageCodec
