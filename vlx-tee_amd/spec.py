"""Wire-format constants and payload sizing of a cold page.

Mirror of research/baseline_codec/cold_page_spec.py (spec:47-67, spec:83-161,
spec:164-253): the 32-byte little-endian header, the AAD record bound to it,
presets, RoPE modes and the payload size (padded to 4 bytes) the reference's
Python wrapper passes as ``expected_payload_bytes``.
"""
from __future__ import annotations

import enum
import struct
from dataclasses import dataclass

MAGIC_ZTCP = 0x5A54
CODEC_VERSION = 1
HEADER_BYTES = 32
TAG_BYTES = 16
HEADER_STRUCT = struct.Struct("<HBBIIHHQQ")


class QuantPreset(enum.IntEnum):
    INT4_SYM = 1
    K8V4_ASYM = 2
    FP8_ONLY = 3
    # extensions (no counterpart in the reference; include/ztcp.h)
    K8V4_ASYM_G64 = 4   # K int8 asymmetric per 64 (scale + zero point), V int4 per 32
    FP8_E4M3 = 5        # K and V OCP e4m3 per 16
    INT4_SYM_G32 = 6    # K and V int4 per 32


class RoPEMode(enum.IntEnum):
    QUANTIZE_ALL = 0
    PRESERVE_FP8 = 1
    PRESERVE_RAW = 2
    PRESERVE_E4M3 = 3   # extension: RoPE columns as e4m3 per 16


def pack_header(preset: int, rope_mode: int, tenant_id_hash: int, model_id_hash: int,
                layer_id: int, head_group_id: int, page_token_hash: int,
                sequence_nonce: int) -> bytes:
    flags = (int(preset) & 0x0F) | ((int(rope_mode) & 0x0F) << 4)
    return HEADER_STRUCT.pack(MAGIC_ZTCP, CODEC_VERSION, flags, tenant_id_hash & 0xFFFFFFFF,
                              model_id_hash & 0xFFFFFFFF, layer_id & 0xFFFF,
                              head_group_id & 0xFFFF, page_token_hash & (2**64 - 1),
                              sequence_nonce & (2**64 - 1))


def unpack_header(b: bytes) -> dict:
    magic, version, flags, tenant, model, layer, hg, tok, seq = HEADER_STRUCT.unpack(b[:HEADER_BYTES])
    return dict(magic=magic, version=version, preset=flags & 0x0F, rope_mode=flags >> 4,
                tenant_id_hash=tenant, model_id_hash=model, layer_id=layer, head_group_id=hg,
                page_token_hash=tok, sequence_nonce=seq)


@dataclass(frozen=True)
class ColdPageAAD:
    """Associated data bound to a cold page's tag: the header fields (spec:83-161).

    ``unpack_header`` raises ``ValueError`` on a wrong magic or version and on
    preset / RoPE-mode nibbles outside the enums, as the reference's does."""

    tenant_id_hash: int
    model_id_hash: int
    layer_id: int
    page_token_hash: int
    sequence_nonce: int
    preset: QuantPreset = QuantPreset.K8V4_ASYM
    rope_mode: RoPEMode = RoPEMode.PRESERVE_FP8
    head_group_id: int = 0

    @classmethod
    def from_context(cls, tenant_id: str, model_id: str, layer_id: int, token_ids,
                     sequence_nonce: int, preset: QuantPreset = QuantPreset.K8V4_ASYM,
                     rope_mode: RoPEMode = RoPEMode.PRESERVE_FP8) -> "ColdPageAAD":
        return cls(tenant_id_hash=hash32(tenant_id), model_id_hash=hash32(model_id),
                   layer_id=layer_id, page_token_hash=hash64_tokens(token_ids),
                   sequence_nonce=sequence_nonce, preset=preset, rope_mode=rope_mode)

    def pack_header(self) -> bytes:
        return pack_header(self.preset, self.rope_mode, self.tenant_id_hash, self.model_id_hash,
                           self.layer_id, self.head_group_id, self.page_token_hash,
                           self.sequence_nonce)

    @classmethod
    def unpack_header(cls, header_bytes: bytes) -> "ColdPageAAD":
        if len(header_bytes) < HEADER_BYTES:
            raise ValueError(f"Header too short: {len(header_bytes)} < {HEADER_BYTES}")
        h = unpack_header(header_bytes)
        if h["magic"] != MAGIC_ZTCP or h["version"] != CODEC_VERSION:
            raise ValueError(f"Invalid cold-page header magic/version: {hex(h['magic'])} v{h['version']}")
        return cls(tenant_id_hash=h["tenant_id_hash"], model_id_hash=h["model_id_hash"],
                   layer_id=h["layer_id"], page_token_hash=h["page_token_hash"],
                   sequence_nonce=h["sequence_nonce"], preset=QuantPreset(h["preset"]),
                   rope_mode=RoPEMode(h["rope_mode"] & 0x0F), head_group_id=h["head_group_id"])


# Section kind of the K columns after the RoPE ones, and of V, per preset.
_KMAIN = {1: "int4", 2: "int8", 3: "int8", 4: "asym8_g64", 5: "e4m3", 6: "int4_g32"}
_VKIND = {1: "int4", 2: "int4", 3: "int8", 4: "int4_g32", 5: "e4m3", 6: "int4_g32"}
# kind -> (elements per group, code bytes per group, parameter bytes per group)
_EXT_GROUP = {"e4m3": (16, 16, 2), "int4_g32": (32, 16, 2), "asym8_g64": (64, 64, 4)}


def _section_bytes(kind: str, vecs: int, width: int) -> int:
    if kind == "raw":
        return vecs * width * 2
    if kind == "int8":  # the reference's per-column formula (cpp:1450-1472)
        return vecs * width + vecs * (width // 16) * 2
    if kind == "int4":
        return vecs * (width // 2) + vecs * (width // 16) * 2
    ges, cb, pb = _EXT_GROUP[kind]
    if width % ges:
        raise ValueError(f"{kind} needs section widths divisible by {ges}")
    return vecs * (width // ges) * (cb + pb)


@dataclass(frozen=True)
class ColdPageGeometry:
    num_tokens: int = 64
    num_kv_heads: int = 8
    head_dim: int = 128
    rope_dim: int = 64
    group_size: int = 16
    hot_element_bytes: int = 2
    is_mla_single_buffer: bool = False

    def __post_init__(self) -> None:
        if self.group_size != 16:
            raise ValueError("the wire format fixes group_size = 16 (cpp:1126)")
        if self.head_dim % 16 or self.head_dim < 16:
            raise ValueError("head_dim must be a positive multiple of 16")
        if self.rope_dim < 0 or self.rope_dim > self.head_dim or self.rope_dim % 16:
            raise ValueError("Invalid rope_dim")

    @property
    def nope_dim(self) -> int:
        return self.head_dim - self.rope_dim

    @property
    def vectors_per_buffer(self) -> int:
        return self.num_tokens * self.num_kv_heads

    @property
    def hot_page_bytes(self) -> int:
        buffers = 1 if self.is_mla_single_buffer else 2
        return buffers * self.vectors_per_buffer * self.head_dim * self.hot_element_bytes

    def required_payload_bytes(self, preset: int, rope_mode: int) -> int:
        """Unpadded payload (cpp:1439-1474; presets 4..6 and RoPE mode 3 are
        this codec's extension kinds, sized from their group geometry)."""
        if preset not in (1, 2, 3, 4, 5, 6) or rope_mode not in (0, 1, 2, 3):
            raise ValueError("Invalid preset or rope_mode")
        vecs, D, R = self.vectors_per_buffer, self.head_dim, self.rope_dim
        req = 0
        if rope_mode != 0 and R > 0:
            req += _section_bytes({1: "int8", 2: "raw", 3: "e4m3"}[rope_mode], vecs, R)
        kq = D if rope_mode == 0 else D - R
        if kq > 0:
            req += _section_bytes(_KMAIN[preset], vecs, kq)
        if not self.is_mla_single_buffer:
            req += _section_bytes(_VKIND[preset], vecs, D)
        return req

    def payload_bytes(self, preset: int, rope_mode: int) -> int:
        """Payload padded to a 4-byte boundary (spec:244-246)."""
        r = self.required_payload_bytes(preset, rope_mode)
        return (r + 3) & ~3

    def cold_blob_bytes(self, preset: int, rope_mode: int) -> int:
        return HEADER_BYTES + self.payload_bytes(preset, rope_mode) + TAG_BYTES

    def compression_ratio(self, preset: int, rope_mode: int) -> float:
        return self.hot_page_bytes / self.cold_blob_bytes(preset, rope_mode)


def hash32(text: str) -> int:
    """32-bit domain identifier hash (spec:70-74): BLAKE2s-32, little-endian."""
    import hashlib

    return int.from_bytes(hashlib.blake2s(text.encode("utf-8"), digest_size=4).digest(), "little")


def hash64_tokens(token_ids) -> int:
    """64-bit token-id hash of a page (spec:77-80): BLAKE2s-64 over LE int32."""
    import hashlib

    buf = struct.pack(f"<{len(token_ids)}i", *token_ids)
    return int.from_bytes(hashlib.blake2s(buf, digest_size=8).digest(), "little")
