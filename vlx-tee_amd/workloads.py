"""Synthetic cold-page workloads (the benchmark configurations).

Each workload fixes a page geometry, a preset / RoPE mode, a value
distribution and the AAD / nonce assignment:
  * values are N(0, sigma) drawn from torch's seeded generator (seed 42) on
    the requested device, cast to the hot dtype;
  * RoPE columns are the leading ``rope_dim`` columns of K (the reference's
    order, cpp:1379-1388);
  * keys come from a seeded stream (seed 7): bytes 0..31 encryption key,
    32..47 MAC key, read as little-endian u64 words (native_fused_codec.py:173-174);
  * page i has token hash i, sequence nonce i and layer i // pages_per_layer;
  * tenant / model hashes are the reference's BLAKE2s-32 of fixed ids.
"""
from __future__ import annotations

import math
import struct
from dataclasses import dataclass

import numpy as np
import torch

from .spec import ColdPageGeometry, hash32


@dataclass(frozen=True)
class Workload:
    name: str
    n_pages: int
    num_tokens: int
    num_heads: int
    head_dim: int
    rope_dim: int
    mla: bool
    preset: int
    rope_mode: int
    pages_per_layer: int
    sigma: float = 1.0            # N(0, sigma) for K (GQA) / latent columns (MLA)
    rope_sigma: float = 1.0       # MLA RoPE columns
    rope_scale: float = 8.0       # GQA: K RoPE columns scaled by this
    outlier_frac: float = 0.0     # fraction of channels scaled by outlier_scale
    outlier_scale: float = 1.0
    tamper_frac: float = 0.0      # ingress stress: pages with one flipped bit

    @property
    def geometry(self) -> ColdPageGeometry:
        return ColdPageGeometry(self.num_tokens, self.num_heads, self.head_dim, self.rope_dim,
                                16, 2, self.mla)

    @property
    def hot_bytes_per_page(self) -> int:
        return self.geometry.hot_page_bytes

    @property
    def blob_bytes(self) -> int:
        return self.geometry.cold_blob_bytes(self.preset, self.rope_mode)

    @property
    def payload_bytes(self) -> int:
        return self.geometry.payload_bytes(self.preset, self.rope_mode)

    @property
    def extension(self) -> bool:
        """Uses the extension presets / RoPE mode (ingress needs ZTCP_EXT_LAYOUTS)."""
        return self.preset > 3 or self.rope_mode > 2


TENANT = "tenant-alpha-bank"
MODEL = "Qwen/Qwen3.6-35B-A3B"
TENANT_HASH = hash32(TENANT)
MODEL_HASH = hash32(MODEL)

WORKLOADS = {
    # 64 GQA pages, INT4_SYM + PRESERVE_FP8, RoPE x8 plus 1% of channels x20
    "c0_int4_gqa64": Workload("c0_int4_gqa64", 64, 16, 4, 128, 64, False, 1, 1, 64,
                              outlier_frac=0.01, outlier_scale=20.0),
    # the same distribution, 256 pages
    "c1_int4_gqa256": Workload("c1_int4_gqa256", 256, 16, 4, 128, 64, False, 1, 1, 256,
                               outlier_frac=0.01, outlier_scale=20.0),
    # 1 GiB BF16 prefix: 4096 tokens x 64 layers, 16-token pages of 8 KV heads
    "c2_k8v4_prefix1g": Workload("c2_k8v4_prefix1g", 16384, 16, 8, 128, 64, False, 2, 1, 256),
    "c2_int4_prefix1g": Workload("c2_int4_prefix1g", 16384, 16, 8, 128, 64, False, 1, 1, 256),
    # the same prefix, INT8 everywhere (the reference's FP8_ONLY), 1% pages tampered
    "c3_fp8only_tamper": Workload("c3_fp8only_tamper", 16384, 16, 8, 128, 64, False, 3, 0, 256,
                                  tamper_frac=0.01),
    # DeepSeek-MLA single buffer: 576 = 64 RoPE + 512 latent per token, 64-token pages
    "c4_mla_int4": Workload("c4_mla_int4", 16384, 64, 1, 576, 64, True, 1, 1, 256, sigma=0.5,
                            rope_sigma=1.0, rope_scale=1.0, outlier_frac=0.02,
                            outlier_scale=16.0),
    # The same three prefixes with the extension kinds, as the workloads are
    # specified: K int8 asymmetric per 64 with the RoPE columns in e4m3 and V
    # int4 per 32 (preset 4 + RoPE mode 3); FP8 e4m3 everywhere with 1% of the
    # pages tampered (preset 5); MLA latent int4 per 32 with e4m3 RoPE (preset
    # 6 + RoPE mode 3).
    "c2_k8v4asym_prefix1g": Workload("c2_k8v4asym_prefix1g", 16384, 16, 8, 128, 64, False, 4, 3, 256),
    "c3_e4m3_tamper": Workload("c3_e4m3_tamper", 16384, 16, 8, 128, 64, False, 5, 0, 256,
                               tamper_frac=0.01),
    "c4_mla_int4g32": Workload("c4_mla_int4g32", 16384, 64, 1, 576, 64, True, 6, 3, 256, sigma=0.5,
                               rope_sigma=1.0, rope_scale=1.0, outlier_frac=0.02,
                               outlier_scale=16.0),
}


def session_keys(seed: int = 7) -> dict:
    """k0..k3 (encryption) and mk0, mk1 (MAC) from a seeded byte stream."""
    raw = np.random.default_rng(seed).integers(0, 256, size=48, dtype=np.uint8).tobytes()
    k0, k1, k2, k3 = struct.unpack("<4Q", raw[:32])
    mk0, mk1 = struct.unpack("<2Q", raw[32:48])
    return dict(k0=k0, k1=k1, k2=k2, k3=k3, mk0=mk0, mk1=mk1)


def page_metadata(w: Workload, first_page: int = 0, n: int | None = None):
    """(token_hashes, sequence_nonces, layer_ids) for pages [first, first + n)."""
    n = w.n_pages if n is None else n
    idx = np.arange(first_page, first_page + n, dtype=np.int64)
    return idx.copy(), idx.astype(np.uint64), (idx // w.pages_per_layer).astype(np.uint16)


def _outlier_channels(gen: torch.Generator, frac: float, ncols: int, device) -> torch.Tensor:
    n = max(1, math.ceil(frac * ncols))
    return torch.randperm(ncols, generator=gen, device=device)[:n]


def generate(w: Workload, device: str | torch.device = "cpu", dtype: torch.dtype = torch.bfloat16,
             seed: int = 42, n_pages: int | None = None):
    """Hot K (and V) pages [n, T, H, D] of `dtype` on `device`."""
    n = w.n_pages if n_pages is None else n_pages
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    shape = (n, w.num_tokens, w.num_heads, w.head_dim)
    R = w.rope_dim
    chunk = max(1, (1 << 26) // (w.num_tokens * w.num_heads * w.head_dim))
    k = torch.empty(shape, dtype=dtype, device=device)
    v = None if w.mla else torch.empty(shape, dtype=dtype, device=device)
    if w.mla:
        ch = _outlier_channels(gen, w.outlier_frac, R, device) if w.outlier_frac and R else None
    else:
        kch = _outlier_channels(gen, w.outlier_frac, w.head_dim, device) if w.outlier_frac else None
        vch = _outlier_channels(gen, w.outlier_frac, w.head_dim, device) if w.outlier_frac else None
    for s in range(0, n, chunk):
        m = min(chunk, n - s)
        x = torch.randn((m,) + shape[1:], generator=gen, device=device, dtype=torch.float32)
        if w.mla:
            x[..., R:] *= w.sigma
            x[..., :R] *= w.rope_sigma
            if ch is not None:
                x[..., ch] *= w.outlier_scale
        else:
            x *= w.sigma
            x[..., :R] *= w.rope_scale
            if kch is not None:
                x[..., kch] *= w.outlier_scale
        k[s:s + m] = x.to(dtype)
        if v is not None:
            y = torch.randn((m,) + shape[1:], generator=gen, device=device, dtype=torch.float32)
            if vch is not None:
                y[..., vch] *= w.outlier_scale
            v[s:s + m] = y.to(dtype)
    return k, v


def tamper_plan(w: Workload, blob_bytes: int, seed: int = 1234):
    """Pages to tamper and, for each, one bit of its header or payload to flip."""
    rng = np.random.default_rng(seed)
    n_t = max(1, int(round(w.tamper_frac * w.n_pages))) if w.tamper_frac else 0
    pages = np.sort(rng.choice(w.n_pages, size=n_t, replace=False)) if n_t else np.zeros(0, np.int64)
    bits = rng.integers(0, (blob_bytes - 16) * 8, size=n_t)  # header + payload bits
    return pages.astype(np.int64), bits.astype(np.int64)
