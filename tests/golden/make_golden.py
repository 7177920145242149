"""Write tests/golden/reference_vectors.json from the reference's own codec.

Runs the reference's C++ codec as compiled by oracle/build.py (oracle/_ref,
built from /root/reference/research/baseline_codec/csrc/fused_cold_page_cpu.cpp)
on seeded FP16 inputs and records, per case, the SHA-256 of the blob batch and
of the decoded K / V, plus the full blob bytes of the smallest case.  Inputs
are regenerated from the recorded seed by `case_inputs`, so the fixture is
data only.  Run in the build container: python tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REPO = HERE.parent.parent
sys.path.insert(0, str(REPO))

KEYS = dict(k0=0x243F6A8885A308D3, k1=0x13198A2E03707344, mk0=0xA4093822299F31D0,
            mk1=0x082EFA98EC4E6C89, k2=0x452821E638D01377, k3=0xBE5466CF34E90C6C)
AAD = dict(tenant=0x9E3779B9, model=0x7F4A7C15, layer=21, head_group=2, base_seq=5000)

CASES = [  # name, tokens, heads, head_dim, rope_dim, mla, pages, seed
    ("tiny", 2, 1, 32, 16, False, 2, 101),
    ("c0_shape", 16, 4, 128, 64, False, 2, 42),
    ("odd_vecs", 3, 3, 48, 16, False, 3, 7),
    ("mla_shape", 64, 1, 576, 64, True, 1, 43),
]


def case_inputs(tokens, heads, head_dim, rope_dim, mla, pages, seed):
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((pages, tokens, heads, head_dim)).astype(np.float32)
    k[..., :rope_dim] *= 8
    k[:, 0, 0, :16] = 0  # an all-zero group
    k = k.astype(np.float16)
    v = None if mla else (rng.standard_normal((pages, tokens, heads, head_dim)) * 0.5).astype(np.float16)
    th = (np.arange(pages, dtype=np.int64) * 0x9E3779B97F4A7C1) & 0x7FFFFFFFFFFFFFFF
    return k, v, th


def main():
    import torch
    from oracle import oracle as O

    ref = O.ref_module()
    assert ref is not None, "compiled reference missing: python oracle/build.py ref"
    out = {"keys": {k: hex(v) for k, v in KEYS.items()}, "aad": AAD, "cases": []}
    for name, T, H, D, R, mla, B, seed in CASES:
        k, v, th = case_inputs(T, H, D, R, mla, B, seed)
        for preset in (1, 2, 3):
            for rm in (0, 1, 2):
                exp = O.payload_bytes(preset, rm, T * H, D, R, not mla)
                blobs = torch.empty((B, 48 + exp), dtype=torch.uint8)
                ref.fused_encode_cold_pages_peak_into_cpu(
                    torch.from_numpy(k), None if v is None else torch.from_numpy(v),
                    torch.from_numpy(th), blobs, preset, rm, R, exp, AAD["tenant"], AAD["model"],
                    AAD["layer"], AAD["head_group"], AAD["base_seq"], KEYS["k0"], KEYS["k1"],
                    KEYS["mk0"], KEYS["mk1"], KEYS["k2"], KEYS["k3"])
                ko = torch.empty((B, T, H, D), dtype=torch.float16)
                vo = None if mla else torch.empty_like(ko)
                ref.fused_decode_cold_pages_peak_into_cpu(
                    blobs, torch.from_numpy(th), ko, vo, R, mla, AAD["tenant"], AAD["model"],
                    AAD["layer"], KEYS["k0"], KEYS["k1"], KEYS["mk0"], KEYS["mk1"], KEYS["k2"],
                    KEYS["k3"])
                entry = dict(name=name, tokens=T, heads=H, head_dim=D, rope_dim=R, mla=mla,
                             pages=B, seed=seed, preset=preset, rope_mode=rm, payload=exp,
                             blobs_sha256=hashlib.sha256(blobs.numpy().tobytes()).hexdigest(),
                             k_sha256=hashlib.sha256(ko.numpy().tobytes()).hexdigest(),
                             v_sha256=None if mla else hashlib.sha256(vo.numpy().tobytes()).hexdigest())
                if name == "tiny":
                    entry["blobs_hex"] = blobs.numpy().tobytes().hex()
                out["cases"].append(entry)
    (HERE / "reference_vectors.json").write_text(json.dumps(out, indent=1) + "\n")
    print(f"wrote {len(out['cases'])} cases")


if __name__ == "__main__":
    main()
