"""Quantizer pins.

* Every finite fp16 value is the amax of some group in a crafted FP16 page;
  the oracle's blob must equal the compiled reference's byte for byte (INT8
  and INT4 sections, all scales, all codes, and the decoded outputs).
* Closed forms: codes are clamp(round-half-even(v / s)), dequantized values
  are q * s rounded once; checked with numpy float32 arithmetic (an
  independent evaluation of the same IEEE operations) for BF16 groups, which
  the reference does not support.
"""
import numpy as np
import torch

KEYS = dict(k0=0x0123456789ABCDEF, k1=0xFEDCBA9876543210, mk0=0x1111222233334444,
            mk1=0x5555666677778888, k2=0xDEADBEEFCAFEF00D, k3=0x0BADC0DE12345678)


def _amax_page():
    """[1, 256, 16, 256] fp16 page whose 65536 groups have every finite fp16 amax."""
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    finite = h[np.isfinite(h.view(np.float16))]
    rng = np.random.default_rng(11)
    reps = np.resize(finite, 65536)
    amax = reps.view(np.float16).astype(np.float32)
    frac = rng.uniform(-1, 1, size=(65536, 16)).astype(np.float32)
    g = (frac * np.abs(amax)[:, None]).astype(np.float16)
    pos = rng.integers(0, 16, size=65536)
    g[np.arange(65536), pos] = reps.view(np.float16)
    # a few exact half-ulp ties and zero groups
    g[:64] = 0
    return g.reshape(1, 256, 16, 256)


def _enc_ref(ref, k, v, preset, rope_mode, rope_dim, exp):
    out = torch.empty((k.shape[0], 48 + exp), dtype=torch.uint8)
    ref.fused_encode_cold_pages_peak_into_cpu(
        torch.from_numpy(k), None if v is None else torch.from_numpy(v),
        torch.arange(k.shape[0], dtype=torch.int64), out, preset, rope_mode, rope_dim, exp,
        0xA1B2C3D4, 0x01020304, 3, 1, 99, KEYS["k0"], KEYS["k1"], KEYS["mk0"], KEYS["mk1"],
        KEYS["k2"], KEYS["k3"])
    return out.numpy()


def _enc_oracle(O, k, v, preset, rope_mode, rope_dim, exp):
    return O.egress_batch(k.view(np.uint16), None if v is None else v.view(np.uint16),
                          np.arange(k.shape[0], dtype=np.int64), dtype=O.FP16, preset=preset,
                          rope_mode=rope_mode, rope_dim=rope_dim, expected_payload_bytes=exp,
                          tenant_id_hash=0xA1B2C3D4, model_id_hash=0x01020304, layer_id=3,
                          head_group_id=1, base_sequence_nonce=99, **KEYS)


def test_every_fp16_amax_int8_int4_vs_reference(O, ref):
    k = _amax_page()
    v = np.ascontiguousarray(k[:, ::-1])
    for preset in (1, 3):  # INT4 K/V, INT8 K/V
        exp = O.payload_bytes(preset, 0, 256 * 16, 256, 0, True)
        a = _enc_ref(ref, k, v, preset, 0, 0, exp)
        b = _enc_oracle(O, k, v, preset, 0, 0, exp)
        assert np.array_equal(a, b), preset
        rc, st, kk, vv = O.ingress_batch(b, np.arange(1), num_tokens=256, num_heads=16,
                                         head_dim=256, rope_dim=0, is_mla_single_buffer=False,
                                         dtype=O.FP16, expected_tenant_hash=0xA1B2C3D4,
                                         expected_model_hash=0x01020304, expected_layer_id=3,
                                         **KEYS)
        assert rc == 0
        ko = torch.empty((1, 256, 16, 256), dtype=torch.float16)
        vo = torch.empty_like(ko)
        ref.fused_decode_cold_pages_peak_into_cpu(
            torch.from_numpy(a), torch.arange(1, dtype=torch.int64), ko, vo, 0, False, 0xA1B2C3D4,
            0x01020304, 3, KEYS["k0"], KEYS["k1"], KEYS["mk0"], KEYS["mk1"], KEYS["k2"], KEYS["k3"])
        assert np.array_equal(ko.numpy().view(np.uint16), kk)
        assert np.array_equal(vo.numpy().view(np.uint16), vv)


def _closed_form(x_f32: np.ndarray, bits: int):
    """numpy float32 evaluation of profile S (cpp:735-753, cpp:806-824)."""
    amax = np.maximum(np.float32(1e-6), np.abs(x_f32).max(axis=1))
    c = np.float32(127.0 if bits == 8 else 7.0)
    s = (amax / c).astype(np.float16)
    inv = np.float32(1.0) / s.astype(np.float32)
    y = x_f32 * inv[:, None]
    r = np.rint(y)
    if bits == 8:
        q = np.clip(r, -127, 127).astype(np.int64)
    else:
        q = np.clip(r + 8, 0, 15).astype(np.int64)
    return q, s


def test_bf16_groups_closed_form(O):
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((50000, 16)) * rng.choice([1e-3, 1, 30, 1e4], size=(50000, 1)))
    xb = torch.from_numpy(x.astype(np.float32)).to(torch.bfloat16)
    bits16 = xb.view(torch.int16).numpy().view(np.uint16)
    xf = xb.float().numpy()
    for b in (8, 4):
        q, s = O.quant_groups(bits16, O.BF16, b)
        qc, sc = _closed_form(xf, b)
        assert np.array_equal(s, sc.view(np.uint16))
        if b == 8:
            assert np.array_equal(q.view(np.int8).astype(np.int64), qc)
        else:
            lo, hi = q & 0xF, q >> 4
            both = np.stack([lo, hi], axis=2).reshape(q.shape[0], 16).astype(np.int64)
            assert np.array_equal(both, qc)
        # dequantize: one rounding of the exact product, to bf16
        out = O.dequant_groups(q, s, O.BF16, b)
        qv = qc if b == 8 else qc - 8
        prod = qv.astype(np.float32) * s.view(np.float16).astype(np.float32)[:, None]
        want = torch.from_numpy(prod).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
        assert np.array_equal(out, want)
