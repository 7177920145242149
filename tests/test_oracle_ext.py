"""Pins of the oracle's extension codes (presets 4..6, RoPE mode 3).

These formats have no counterpart in the reference, so nothing in it pins
them.  Each oracle function is checked against something that does not
restate it:
  * e4m3 conversion and decode: torch.float8_e4m3fn (a library conversion),
    on every bf16 pattern, random fp32 values and every rounding tie;
  * the e4m3 group quantizer: numpy's fp32 division / float16 rounding for
    the scale and torch's e4m3 conversion for the codes; dequantization by
    torch's e4m3 decode, fp32 product and bf16 / fp16 rounding;
  * int4 per 32: reduction to the reference-pinned int4 per-16 quantizer
    (scale = the larger of the two halves' scales, the dominant half's codes
    equal), plus the error bound;
  * asymmetric int8 per 64: invariants a plausible mistake breaks (zero is
    exact, codes span [0, 255] from the group minimum to its maximum, the
    error bound, the scale by numpy's division and float16 rounding), and
    exact ties of codes and zero points, which must round to even;
  * page sizing and byte maps: section offsets computed from the format, and
    the decrypted payload compared with group-wise quantization.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O

KEYS = dict(k0=0x0123456789ABCDEF, k1=0xFEDCBA9876543210, mk0=0x1111222233334444,
            mk1=0x5555666677778888, k2=0x0F1E2D3C4B5A6978, k3=0x8796A5B4C3D2E1F0)


def _hot(x: np.ndarray, dtype: int) -> np.ndarray:
    t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32))
    t = t.bfloat16() if dtype == O.BF16 else t.half()
    return t.view(torch.int16).numpy().view(np.uint16)


def _hot_f32(bits: np.ndarray, dtype: int) -> np.ndarray:
    t = torch.from_numpy(np.ascontiguousarray(bits).view(np.int16))
    t = t.view(torch.bfloat16) if dtype == O.BF16 else t.view(torch.float16)
    return t.float().numpy()


def _torch_e4m3(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(
        torch.float8_e4m3fn).view(torch.uint8).numpy()


def _round_hot(x: np.ndarray, dtype: int) -> np.ndarray:
    return _hot(x, dtype)


# ---- e4m3 conversion ---------------------------------------------------------

def test_e4m3_conversion_matches_torch_on_every_bf16_pattern():
    x = (np.arange(1 << 16, dtype=np.uint32) << 16).view(np.float32)
    x = x[~np.isnan(x)]
    np.testing.assert_array_equal(O.f32_to_e4m3(x), _torch_e4m3(np.clip(x, -448, 448)))


def test_e4m3_conversion_ties_and_random():
    finite = O.e4m3_to_f32(np.arange(256, dtype=np.uint8))
    pos = np.unique(finite[np.isfinite(finite) & (finite >= 0)]).astype(np.float64)
    mids = ((pos[:-1] + pos[1:]) / 2).astype(np.float32)  # exact ties in fp32
    near = np.concatenate([mids, np.nextafter(mids, np.float32(0)), np.nextafter(mids, np.float32(1e9))])
    rng = np.random.default_rng(3)
    x = np.concatenate([near, -near, rng.standard_normal(400_000).astype(np.float32) * 60,
                        rng.standard_normal(100_000).astype(np.float32) * 0.003,
                        np.array([np.inf, -np.inf, 1e30, -1e30, 448, -448, 464, 480], np.float32)])
    np.testing.assert_array_equal(O.f32_to_e4m3(x), _torch_e4m3(np.clip(x, -448, 448)))
    assert O.f32_to_e4m3(np.array([np.nan], np.float32))[0] == 0x7F


def test_e4m3_decode_matches_torch():
    c = np.arange(256, dtype=np.uint8)
    got = O.e4m3_to_f32(c)
    want = torch.from_numpy(c).view(torch.float8_e4m3fn).float().numpy()
    same = (got == want) | (np.isnan(got) & np.isnan(want))
    assert same.all()
    np.testing.assert_array_equal(np.signbit(got[~np.isnan(got)]), np.signbit(want[~np.isnan(want)]))


# ---- group quantizers ----------------------------------------------------------

def _groups(rng, n, ges, dtype, outliers=True):
    x = rng.standard_normal((n, ges)).astype(np.float32)
    if outliers:
        x[::7] *= 40.0
        x[1::11] *= 1e-3
    x[3] = 0.0                       # all-zero group (amax clamp 1e-6)
    x[4] = np.abs(x[4])              # one-signed groups
    x[5] = -np.abs(x[5])
    return _hot(x, dtype)


@pytest.mark.parametrize("dtype", [O.FP16, O.BF16])
def test_e4m3_group_quantizer(dtype):
    rng = np.random.default_rng(11)
    src = _groups(rng, 4000, 16, dtype)
    q, prm = O.quant_groups_ext(src, dtype, O.SEC_E4M3)
    v = _hot_f32(src, dtype)
    amax = np.maximum(np.float32(1e-6), np.abs(v).max(axis=1))
    scale = (amax / np.float32(448.0)).astype(np.float16)
    np.testing.assert_array_equal(prm[:, 0], scale.view(np.uint16))
    assert (prm[:, 1] == 0).all()
    with np.errstate(divide="ignore", invalid="ignore"):
        inv = (np.float32(1.0) / scale.astype(np.float32))[:, None]
        x = v * inv
    # a NaN product (scale underflowed to 0) is code 0
    np.testing.assert_array_equal(q, _torch_e4m3(np.clip(np.nan_to_num(x, nan=0.0), -448, 448)))
    if dtype == O.FP16:
        assert (prm[3, 0] == 0) and not q[3].any()  # all-zero group: fp16 scale underflows
    # dequantization: torch decode, fp32 product, one rounding to the hot dtype
    out = O.dequant_groups_ext(q, prm, dtype, O.SEC_E4M3)
    dec = torch.from_numpy(q).view(torch.float8_e4m3fn).float().numpy()
    want = _round_hot(dec * scale.astype(np.float32)[:, None], dtype)
    np.testing.assert_array_equal(out, want)


@pytest.mark.parametrize("dtype", [O.FP16, O.BF16])
def test_int4_g32_reduces_to_reference_int4_g16(dtype):
    rng = np.random.default_rng(12)
    src = _groups(rng, 3000, 32, dtype)
    q32, prm = O.quant_groups_ext(src, dtype, O.SEC_INT4G32)
    q16, s16 = O.quant_groups(src.reshape(-1, 16), dtype, 4)   # pinned against the reference
    s16 = s16.reshape(-1, 2)
    f16 = lambda b: b.view(np.float16).astype(np.float32)  # noqa: E731
    # scale = fp16(max(amax_a, amax_b) / 7) = the larger of the halves' scales
    np.testing.assert_array_equal(f16(prm[:, 0]), np.maximum(f16(s16[:, 0]), f16(s16[:, 1])))
    # the half that holds the group's absmax has the per-16 codes
    v = np.abs(_hot_f32(src, dtype)).reshape(-1, 2, 16).max(axis=2)
    dom = np.where(v[:, 0] >= v[:, 1], 0, 1)
    q16 = q16.reshape(-1, 2, 8)
    np.testing.assert_array_equal(q32.reshape(-1, 2, 8)[np.arange(len(dom)), dom],
                                  q16[np.arange(len(dom)), dom])
    # the other half: error bound |deq - v| <= s / 2 (no clamping below absmax)
    out = _hot_f32(O.dequant_groups_ext(q32, prm, dtype, O.SEC_INT4G32), dtype)
    s = f16(prm[:, 0])[:, None]
    x = _hot_f32(src, dtype)
    tol = s * 0.5 * (1 + 2.0 ** -8) + np.abs(x) * 2.0 ** -7
    assert (np.abs(out - x) <= tol).all()


@pytest.mark.parametrize("dtype", [O.FP16, O.BF16])
def test_asym8_g64_invariants(dtype):
    rng = np.random.default_rng(13)
    src = _groups(rng, 3000, 64, dtype)
    x = _hot_f32(src, dtype)
    x[6] = 0.0
    src[6] = 0
    x[7, 0] = 0.0
    src[7, 0] = 0
    q, prm = O.quant_groups_ext(src, dtype, O.SEC_ASYM8)
    lo = np.minimum(np.float32(0), x.min(axis=1))
    hi = np.maximum(np.float32(0), x.max(axis=1))
    rng_ = np.maximum(np.float32(1e-6), hi - lo)
    s = (rng_ / np.float32(255.0)).astype(np.float16)
    np.testing.assert_array_equal(prm[:, 0], s.view(np.uint16))
    s = s.astype(np.float32)
    z = prm[:, 1].astype(np.int64)
    assert (z >= 0).all() and (z <= 255).all()
    # the zero point maps to exactly 0, the group's minimum to code ~0 and its
    # maximum to code ~255 (one code of slack for the fp16 scale rounding)
    zero_in = x == 0
    assert (q.astype(np.int64)[zero_in] == np.broadcast_to(z[:, None], q.shape)[zero_in]).all()
    qi = q.astype(np.int64)
    rows = np.arange(len(q))
    assert (qi[rows, x.argmin(axis=1)] <= 1).all()
    busy = hi > 0
    assert (qi[rows, x.argmax(axis=1)][busy] >= 254).all()
    # one-signed groups: all-positive has z = 0, all-negative z = 255 (or 254)
    assert z[4] == 0 and z[5] >= 254
    # dequantized = (q - z) * s, exact in fp32, then one rounding
    out = O.dequant_groups_ext(q, prm, dtype, O.SEC_ASYM8)
    want = _round_hot((qi - z[:, None]).astype(np.float32) * s[:, None], dtype)
    np.testing.assert_array_equal(out, want)
    outf = _hot_f32(out, dtype)
    assert (outf[zero_in] == 0).all()
    tol = s[:, None] * 0.5 * (1 + 2.0 ** -8) + np.abs(x) * 2.0 ** -7 + s[:, None] * 2.0 ** -10
    assert (np.abs(outf - x) <= tol).all()


@pytest.mark.parametrize("dtype", [O.FP16, O.BF16])
def test_asym8_g64_ties_round_to_even(dtype):
    """Codes and zero points that fall exactly halfway between two integers
    round to the even one.  Groups whose range is 255 / 16 get the scale
    1 / 16 exactly (an fp16 power of two, so v * inv is exact), and values
    (2k + 1) / 32 then sit on the tie k + 1/2; a half-away-from-zero or
    truncating rounding fails here, where the invariants above cannot see it."""
    k = np.arange(128)
    ties = (2 * k + 1) / 32.0                       # v * 16 = k + 1/2
    even = np.where(k % 2 == 0, k, k + 1)           # the even neighbour
    # all-positive group: lo = 0, hi = 255/16, z = 0
    pos = np.concatenate([[0.0, 255 / 16], ties[:62]])
    # all-negative values with hi = 0: lo = -255/16, z = 255; -(k + 1/2) -> -even
    neg = np.concatenate([[0.0, -255 / 16], -ties[:62]])
    groups = [pos, neg]
    want_q = [np.concatenate([[0, 255], even[:62]]),
              np.concatenate([[255, 0], 255 - even[:62]])]
    want_z = [0, 255]
    if dtype == O.FP16:
        # the zero point on a tie: lo = -253/32 (-lo * 16 = 126.5 -> 126),
        # hi = 257/32 (hi * 16 = 128.5 -> 128, code 254), so the range is
        # 510/32 = 255/16 again
        mixed = np.concatenate([[-253 / 32, 257 / 32], ties[:31], -ties[:31]])
        groups.append(mixed)
        want_z.append(126)
        want_q.append(np.concatenate([[0, 254], 126 + even[:31], 126 - even[:31]]))
    src = np.stack([_hot(np.asarray(g, dtype=np.float32), dtype) for g in groups])
    assert (_hot_f32(src, dtype) == np.stack(groups).astype(np.float32)).all()  # exactly representable
    q, prm = O.quant_groups_ext(src, dtype, O.SEC_ASYM8)
    assert (prm[:, 0] == np.float16(1 / 16).view(np.uint16)).all()
    np.testing.assert_array_equal(prm[:, 1], want_z)
    np.testing.assert_array_equal(q.astype(np.int64), np.stack(want_q))


# ---- sizing, byte maps and round trips ------------------------------------------

# (preset, rope_mode, T, H, D, R, mla) -> expected payload bytes, from the format:
# c2 shape (16 x 8 x 128, rope 64), 128 vecs:
#   preset 4 + rope 3: rope e4m3 128*64 + 128*4*2 = 9216; K asym8 128*1*(64+4) = 8704;
#                      V int4/32 128*4*(16+2) = 9216  -> 27136
#   preset 5 + rope 0: K e4m3 128*8*18 = 18432; V the same -> 36864
#   preset 6 + rope 1: rope int8 9216; K int4/32 128*2*18 = 4608; V 9216 -> 23040
# c4 shape (64 x 1 x 576, rope 64, MLA), 64 vecs:
#   preset 6 + rope 3: rope e4m3 64*4*18 = 4608; latent int4/32 64*16*18 = 18432 -> 23040
#   preset 4 + rope 1: rope int8 4608; latent asym8 64*8*68 = 34816 -> 39424
SIZES = [
    ((4, 3, 16, 8, 128, 64, False), 27136),
    ((5, 0, 16, 8, 128, 64, False), 36864),
    ((6, 1, 16, 8, 128, 64, False), 23040),
    ((6, 3, 64, 1, 576, 64, True), 23040),
    ((4, 1, 64, 1, 576, 64, True), 39424),
    ((2, 3, 16, 8, 128, 64, False), 9216 + 9216 + 8192 + 2048),
]


@pytest.mark.parametrize("case,payload", SIZES)
def test_extension_sizes(case, payload):
    preset, rm, T, H, D, R, mla = case
    assert O.required_payload(preset, rm, T * H, D, R, not mla) == payload


def test_extension_invalid_geometry():
    # asym8 needs 64-column sections, int4/32 needs 32-column sections
    assert O.required_payload(4, 1, 64, 128, 16, True) == -1   # K main 112 columns
    assert O.required_payload(6, 1, 64, 128, 16, True) == -1
    assert O.required_payload(6, 1, 64, 128, 32, True) != -1
    assert O.required_payload(7, 1, 64, 128, 64, True) == -1
    assert O.required_payload(1, 4, 64, 128, 64, True) == -1


def _pages(rng, B, T, H, D, R, mla, dtype):
    k = rng.standard_normal((B, T, H, D)).astype(np.float32)
    k[..., :R] *= 8.0
    v = None if mla else rng.standard_normal((B, T, H, D)).astype(np.float32)
    return _hot(k, dtype), (None if v is None else _hot(v, dtype))


def _decrypt_payload(blob: np.ndarray, payload: int, seq: int, layer: int, hg: int) -> np.ndarray:
    key = b"".join(int(KEYS[n]).to_bytes(8, "little") for n in ("k0", "k1", "k2", "k3"))
    nonce = seq.to_bytes(8, "little") + ((layer << 16) | hg).to_bytes(4, "little")
    return np.frombuffer(O.chacha20_xor(blob[32:32 + payload].tobytes(), key, 1, nonce), np.uint8)


@pytest.mark.parametrize("preset,rm,T,H,D,R,mla", [
    (4, 3, 16, 8, 128, 64, False), (5, 1, 16, 4, 128, 64, False), (6, 3, 64, 1, 576, 64, True),
    (4, 0, 4, 2, 128, 0, False), (5, 3, 8, 2, 64, 32, False), (6, 2, 4, 4, 128, 64, False),
])
@pytest.mark.parametrize("dtype", [O.FP16, O.BF16])
def test_extension_byte_map_and_round_trip(preset, rm, T, H, D, R, mla, dtype):
    rng = np.random.default_rng(preset * 100 + rm)
    B = 3
    k, v = _pages(rng, B, T, H, D, R, mla, dtype)
    th = np.arange(B, dtype=np.int64) + 5
    kw = dict(tenant_id_hash=1, model_id_hash=2, layer_id=3, head_group_id=4, base_sequence_nonce=50)
    blobs = O.egress_batch(k, v, th, dtype=dtype, preset=preset, rope_mode=rm, rope_dim=R, **kw, **KEYS)
    payload = blobs.shape[1] - 48
    assert payload == O.payload_bytes(preset, rm, T * H, D, R, not mla)
    assert blobs[0, 3] == preset | (rm << 4)
    vecs = T * H
    kinds = {1: (1, 2, 2), 2: (0, 0, 1), 3: (0, 0, 0), 4: (5, 5, 4), 5: (3, 3, 3), 6: (4, 4, 4)}
    rope_kind = {1: 0, 2: 2, 3: 3}
    km, _, vk = kinds[preset]
    vk = {1: 1, 2: 1, 3: 0, 4: 4, 5: 3, 6: 4}[preset]
    km = {1: 1, 2: 0, 3: 0, 4: 5, 5: 3, 6: 4}[preset]
    secs = []
    if rm and R:
        secs.append((rope_kind[rm], 0, 0, R))
    kq = D if rm == 0 else D - R
    if kq:
        secs.append((km, 0, 0 if rm == 0 else R, kq))
    if not mla:
        secs.append((vk, 1, 0, D))
    geom = {0: (16, 16, 2), 1: (16, 8, 2), 3: (16, 16, 2), 4: (32, 16, 2), 5: (64, 64, 4)}
    for b in range(B):
        plain = _decrypt_payload(blobs[b], payload, 50 + b, 3, 4)
        off = 0
        for kind, src, col, width in secs:
            buf = (k if src == 0 else v)[b].reshape(vecs, D)[:, col:col + width]
            if kind == 2:
                n = vecs * width * 2
                np.testing.assert_array_equal(plain[off:off + n], np.ascontiguousarray(buf).view(np.uint8).ravel())
                off += n
                continue
            ges, cb, pb = geom[kind]
            grp = np.ascontiguousarray(buf).reshape(-1, ges)
            if kind in (0, 1):
                q, sc = O.quant_groups(grp, dtype, 8 if kind == 0 else 4)
                prm = sc.view(np.uint8).reshape(-1, 2)
            else:
                q, p2 = O.quant_groups_ext(grp, dtype, kind)
                prm = p2.view(np.uint8).reshape(-1, 4)[:, :pb]
            ng = grp.shape[0]
            np.testing.assert_array_equal(plain[off:off + ng * cb], q.ravel())
            off += ng * cb
            np.testing.assert_array_equal(plain[off:off + ng * pb], prm.ravel())
            off += ng * pb
        assert not plain[off:].any()
    rc, st, ko, vo = O.ingress_batch(blobs, th, num_tokens=T, num_heads=H, head_dim=D, rope_dim=R,
                                     is_mla_single_buffer=mla, dtype=dtype, expected_tenant_hash=1,
                                     expected_model_hash=2, expected_layer_id=3, **KEYS)
    assert rc == 0 and not st.any()
    for src, out in ((k, ko), (v, vo)):
        if src is None:
            continue
        x, y = _hot_f32(src, dtype), _hot_f32(out, dtype)
        err = np.abs(x - y) / (np.abs(x).max() + 1e-6)
        assert err.max() < 0.1
    bad = blobs.copy()
    bad[1, 40] ^= 0x10
    rc, st, _, _ = O.ingress_batch(bad, th, num_tokens=T, num_heads=H, head_dim=D, rope_dim=R,
                                   is_mla_single_buffer=mla, dtype=dtype, expected_tenant_hash=1,
                                   expected_model_hash=2, expected_layer_id=3,
                                   all_or_nothing=False, **KEYS)
    assert rc == 3 and list(st) == [0, 3, 0]
