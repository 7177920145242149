"""A seeded sweep of random page geometries, presets and batch sizes: the HIP
path against the oracle, through the C ABI.

The fixed geometry lists of the other GPU tests pin the shapes the
reference's configurations use; this sweep draws tokens, heads, head_dim,
rope_dim, MLA, preset x RoPE mode (the extension layouts included), hot
dtype and page count (one page, the small-batch kernels' limit of four
pages per workgroup on either side, partial workgroups of the row
pipeline) from a fixed seed, so that shapes nobody listed go through
whichever kernel the launcher picks for them.  Every case must give
byte-identical blobs and bit-identical decoded pages, and a copy with one
flipped bit must get the oracle's per-page verdicts and outputs.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

KEYS = dict(k0=0x243F6A8885A308D3, k1=0x13198A2E03707344, mk0=0xA4093822299F31D0,
            mk1=0x082EFA98EC4E6C89, k2=0x452821E638D01377, k3=0xBE5466CF34E90C6C)
TEN, MOD, LAYER, HG, BASE = 0x5EED5EED, 0x0DDBA11, 11, 2, 77_000
DT = {"fp16": torch.float16, "bf16": torch.bfloat16}
# pages per call: one, the small-batch kernels' range and its edges
# (4 pages per workgroup on 256 CUs), and row-pipeline batches with a
# partial last workgroup
PAGE_COUNTS = [1, 3, 64, 255, 1024, 1025, 1500]
PRESET_MODES = [(p, r) for p in (1, 2, 3) for r in (0, 1, 2)] + [(4, 3), (5, 0), (5, 3), (6, 1), (6, 3), (4, 1)]


def _cases(n=64, seed=20261202):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        mla = bool(rng.random() < 0.25)
        T = int(rng.choice([1, 2, 3, 5, 8, 16, 32]))
        H = 1 if mla else int(rng.choice([1, 2, 3, 4, 8]))
        D = int(rng.choice([16, 32, 48, 64, 128, 192, 256] + ([576] if mla else [])))
        R = int(rng.choice([r for r in (0, 16, 32, 64) if r <= D]))
        preset, rm = PRESET_MODES[int(rng.integers(len(PRESET_MODES)))]
        B = int(rng.choice(PAGE_COUNTS))
        dt = str(rng.choice(["fp16", "bf16"]))
        if O.payload_bytes(preset, rm, T * H, D, R, not mla) <= 0:
            continue
        if B * T * H * D > (1 << 23):  # keep the oracle's share of each case short
            B = max(1, (1 << 23) // (T * H * D))
        out.append((T, H, D, R, mla, preset, rm, B, dt, int(rng.integers(1 << 30))))
    return out


CASES = _cases()


def _bits(t):
    return None if t is None else t.contiguous().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize(
    "case", CASES,
    ids=lambda c: f"T{c[0]}H{c[1]}D{c[2]}R{c[3]}{'m' if c[4] else ''}-p{c[5]}r{c[6]}-B{c[7]}-{c[8]}")
def test_random_geometry_matches_oracle(hip, O, case):
    T, H, D, R, mla, preset, rm, B, dt, seed = case
    ext = preset >= 4 or rm == 3
    odt = O.BF16 if dt == "bf16" else O.FP16
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((B, T, H, D)).astype(np.float32) * 0.8
    if R:
        k[..., :R] *= 6
    v = None if mla else (rng.standard_normal((B, T, H, D)) * 0.5).astype(np.float32)
    k[0, 0, 0, :16] = 0  # an all-zero group
    kt = torch.from_numpy(k).to(DT[dt])
    vt = None if v is None else torch.from_numpy(v).to(DT[dt])
    th = rng.integers(0, 1 << 62, size=B, dtype=np.int64)
    exp = O.payload_bytes(preset, rm, T * H, D, R, not mla)
    dev = torch.device("cuda")

    blobs = torch.full((B, 48 + exp), 0xA5, dtype=torch.uint8, device=dev)
    hip.fused_encode_cold_pages_peak_into(kt.to(dev), None if vt is None else vt.to(dev), torch.from_numpy(th),
                                          blobs, preset, rm, R, exp, TEN, MOD, LAYER, HG, BASE, KEYS["k0"],
                                          KEYS["k1"], KEYS["mk0"], KEYS["mk1"], KEYS["k2"], KEYS["k3"],
                                          ext_layouts=ext)
    torch.cuda.synchronize()
    want = O.egress_batch(_bits(kt), _bits(vt), th, dtype=odt, preset=preset, rope_mode=rm, rope_dim=R,
                          expected_payload_bytes=exp, tenant_id_hash=TEN, model_id_hash=MOD, layer_id=LAYER,
                          head_group_id=HG, base_sequence_nonce=BASE, **KEYS)
    got = blobs.cpu().numpy()
    assert np.array_equal(got, want), "blobs differ from the oracle's"

    def ingress(b, per_page):
        ko = torch.full((B, T, H, D), 3.0, dtype=DT[dt], device=dev)
        vo = None if mla else torch.full_like(ko, 3.0)
        st = torch.full((B,), -9, dtype=torch.int32, device=dev)
        err = None
        try:
            hip.fused_decode_cold_pages_peak_into(torch.from_numpy(b).to(dev), torch.from_numpy(th), ko, vo, R, mla,
                                                  TEN, MOD, LAYER, KEYS["k0"], KEYS["k1"], KEYS["mk0"], KEYS["mk1"],
                                                  KEYS["k2"], KEYS["k3"], page_status=st, per_page=per_page,
                                                  ext_layouts=ext)
        except RuntimeError as e:
            err = str(e)
        torch.cuda.synchronize()
        rc, ost, ok, ov = O.ingress_batch(b, th, num_tokens=T, num_heads=H, head_dim=D, rope_dim=R,
                                          is_mla_single_buffer=mla, dtype=odt, expected_tenant_hash=TEN,
                                          expected_model_hash=MOD, expected_layer_id=LAYER,
                                          all_or_nothing=not per_page, **KEYS)
        return err, st.cpu().numpy(), _bits(ko.cpu()), _bits(None if vo is None else vo.cpu()), rc, ost, ok, ov

    err, st, gk, gv, rc, ost, ok, ov = ingress(want, per_page=False)
    assert err is None and rc == 0 and (st == 0).all()
    assert np.array_equal(gk, ok) and (gv is None or np.array_equal(gv, ov)), "decoded pages differ"

    # one flipped bit in one page (header, payload or tag): the oracle's
    # per-page verdicts, and that page's outputs zeroed as the oracle's are
    bad = want.copy()
    page = B // 2
    byte = int(rng.integers(bad.shape[1]))
    bad[page, byte] ^= np.uint8(1 << int(rng.integers(8)))
    err, st, gk, gv, rc, ost, ok, ov = ingress(bad, per_page=True)
    assert np.array_equal(st, ost), (st[page], ost[page], byte)
    assert st[page] != 0 and (np.delete(st, page) == 0).all()
    assert np.array_equal(gk, ok) and (gv is None or np.array_equal(gv, ov)), "outputs after tamper differ"
