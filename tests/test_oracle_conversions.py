"""fp16 / bf16 conversions of the oracle against numpy and torch.

fp32 -> fp16 is the rounding every wire scale goes through; fp32 -> bf16 is
the BF16 dequantize rounding.  Both are checked against library routines:
exhaustively on the 16-bit side, and on every fp32 pattern whose low 13 bits
sit at or next to a rounding boundary (all exponents, all signs), plus a
random sample.
"""
import numpy as np
import torch


def _boundary_patterns() -> np.ndarray:
    hi = np.arange(0, 1 << 19, dtype=np.uint32) << 13           # sign, exponent, top mantissa
    lows = np.array([0, 1, 0x0FFF, 0x1000, 0x1001, 0x17FF, 0x1800, 0x1FFF], dtype=np.uint32)
    return (hi[:, None] | lows[None, :]).reshape(-1)


def test_f16_to_f32_exhaustive(O):
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    got = O.f16_bits_to_f32(h)
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(got.view(np.uint32)[~nan], want.view(np.uint32)[~nan])
    assert np.isnan(got[nan]).all()


def test_f32_to_f16_boundaries(O):
    bits = _boundary_patterns()
    f = bits.view(np.float32)
    got = O.f32_to_f16_bits(f)
    with np.errstate(over="ignore", invalid="ignore"):
        want = f.astype(np.float16).view(np.uint16)
    nan = np.isnan(f)
    assert np.array_equal(got[~nan], want[~nan])
    # NaN keeps its sign and becomes the quiet 0x7E00 payload (c10 software path)
    assert np.array_equal(got[nan] & 0x7FFF, np.full(nan.sum(), 0x7E00, np.uint16))


def test_f32_to_f16_random(O):
    bits = np.random.default_rng(0).integers(0, 2**32, size=1 << 22, dtype=np.uint64).astype(np.uint32)
    f = bits.view(np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        want = f.astype(np.float16).view(np.uint16)
    nan = np.isnan(f)
    assert np.array_equal(O.f32_to_f16_bits(f)[~nan], want[~nan])


def test_f32_to_bf16_boundaries(O):
    bits = _boundary_patterns()
    # bf16 rounds at bit 16: also probe its own boundaries
    hi = np.arange(0, 1 << 16, dtype=np.uint32) << 16
    lows = np.array([0, 1, 0x7FFF, 0x8000, 0x8001, 0xFFFF], dtype=np.uint32)
    bits = np.concatenate([bits, (hi[:, None] | lows[None, :]).reshape(-1)])
    f = bits.view(np.float32)
    got = O.f32_to_bf16_bits(f)
    want = torch.from_numpy(f.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    nan = np.isnan(f)
    assert np.array_equal(got[~nan], want[~nan])
    assert (got[nan] == 0x7FC0).all()
