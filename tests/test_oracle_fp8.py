"""Pins of the e4m3fn codec (oracle/fp8.py) -- CPU only."""
import numpy as np
import torch

from oracle import fp8


def test_decode_table_known_values():
    d = fp8.decode_table()
    assert d[0x00] == 0.0 and d[0x80] == 0.0 and np.signbit(d[0x80])
    assert d[0x01] == 2.0 ** -9            # smallest subnormal
    assert d[0x07] == 7 * 2.0 ** -9        # largest subnormal
    assert d[0x08] == 2.0 ** -6            # smallest normal
    assert d[0x38] == 1.0                  # exponent field 7 = bias
    assert d[0x7E] == 448.0 and d[0xFE] == -448.0
    assert np.isnan(d[0x7F]) and np.isnan(d[0xFF])
    assert np.sum(np.isnan(d)) == 2        # no infinities, two NaN codes


def test_encode_matches_torch_on_every_bf16_times_scales():
    """Exhaustive: every bf16 bit pattern divided by several scales (the act_quant input
    set) -- the nearest-neighbour codec and torch's cast agree bit for bit."""
    f = (np.arange(65536, dtype=np.uint32) << 16).view(np.float32)
    for s in (1.0, 3.0, 0.1, 1e-3, 448 / 3.7, 2.0 ** -20):
        with np.errstate(all="ignore"):
            v = (f / np.float32(s)).astype(np.float32)
        v = v[np.isfinite(v)]
        th = torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
        assert np.array_equal(fp8.encode(v), th)


def test_encode_round_to_nearest_even_ties():
    # 1.0625 is halfway between 1.0 (0x38, even) and 1.125 (0x39): ties to even
    assert fp8.encode(np.float32(1.0625)) == 0x38
    # 1.1875 is halfway between 1.125 (0x39) and 1.25 (0x3A, even)
    assert fp8.encode(np.float32(1.1875)) == 0x3A
    # halfway between the two smallest subnormals -> even (0)
    assert fp8.encode(np.float32(2.0 ** -10)) == 0x00
    assert fp8.encode(np.float32(3 * 2.0 ** -10)) == 0x02
    assert fp8.encode(np.float32(464.0)) == 0x7E      # ties down to 448 (mantissa 110)
    assert fp8.encode(np.float32(470.0)) == 0x7F      # overflow is NaN
    assert fp8.encode(np.float32(-1e-30)) == 0x80     # sign of zero kept


def test_decode_encode_roundtrip():
    codes = np.arange(256, dtype=np.uint8)
    finite = ~np.isnan(fp8.decode(codes))
    assert np.array_equal(fp8.encode(fp8.decode(codes[finite])), codes[finite])
