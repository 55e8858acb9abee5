"""The C E4M3FN codec oracle (oracle/fp8_e4m3.c) against torch's float8_e4m3fn
casts and the reference's known-answer table (CPU only)."""
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import fp8

GOLDEN = Path(__file__).resolve().parent / "golden" / "e4m3.npz"


def test_decode_all_256_codes_match_torch():
    codes = np.arange(256, dtype=np.uint8)
    got = fp8.decode(codes)
    want = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert set(np.flatnonzero(nan)) == {0x7F, 0xFF}
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))  # bit-exact, -0 included


def test_decode_matches_golden_table():
    g = np.load(GOLDEN)
    got = fp8.decode(g["decode_codes"])
    want = g["decode_values"]
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    assert np.array_equal(got[ok].view(np.uint32), want[ok].view(np.uint32))


def test_encode_known_answer_table():
    """flash_attn_mps tests/test_cache.py:39-54: every finite code, every
    midpoint (ties to even), both signs, saturation at +-1000 and +-inf."""
    g = np.load(GOLDEN)
    assert np.array_equal(fp8.encode(g["encode_inputs"]), g["encode_codes"])


@pytest.mark.parametrize("scale", [0.5, 2.0, 4.0])
def test_encode_scaled_known_answers(scale):
    """Scaled stores encode x / scale: x = value * scale recovers the table."""
    g = np.load(GOLDEN)
    values = g["encode_inputs"].astype(np.float32)
    x = (values * np.float32(scale)).reshape(-1, 1, 1)
    codes = fp8.encode_scaled(x, np.array([scale], dtype=np.float32)).reshape(-1)
    assert np.array_equal(codes, g["encode_codes"])


def test_encode_per_head_scales():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((64, 3, 8)).astype(np.float32) * 50
    scale = np.array([0.5, 0.01, 3.0], dtype=np.float32)
    got = fp8.encode_scaled(x, scale)
    want = torch.from_numpy(x / scale[None, :, None]).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8)
    assert np.array_equal(got, want.numpy())


def test_nan_encodes_to_signed_0x7f():
    nans = np.array([np.nan, -np.nan], dtype=np.float32)
    nans[1] = -np.abs(nans[1])
    assert fp8.encode(nans).tolist() == [0x7F, 0xFF]


def test_encode_float32_sweep_matches_torch():
    """~1.05M float32 bit patterns (stride 4099 over all 2^32, every sign,
    exponent, subnormal and saturating range) against torch's RNE cast."""
    stride = 4099
    count = (1 << 32) // stride
    got = fp8.sweep(0, stride, count)
    bits = (np.arange(count, dtype=np.uint64) * stride).astype(np.uint32)
    x = bits.view(np.float32)
    finite = ~np.isnan(x)
    want = torch.from_numpy(x[finite].copy()).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(got[finite], want)
    sign = (bits[~finite] >> 31).astype(np.uint8)
    assert np.array_equal(got[~finite], (sign << 7) | 0x7F)


def test_subnormal_boundaries():
    """Subnormals are m * 2^-9: 2^-10 ties to 0 (even), 3 * 2^-10 to code 2,
    2^-6 is the first normal code 0x08, 448 = 0x7E."""
    x = np.array([2.0 ** -9, 2.0 ** -10, 3 * 2.0 ** -10, 2.0 ** -6, 448.0, 464.0, -2.0 ** -9], dtype=np.float32)
    assert fp8.encode(x).tolist() == [0x01, 0x00, 0x02, 0x08, 0x7E, 0x7E, 0x81]
