"""Pins oracle/numerics.py against torch's own casts (library routines)."""
import numpy as np
import torch

from oracle.numerics import (bf16_encode, e4m3_decode, e4m3_decode_table, e4m3_encode)


def test_e4m3_decode_all_codes_match_torch():
    ours = e4m3_decode(np.arange(256))
    ref = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(ours, ref, equal_nan=True)


def test_e4m3_known_values():
    t = e4m3_decode_table()
    assert t[0x7E] == 448.0 and np.isnan(t[0x7F]) and t[0x01] == 2.0 ** -9
    assert t[0x08] == 2.0 ** -6 and t[0x38] == 1.0 and t[0xB8] == -1.0


def test_e4m3_encode_exhaustive_bf16_matches_torch():
    f = (np.arange(65536, dtype=np.uint32) << 16).view(np.float32)
    fin = np.isfinite(f)
    ref = torch.from_numpy(f.copy()).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(e4m3_encode(f)[fin], ref[fin])


def test_e4m3_encode_random_fp32_matches_torch():
    rng = np.random.default_rng(0)
    f = (rng.standard_normal(10**6) * np.exp(rng.uniform(-12, 6, 10**6))).astype(np.float32)
    ref = torch.from_numpy(f).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(e4m3_encode(f), ref)


def test_e4m3_ties_round_to_even():
    # 1.0625 is halfway between 1.0 (0x38) and 1.125 (0x39): even mantissa wins.
    assert e4m3_encode(np.float32([1.0625, 1.1875]))[0] == 0x38
    assert e4m3_encode(np.float32([1.1875]))[0] == 0x3A


def test_bf16_encode_matches_torch():
    rng = np.random.default_rng(1)
    f = (rng.standard_normal(10**6) * 100).astype(np.float32)
    ref = torch.from_numpy(f).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(bf16_encode(f), ref)
