"""Pins the oracle's bf16 conversions against torch's own (an independent implementation)."""
import numpy as np
import torch

from oracle.bf16 import bf16_bits_to_f32, f16_bits_to_f32, f32_to_bf16_bits, f32_to_f16_bits


def _torch_bits(a: np.ndarray) -> np.ndarray:
    return torch.from_numpy(a).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def test_rne_ties_and_specials_match_torch():
    # every 16-bit upper half with lower halves at the rounding boundary and around it
    hi = np.arange(0, 1 << 16, dtype=np.uint32) << 16
    lows = np.array([0x0000, 0x0001, 0x7FFF, 0x8000, 0x8001, 0xFFFF], dtype=np.uint32)
    u = (hi[:, None] | lows[None, :]).reshape(-1)
    a = u.view(np.float32)
    mine = f32_to_bf16_bits(a)
    ref = _torch_bits(a)
    nan = np.isnan(a)
    assert np.array_equal(mine[~nan], ref[~nan])
    # every NaN maps to a NaN; the oracle's choice is the canonical quiet NaN
    assert np.all(np.isnan(bf16_bits_to_f32(mine[nan])))
    assert np.all(mine[nan] == 0x7FC0)


def test_random_values_match_torch():
    r = np.random.default_rng(7)
    a = (r.standard_normal(1 << 20) * np.exp(r.uniform(-40, 40, 1 << 20))).astype(np.float32)
    assert np.array_equal(f32_to_bf16_bits(a), _torch_bits(a))


def test_widening_is_exact():
    b = np.arange(0, 1 << 16, dtype=np.uint32).astype(np.uint16)
    f = bf16_bits_to_f32(b)
    t = torch.from_numpy(b.view(np.int16)).view(torch.bfloat16).float().numpy()
    same = (f.view(np.uint32) == t.view(np.uint32)) | (np.isnan(f) & np.isnan(t))
    assert same.all()
    # round trip of every non-NaN pattern
    ok = ~np.isnan(f)
    assert np.array_equal(f32_to_bf16_bits(f[ok]), b[ok])


def test_half_helpers_round_trip():
    b = np.arange(0, 1 << 16, dtype=np.uint32).astype(np.uint16)
    f = f16_bits_to_f32(b)
    ok = ~np.isnan(f)
    assert np.array_equal(f32_to_f16_bits(f[ok]), b[ok])
