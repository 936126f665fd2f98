"""Pins oracle/cpu_path.py (the reference's CPU int4 linear in torch ops, and torch's CPU
int4 operator pair) against the float64 closed form of the qsz contract
(oracle/gptq_ref.py: effective_weight, int4pack_mm)."""
import numpy as np
import pytest
import torch

from oracle import cpu_path as C
from oracle import gptq_ref as G
from oracle.bf16 import bf16_bits_to_f32


def _case(n, k, g, m, seed):
    r = np.random.default_rng(seed)
    q = r.integers(0, 16, (n, k), dtype=np.uint8)
    qsz = torch.stack([torch.from_numpy(r.uniform(0.002, 0.02, (k // g, n)).astype(np.float32)),
                       torch.from_numpy(r.uniform(-0.1, 0.1, (k // g, n)).astype(np.float32))],
                      2).bfloat16()
    x = torch.from_numpy(r.standard_normal((m, k)).astype(np.float32)).bfloat16()
    return q, qsz, x


def _bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("n,k,g,m", [(256, 512, 128, 1), (128, 1024, 32, 3), (64, 512, 256, 16)])
def test_cpu_paths_match_closed_form(n, k, g, m):
    q, qsz, x = _case(n, k, g, m, seed=n + k + g + m)
    # the dequant is the closed form bit for bit
    w = C.effective_weight(torch.from_numpy(q), qsz, g).numpy()
    np.testing.assert_array_equal(w, G.effective_weight(q, _bits(qsz), g))
    ref = G.int4pack_mm(bf16_bits_to_f32(_bits(x)), q, _bits(qsz), g)
    y32 = C.linear_fp32(x, torch.from_numpy(q), qsz, g).numpy()
    assert np.linalg.norm(y32 - ref) / np.linalg.norm(ref) < 1e-5          # fp32 sums
    y4 = C.int4pack_mm_cpu(x, C.pack_for_cpu(torch.from_numpy(q)), g, qsz).float().numpy()
    assert np.linalg.norm(y4 - ref) / np.linalg.norm(ref) < 5e-3           # bf16 output
    # a transposed group order of the metadata does not pass
    bad = C.linear_fp32(x, torch.from_numpy(q), qsz.flip(0), g).numpy()
    assert np.linalg.norm(bad - ref) / np.linalg.norm(ref) > 5e-2
