"""The device-side sampler against the reference's own sampler, on the CPU.

moss_tts_lite_amd.generate.sample_rows replaces ``torch.multinomial`` by the draw it makes
internally (``q = exponential_(1)`` over the probabilities' shape, ``argmax(p / q)``) and
``torch.unique`` by presence masks.  ``tests/golden/generate_fixtures.npz`` holds what the
reference's ``sample_token`` (moss_tts_lite/sampling.py:70-99, run on the CPU by
``tests/golden/make_generate_fixtures.py``) returned for the argument combinations the
reference's own tests use (tests/test_core.py:230-246), and the generator state it left; the
device sampler must give the same tokens and leave the same state.
"""
import os

import numpy as np
import pytest
import torch

from moss_tts_lite_amd import generate as GEN
from tests.golden.make_generate_fixtures import SAMPLE_GRID, sample_grid_logits

FIXTURES = os.path.join(os.path.dirname(__file__), "golden", "generate_fixtures.npz")


def _history_masks(prev, v):
    seen = torch.zeros(v, dtype=torch.bool)
    seen[prev.reshape(-1)] = True
    return seen


@pytest.fixture(scope="module")
def fixtures():
    return np.load(FIXTURES)


@pytest.mark.parametrize("i", range(len(SAMPLE_GRID)))
def test_sample_rows_matches_reference_sample_token(fixtures, i):
    tk, tp, rep, dt, shape = SAMPLE_GRID[i]
    lg, prev = sample_grid_logits(i, shape, dt)
    torch.manual_seed(42)
    got = GEN.sample_rows(lg.clone(), seen=_history_masks(prev, shape[1]), penalty=rep, top_p=tp,
                          top_k=tk, do_sample=True)
    after = torch.rand(3)
    want = fixtures["sample_tokens"][i][:shape[0]]
    assert got.tolist() == want.tolist(), (tk, tp, rep, dt, shape)
    assert torch.equal(after, torch.from_numpy(fixtures["sample_after"][i]))   # same generator state


def test_sample_rows_greedy_and_penalty_values():
    lg = torch.tensor([[2.0, -1.0, 0.5, -3.0, 1.0]]).bfloat16()
    seen = torch.tensor([True, True, False, True, False])
    out = GEN.penalize(lg, seen, 2.0)
    assert torch.equal(out, torch.tensor([[1.0, -2.0, 0.5, -6.0, 1.0]]).bfloat16())
    assert int(GEN.sample_rows(lg, do_sample=False)[0]) == 0
    assert int(GEN.sample_rows(lg, seen=seen, penalty=4.0, do_sample=False)[0]) == 4


def test_top_filters_keep_what_the_definitions_say():
    x = torch.tensor([[3.0, 1.0, 2.0, 0.0, -1.0]])
    k = GEN.filter_top_k(x.clone(), 2)
    assert torch.isinf(k).tolist() == [[False, True, False, True, True]]
    # softmax of x: 0.6364, 0.0861, 0.2341, 0.0317, 0.0117; cumulative past 0.8 after two
    p = GEN.filter_top_p(x.clone(), 0.8)
    assert torch.isinf(p).tolist() == [[False, True, False, True, True]]
    p = GEN.filter_top_p(x.clone(), 0.5)        # the most likely token always stays
    assert torch.isinf(p).tolist() == [[False, True, True, True, True]]
