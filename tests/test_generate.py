"""The device-side sampler against the reference's sampling ops, on the CPU.

moss_tts_lite_amd.generate.sample_rows replaces ``torch.multinomial`` by the draw it makes
internally (``q = exponential_(1)`` over the probabilities' shape, ``argmax(p / q)``) and
``torch.unique`` by presence masks; the tokens and the generator's state afterwards must
equal the reference's ``sample_token`` (restated in tests/_generate_ref.py from
moss_tts_lite/sampling.py) for every argument combination the reference's own tests use
(tests/test_core.py:230-246).
"""
import pytest
import torch

from moss_tts_lite_amd import generate as GEN
from tests import _generate_ref as R


def _history_masks(prev, v):
    seen = torch.zeros(v, dtype=torch.bool)
    seen[prev.reshape(-1)] = True
    return seen


@pytest.mark.parametrize("tk,tp", [(None, None), (25, 0.8), (50, 1.0), (None, 0.95), (5, None)])
@pytest.mark.parametrize("rep", [1.0, 1.2])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_sample_rows_matches_sample_token(tk, tp, rep, dtype):
    g = torch.Generator().manual_seed(3)
    for rows, v in ((1, 50), (31, 1025)):
        lg = (torch.randn(rows, v, generator=g) * 2).to(dtype)
        prev = torch.randint(0, v, (1, 9, 3), generator=g)
        torch.manual_seed(42)
        a = R.sample_token(lg.clone(), prev_tokens=prev, repetition_penalty=rep, top_p=tp,
                           top_k=tk, do_sample=True)
        after_a = torch.rand(3)
        torch.manual_seed(42)
        b = GEN.sample_rows(lg.clone(), seen=_history_masks(prev, v), penalty=rep, top_p=tp,
                            top_k=tk, do_sample=True)
        after_b = torch.rand(3)
        assert torch.equal(a, b), (tk, tp, rep, rows)
        assert torch.equal(after_a, after_b)       # the generator advanced alike


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
