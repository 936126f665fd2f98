"""The captured MOSS decode step against the reference's own eager model.

``tests/golden/moss_step_fixtures.npz`` holds what moss_tts_lite/model.py computes on the
CPU for the seeded tiny MOSS model of ``tests/_moss_tiny.py``:
- ``prefill`` of 6 rows, then ``step`` x 3;
- the final-normed hidden state of each point, the text logits at sampled rows, the audio
  logits (pad column -inf) and the 2-way logits.

Here the same model runs as int4 GPTQ weights (act-order groups, or contiguous groups) on
``FastMossDecoder``. The path is the batched prefill, then graph replays of both head
variants at each step position. Bar: rel-L2 <= 1e-2 (bf16 step outputs). The text and
audio2 replays at one position agree on the hidden state bit for bit.
"""
import os

import numpy as np
import pytest
import torch

from oracle.bf16 import bf16_bits_to_f32
from tests import _moss_tiny as T

pytestmark = pytest.mark.gpu

FIX = os.path.join(os.path.dirname(__file__), "golden", "moss_step_fixtures.npz")
BAR = 1e-2


def rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


def fb(t):
    return t.float().cpu().numpy()


@pytest.mark.parametrize("plan", ["strip", "unfused"])
@pytest.mark.parametrize("tag", ["ao", "ct"])
def test_moss_decoder_matches_reference_model(dev, tag, plan):
    from moss_tts_lite_amd.fast import FastMossDecoder

    model = T.device_backbone(T.generate(T.SEED, tag == "ao"), dev, max_seq=64)
    _check_decoder(FastMossDecoder(model, plan=plan), tag, plan)


# bf16-keep lists in the reference's form (gptq.py:645-650): every v_proj kept, and
# up_proj of layer 0 as in the shipped presets' layers that keep it
KEEPS = {"int4": (), "keep_v_up": [(0, "v"), (1, "v"), (0, "up")]}


@pytest.mark.parametrize("keep", list(KEEPS))
def test_moss_decoder_on_reference_records(dev, keep):
    """The reference's own ``(codes, qsz)`` records through ``W4Dispatch`` and
    ``layers_from_dispatch``: the qsz read in place by the strip kernels, v/up kept bf16."""
    from moss_tts_lite_amd.fast import FastMossDecoder

    model = T.dispatch_backbone(T.generate(T.SEED, False), dev, max_seq=64, keep=KEEPS[keep])
    dec = FastMossDecoder(model)
    assert dec.up_keep == [keep != "int4", False]
    assert dec.v_keep == [keep != "int4"] * 2
    _check_decoder(dec, "ct", keep)


def _check_decoder(dec, tag, label):
    fix = dict(np.load(FIX))
    f = bf16_bits_to_f32
    rows, n_prompt = fix["rows"], int(fix["prompt_rows"])
    hf0 = fb(dec.prefill(torch.from_numpy(rows[:n_prompt])))
    err = rel_l2(hf0, f(fix[f"{tag}_hf"][0]))
    print(f"{tag}/{label} prefill: hf rel_l2={err:.2e}")
    assert err < BAR
    dec.capture()
    idx = fix[f"{tag}_lt_idx"]
    keep = np.arange(T.AUDIO_VOCAB) != T.AUDIO_PAD
    for s in range(rows.shape[0] - n_prompt):
        p, i = n_prompt + s, s + 1
        row = torch.from_numpy(rows[p])
        lt, la, hf, _ = (t.clone() for t in dec.step(row, p, False))
        _, la2, hf2, two = (t.clone() for t in dec.step(row, p, True))
        assert torch.equal(hf, hf2) and torch.equal(la, la2)
        assert np.isneginf(fb(la)[:, T.AUDIO_PAD]).all()
        errs = {"hf": rel_l2(fb(hf), f(fix[f"{tag}_hf"][i])),
                "lt": rel_l2(fb(lt)[idx], f(fix[f"{tag}_lt"][i])),
                "la": rel_l2(fb(la)[:, keep], f(fix[f"{tag}_la"][i])[:, keep]),
                "two": rel_l2(fb(two), f(fix[f"{tag}_two"][i]))}
        print(f"{tag}/{label} pos {p}: " + " ".join(f"{k}={v:.2e}" for k, v in errs.items()))
        assert max(errs.values()) < BAR, (p, errs)
    # positions outside the cache and host ids outside a table are refused before replay
    with pytest.raises(ValueError):
        dec.step(torch.from_numpy(rows[0]), 64)
    bad = rows[0].copy()
    bad[3] = T.AUDIO_VOCAB
    with pytest.raises(ValueError):
        dec.step(torch.from_numpy(bad), 9)
