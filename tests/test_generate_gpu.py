"""Device-side MOSS generation against the reference's own generation loop, on the GPU.

``tests/golden/generate_fixtures.npz`` holds the decisions of the reference's
``generate_fast`` (moss_tts_lite/fast.py:343-610), run on the CPU by
``tests/golden/make_generate_fixtures.py`` over the scripted head outputs of
``tests/_generate_script.py``.  Here moss_tts_lite_amd.generate.generate_fast (sampling on the
device, one overlapped host read per step) drives a FastMossDecoder over the seeded tiny MOSS
model whose head outputs are overwritten with the same scripted logits after every head
pass; the text tokens, the audio frames, the stop fields, the (position, audio2) of every
step and the shapes of the random draws, in order, must be the reference's.  Also: on this
GPU ``torch.multinomial(p, 1)`` equals ``argmax(p / exponential_(1))`` drawn from the same
generator, in the dtypes and shapes generation uses.
"""
import json
import os

import numpy as np
import pytest
import torch

from moss_tts_lite_amd import generate as GEN
from tests import _generate_script as S
from tests import _moss_tiny as T

pytestmark = pytest.mark.gpu

FIXTURES = os.path.join(os.path.dirname(__file__), "golden", "generate_fixtures.npz")


@pytest.mark.parametrize("rows,v", [(1, 1025), (31, 1025), (1, 151664), (7, 2)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_multinomial_is_the_exponential_argmax(dev, rows, v, dtype):
    for t in range(20):
        g0 = torch.Generator(device=dev).manual_seed(100 + t)
        p = torch.softmax((torch.randn(rows, v, device=dev, generator=g0) * 3).to(dtype), -1)
        g1 = torch.Generator(device=dev).manual_seed(7 + t)
        g2 = torch.Generator(device=dev).manual_seed(7 + t)
        a = torch.multinomial(p, 1, generator=g1)[:, 0]
        b = torch.argmax(p / torch.empty_like(p).exponential_(1, generator=g2), dim=-1)
        assert torch.equal(a, b)
        assert torch.equal(torch.rand(4, device=dev, generator=g1),
                           torch.rand(4, device=dev, generator=g2))


@pytest.fixture(scope="module")
def decoder(dev):
    from moss_tts_lite_amd.fast import FastMossDecoder
    model = T.device_backbone(T.generate(T.SEED, True), dev, max_seq=320, full_text_embedding=True)
    return FastMossDecoder(model)


@pytest.fixture(scope="module")
def fixtures():
    return np.load(FIXTURES)


@pytest.mark.parametrize("case", sorted(S.CASES))
def test_generate_fast_matches_reference_fixture(dev, decoder, fixtures, case, monkeypatch):
    spec = S.CASES[case]
    p = case + "/"
    script = S.Script(case, vocab=decoder.lt.numel())
    assert decoder.lt.numel() == S.TEXT_VOCAB
    assert script.checksum(6) == float(fixtures[p + "checksum"])    # the same scripted logits
    prompt = S.prompt(spec["prompt"])
    assert np.array_equal(prompt.numpy(), fixtures[p + "prompt"])

    heads, backbone = decoder.replay_heads, decoder.replay_backbone
    flags, positions, draws = [], [], []

    def scripted_heads(audio2=False):
        heads(audio2)
        k = len(flags)
        lt, la, two = script.heads(k)
        if k == 0 or not audio2:                 # what this pass of the heads refreshes
            decoder.lt.copy_(lt)
        if k == 0 or audio2:
            decoder.two.copy_(two)
        decoder.la.copy_(la)
        flags.append(bool(audio2))

    def recorded_backbone(pos):
        positions.append(int(pos))
        backbone(pos)

    real_exponential = torch.Tensor.exponential_

    def recorded_exponential(self, *a, **k):
        draws.append(list(self.shape))
        return real_exponential(self, *a, **k)

    monkeypatch.setattr(decoder, "replay_heads", scripted_heads)
    monkeypatch.setattr(decoder, "replay_backbone", recorded_backbone)
    monkeypatch.setattr(torch.Tensor, "exponential_", recorded_exponential)
    res = GEN.generate_fast(decoder, {"input_ids": prompt}, max_new_tokens=spec["n"], seed=5,
                            **spec["kwargs"])
    monkeypatch.undo()
    want = json.loads(str(fixtures[p + "result"]))
    print(f"{case}: {res.n_steps} steps, reason {res.watchdog_reason!r}, "
          f"{len(draws)} draws (reference {len(fixtures[p + 'draws'])})")
    assert res.text_ids.tolist() == fixtures[p + "text_ids"].tolist()
    assert np.array_equal(res.audio_frames.numpy(), fixtures[p + "audio_frames"])
    assert (res.finished, res.n_steps) == (want["finished"], want["n_steps"])
    assert (res.watchdog_triggered, res.watchdog_reason) == (want["watchdog_triggered"],
                                                              want["watchdog_reason"])
    assert res.watchdog_stats == want["watchdog_stats"]
    calls = fixtures[p + "calls"]                # the reference's step(pos, audio2), steps 1..
    assert flags[1:] == [bool(a) for a in calls[:, 1]]
    # the backbone of the step after the last one is queued before the host's decision
    assert positions[:len(calls)] == calls[:, 0].tolist()
    assert len(positions) - len(calls) in (0, 1)
    assert draws == fixtures[p + "draws"].tolist()


def test_capture_outside_inference_mode_after_generation(dev):
    # generation captures its graphs under inference mode; a decoder captured afterwards
    # outside it must still capture and replay (the default generator's graph state is
    # shared by every capture of the process)
    from moss_tts_lite_amd.fast import FastMossDecoder
    model = T.device_backbone(T.generate(T.SEED, True), dev, max_seq=64, full_text_embedding=True)
    first = FastMossDecoder(model)
    GEN.generate_fast(first, {"input_ids": S.prompt("audio")}, max_new_tokens=4, seed=5)
    second = FastMossDecoder(model)
    assert not torch.is_inference_mode_enabled()
    second.prefill(S.prompt("audio")[0])
    second.capture()
    lt, la, _, _ = second.step(None, 8, audio2=True)
    torch.cuda.synchronize()
    pad = GEN.AUDIO_PAD_CODE                  # the heads' pad code is -inf by design
    assert torch.isfinite(la[:, :pad].float()).all() and bool((la[:, pad] == float("-inf")).all())
