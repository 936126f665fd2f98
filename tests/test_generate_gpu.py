"""Device-side MOSS generation against the reference's host loop, on the GPU.

moss_tts_lite_amd.generate.generate_fast (sampling on the device, one overlapped host read
per step) and the reference's generate_fast restated in tests/_generate_ref.py (every
decision read back to the host, torch.multinomial, torch.unique) drive the same
FastMossDecoder over the seeded tiny MOSS model from the same seed; the text tokens, the
audio frames and the stop reason must be identical.  Also: on this GPU
``torch.multinomial(p, 1)`` equals ``argmax(p / exponential_(1))`` drawn from the same
generator, in the dtypes and shapes generation uses.
"""
import pytest
import torch

from moss_tts_lite_amd import generate as GEN
from tests import _generate_ref as R
from tests import _moss_tiny as T

pytestmark = pytest.mark.gpu


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
    model = T.device_backbone(T.generate(T.SEED, True), dev, max_seq=192, full_text_embedding=True)
    return FastMossDecoder(model)


def _prompt(kind):
    g = torch.Generator().manual_seed(11)
    rows = torch.full((8, 33), GEN.AUDIO_PAD_CODE, dtype=torch.long)
    rows[:, 0] = torch.randint(100, 8000, (8,), generator=g)
    if kind == "audio":                       # a continuation: audio already started
        rows[-1, 0] = GEN.AUDIO_START_TOKEN_ID
        rows[3, 1:] = torch.randint(0, 1024, (32,), generator=g)
    return rows[None]


CASES = {
    "audio_sampled": dict(prompt="audio"),
    "audio_greedy": dict(prompt="audio", greedy=True),
    "audio_penalty": dict(prompt="audio", audio_repetition_penalty=1.3, audio_top_k=40),
    "audio_text_sampled_2way": dict(prompt="audio", text_temperature=1.0, text_top_k=2),
    "text_first": dict(prompt="text", text_top_p=0.9),
    # channel 0 pinned to a low-energy code (see the test): three such frames in a row
    # stop the segment
    "watchdog": dict(prompt="audio", watchdog_silence_frames=3),
}


@pytest.mark.parametrize("case", list(CASES))
def test_generate_fast_matches_reference_loop(dev, decoder, case, monkeypatch):
    kw = dict(CASES[case])
    prompt = _prompt(kw.pop("prompt"))
    n = kw.pop("n", 90)
    if case == "watchdog":      # channel 0's logits after every head pass: only code 9 finite
        heads, step = decoder.replay_heads, decoder.step

        def pin():
            decoder.la[0].fill_(float("-inf"))
            decoder.la[0, 9] = 1.0

        def pinned_heads(audio2=False):
            heads(audio2)
            pin()

        def pinned_step(row, pos, audio2=False):
            out = step(row, pos, audio2)
            pin()
            return out

        monkeypatch.setattr(decoder, "replay_heads", pinned_heads)
        monkeypatch.setattr(decoder, "step", pinned_step)
    ref_text, ref_audio, ref_reason = R.generate(decoder, prompt, max_new_tokens=n, seed=5, **kw)
    stats = {}
    res = GEN.generate_fast(decoder, {"input_ids": prompt}, max_new_tokens=n, seed=5, stats=stats,
                            **kw)
    print(f"{case}: {res.n_steps} steps, text {sorted(set(res.text_ids.tolist()))[:6]}, "
          f"reason {res.watchdog_reason!r}, host wait {stats['host_wait_s'] * 1e3:.1f} ms")
    assert res.text_ids.tolist() == ref_text
    assert torch.equal(res.audio_frames, ref_audio)
    assert res.watchdog_reason == ref_reason
    assert res.n_steps == len(ref_text)
    if case == "watchdog":
        assert ref_reason == "silence" and res.watchdog_triggered


def test_capture_outside_inference_mode_after_generation(dev):
    # generation captures its graphs under inference mode; a decoder captured afterwards
    # outside it must still capture and replay (the default generator's graph state is
    # shared by every capture of the process)
    from moss_tts_lite_amd.fast import FastMossDecoder
    model = T.device_backbone(T.generate(T.SEED, True), dev, max_seq=64, full_text_embedding=True)
    first = FastMossDecoder(model)
    GEN.generate_fast(first, {"input_ids": _prompt("audio")}, max_new_tokens=4, seed=5)
    second = FastMossDecoder(model)
    assert not torch.is_inference_mode_enabled()
    second.prefill(_prompt("audio")[0])
    second.capture()
    lt, la, _, _ = second.step(None, 8, audio2=True)
    torch.cuda.synchronize()
    pad = GEN.AUDIO_PAD_CODE                  # the heads' pad code is -inf by design
    assert torch.isfinite(la[:, :pad].float()).all() and bool((la[:, pad] == float("-inf")).all())
