"""Scripted head outputs that drive the MOSS generation loop through chosen paths.

A case is an argument set of ``generate_fast``, a prompt and a script.  The script gives,
for every time step t, the logits the three heads "produce" at that step: text ``lt [V]``,
audio ``la [32, 1025]`` (pad column -inf, as the heads make it) and 2-way ``two [2]``.  The
delay-pattern state machine decides which of them a step reads; the script is written so
that the decisions follow a planned path (audio start, generation and delay slots, the
32-step delay window, the audio end, ``<|im_end|>``, the masks of step 0 and of the first
32 steps, both watchdog triggers).

The same numbers feed two runs:
- ``tests/golden/make_generate_fixtures.py`` runs the reference's own ``generate_fast``
  (moss_tts_lite/fast.py:343-610) on the CPU over a stand-in decoder that returns them, and
  stores its decisions;
- ``tests/test_generate_gpu.py`` overwrites the device decoder's head outputs with them after
  every head pass and holds ``moss_tts_lite_amd.generate.generate_fast`` to those decisions.

Text candidates get well separated values (80, 40, 20, ...) over a baseline in (-1, 1), so
the winner after the loop's masks is the first candidate they leave, and sampled steps
pick it with probability 1 - O(e^-20): the outcome does not depend on the random stream.
In the "random" audio mode the audio logits are N(0, 4) draws (greedy cases: the argmax,
with the repetition penalty where a case sets one, is then a real decision over the
history); in the "dominant" mode each channel has one code at 80.
"""
from __future__ import annotations

import numpy as np
import torch

from moss_tts_lite_amd.generate import (AUDIO_DELAY_SLOT_TOKEN_ID as DELAY, AUDIO_END_TOKEN_ID as END,
                                        AUDIO_GEN_SLOT_TOKEN_ID as GEN, AUDIO_PAD_CODE,
                                        AUDIO_START_TOKEN_ID as START, IM_END_TOKEN_ID as IM_END,
                                        N_VQ, PAD_TOKEN_ID as PAD)

TEXT_VOCAB = 151664          # the text head rows of the tiny MOSS model (tests/_moss_tiny.py)
AUDIO_VOCAB = AUDIO_PAD_CODE + 1
SPEECH_CODE, SILENT_CODE = 500, 9      # channel 0: outside / inside the watchdog's low-energy set
CAND_VALUES = (80.0, 40.0, 20.0, 10.0)


def prompt(kind: str) -> torch.Tensor:
    """[1, 8, 33] int64: text rows, or (``"audio"``) a continuation whose last row starts audio."""
    r = np.random.default_rng(11)
    rows = np.full((8, 1 + N_VQ), AUDIO_PAD_CODE, np.int64)
    rows[:, 0] = r.integers(100, 8000, 8)
    if kind == "audio":
        rows[-1, 0] = START
        rows[3, 1:] = r.integers(0, 1024, N_VQ)
    return torch.from_numpy(rows)[None]


# ------------------------------------------------------------------------------ the cases
def _c(prompt_kind, n, audio, text, two, ch0=None, **kwargs):
    return dict(prompt=prompt_kind, n=n, audio=audio, text=text, two=two, ch0=ch0, kwargs=kwargs)


def _text_cycle(t):
    # step 0: the delay slot and im_end are masked (pre-exclusion, step 0, t <= 32); step 1: the
    # slot/end/pad tokens are pre-excluded; step 2 starts audio; afterwards im_end, masked
    # until step 33
    if t == 0:
        return [DELAY, IM_END, 5001]
    if t == 1:
        return [GEN, END, PAD, 5002]
    if t == 2:
        return [START]
    return [IM_END, 5003 + t]


CASES = {
    # text, audio start, 40 generation slots, a delay slot, the window, audio end, im_end
    "greedy_text_audio_cycle": _c("text", 100, "random", _text_cycle,
                                  lambda t: 1 if t >= 43 else 0, greedy=True),
    # continuation: the 2-way head at step 0 with the delay slot masked; a second segment
    # opened from text mode; stops at max_new_tokens
    "greedy_continuation_t0": _c("audio", 60, "random", lambda t: [START],
                                 lambda t: 1 if t == 0 or t == 10 else 0, greedy=True),
    # the repetition penalty over the history decides greedy audio codes
    "greedy_penalty": _c("audio", 50, "random", lambda t: [START],
                         lambda t: 1 if t == 30 else 0, greedy=True,
                         audio_repetition_penalty=1.3),
    # silence trigger with the threshold raised by max_requested_pause_s (5 -> 32 frames)
    "watchdog_silence_pause": _c("audio", 100, "random", lambda t: [START], lambda t: 0,
                                 lambda t: SPEECH_CODE if t < 10 else SILENT_CODE, greedy=True,
                                 watchdog_silence_frames=5, max_requested_pause_s=0.5),
    # segment bound 2 x the longest completed segment (53 frames -> 106) over a floor of 20
    "watchdog_max_segment_peak": _c("audio", 260, "random", lambda t: [START],
                                    lambda t: 1 if t == 20 else 0,
                                    lambda t: SILENT_CODE if t >= 112 else SPEECH_CODE,
                                    greedy=True, watchdog_max_segment_frames=20),
    # the floor of 60 frames holds the max-segment trigger back past 32 silent frames
    "watchdog_floor": _c("audio", 140, "random", lambda t: [START], lambda t: 0,
                         lambda t: SPEECH_CODE if t < 10 else SILENT_CODE, greedy=True,
                         watchdog_max_segment_frames=60),
    # im_end is masked through step 32 and taken at step 33
    "text_im_end_mask": _c("text", 40, "random", lambda t: [IM_END, 6000 + t], lambda t: 0,
                           greedy=True),
    # sampled text and audio (the 2-way choice through the text buffer), penalty and top-p
    "sampled_text_audio_cycle": _c("text", 90, "dominant", _text_cycle,
                                   lambda t: 1 if t >= 40 else 0, text_top_p=0.9,
                                   audio_repetition_penalty=1.3),
    # sampled 2-way at step 0 (delay slot masked in the text buffer), top-k 2
    "sampled_continuation_t0": _c("audio", 50, "dominant", lambda t: [START],
                                  lambda t: 1 if t == 0 or t >= 25 else 0, text_temperature=1.0,
                                  text_top_k=2),
}


# ------------------------------------------------------------------------------ the logits
def _bf16(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16)


class Script:
    """The head outputs of one case, step by step (CPU bf16 tensors)."""

    def __init__(self, name: str, vocab: int = TEXT_VOCAB):
        self.case = CASES[name]
        self.seed = 1000 + sorted(CASES).index(name)
        self.vocab = vocab
        r = np.random.default_rng(self.seed)
        self.text_base = r.uniform(-1.0, 1.0, vocab).astype(np.float32)

    def text(self, t: int) -> torch.Tensor:
        lt = self.text_base.copy()
        for v, tok in zip(CAND_VALUES, self.case["text"](t)):
            lt[tok] = v
        return _bf16(lt)

    def two(self, t: int) -> torch.Tensor:
        two = np.zeros(2, np.float32)
        two[self.case["two"](t)] = CAND_VALUES[0]
        return _bf16(two)

    def audio(self, t: int) -> torch.Tensor:
        r = np.random.default_rng((self.seed, t))
        if self.case["audio"] == "random":
            la = 2.0 * r.standard_normal((N_VQ, AUDIO_VOCAB)).astype(np.float32)
            top = 50.0
        else:
            la = r.uniform(-1.0, 1.0, (N_VQ, AUDIO_VOCAB)).astype(np.float32)
            la[np.arange(N_VQ), r.integers(0, AUDIO_PAD_CODE, N_VQ)] = CAND_VALUES[0]
            top = CAND_VALUES[0]
        if self.case["ch0"] is not None:
            la[0, self.case["ch0"](t)] = top + 10.0
        la[:, AUDIO_PAD_CODE] = -np.inf
        return _bf16(la)

    def heads(self, t: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        return self.text(t), self.audio(t), self.two(t)

    def checksum(self, steps: int) -> float:
        """A float64 sum over the first ``steps`` steps' logits (finite entries): ties a
        fixture to the numbers this module generates."""
        s = 0.0
        for t in range(steps):
            lt, la, two = self.heads(t)
            la = la.double()
            s += float(lt.double().sum()) + float(la[torch.isfinite(la)].sum()) + float(two.double().sum())
        return s
