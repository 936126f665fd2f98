"""Write ``tests/golden/generate_fixtures.npz``: the reference's own generation loop and
sampler, run on the CPU.

Runs in the build container only, where the reference checkout exists.  It imports
``moss_tts_lite/fast.py`` (with the ``model``, ``sampling`` and ``generate`` modules it
imports; torch only) by path under a private package name and runs:

1. ``sample_token`` (sampling.py:70-99) over a grid of the arguments the reference's tests use
   (tests/test_core.py:230-246): logits from a seeded numpy generator, ``torch.manual_seed(42)``
   before each call; stored: the tokens and ``torch.rand(3)`` drawn afterwards (the generator
   state the call leaves).
2. ``generate_fast`` (fast.py:343-610) for every case of ``tests/_generate_script.py``, over a
   CPU stand-in for ``FastMossTTS`` whose ``prefill``/``step`` return the case's scripted head
   outputs (``step`` refreshes the text or the 2-way output by its ``audio2`` flag and the
   audio output always, as the reference's captured graphs do, fast.py:174-195).  Stored per
   case: the text ids, the audio frames, ``finished``, ``n_steps``, the watchdog fields, the
   ``(pos, audio2)`` of every ``step`` call, the shapes of the ``torch.multinomial`` calls in
   order (the random stream's consumption), the prompt and a checksum of the scripted logits.

Nothing of the reference is stored.  Usage:
    python tests/golden/make_generate_fixtures.py
"""
from __future__ import annotations

import importlib
import json
import os
import sys
import types

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
REFERENCE_PACKAGE = "/root/reference/moss_tts_lite"
OUT = os.path.join(HERE, "generate_fixtures.npz")
CHECKSUM_STEPS = 6

SAMPLE_GRID = [(tk, tp, rep, dt, shape)
               for tk, tp in [(None, None), (25, 0.8), (50, 1.0), (None, 0.95), (5, None)]
               for rep in (1.0, 1.2) for dt in ("float32", "bfloat16")
               for shape in ((1, 50), (31, 1025))]


def load_reference():
    sys.dont_write_bytecode = True      # write nothing into the reference checkout
    pkg = types.ModuleType("_moss_reference")
    pkg.__path__ = [REFERENCE_PACKAGE]
    sys.modules["_moss_reference"] = pkg
    return (importlib.import_module("_moss_reference.fast"),
            importlib.import_module("_moss_reference.sampling"))


def sample_grid_logits(i: int, shape, dtype: str):
    """Logits and history of grid entry i (also rebuilt by tests/test_generate.py)."""
    import numpy as np
    import torch
    r = np.random.default_rng(500 + i)
    lg = torch.from_numpy(2.0 * r.standard_normal(shape).astype(np.float32)).to(getattr(torch, dtype))
    prev = torch.from_numpy(r.integers(0, shape[1], (1, 9, 3)))
    return lg, prev


class _Standin:
    """What ``generate_fast`` reads of a ``FastMossTTS``: ``m`` (device, cache length, the
    2-way head and the head functions of step 0), ``prefill``, ``capture``, ``step``,
    ``ids_row`` and ``lt_buf``; the heads' outputs come from the script."""

    def __init__(self, script):
        import torch
        self.script = script
        self.calls = []
        lt, la, two = script.heads(0)
        m = types.SimpleNamespace()
        m.device = torch.device("cpu")
        m.max_seq_len = 4096
        m.head_2way = torch.eye(2, dtype=torch.bfloat16)     # F.linear(h, I) == h: step 0's 2-way
        m.text_logits = lambda h: lt
        m.audio_logits = lambda h: la
        self.m = m
        self._two0 = two
        self.lt_static, self.la_static, self.two_static = lt.clone(), la.clone(), two.clone()
        self.lt_buf = torch.full((lt.shape[0],), float("-inf"), dtype=torch.bfloat16)
        self.ids_row = torch.zeros(1, 1, 33, dtype=torch.long)
        self.h_final = torch.zeros(1, 2, dtype=torch.bfloat16)

    def prefill(self, input_ids):
        return types.SimpleNamespace(last_hidden=self._two0.view(1, 1, 2))

    def capture(self):
        pass

    def step(self, row, pos, audio2=False):
        self.calls.append((int(pos), bool(audio2)))
        lt, la, two = self.script.heads(len(self.calls))
        if audio2:
            self.two_static = two
        else:
            self.lt_static = lt
        self.la_static = la
        return self.lt_static, self.la_static, self.h_final, self.two_static


def main():
    import numpy as np
    import torch

    import __graft_entry__
    __graft_entry__.import_package()
    from tests import _generate_script as S

    fast, sampling = load_reference()
    out = {}

    # 1. the sampler over the argument grid
    toks, after = [], []
    for i, (tk, tp, rep, dt, shape) in enumerate(SAMPLE_GRID):
        lg, prev = sample_grid_logits(i, shape, dt)
        torch.manual_seed(42)
        t = sampling.sample_token(lg.clone(), prev_tokens=prev, repetition_penalty=rep, top_p=tp,
                                  top_k=tk, do_sample=True)
        toks.append(np.pad(t.numpy().astype(np.int64), (0, 31 - t.numel()), constant_values=-1))
        after.append(torch.rand(3).numpy())
    out["sample_tokens"] = np.stack(toks)
    out["sample_after"] = np.stack(after)

    # 2. the generation loop, case by case
    real_multinomial = torch.multinomial
    for name in sorted(S.CASES):
        case = S.CASES[name]
        script = S.Script(name)
        dec = _Standin(script)
        draws = []

        def multinomial(p, *a, **k):
            draws.append(list(p.shape))
            return real_multinomial(p, *a, **k)

        torch.multinomial = multinomial
        try:
            res = fast.generate_fast(dec, {"input_ids": S.prompt(case["prompt"])},
                                     max_new_tokens=case["n"], seed=5, **case["kwargs"])
        finally:
            torch.multinomial = real_multinomial
        p = f"{name}/"
        out[p + "text_ids"] = res.text_ids.numpy().astype(np.int64)
        out[p + "audio_frames"] = res.audio_frames.numpy().astype(np.int64)
        out[p + "calls"] = np.array(dec.calls, np.int64).reshape(-1, 2)
        out[p + "draws"] = np.array(draws, np.int64).reshape(-1, 2)
        out[p + "prompt"] = S.prompt(case["prompt"]).numpy()
        out[p + "checksum"] = np.float64(script.checksum(CHECKSUM_STEPS))
        out[p + "result"] = np.array(json.dumps({
            "finished": bool(res.finished), "n_steps": int(res.n_steps),
            "watchdog_triggered": bool(res.watchdog_triggered),
            "watchdog_reason": res.watchdog_reason, "watchdog_stats": res.watchdog_stats}))
        text = res.text_ids.tolist()
        print(f"{name}: {res.n_steps} steps, reason {res.watchdog_reason!r}, finished {res.finished}, "
              f"{len(draws)} draws, starts {text.count(S.START)}, ends {text.count(S.END)}, "
              f"delay {text.count(S.DELAY)}, gen {text.count(S.GEN)}, im_end {text.count(S.IM_END)}")
    np.savez_compressed(OUT, **out)
    print("wrote", OUT)


if __name__ == "__main__":
    main()
