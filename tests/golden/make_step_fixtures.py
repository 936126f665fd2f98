"""Write ``tests/golden/moss_step_fixtures.npz``: the reference's own eager MOSS step on the
seeded tiny model of ``tests/_moss_tiny.py``.

Runs in the build container only, where the reference checkout exists. It loads
``moss_tts_lite/model.py`` by path (it needs torch only; nothing else of the reference is
imported) and runs ``MossTTSModel`` on the CPU in bf16:
- ``prefill`` of a 6-row prompt, then ``step`` x 3 (model.py:195-233);
- after each, ``text_logits``, ``audio_logits`` and ``text_logits_2way`` (model.py:240-295).

Stored, for two versions of the model (act-order groups ``ao_``, contiguous groups ``ct_``):
- the id rows;
- the final-normed hidden state of each point;
- each layer's output at that row (``_layer`` observed through a wrapper), and inside that
  layer call the outputs of its seven ``F.linear`` calls and the operands and result of its
  ``F.scaled_dot_product_attention`` call (the roped q, the new k and v cache rows), all at
  that row;
- the 2-way and audio logits in full, and the text logits at sampled rows (the pad column of
  the audio logits is ``-inf``).

Also stored: where the reference's RoPE tables (``MossTTSModel._rope_tables`` at 2048
positions on the CPU, model.py:115-124) differ from the oracle's float64-rounded tables,
plus a sha256 of the reference tables' bits.

No weights are stored: the tests rebuild them from the seed. Usage:
    python tests/golden/make_step_fixtures.py
"""
from __future__ import annotations

import hashlib
import importlib.util
import os
import sys
import types

sys.dont_write_bytecode = True          # write nothing into the reference checkout

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
REFERENCE_MODEL = "/root/reference/moss_tts_lite/model.py"
OUT = os.path.join(HERE, "moss_step_fixtures.npz")

PROMPT_ROWS, STEPS, SAMPLED_TEXT_ROWS = 6, 3, 4096


def load_reference_model():
    spec = importlib.util.spec_from_file_location("_moss_reference_model", REFERENCE_MODEL)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[spec.name] = mod            # dataclasses resolve the module by name
    spec.loader.exec_module(mod)
    return mod


def bits(t):
    import numpy as np
    import torch
    return t.detach().to(torch.bfloat16).contiguous().view(torch.int16).numpy().view(np.uint16)


def run_model(ref, act_order: bool, rows):
    import numpy as np
    import torch

    from tests import _moss_tiny as T

    m = T.generate(T.SEED, act_order)
    sd = {k: torch.from_numpy(v).to(torch.bfloat16) for k, v in T.reference_state_dict(m).items()}
    model = ref.MossTTSModel(sd, device="cpu", dtype=torch.bfloat16, max_seq_len=64)
    # observe each layer call: its output, the seven F.linear outputs and the SDPA
    # operands and result, all at the call's last row (the point's row)
    calls = []
    inner = model._layer
    real_f = ref.F

    def linear(x, w, *a, **k):
        y = real_f.linear(x, w, *a, **k)
        if calls and "open" in calls[-1]:
            calls[-1]["lin"].append(y[0, -1].clone())
        return y

    def sdpa(q, keys, vals, *a, **k):
        y = real_f.scaled_dot_product_attention(q, keys, vals, *a, **k)
        c = calls[-1]
        c["q"], c["k"], c["v"], c["a"] = (q[0, :, -1].clone(), keys[0, 0, -1].clone(),
                                          vals[0, 0, -1].clone(), y[0, :, -1].clone())
        return y

    def observed(li, h, s0):
        calls.append({"open": True, "lin": []})
        out = inner(li, h, s0)
        del calls[-1]["open"]
        calls[-1]["out"] = out[0, -1].clone()
        return out

    shim = types.SimpleNamespace(**{n: getattr(real_f, n) for n in dir(real_f)
                                    if not n.startswith("_")})
    shim.linear, shim.scaled_dot_product_attention = linear, sdpa
    model._layer = observed
    ref.F = shim
    try:
        ids = torch.from_numpy(rows)
        points = [model.prefill(ids[None, :PROMPT_ROWS]).last_hidden[:, -1:]]
        for t in range(STEPS):
            points.append(model.step(ids[PROMPT_ROWS + t][None]).last_hidden)
    finally:
        ref.F = real_f
    hf, lt, la, two = [], [], [], []
    for h in points:
        hf.append(bits(h[0, 0]))
        lt.append(model.text_logits(h).float())
        la.append(bits(model.audio_logits(h)))
        two.append(bits(model.text_logits_2way(h)))
    n = model.n_layers
    res = {"hf": np.stack(hf), "la": np.stack(la), "two": np.stack(two)}

    def per_call(get):
        return np.stack([np.stack([get(calls[p * n + li]) for li in range(n)])
                         for p in range(len(points))])
    res["layer_h"] = per_call(lambda c: bits(c["out"]))
    for j, name in enumerate(("q", "k", "v", "o", "gate", "up", "down")):
        res[f"lin_{name}"] = per_call(lambda c, j=j: bits(c["lin"][j]))
    for name in ("q", "k", "v", "a"):
        res[f"sdpa_{name}"] = per_call(lambda c, name=name: bits(c[name]))
    return res, lt


def main() -> None:
    import numpy as np
    import torch

    from oracle import decode_ref as D
    from oracle.bf16 import f32_to_bf16_bits
    from tests import _moss_tiny as T

    if not os.path.exists(REFERENCE_MODEL):
        raise SystemExit(f"{REFERENCE_MODEL} not found: fixtures are written in the build container")
    ref = load_reference_model()
    r = np.random.default_rng(T.SEED + 1)
    n_rows = PROMPT_ROWS + STEPS
    rows = np.concatenate([r.integers(0, T.EMBED_ROWS, (n_rows, 1)),
                           r.integers(0, T.AUDIO_VOCAB, (n_rows, T.N_VQ))], 1).astype(np.int64)
    rows[2, 5] = T.AUDIO_PAD                 # a pad code among the audio ids
    out = {"rows": rows, "seed": np.int64(T.SEED), "prompt_rows": np.int64(PROMPT_ROWS),
           "torch_version": np.array(torch.__version__)}
    sample = r.choice(T.TEXT_VOCAB, SAMPLED_TEXT_ROWS, replace=False)
    for tag, act_order in (("ao", True), ("ct", False)):
        res, lt = run_model(ref, act_order, rows)
        idx = set(sample.tolist()) | set(T.TWO_WAY)
        for lg in lt:
            idx |= set(torch.topk(lg, 8).indices.tolist())
        idx = np.array(sorted(idx), dtype=np.int64)
        res["lt_idx"] = idx
        res["lt"] = np.stack([bits(lg[torch.from_numpy(idx)]) for lg in lt])
        res["lt_argmax"] = np.array([int(torch.argmax(lg)) for lg in lt], dtype=np.int64)
        for k, v in res.items():
            out[f"{tag}_{k}"] = v
    # the reference's RoPE tables vs the oracle's correctly rounded ones
    cos, sin = ref.MossTTSModel._rope_tables(2048, torch.device("cpu"), torch.bfloat16, 128)
    ocos, osin = D.rope_tables(2048, 128)
    for name, rt, ot in (("cos", cos, ocos), ("sin", sin, osin)):
        rb = bits(rt)
        ob = f32_to_bf16_bits(ot)
        diff = np.flatnonzero(rb.reshape(-1) != ob.reshape(-1))
        out[f"rope_{name}_diff_idx"] = diff.astype(np.int64)
        out[f"rope_{name}_diff_bits"] = rb.reshape(-1)[diff]
        out[f"rope_{name}_sha256"] = np.array(hashlib.sha256(rb.tobytes()).hexdigest())
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT}: {sorted(out)}")


if __name__ == "__main__":
    main()
