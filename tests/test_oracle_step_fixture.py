"""Pins the oracle's step composition (oracle/decode_ref.py: ``decoder_layer``,
``moss_decode_step``) to the reference's own eager MOSS model.

``tests/golden/moss_step_fixtures.npz`` holds the outputs of moss_tts_lite/model.py
(``MossTTSModel.prefill/step``, ``text_logits``, ``audio_logits``, ``text_logits_2way``),
run on the CPU in bf16 over the seeded tiny model of ``tests/_moss_tiny.py``. It also holds
what each layer call computes inside: its seven linear outputs and the operands and result
of its attention. Its writer is ``tests/golden/make_step_fixtures.py``. The weights are
rebuilt here from the seed.

Bars:
- Each oracle piece, run on the reference's own inputs, matches the reference bit for bit,
  up to isolated rounding flips (at most 2 elements of a vector; the float64 products and
  the order of fp32 score sums can move one value across a bf16 rounding boundary).
- The composed oracle is within rel-L2 1e-3 of the reference on every layer output, final
  hidden state and head. It is bit-exact at every hidden state of these points; the heads
  differ by accumulation order only.
- Negative controls plant one plausible slip each in a copy of the composition (norm order,
  residual source, SwiGLU operand order, final norm, RoPE position). Each must miss the
  fixture by more than 1e-2.
"""
import functools
import hashlib
import os

import numpy as np
import pytest

from oracle import decode_ref as D
from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits, round_bf16
from tests import _moss_tiny as T

FIX = os.path.join(os.path.dirname(__file__), "golden", "moss_step_fixtures.npz")
BAR = 1e-3
SLIP_BAR = 1e-2


def rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


@pytest.fixture(scope="module")
def fix():
    return dict(np.load(FIX))


@functools.lru_cache(maxsize=2)
def _ow(tag):
    return T.oracle_weights(T.generate(T.SEED, tag == "ao"))


def _run_points(fix, ow, layer=D.decoder_layer, step=D.moss_decode_step):
    """Prompt rows through ``layer`` one position at a time, then the fixture's steps
    through ``step``. Returns per point: (per-layer h of that row, hf, lt, la, two)."""
    rows, n_prompt = fix["rows"], int(fix["prompt_rows"])
    cos, sin = D.rope_tables(64, T.HEAD_DIM)
    kc = np.zeros((T.N_LAYERS, T.N_KV, 64, T.HEAD_DIM), np.float32)
    vc = np.zeros_like(kc)
    tables = [ow["embed_tokens"]] + list(ow["emb_ext"])
    for p in range(n_prompt):
        h = D.embed_sum(rows[p], tables)
        lh = []
        for li, lw in enumerate(ow["layers"]):
            h = layer(h, lw, kc[li], vc[li], p, cos, sin, T.N_HEADS, T.N_KV, T.HEAD_DIM)
            lh.append(h)
    hf = D.rms_norm(h, ow["final_norm"])
    lt, la, _ = D.moss_heads(hf, ow["head"], ow["head_audio"], ow["head_2way"], T.AUDIO_PAD, False)
    two = D.bf16_linear_rows(hf, ow["head_2way"])
    points = [(np.stack(lh), hf, lt, la, two)]
    for s in range(rows.shape[0] - n_prompt):
        p = n_prompt + s
        lt, la, hf, _ = step(rows[p], p, ow, kc, vc, cos, sin, T.N_HEADS, T.N_KV, T.HEAD_DIM,
                             T.AUDIO_PAD, False)
        two = D.bf16_linear_rows(hf, ow["head_2way"])
        points.append((None, hf, lt, la, two))
    return points


def _errors(fix, tag, points):
    f = bf16_bits_to_f32
    errs = []
    idx = fix[f"{tag}_lt_idx"]
    keep = np.arange(T.AUDIO_VOCAB) != T.AUDIO_PAD
    for i, (lh, hf, lt, la, two) in enumerate(points):
        e = {"hf": rel_l2(hf, f(fix[f"{tag}_hf"][i])),
             "lt": rel_l2(lt[idx], f(fix[f"{tag}_lt"][i])),
             "la": rel_l2(la[:, keep], f(fix[f"{tag}_la"][i])[:, keep]),
             "two": rel_l2(two, f(fix[f"{tag}_two"][i]))}
        if lh is not None:
            for li in range(T.N_LAYERS):
                e[f"layer{li}"] = rel_l2(lh[li], f(fix[f"{tag}_layer_h"][i, li]))
        errs.append(e)
    return errs


@pytest.mark.parametrize("tag", ["ao", "ct"])
def test_oracle_step_matches_reference_model(fix, tag):
    ow = _ow(tag)
    points = _run_points(fix, ow)
    errs = _errors(fix, tag, points)
    for i, e in enumerate(errs):
        print(tag, i, " ".join(f"{k}={v:.2e}" for k, v in e.items()))
        assert max(e.values()) < BAR, (i, e)
    # the pad column is -inf in both; the greedy text token agrees where it is clear
    f = bf16_bits_to_f32
    for i, (_, _, lt, la, _) in enumerate(points):
        assert np.isneginf(la[:, T.AUDIO_PAD]).all()
        assert np.isneginf(f(fix[f"{tag}_la"][i])[:, T.AUDIO_PAD]).all()
        top2 = np.sort(lt)[-2:]
        if top2[1] - top2[0] > 0.05:
            assert int(np.argmax(lt)) == int(fix[f"{tag}_lt_argmax"][i])


@pytest.mark.parametrize("tag", ["ao", "ct"])
def test_oracle_pieces_on_reference_inputs(fix, tag):
    # every piece of the layer, fed the reference's own inputs at each point's row
    ow = _ow(tag)
    f = bf16_bits_to_f32
    rows, n_prompt = fix["rows"], int(fix["prompt_rows"])
    cos, sin = D.rope_tables(64, T.HEAD_DIM)
    kc = np.zeros((T.N_LAYERS, T.N_KV, 64, T.HEAD_DIM), np.float32)
    vc = np.zeros_like(kc)
    tables = [ow["embed_tokens"]] + list(ow["emb_ext"])
    flips = {}
    for p in range(rows.shape[0]):
        h = D.embed_sum(rows[p], tables)
        pi = p - n_prompt + 1
        for li, lw in enumerate(ow["layers"]):
            if pi >= 0:
                def g(k):
                    return f(fix[f"{tag}_{k}"][pi, li])
                hin = h if li == 0 else g_prev
                x = D.rms_norm(hin, lw["input_layernorm"])
                q = D.rms_norm(g("lin_q").reshape(T.N_HEADS, -1), lw["q_norm"])
                k = D.rms_norm(g("lin_k").reshape(T.N_KV, -1), lw["k_norm"])
                kk, vv = kc[li].copy(), vc[li].copy()
                kk[:, p], vv[:, p] = g("sdpa_k"), g("sdpa_v")
                hm = round_bf16(hin + g("lin_o"))
                x2 = D.rms_norm(hm, lw["post_attention_layernorm"])
                pieces = {
                    "q": (D.linear(x, lw["q"]), g("lin_q")),
                    "k": (D.linear(x, lw["k"]), g("lin_k")),
                    "v": (D.linear(x, lw["v"]), g("lin_v")),
                    "q norm+rope": (D.apply_rope(q, cos[p], sin[p]), g("sdpa_q")),
                    "k norm+rope": (D.apply_rope(k, cos[p], sin[p]), g("sdpa_k")),
                    "attention": (D.attention(g("sdpa_q"), kk[:, :p + 1], vv[:, :p + 1],
                                              1.0 / np.sqrt(T.HEAD_DIM)), g("sdpa_a")),
                    "o": (D.linear(g("sdpa_a").reshape(-1), lw["o"]), g("lin_o")),
                    "gate": (D.linear(x2, lw["gate"]), g("lin_gate")),
                    "up": (D.linear(x2, lw["up"]), g("lin_up")),
                    "down": (D.linear(D.silu_mul(g("lin_gate"), g("lin_up")), lw["down"]),
                             g("lin_down")),
                    "residuals": (round_bf16(hm + g("lin_down")), g("layer_h")),
                }
                for name, (ours, ref) in pieces.items():
                    n = int((ours.reshape(-1) != ref.reshape(-1)).sum())
                    flips[name] = flips.get(name, 0) + n
                    assert n <= 2, (p, li, name, n)
                g_prev = g("layer_h")
            h = D.decoder_layer(h, lw, kc[li], vc[li], p, cos, sin, T.N_HEADS, T.N_KV, T.HEAD_DIM)
    print(tag, "isolated rounding flips per piece:", flips)


# -- negative controls: one slip each, planted in a copy of the composition -----------

def _layer_slip(slip):
    def layer(h, lw, k_cache, v_cache, pos, cos, sin, n_heads, n_kv, head_dim, eps=1e-6):
        x = D.rms_norm(h, lw["input_layernorm"], eps)
        q = D.linear(x, lw["q"]).reshape(n_heads, head_dim)
        k = D.linear(x, lw["k"]).reshape(n_kv, head_dim)
        v = D.linear(x, lw["v"]).reshape(n_kv, head_dim)
        rp = pos + 1 if slip == "rope position off by one" else pos
        if slip == "q/k norm after RoPE":
            q = D.rms_norm(D.apply_rope(q, cos[rp], sin[rp]), lw["q_norm"], eps)
            k = D.rms_norm(D.apply_rope(k, cos[rp], sin[rp]), lw["k_norm"], eps)
        else:
            q = D.apply_rope(D.rms_norm(q, lw["q_norm"], eps), cos[rp], sin[rp])
            k = D.apply_rope(D.rms_norm(k, lw["k_norm"], eps), cos[rp], sin[rp])
        k_cache[:, pos] = k
        v_cache[:, pos] = v
        a = D.attention(q, k_cache[:, :pos + 1], v_cache[:, :pos + 1], 1.0 / np.sqrt(head_dim))
        base = x if slip == "residual from the normed input" else h
        h = round_bf16(base + D.linear(a.reshape(-1), lw["o"]))
        x = D.rms_norm(h, lw["post_attention_layernorm"], eps)
        g, u = D.linear(x, lw["gate"]), D.linear(x, lw["up"])
        act = D.silu_mul(u, g) if slip == "SiLU on up, not gate" else D.silu_mul(g, u)
        return round_bf16(h + D.linear(act, lw["down"]))
    return layer


def _step_without_final_norm(row, pos, weights, k_cache, v_cache, cos, sin, n_heads, n_kv,
                             head_dim, pad_code, audio2=False, eps=1e-6):
    h = D.embed_sum(row, [weights["embed_tokens"]] + list(weights["emb_ext"]))
    for li, lw in enumerate(weights["layers"]):
        h = D.decoder_layer(h, lw, k_cache[li], v_cache[li], pos, cos, sin, n_heads, n_kv,
                            head_dim, eps)
    lt, la, two = D.moss_heads(h, weights["head"], weights["head_audio"], weights["head_2way"],
                               pad_code, audio2)
    return lt, la, h, two


@pytest.mark.parametrize("slip", ["q/k norm after RoPE", "residual from the normed input",
                                  "SiLU on up, not gate", "rope position off by one",
                                  "no final norm"])
def test_planted_composition_slips_miss_the_fixture(fix, slip):
    ow = _ow("ao")
    if slip == "no final norm":
        points = _run_points(fix, ow, step=_step_without_final_norm)
    else:
        points = _run_points(fix, ow, layer=_layer_slip(slip))
    worst = max(max(e.values()) for e in _errors(fix, "ao", points))
    print(f"{slip}: worst rel_l2 {worst:.2e}")
    assert worst > SLIP_BAR, slip


def test_slip_free_copy_reproduces_the_oracle_layer(fix):
    # the planted-slip copy without a slip is the oracle's layer, bit for bit
    ow = _ow("ao")
    a = _run_points(fix, ow)
    b = _run_points(fix, ow, layer=_layer_slip(None))
    for pa, pb in zip(a, b):
        np.testing.assert_array_equal(pa[1], pb[1])


# -- RoPE tables -----------------------------------------------------------------------

def reference_rope_bits(fix, name):
    """The reference's CPU tables (model.py:115-124) at 2048 positions: the oracle's
    tables with the fixture's differing entries put back, checked by their sha256."""
    cos, sin = D.rope_tables(2048, T.HEAD_DIM)
    b = f32_to_bf16_bits(cos if name == "cos" else sin).reshape(-1).copy()
    b[fix[f"rope_{name}_diff_idx"]] = fix[f"rope_{name}_diff_bits"]
    assert hashlib.sha256(b.tobytes()).hexdigest() == str(fix[f"rope_{name}_sha256"])
    return b


@pytest.mark.parametrize("name", ["cos", "sin"])
def test_oracle_rope_tables_match_reference(fix, name):
    # the oracle rounds float64 cos/sin of the fp32 angles; the reference's CPU chain uses
    # torch's fp32 cos/sin, whose range reduction is good to about |angle| * 2**-23 (the
    # angles reach 2047 rad). Equal below position 128; elsewhere one bf16 ulp apart, or
    # 2.5e-4 where a value near zero has a finer ulp than that error.
    ref = bf16_bits_to_f32(reference_rope_bits(fix, name)).reshape(2048, T.HEAD_DIM)
    cos, sin = D.rope_tables(2048, T.HEAD_DIM)
    ours = cos if name == "cos" else sin
    d = np.abs(ours - ref)
    assert np.array_equal(ours[:128], ref[:128])
    assert (d <= np.maximum(np.abs(ref) * 2.0 ** -7, 2.5e-4)).all()
    n_diff = int((d > 0).sum())
    print(f"{name}: {n_diff} of {d.size} entries differ, max {d.max():.2e}")
    assert n_diff == fix[f"rope_{name}_diff_idx"].size and n_diff < 300
