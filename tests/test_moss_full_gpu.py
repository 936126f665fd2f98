"""The MOSS-TTS decode step at the reference's full shape, on the reference's own weight
records.

Shape (moss_tts_lite/model.py:9-24): the Qwen3-8B backbone (36 layers, hidden 4096, 32/8
heads, SwiGLU 12288), the 33-way summed embedding (text 155648 rows + 32 audio tables of
1025), the text head 155648 x 4096, 32 audio heads of 1025 and the 2-way head.  Weights
(random, seeded): every int4 linear is a ``(packed, qsz)`` record of group 32 -- codes
packed by torch's own ``_convert_weight_to_int4pack`` (the reference's pack_fast,
gptq.py:66-77) and the bf16 (scale, zero) pairs -- with the bf16 keeps of the w2 preset
(every v_proj, and up_proj of layers 6, 7, 9 and 35; moss_tts_lite/export.py:59-72),
installed through ``W4Dispatch`` (gptq.py:641-697) as the reference installs them.

- 256 prompt rows on the batched prefill; then graph replay equals the eager step bit for
  bit in both head variants (text: lt, la, h_final; audio2: two, la, h_final) and in the
  KV caches (the reference's phase0 gate, tests/test_fast.py:57-93).
- Graph-replayed steps over random id rows fill the cache to position 1279; there one
  teacher-forced eager step runs layer by layer.  The embedding sum equals the oracle's
  bit for bit.  The oracle (oracle/decode_ref.py; weights from the codes and qsz the
  records were packed from, oracle/gptq_ref.effective_weight) takes each layer's input from
  the device and must match its output within rel-L2 1e-2; the final norm and the three
  heads on the device's final hidden state as well.
- The oracle also runs the step free from the embedding through all 36 layers; it is held
  to 3x the spread between two fp32 summation orders of the device (the same step with
  o, gate|up and down on other K splits: 4 instead of 8 128-channel blocks per wave, down
  16 instead of 6), and at least 1e-2: text and audio logits in relative L2, the 2-way
  head's two logits each within 3x the largest absolute spread over the text logits.
"""
import time
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest
import torch

from oracle import decode_ref as D
from oracle import gptq_ref as G

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(600)]

PROMPT, LAST, GROUP, SEED = 256, 1279, 32, 2024
NAMES = ("q", "k", "v", "o", "gate", "up", "down")
KEEP = {(li, "v") for li in range(36)} | {(li, "up") for li in (6, 7, 9, 35)}
# other K splits of the strip launches: the noise floor of fp32 summation order
FLOOR_GEOMETRY = {"o": {"nb": 4}, "gate_up": {"nb": 4}, "down": {"nb": 16}}


def fb(t):
    return t.float().cpu().numpy()


def rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


def _shapes(cfg):
    h, d = cfg.hidden, cfg.head_dim
    return {"q": (cfg.n_heads * d, h), "k": (cfg.n_kv_heads * d, h),
            "v": (cfg.n_kv_heads * d, h), "o": (h, cfg.n_heads * d),
            "gate": (cfg.intermediate, h), "up": (cfg.intermediate, h),
            "down": (h, cfg.intermediate)}


def _record(li, name, shape, dev):
    """One linear, regenerated from its seed: ``{"w": bf16 [N, K]}`` for a kept linear,
    else ``{"codes": uint8 [N, K], "qsz": bf16 [K/32, N, 2]}`` with codes uniform 0..15,
    scales U(0.002, 0.02) and zeros (8 - z) * scale, z uniform 6..9."""
    n, k = shape
    g = torch.Generator(device=dev)
    g.manual_seed(SEED + 64 * li + NAMES.index(name))
    if (li, name) in KEEP:
        return {"w": (torch.randn(n, k, device=dev, generator=g) * 0.02).bfloat16()}
    codes = torch.randint(0, 16, (n, k), dtype=torch.uint8, device=dev, generator=g)
    sc = torch.rand(k // GROUP, n, device=dev, generator=g) * 0.018 + 0.002
    z = torch.randint(6, 10, (k // GROUP, n), device=dev, generator=g)
    return {"codes": codes, "qsz": torch.stack([sc, (8 - z) * sc], -1).bfloat16()}


def _packed(codes):
    """torch's int4 tiles of the codes: the reference's pre-pack (even k in the high
    nibble, gptq.py:76) through ``_convert_weight_to_int4pack`` with 8 inner k-tiles."""
    pre = (codes[:, 1::2] | (codes[:, 0::2] << 4)).contiguous()
    return torch.ops.aten._convert_weight_to_int4pack(pre, 8)


def _host_layer(li, shapes, dev):
    out = {}
    for name, shape in shapes.items():
        rec = _record(li, name, shape, dev)
        if "w" in rec:
            out[name] = ("w", fb(rec["w"]))
        else:
            out[name] = ("q", rec["codes"].cpu().numpy(),
                         rec["qsz"].cpu().view(torch.int16).numpy().view(np.uint16))
    return out


def _oracle_layer(host, norms):
    """float64 ``[K, N]`` matrices of one layer and its norms."""
    lw = dict(norms)
    for name, rec in host.items():
        w = rec[1] if rec[0] == "w" else G.effective_weight(rec[1], rec[2], GROUP)
        lw[name] = np.ascontiguousarray(w.T, dtype=np.float64)
    return lw


def test_moss_full_shape_graph_replay_and_last_position_vs_oracle(dev):
    from moss_tts_lite_amd.fast import FastMossDecoder
    from moss_tts_lite_amd.gptq import W4Dispatch
    from moss_tts_lite_amd.model import Int4Backbone, layers_from_dispatch, moss_config

    t0 = time.time()
    cfg = moss_config(group_size=GROUP, act_order=False, max_seq=LAST + 1)
    shapes = _shapes(cfg)
    layers, state = [], {}
    for li in range(cfg.n_layers):
        lw, recs = {}, {}
        for name, shape in shapes.items():
            rec = _record(li, name, shape, dev)
            if "w" in rec:
                lw[name] = rec["w"]
            else:
                recs[name] = {"packed": _packed(rec["codes"]), "qsz": rec["qsz"]}
        layers.append(lw)
        state[li] = recs
    disp = W4Dispatch(layers, w4_group_size=GROUP, bf16_keep=sorted(KEEP), state=state, device=dev)
    del state
    gen = torch.Generator(device=dev)
    gen.manual_seed(SEED + 1)
    h = cfg.hidden

    def normal(*shape, std):
        return (torch.randn(*shape, device=dev, generator=gen) * std).bfloat16()

    def norm_w(n):
        return (1.0 + torch.randn(n, device=dev, generator=gen) * 0.05).bfloat16()

    norms = [{"input_layernorm": norm_w(h), "post_attention_layernorm": norm_w(h),
              "q_norm": norm_w(cfg.head_dim), "k_norm": norm_w(cfg.head_dim)}
             for _ in range(cfg.n_layers)]
    norms_host = [{k: fb(v) for k, v in n.items()} for n in norms]
    w = {"embed_tokens": normal(cfg.text_embed_rows, h, std=1.0), "final_norm": norm_w(h),
         "head": normal(cfg.vocab, h, std=0.02), "layers": layers_from_dispatch(disp, norms),
         "emb_ext": [normal(cfg.audio_vocab, h, std=1.0) for _ in range(cfg.n_vq)],
         "head_audio": normal(cfg.n_vq, cfg.audio_vocab, h, std=0.02)}
    del disp, layers, norms
    model = Int4Backbone(cfg, w, dev)
    del w
    dec = FastMossDecoder(model)
    g = torch.Generator().manual_seed(SEED)
    rows = torch.cat([torch.randint(0, cfg.text_embed_rows, (LAST + 1, 1), generator=g),
                      torch.randint(0, cfg.audio_vocab - 1, (LAST + 1, cfg.n_vq), generator=g)], 1)
    rows_dev = rows.to(dev)
    dec.prefill(rows[:PROMPT])
    dec.capture()
    torch.cuda.synchronize()
    print(f"MOSS full shape: built and prefilled in {time.time() - t0:.1f} s", flush=True)

    # graph replay == eager, bit for bit, from the same state, both head variants
    kv0 = (model.k_cache.clone(), model.v_cache.clone())
    variants = (False, True, True, False)
    eager = []
    for i, audio2 in enumerate(variants):
        dec.ids.copy_(rows_dev[PROMPT + i])
        dec.pos.fill_(PROMPT + i)
        dec.run_step(audio2)
        eager.append(tuple(t.clone() for t in
                           ((dec.two if audio2 else dec.lt), dec.la, dec.h_final)))
    kv_eager = (model.k_cache.clone(), model.v_cache.clone())
    model.k_cache.copy_(kv0[0])
    model.v_cache.copy_(kv0[1])
    del kv0
    for i, audio2 in enumerate(variants):
        lt, la, hf, two = dec.step(rows_dev[PROMPT + i], PROMPT + i, audio2)
        got = ((two if audio2 else lt), la, hf)
        for name, a, b in zip(("lt/two", "la", "h_final"), got, eager[i]):
            assert torch.equal(a, b), (i, audio2, name)
    assert torch.equal(model.k_cache, kv_eager[0]) and torch.equal(model.v_cache, kv_eager[1])
    del eager, kv_eager

    # graph replays over random rows up to the last position
    for p in range(PROMPT + len(variants), LAST):
        dec.step(rows_dev[p], p, audio2=bool(p % 3 == 0))
    torch.cuda.synchronize()
    kv_before = (model.k_cache.clone(), model.v_cache.clone())

    # the same step with other K splits: the noise floor of fp32 summation order
    alt = FastMossDecoder(model, strip_geometry=FLOOR_GEOMETRY)
    alt.ids.copy_(rows_dev[LAST])
    alt.pos.fill_(LAST)
    alt.run_step(False)
    alt_lt, alt_la = fb(alt.lt), fb(alt.la)
    alt.run_step(True)
    alt_two = fb(alt.two)
    model.k_cache.copy_(kv_before[0])
    model.v_cache.copy_(kv_before[1])
    del alt

    # the teacher-forced step, layer by layer
    dec.ids.copy_(rows_dev[LAST])
    dec.pos.fill_(LAST)
    dec._run(dec._embed)
    h_dev = [fb(dec.h)]
    for li in range(cfg.n_layers):
        dec.run_layer(li)
        h_dev.append(fb(dec.h))
    dec._run(dec._final_variant(False))
    lt, la, hf_dev = fb(dec.lt), fb(dec.la), fb(dec.h_final)
    dec._run(dec._final_variant(True))
    two, la2 = fb(dec.two), fb(dec.la)
    assert np.array_equal(la, la2)
    print(f"MOSS full shape: decoded to position {LAST} at {time.time() - t0:.1f} s", flush=True)

    row = rows[LAST].numpy()
    tables = [fb(model.embed_tokens[int(row[0])])[None]] + \
        [fb(model.emb_ext[j][int(row[1 + j])])[None] for j in range(cfg.n_vq)]
    h_free = D.embed_sum(np.zeros(1 + cfg.n_vq, np.int64), tables)
    assert np.array_equal(h_free, h_dev[0])

    cos, sin = D.rope_tables(cfg.max_seq, cfg.head_dim)
    layer_err = []
    with ThreadPoolExecutor(6) as pool:
        pending = {}
        for li in range(cfg.n_layers):
            for lj in range(li, min(li + 6, cfg.n_layers)):
                if lj not in pending:
                    pending[lj] = pool.submit(_oracle_layer, _host_layer(lj, shapes, dev),
                                              norms_host[lj])
            lw = pending.pop(li).result()
            kc, vc = fb(kv_before[0][li]), fb(kv_before[1][li])     # positions 0..1278
            forced = D.decoder_layer(h_dev[li], lw, kc.copy(), vc.copy(), LAST, cos, sin,
                                     cfg.n_heads, cfg.n_kv_heads, cfg.head_dim)
            layer_err.append(rel_l2(h_dev[li + 1], forced))
            h_free = D.decoder_layer(h_free, lw, kc, vc, LAST, cos, sin, cfg.n_heads,
                                     cfg.n_kv_heads, cfg.head_dim)
            del lw
            if li % 6 == 5:
                print(f"MOSS full shape oracle: layer {li} at {time.time() - t0:.1f} s, "
                      f"teacher-forced h rel_l2 {layer_err[-1]:.2e}", flush=True)

    fnorm = fb(model.final_norm)
    head_text = fb(model.head)
    head_audio = fb(model.head_audio).reshape(cfg.n_vq, cfg.audio_vocab, h)
    head_2way = fb(model.head_2way)
    pad = cfg.audio_pad_code

    def heads(hf):
        lt_o, la_o, _ = D.moss_heads(hf, head_text, head_audio, head_2way, pad, False)
        _, _, two_o = D.moss_heads(hf, head_text, head_audio[:1], head_2way, pad, True)
        return lt_o, la_o, two_o

    def audio_err(a, b):
        assert np.array_equal(np.isinf(a), np.isinf(b)) and np.all(np.isinf(b[:, pad]))
        keep = np.ones(cfg.audio_vocab, bool)
        keep[pad] = False
        return rel_l2(a[:, keep], b[:, keep])

    norm_err = rel_l2(hf_dev, D.rms_norm(h_dev[-1], fnorm))
    lt_o, la_o, two_o = heads(hf_dev)
    head_err = {"text": rel_l2(lt, lt_o), "audio": audio_err(la, la_o), "2way": rel_l2(two, two_o)}
    lt_f, la_f, two_f = heads(D.rms_norm(h_free, fnorm))
    free_err = {"text": rel_l2(lt, lt_f), "audio": audio_err(la, la_f), "2way": rel_l2(two, two_f)}
    floor = {"text": rel_l2(lt, alt_lt), "audio": audio_err(la, alt_la), "2way": rel_l2(two, alt_two)}
    print(f"MOSS full shape step at position {LAST}: per-layer teacher-forced h rel_l2 max "
          f"{max(layer_err):.2e} mean {np.mean(layer_err):.2e} (kept-up layers 6/7/9/35: "
          f"{', '.join(f'{layer_err[i]:.2e}' for i in (6, 7, 9, 35))}); final norm {norm_err:.2e}; "
          f"heads on the device's h_final: " +
          ", ".join(f"{k} {v:.2e}" for k, v in head_err.items()) +
          "; free-running: " + ", ".join(f"{k} {free_err[k]:.2e} (floor {floor[k]:.2e})"
                                         for k in free_err) +
          f"; greedy text {int(np.argmax(lt))} vs oracle {int(np.argmax(lt_f))}", flush=True)
    # The 2-way head's two logits: a relative L2 over two entries, and the floor beside it,
    # are single draws (0.129 against 0.070 and 0.146 against 0.025 on two runs of the same
    # weights, while text and audio sat at 1.2-1.4x their floors).  They are text-head rows
    # on the same final state, so each is held to 3x the largest absolute spread the two
    # summation orders give over all text logits.
    two_abs = float(np.max(np.abs(np.asarray(two, np.float64) - np.asarray(two_f, np.float64))))
    text_spread = float(np.max(np.abs(np.asarray(lt, np.float64) - np.asarray(alt_lt, np.float64))))
    print(f"MOSS full shape 2-way head, free-running: max abs error {two_abs:.3e}; largest "
          f"abs spread of the text logits between summation orders {text_spread:.3e}", flush=True)
    assert max(layer_err) < 1e-2
    assert norm_err < 1e-2
    assert all(v < 1e-2 for v in head_err.values()), head_err
    for k in ("text", "audio"):
        assert free_err[k] < max(1e-2, 3 * floor[k]), (k, free_err[k], floor[k])
    assert two_abs < 3 * text_spread, (two_abs, text_spread)
