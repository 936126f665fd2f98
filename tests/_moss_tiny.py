"""A seeded tiny MOSS-TTS model, shared by the step-fixture writer and the tests.

The model has the reference's structure (moss_tts_lite/model.py:46-112): 32 audio
codebooks with their embedding tables and heads, a text head long enough for the 2-way
rows 151656/151662, q/k RMSNorm, GQA with 4 query heads on 1 kv head (the 8B model's
ratio), head_dim 128. Only the widths are small: hidden 512, intermediate 1024, 2 layers,
and the text embedding has 8192 rows (the reference reads its row count from the table,
apart from the head's, model.py:60-97).

Every int4 linear is defined by codes, zero points and power-of-two scales:
``W[n, k] = (q[n, k] - z[g(k), n]) * 2**-e[g(k), n]``, with ``g(k)`` an act-order group
index. Those products are exact bf16 values. So one set of numbers feeds three consumers
unchanged:
- the reference's bf16 ``MossTTSModel`` (dense weights);
- the oracle (float32 ``[K, N]`` matrices);
- the device backbone (AutoGPTQ ``qweight/qzeros/scales/g_idx``, or the reference's own
  ``(codes, qsz)`` records with ``scale = s``, ``zero = (8 - z) * s``).

Nothing is stored but the seed. ``generate`` rebuilds every array from it with numpy.
"""
from __future__ import annotations

import functools

import numpy as np

from oracle import gptq_ref as G
from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits, f32_to_f16_bits

SEED = 4242
HIDDEN, N_HEADS, N_KV, HEAD_DIM = 512, 4, 1, 128
INTER, N_LAYERS, GROUP = 1024, 2, 128
TEXT_VOCAB, N_VQ, AUDIO_VOCAB, AUDIO_PAD = 151664, 32, 1025, 1024
EMBED_ROWS = 8192                    # text embedding rows (the head has TEXT_VOCAB)
TWO_WAY = (151656, 151662)           # moss_tts_lite/model.py:21-22
# the int4 linears and the input each one reads ("site": same input, same act-order)
LINEARS = {"q": ("attn_in", N_HEADS * HEAD_DIM, HIDDEN), "k": ("attn_in", N_KV * HEAD_DIM, HIDDEN),
           "v": ("attn_in", N_KV * HEAD_DIM, HIDDEN), "o": ("o_in", HIDDEN, N_HEADS * HEAD_DIM),
           "gate": ("mlp_in", INTER, HIDDEN), "up": ("mlp_in", INTER, HIDDEN),
           "down": ("down_in", HIDDEN, INTER)}
SITE_K = {"attn_in": HIDDEN, "o_in": N_HEADS * HEAD_DIM, "mlp_in": HIDDEN, "down_in": INTER}


def _bf16(x) -> np.ndarray:
    return f32_to_bf16_bits(np.asarray(x, np.float32))


def _normal_bf16(r, shape, std: float, rows: int = 4096) -> np.ndarray:
    """bf16 bits of ``std * N(0, 1)`` drawn ``rows`` leading rows at a time (small
    temporaries that the allocator reuses)."""
    out = np.empty(shape, np.uint16)
    flat = out.reshape(shape[0], -1) if len(shape) > 1 else out.reshape(-1, 1)
    for r0 in range(0, flat.shape[0], rows):
        n = min(rows, flat.shape[0] - r0)
        flat[r0:r0 + n] = _bf16(std * r.standard_normal((n, flat.shape[1]), dtype=np.float32))
    return out


@functools.lru_cache(maxsize=2)
def generate(seed: int = SEED, act_order: bool = True) -> dict:
    """Every array of the model, as numpy (bf16 tensors as uint16 bit patterns).
    ``act_order=False``: every linear's groups are contiguous runs of K (``g_idx = k // g``),
    the only form the reference's ``(codes, qsz)`` records express."""
    r = np.random.default_rng(seed)
    m = {"layers": [], "act_order": act_order}
    for _ in range(N_LAYERS):
        lyr = {
            "input_layernorm": _bf16(1.0 + 0.1 * r.standard_normal(HIDDEN)),
            "post_attention_layernorm": _bf16(1.0 + 0.1 * r.standard_normal(HIDDEN)),
            # wide q/k norm weights: the norm must come before RoPE for a match
            "q_norm": _bf16(r.uniform(0.25, 2.5, HEAD_DIM)),
            "k_norm": _bf16(r.uniform(0.25, 2.5, HEAD_DIM)),
        }
        perm = {s: r.permutation(k) for s, k in SITE_K.items()}
        for name, (site, n, k) in LINEARS.items():
            gi = G.actorder_g_idx(perm[site], GROUP) if act_order else G.trivial_g_idx(k, GROUP)
            lyr[name] = {"codes": r.integers(0, 16, (n, k), dtype=np.uint8),
                         "z": r.integers(6, 10, (k // GROUP, n), dtype=np.uint8),
                         "e": r.integers(7, 10, (k // GROUP, n), dtype=np.int32),
                         "g_idx": gi}
        m["layers"].append(lyr)
    m["final_norm"] = _bf16(1.0 + 0.1 * r.standard_normal(HIDDEN))
    m["embed_tokens"] = _normal_bf16(r, (EMBED_ROWS, HIDDEN), 1.0)
    m["emb_ext"] = _normal_bf16(r, (N_VQ * AUDIO_VOCAB, HIDDEN), 0.5).reshape(N_VQ, AUDIO_VOCAB, HIDDEN)
    m["head"] = _normal_bf16(r, (TEXT_VOCAB, HIDDEN), 0.02)
    m["head_audio"] = _normal_bf16(r, (N_VQ * AUDIO_VOCAB, HIDDEN), 0.02).reshape(
        N_VQ, AUDIO_VOCAB, HIDDEN)
    return m


def scales(lin: dict) -> np.ndarray:
    """float32 ``[K/g, N]`` scales ``2**-e`` (exact in fp16 and bf16)."""
    return np.ldexp(np.float32(1.0), -lin["e"]).astype(np.float32)


def dense_nk(lin: dict) -> np.ndarray:
    """float32 ``[N, K]`` weight (out, in) -- exact bf16 values."""
    gi = lin["g_idx"].astype(np.int64)
    z = lin["z"].astype(np.float32)[gi].T                       # [N, K]
    s = scales(lin)[gi].T
    return ((lin["codes"].astype(np.float32) - z) * s).astype(np.float32)


def gptq_buffers(lin: dict) -> dict:
    """AutoGPTQ buffers: ``qweight [K/8, N]``, ``qzeros [K/g, N/8]``, fp16 ``scales``
    bit patterns ``[K/g, N]`` and ``g_idx [K]``."""
    return {"qweight": G.pack_qweight(lin["codes"].T), "qzeros": G.pack_qzeros(lin["z"]),
            "scales": f32_to_f16_bits(scales(lin)), "g_idx": lin["g_idx"]}


def qsz_record(lin: dict) -> dict:
    """The reference's ``(codes, qsz)`` form of the same weight (gptq.py:73-97):
    codes uint8 ``[N, K]`` and qsz bf16 bits ``[K/g, N, 2]`` with scale ``s`` and zero
    ``(8 - z) * s``, so ``(q - 8) * scale + zero == (q - z) * s``. Only for linears without
    act-order: the reference's groups are contiguous runs of K."""
    if not np.array_equal(lin["g_idx"], G.trivial_g_idx(lin["codes"].shape[1], GROUP)):
        raise ValueError("the (codes, qsz) form has contiguous groups only")
    s = scales(lin)
    zero = ((8.0 - lin["z"].astype(np.float32)) * s).astype(np.float32)
    return {"q": lin["codes"], "qsz": _bf16(np.stack([s, zero], -1))}


def reference_state_dict(m: dict) -> dict:
    """Checkpoint-named float32 arrays in the reference's key scheme (model.py:60-101)."""
    f = bf16_bits_to_f32
    sd = {"language_model.embed_tokens.weight": f(m["embed_tokens"]),
          "language_model.norm.weight": f(m["final_norm"]),
          "lm_heads.0.weight": f(m["head"])}
    proj = {"q": "self_attn.q_proj", "k": "self_attn.k_proj", "v": "self_attn.v_proj",
            "o": "self_attn.o_proj", "gate": "mlp.gate_proj", "up": "mlp.up_proj",
            "down": "mlp.down_proj"}
    for i, lyr in enumerate(m["layers"]):
        p = f"language_model.layers.{i}"
        sd[f"{p}.input_layernorm.weight"] = f(lyr["input_layernorm"])
        sd[f"{p}.post_attention_layernorm.weight"] = f(lyr["post_attention_layernorm"])
        sd[f"{p}.self_attn.q_norm.weight"] = f(lyr["q_norm"])
        sd[f"{p}.self_attn.k_norm.weight"] = f(lyr["k_norm"])
        for name, key in proj.items():
            sd[f"{p}.{key}.weight"] = dense_nk(lyr[name])
    for i in range(N_VQ):
        sd[f"emb_ext.{i}.weight"] = f(m["emb_ext"][i])
        sd[f"lm_heads.{i + 1}.weight"] = f(m["head_audio"][i])
    return sd


def oracle_weights(m: dict) -> dict:
    """The oracle's weight dict (``decode_ref.moss_decode_step``): float32, ``[K, N]``."""
    f = bf16_bits_to_f32
    layers = []
    for lyr in m["layers"]:
        lw = {k: f(lyr[k]) for k in ("input_layernorm", "post_attention_layernorm", "q_norm",
                                     "k_norm")}
        lw.update({name: np.ascontiguousarray(dense_nk(lyr[name]).T) for name in LINEARS})
        layers.append(lw)
    head = f(m["head"])
    return {"embed_tokens": f(m["embed_tokens"]), "emb_ext": list(f(m["emb_ext"])),
            "final_norm": f(m["final_norm"]), "head": head, "head_audio": f(m["head_audio"]),
            "head_2way": head[list(TWO_WAY)], "layers": layers}


def backbone_config(max_seq: int = 64, act_order: bool = True, embed_rows: int = EMBED_ROWS):
    from moss_tts_lite_amd.model import BackboneConfig
    return BackboneConfig(hidden=HIDDEN, n_heads=N_HEADS, n_kv_heads=N_KV, head_dim=HEAD_DIM,
                          intermediate=INTER, n_layers=N_LAYERS, vocab=TEXT_VOCAB,
                          group_size=GROUP, act_order=act_order, max_seq=max_seq, n_vq=N_VQ,
                          audio_vocab=AUDIO_VOCAB, audio_pad_code=AUDIO_PAD, two_way_ids=TWO_WAY,
                          embed_vocab=embed_rows)


def device_backbone(m: dict, dev, max_seq: int = 64, full_text_embedding: bool = False):
    """The int4 device backbone of the same model (AutoGPTQ buffers, act-order): q|k|v
    fused along N, gate|up in the 32-column interleave.  ``full_text_embedding``: a text
    embedding of all TEXT_VOCAB rows (seeded on the device) instead of the model's 8192, so
    that the special tokens (AUDIO_START and the slots) can be fed back as ids."""
    import torch

    from moss_tts_lite_amd.gptq import GPTQLinear, fuse_gptq_linears, interleave_gate_up
    from moss_tts_lite_amd.model import Int4Backbone

    def t(a):
        return torch.from_numpy(np.ascontiguousarray(a)).to(dev)

    def bf(a):
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16)

    def lin(d):
        b = gptq_buffers(d)
        return GPTQLinear.from_buffers(t(b["qweight"]), t(b["qzeros"]),
                                       t(b["scales"].view(np.float16)), t(b["g_idx"]), GROUP)

    layers = []
    for lyr in m["layers"]:
        dl = {k: bf(lyr[k]) for k in ("input_layernorm", "post_attention_layernorm", "q_norm",
                                      "k_norm")}
        dl["qkv"] = fuse_gptq_linears([lin(lyr["q"]), lin(lyr["k"]), lin(lyr["v"])])
        dl["o"] = lin(lyr["o"])
        dl["gate_up"] = interleave_gate_up(lin(lyr["gate"]), lin(lyr["up"]))
        dl["down"] = lin(lyr["down"])
        layers.append(dl)
    w = {"embed_tokens": bf(m["embed_tokens"]), "final_norm": bf(m["final_norm"]),
         "head": bf(m["head"]), "layers": layers,
         "emb_ext": [bf(e) for e in m["emb_ext"]], "head_audio": bf(m["head_audio"])}
    rows = EMBED_ROWS
    if full_text_embedding:
        g = torch.Generator(device=dev).manual_seed(SEED)
        w["embed_tokens"] = torch.randn(TEXT_VOCAB, HIDDEN, generator=g, device=dev).bfloat16()
        rows = TEXT_VOCAB
    return Int4Backbone(backbone_config(max_seq, m["act_order"], rows), w, dev)


def dispatch_backbone(m: dict, dev, max_seq: int = 64, keep=()):
    """The same model through the reference's own per-linear records: a ``W4Dispatch``
    over the layers' dense bf16 weights with a state of ``(codes, qsz)`` records
    (:func:`qsz_record`) for every linear not in ``keep`` (the reference's bf16-keep list,
    gptq.py:645-650), assembled by ``layers_from_dispatch``. Contiguous groups only."""
    import torch

    from moss_tts_lite_amd.gptq import W4Dispatch
    from moss_tts_lite_amd.model import Int4Backbone, layers_from_dispatch

    def bf(a):
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).to(dev)

    dense = [{name: bf(_bf16(dense_nk(lyr[name]))) for name in LINEARS} for lyr in m["layers"]]
    state = {}
    for li, lyr in enumerate(m["layers"]):
        state[li] = {}
        for name in LINEARS:
            rec = qsz_record(lyr[name])
            state[li][name] = {"q": torch.from_numpy(rec["q"]),
                               "qsz": torch.from_numpy(rec["qsz"].view(np.int16)).view(torch.bfloat16)}
    disp = W4Dispatch(dense, w4_group_size=GROUP, bf16_keep=keep, state=state, device=dev)
    norms = [{k: bf(lyr[k]) for k in ("input_layernorm", "post_attention_layernorm", "q_norm",
                                      "k_norm")} for lyr in m["layers"]]
    w = {"embed_tokens": bf(m["embed_tokens"]), "final_norm": bf(m["final_norm"]),
         "head": bf(m["head"]), "layers": layers_from_dispatch(disp, norms),
         "emb_ext": [bf(e) for e in m["emb_ext"]], "head_audio": bf(m["head_audio"])}
    return Int4Backbone(backbone_config(max_seq, False), w, dev)
