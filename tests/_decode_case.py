"""Builds one decode-step case twice from the same seeded numpy buffers: the device
``Int4Backbone`` (AutoGPTQ buffers, act-order) and the oracle's float weights."""
import numpy as np
import torch

from moss_tts_lite_amd.gptq import GPTQLinear
from moss_tts_lite_amd.model import BackboneConfig, Int4Backbone
from oracle import gptq_ref as G
from oracle import synth
from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits


def small_config(**kw) -> BackboneConfig:
    base = dict(hidden=512, n_heads=4, n_kv_heads=2, head_dim=128, intermediate=1024,
                n_layers=2, vocab=1000, group_size=128, act_order=True, max_seq=96)
    base.update(kw)
    return BackboneConfig(**base)


def _bf16_bits(r, shape, std=1.0, mean=0.0):
    return f32_to_bf16_bits((mean + std * r.standard_normal(size=shape)).astype(np.float32))


def _gptq_np(r, k, n, g, act_order):
    qweight = synth.random_qweight(r, k, n)
    scales = synth.random_scales(r, k // g, n)
    qzeros = synth.random_qzeros(r, k // g, n)
    g_idx = G.actorder_g_idx(r.permutation(k), g) if act_order else G.trivial_g_idx(k, g)
    return dict(qweight=qweight, qzeros=qzeros, scales=scales, g_idx=g_idx)


def _to_linear(d, g, dev):
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    return GPTQLinear.from_buffers(t(d["qweight"]), t(d["qzeros"]),
                                   t(d["scales"].view(np.float16)), t(d["g_idx"]), g)


def _dequant(d, g):
    return G.gptq_dequant(d["qweight"], d["qzeros"], d["scales"], d["g_idx"], g)


def gate_up_columns(inter: int):
    """Fused column index of gate[j] and up[j] in the 32-column interleave."""
    j = np.arange(inter)
    gate = (j // 32) * 64 + j % 32
    return gate, gate + 32


def build_case(cfg: BackboneConfig, seed: int, dev, v_keep: bool = False):
    """``v_keep``: each layer's v_proj stays a bf16 weight (q|k int4), as in the shipped
    GPTQ presets."""
    r = synth.rng(seed)
    h, g, hd = cfg.hidden, cfg.group_size, cfg.head_dim
    qn, kn = cfg.n_heads * hd, cfg.n_kv_heads * hd
    np_layers, dev_layers = [], []
    for _ in range(cfg.n_layers):
        norms = {k: _bf16_bits(r, n, std=0.05, mean=1.0) for k, n in
                 (("input_layernorm", h), ("post_attention_layernorm", h), ("q_norm", hd),
                  ("k_norm", hd))}
        lin = {"qkv": _gptq_np(r, h, cfg.qkv_out - (kn if v_keep else 0), g, cfg.act_order),
               "o": _gptq_np(r, h, h, g, cfg.act_order),
               "gate_up": _gptq_np(r, h, 2 * cfg.intermediate, g, cfg.act_order),
               "down": _gptq_np(r, cfg.intermediate, h, g, cfg.act_order)}
        v_bits = _bf16_bits(r, (kn, h), std=0.05) if v_keep else None
        w_qkv = _dequant(lin["qkv"], g)
        w_gu = _dequant(lin["gate_up"], g)
        gcol, ucol = gate_up_columns(cfg.intermediate)
        lw = {k: bf16_bits_to_f32(v) for k, v in norms.items()}
        lw.update(q=w_qkv[:, :qn], k=w_qkv[:, qn:qn + kn],
                  v=bf16_bits_to_f32(v_bits).T if v_keep else w_qkv[:, qn + kn:],
                  o=_dequant(lin["o"], g), gate=w_gu[:, gcol], up=w_gu[:, ucol],
                  down=_dequant(lin["down"], g))
        np_layers.append(lw)
        dl = {k: torch.from_numpy(v.view(np.int16)).view(torch.bfloat16) for k, v in norms.items()}
        dl.update({k: _to_linear(v, g, dev) for k, v in lin.items()})
        if v_keep:
            dl["v"] = torch.from_numpy(v_bits.view(np.int16)).view(torch.bfloat16).to(dev)
        dev_layers.append(dl)
    emb = _bf16_bits(r, (cfg.vocab, h), std=1.0)
    head = _bf16_bits(r, (cfg.vocab, h), std=0.02)
    fnorm = _bf16_bits(r, h, std=0.05, mean=1.0)
    t16 = lambda a: torch.from_numpy(a.view(np.int16)).view(torch.bfloat16)  # noqa: E731
    dev_w = {"embed_tokens": t16(emb), "final_norm": t16(fnorm), "head": t16(head),
             "layers": dev_layers}
    oracle_w = {"embed_tokens": bf16_bits_to_f32(emb), "final_norm": bf16_bits_to_f32(fnorm),
                "head": bf16_bits_to_f32(head), "layers": np_layers}
    if cfg.n_vq:
        ext = [_bf16_bits(r, (cfg.audio_vocab, h), std=1.0) for _ in range(cfg.n_vq)]
        ha = _bf16_bits(r, (cfg.n_vq, cfg.audio_vocab, h), std=0.02)
        dev_w.update(emb_ext=[t16(e) for e in ext], head_audio=t16(ha))
        oracle_w.update(emb_ext=[bf16_bits_to_f32(e) for e in ext],
                        head_audio=bf16_bits_to_f32(ha),
                        head_2way=bf16_bits_to_f32(head)[list(cfg.two_way_ids)])
    model = Int4Backbone(cfg, dev_w, dev)
    return model, oracle_w


def slots16(h) -> np.ndarray:
    """Sums of squares of h per 16 columns in the kernels' fixed order: four float32
    chains over 4 consecutive columns (h*h is exact for bf16 h, so the fma is an add),
    joined as (c0 + c1) + (c2 + c3)."""
    h = np.asarray(h, np.float32).reshape(-1)
    pad = np.zeros(((h.size + 15) // 16) * 16, np.float32)
    pad[:h.size] = h
    sq = pad.reshape(-1, 4, 4) ** 2                   # slot, chain, column
    c = np.zeros(sq.shape[:2], np.float32)
    for j in range(4):
        c = (c + sq[:, :, j]).astype(np.float32)
    return ((c[:, 0] + c[:, 1]) + (c[:, 2] + c[:, 3])).astype(np.float32)


def silu_mul_check(got_bits, g, u):
    """Compare SwiGLU outputs ``bf16(silu(bf16 g) * bf16 u)`` (uint16 bits) with numpy's
    correctly rounded form.  The kernels take silu from the hardware exp2 and reciprocal, so
    silu(g) may round to the other bf16 neighbour of the exact quotient where that quotient
    lies within a few fp32 ulps of a rounding boundary; the product then differs by up to
    2 bf16 ulps.  Returns (share of outputs equal bit for bit, every output equal to the
    product with silu rounded to the exact bf16 value or one of its two neighbours)."""
    rb = lambda v: bf16_bits_to_f32(f32_to_bf16_bits(np.asarray(v, np.float32)))  # noqa: E731
    g = rb(g)
    ub = rb(u)
    sg_bits = f32_to_bf16_bits((g / (np.float32(1) + np.exp(-g))).astype(np.float32)).astype(np.int64)
    got = np.asarray(got_bits).astype(np.int64)
    exact = f32_to_bf16_bits((bf16_bits_to_f32(sg_bits.astype(np.uint16)) * ub).astype(np.float32))
    ok = got == exact
    for d in (1, -1):
        nb = ((sg_bits + d) & 0xFFFF).astype(np.uint16)
        ok |= got == f32_to_bf16_bits((bf16_bits_to_f32(nb) * ub).astype(np.float32))
    return float(np.mean(got == exact)), bool(ok.all())
