"""Device-resident int4 GPTQ backbone of the decode step (Qwen3-8B-shaped stand-in).

Mirrors the state ``MossTTSModel`` owns (moss_tts_lite/model.py:46-124): embedding,
per-layer norms and projections, final norm, output head, RoPE tables and the dense
bf16 KV cache ``[layers, kv_heads, max_seq, head_dim]`` (model.py:110-112).  The
seven projections of a layer are held as four GPTQ linears: fused q|k|v, o,
gate/up interleaved in 32-column blocks (the layout the fused SiLU*up epilogue
reads), and down.
"""
from __future__ import annotations

import dataclasses
import math

import torch

from .gptq import (GPTQLinear, QszLinear, W4Dispatch, fuse_qsz_linears,
                   interleave_qsz_gate_up)

ROPE_THETA = 1_000_000.0
RMS_EPS = 1e-6
_NORMS = ("input_layernorm", "post_attention_layernorm", "q_norm", "k_norm")


@dataclasses.dataclass
class BackboneConfig:
    hidden: int = 4096
    n_heads: int = 32
    n_kv_heads: int = 8
    head_dim: int = 128
    intermediate: int = 12288
    n_layers: int = 36
    vocab: int = 151936
    group_size: int = 128
    act_order: bool = True
    rope_theta: float = ROPE_THETA
    eps: float = RMS_EPS
    max_seq: int = 2048
    # MOSS-TTS output side (moss_tts_lite/model.py:9-24, 89-101): n_vq audio codebooks,
    # each with an embedding table and a head of audio_vocab rows (pad code masked to
    # -inf), and a 2-way head made of two text-head rows.  n_vq = 0: one text head.
    n_vq: int = 0
    audio_vocab: int = 1025
    audio_pad_code: int = 1024
    two_way_ids: tuple = (151656, 151662)
    # rows of the text embedding when they differ from the head's (the reference reads
    # the two from separate tensors, model.py:60-97); None: the same as ``vocab``
    embed_vocab: int | None = None

    @property
    def text_embed_rows(self) -> int:
        return self.vocab if self.embed_vocab is None else self.embed_vocab

    @property
    def qkv_out(self) -> int:
        return (self.n_heads + 2 * self.n_kv_heads) * self.head_dim

    def validate(self) -> None:
        if self.head_dim != 128:
            raise ValueError("head_dim must be 128")
        if self.n_heads % self.n_kv_heads:
            raise ValueError("n_heads must be a multiple of n_kv_heads")
        if self.n_heads * self.head_dim != self.hidden:
            raise ValueError("hidden must equal n_heads * head_dim")
        if self.intermediate % 64 or self.hidden % self.group_size or \
                self.intermediate % self.group_size:
            raise ValueError("intermediate must be a multiple of 64 and of the group size")
        if self.n_vq:
            if not 0 <= self.audio_pad_code < self.audio_vocab:
                raise ValueError("audio_pad_code must index an audio head row")
            if len(self.two_way_ids) != 2 or not all(0 <= i < self.vocab for i in self.two_way_ids):
                raise ValueError("two_way_ids must be two text-vocabulary rows")


def moss_config(**kw) -> BackboneConfig:
    """MOSS-TTS shape: Qwen3-8B backbone, text vocabulary 155648 (model.py:14), 32 audio
    codebooks of 1025 codes (model.py:9-12)."""
    base = dict(vocab=155648, n_vq=32)
    base.update(kw)
    return BackboneConfig(**base)


def gate_up_columns_for(order: torch.Tensor, block: int = 32) -> torch.Tensor:
    """Fused gate|up column order that emits intermediate channel ``order[j]`` at j.

    Fused column of (gate, j) is ``64*(j//32) + j%32`` and of (up, j) that plus 32.
    """
    order = order.to(torch.long)
    j = torch.arange(order.numel(), device=order.device)
    new_g = 2 * block * (j // block) + j % block
    old_g = 2 * block * (order // block) + order % block
    cols = torch.empty(2 * order.numel(), dtype=torch.long, device=order.device)
    cols[new_g] = old_g
    cols[new_g + block] = old_g + block
    return cols


def rope_tables(n: int, head_dim: int, theta: float, device, dtype=torch.bfloat16):
    """cos/sin ``[n, head_dim]``: the reference's fp32 chain (model.py:115-124), computed on
    ``device`` as the reference computes it on its own device. The chain fixes the rounding:
    fp32 inverse frequencies, fp32 angles ``pos * inv`` duplicated, fp32 cos/sin, then one
    rounding to ``dtype``."""
    dev = torch.device(device)
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32, device=dev) / head_dim))
    pos = torch.arange(n, dtype=torch.float32, device=dev)
    freqs = torch.outer(pos, inv)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


class Int4Backbone:
    """Weights, caches and tables of the decoder on one device.

    Each layer's int4 projections are :class:`GPTQLinear` (AutoGPTQ buffers) or
    :class:`QszLinear` (the reference's ``(packed, qsz)`` records, see
    :func:`layers_from_dispatch`).  Two projections may stay bf16 as in the reference's
    presets (gptq.py:645-650): ``"v"`` (then ``"qkv"`` holds q|k) and ``"up"`` (then the
    layer holds ``"gate"``, an int4 linear of ``intermediate`` columns, instead of the
    interleaved ``"gate_up"``).
    """

    def __init__(self, cfg: BackboneConfig, weights: dict, device="cuda"):
        cfg.validate()
        self.cfg = cfg
        self.device = torch.device(device)
        dev = self.device

        def T(t):
            return t.to(device=dev, dtype=torch.bfloat16).contiguous()

        self.embed_tokens = T(weights["embed_tokens"])
        self.final_norm = T(weights["final_norm"])
        self.head = T(weights["head"])
        if tuple(self.embed_tokens.shape) != (cfg.text_embed_rows, cfg.hidden):
            raise ValueError(f"embed_tokens must be [{cfg.text_embed_rows}, {cfg.hidden}]")
        if tuple(self.head.shape) != (cfg.vocab, cfg.hidden):
            raise ValueError(f"head must be [{cfg.vocab}, {cfg.hidden}]")
        self.emb_ext, self.head_audio, self.head_2way = [], None, None
        if cfg.n_vq:
            self.emb_ext = [T(t) for t in weights["emb_ext"]]
            if len(self.emb_ext) != cfg.n_vq:
                raise ValueError("need one audio embedding table per codebook")
            # the 32 audio heads stacked as one [n_vq * audio_vocab, hidden] matrix
            self.head_audio = T(weights["head_audio"]).reshape(cfg.n_vq * cfg.audio_vocab,
                                                               cfg.hidden)
            self.head_2way = self.head[list(cfg.two_way_ids)].contiguous()
        self.layers = []
        for lw in weights["layers"]:
            lyr = {k: T(lw[k]) for k in _NORMS}
            up_keep = "up" in lw
            for k in ("qkv", "o", "gate" if up_keep else "gate_up", "down"):
                lin = lw[k]
                if not isinstance(lin, (GPTQLinear, QszLinear)):
                    raise TypeError(f"layer weight {k} must be a GPTQLinear or QszLinear")
                lin.post_init()
                lin.drop_original()
                lyr["gate_up" if k == "gate" else k] = lin
            # v_proj kept in bf16 (the shipped GPTQ presets, export.py:59-72): "qkv" then
            # holds q|k only and "v" the bf16 weight [kv_heads * head_dim, hidden]
            nv = cfg.n_kv_heads * cfg.head_dim
            if "v" in lw:
                v = lw["v"]
                if v.dtype != torch.bfloat16 or tuple(v.shape) != (nv, cfg.hidden):
                    raise ValueError(f"kept v must be bfloat16 [{nv}, {cfg.hidden}]")
                lyr["v_keep"] = T(v)
                if lyr["qkv"].out_features != cfg.qkv_out - nv:
                    raise ValueError("with a kept v, qkv must hold q|k only")
            elif lyr["qkv"].out_features != cfg.qkv_out:
                raise ValueError("qkv must hold q|k|v")
            perm_down = lyr["down"].perm
            if up_keep:
                # up_proj kept in bf16: "gate_up" holds the int4 gate alone; SiLU*up is a
                # separate elementwise pass, so down must read its input in natural order
                up = lw["up"]
                if up.dtype != torch.bfloat16 or tuple(up.shape) != (cfg.intermediate, cfg.hidden):
                    raise ValueError(f"kept up must be bfloat16 [{cfg.intermediate}, {cfg.hidden}]")
                if lyr["gate_up"].out_features != cfg.intermediate:
                    raise ValueError("with a kept up, gate must have intermediate columns")
                if perm_down is not None:
                    raise ValueError("a kept up needs a down projection without act-order")
                lyr["up_keep"] = T(up)
            elif lyr["gate_up"].out_features != 2 * cfg.intermediate:
                raise ValueError("gate_up must hold 2 * intermediate columns")
            # gate|up emits its SiLU*up channels already in the down projection's
            # act-order input order, so the down GEMV reads them without a gather.
            lyr["act_in_down_order"] = perm_down is not None
            if perm_down is not None:
                lyr["gate_up"].reorder_output_columns(gate_up_columns_for(perm_down))
            self.layers.append(lyr)
        self.rope_cos, self.rope_sin = rope_tables(cfg.max_seq, cfg.head_dim, cfg.rope_theta, dev)
        self.k_cache = torch.zeros(cfg.n_layers, cfg.n_kv_heads, cfg.max_seq, cfg.head_dim,
                                   dtype=torch.bfloat16, device=dev)
        self.v_cache = torch.zeros_like(self.k_cache)

    def reset_cache(self) -> None:
        self.k_cache.zero_()
        self.v_cache.zero_()

    def keep_strip_copies_only(self) -> "Int4Backbone":
        """One resident int4 copy per linear: each GPTQ linear keeps its strip copy (with
        strip-ordered metadata) and frees its AutoGPTQ and split-K copies, one linear at a
        time.  Afterwards the model runs the decode step's strip plan and the prompt-length
        GEMMs, which read only the strip copies; the other launch plans need the freed
        copies and raise ``RuntimeError`` at construction."""
        for lyr in self.layers:
            for k in ("qkv", "o", "gate_up", "down"):
                lyr[k].keep_strip_only()
        return self

    def int4_weight_bytes(self) -> int:
        """Device bytes of every resident int4 weight copy (codes, not metadata)."""
        seen, total = set(), 0
        for lyr in self.layers:
            for k in ("qkv", "o", "gate_up", "down"):
                lin = lyr[k]
                copies = ((lin.packed,) if isinstance(lin, QszLinear) else
                          (lin.qweight, lin._kernel_qweight, lin._tiled, lin._strip))
                for t in copies:
                    if t is not None and t.numel() and t.data_ptr() not in seen:
                        seen.add(t.data_ptr())
                        total += t.numel() * t.element_size()
        return total


def layers_from_dispatch(disp: W4Dispatch, norms: list[dict]) -> list[dict]:
    """Backbone layer weights from the reference's per-linear records: the
    ``(packed, qsz)`` pairs a :class:`W4Dispatch` installed (fast.py:73-121,
    gptq.py:641-697) and the bf16 weights it kept.

    q|k|v are concatenated along N, as fast_native.py:146-161 concatenates them
    (``torch.cat`` of the packed tensors on dim 0 and of the qsz on dim 1); gate and up
    are interleaved in whole 16-column strips for the SiLU*up epilogue.  v_proj and
    up_proj may be kept bf16; every other projection must be int4.  ``norms[li]`` holds
    the layer's four norm weights."""
    out = []
    for li, lw in enumerate(disp.layers):
        qd = disp.qlayers[li] or {}
        missing = [n for n in ("q", "k", "o", "gate", "down") if n not in qd]
        if missing:
            raise ValueError(f"layer {li}: {missing} must be int4 for the decode step")

        def lin(name):
            packed, qsz = qd[name]
            return QszLinear(packed, qsz, disp.group_size_map[li][name])

        layer = {k: norms[li][k] for k in _NORMS}
        if "v" in qd:
            layer["qkv"] = fuse_qsz_linears([lin("q"), lin("k"), lin("v")])
        else:
            layer["qkv"] = fuse_qsz_linears([lin("q"), lin("k")])
            layer["v"] = lw["v"]
        layer["o"] = lin("o")
        if "up" in qd:
            layer["gate_up"] = interleave_qsz_gate_up(lin("gate"), lin("up"))
        else:
            layer["gate"] = lin("gate")
            layer["up"] = lw["up"]
        layer["down"] = lin("down")
        out.append(layer)
    return out


def _random_gptq(gen, dev, k: int, n: int, g: int, perm: torch.Tensor | None) -> GPTQLinear:
    """A GPTQ linear with the benchmark distributions: nibbles uniform 0..15, scales
    U(0.002, 0.02), zero nibbles uniform 6..9, act-order g_idx from ``perm``."""
    qweight = torch.randint(-2**31, 2**31 - 1, (k // 8, n), dtype=torch.int32, device=dev,
                            generator=gen)
    scales = (torch.rand(k // g, n, device=dev, generator=gen) * 0.018 + 0.002).half()
    z = torch.randint(6, 10, (k // g, n), dtype=torch.int64, device=dev, generator=gen)
    z = z.reshape(k // g, n // 8, 8)
    zw = torch.zeros(k // g, n // 8, dtype=torch.int64, device=dev)
    for j in range(8):
        zw |= z[..., j] << (4 * j)
    qzeros = ((zw + 2**31) % 2**32 - 2**31).to(torch.int32)
    g_idx = None
    if perm is not None:
        g_idx = torch.empty(k, dtype=torch.int32, device=dev)
        g_idx[perm] = (torch.arange(k, device=dev) // g).to(torch.int32)
    return GPTQLinear.from_buffers(qweight, qzeros, scales, g_idx, g)


def random_weights(cfg: BackboneConfig, seed: int = 1234, device="cuda",
                   v_keep: bool = False) -> dict:
    """Random-init weights of the configured shape, generated on the device; with
    ``v_keep`` each layer's v_proj stays bf16 (q|k int4), as in the shipped presets."""
    dev = torch.device(device)
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    h, g = cfg.hidden, cfg.group_size

    def normal(*shape, std, rows: int = 8192):
        # drawn a block of leading rows at a time: no float32 copy of a whole table
        out = torch.empty(*shape, dtype=torch.bfloat16, device=dev)
        flat = out.view(shape[0], -1)
        for r0 in range(0, shape[0], rows):
            blk = flat[r0:r0 + rows]
            blk.copy_(torch.randn(blk.shape, device=dev, generator=gen) * std)
        return out

    def norm_w(n):
        return (1.0 + torch.randn(n, device=dev, generator=gen) * 0.05).bfloat16()

    def perm(k):
        return torch.randperm(k, device=dev, generator=gen) if cfg.act_order else None

    layers = []
    nv = cfg.n_kv_heads * cfg.head_dim
    for _ in range(cfg.n_layers):
        lw = {
            "input_layernorm": norm_w(h), "post_attention_layernorm": norm_w(h),
            "q_norm": norm_w(cfg.head_dim), "k_norm": norm_w(cfg.head_dim),
            "qkv": _random_gptq(gen, dev, h, cfg.qkv_out - (nv if v_keep else 0), g, perm(h)),
            "o": _random_gptq(gen, dev, h, h, g, perm(h)),
            "gate_up": _random_gptq(gen, dev, h, 2 * cfg.intermediate, g, perm(h)),
            "down": _random_gptq(gen, dev, cfg.intermediate, h, g, perm(cfg.intermediate)),
        }
        if v_keep:
            lw["v"] = normal(nv, h, std=0.02)
        layers.append(lw)
    out = {"embed_tokens": normal(cfg.text_embed_rows, h, std=1.0), "final_norm": norm_w(h),
           "head": normal(cfg.vocab, h, std=0.02), "layers": layers}
    if cfg.n_vq:
        out["emb_ext"] = [normal(cfg.audio_vocab, h, std=1.0) for _ in range(cfg.n_vq)]
        out["head_audio"] = normal(cfg.n_vq, cfg.audio_vocab, h, std=0.02)
    return out


def attention_scale(cfg: BackboneConfig) -> float:
    return 1.0 / math.sqrt(cfg.head_dim)
