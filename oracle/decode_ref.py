"""One batch-1 decode step of the Qwen3-shaped backbone on the CPU (oracle; test
infrastructure only).

Restates moss_tts_lite/model.py:34-44 (RMSNorm, rotate_half), 115-124 (RoPE tables),
163-197 (the layer) and fast.py:123-194 (the step pieces) in numpy.  Every bf16
tensor op of the reference computes in fp32 and rounds to bf16; the oracle does the
same at the same points.  Linear layers and attention accumulate in float64 (the
exact result the fp32 kernels approximate), then round.

Pinning: ``rms_norm`` against torch's own bf16 chain and closed-form properties;
``rope_tables`` against float64 trigonometry (<= 1 bf16 ulp); ``attention`` against a
float64 brute-force softmax and torch's CPU SDPA; see tests/test_oracle_decode.py.
The composition (``decoder_layer``, ``decode_step``, ``moss_decode_step``, ``moss_heads``)
and every piece on the reference's own operands are pinned to the reference's eager
``MossTTSModel`` run on the CPU (tests/golden/moss_step_fixtures.npz,
tests/test_oracle_step_fixture.py), with planted composition slips as negative controls.
"""
from __future__ import annotations

import numpy as np

from .bf16 import round_bf16


def rms_norm(x: np.ndarray, w: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    """Qwen3RMSNorm on bf16 values (model.py:34-40): fp32 mean of squares, then
    ``bf16(w * bf16(x * rsqrt(mean + eps)))``; reduces over the last axis."""
    x = np.asarray(x, np.float32)
    var = np.mean(x.astype(np.float64) ** 2, axis=-1, keepdims=True).astype(np.float32)
    r = (np.float32(1.0) / np.sqrt(var + np.float32(eps))).astype(np.float32)
    return round_bf16(np.asarray(w, np.float32) * round_bf16(x * r))


def rotate_half(x: np.ndarray) -> np.ndarray:
    """``cat(-x2, x1)`` over the last axis (model.py:42-44)."""
    h = x.shape[-1] // 2
    return np.concatenate([-x[..., h:], x[..., :h]], axis=-1)


def rope_tables(n: int, head_dim: int, theta: float = 1e6):
    """cos/sin ``[n, head_dim]`` as bf16 values (model.py:115-124): the fp32 chain
    ``inv = 1/theta**(2i/d)``, ``freqs = pos*inv`` duplicated, cos/sin, rounded to bf16."""
    i = np.arange(0, head_dim, 2, dtype=np.float32)
    inv = (np.float32(1.0) / np.power(np.float32(theta), i / np.float32(head_dim))).astype(np.float32)
    freqs = np.outer(np.arange(n, dtype=np.float32), inv).astype(np.float32)
    emb = np.concatenate([freqs, freqs], axis=-1)
    return round_bf16(np.cos(emb.astype(np.float64)).astype(np.float32)), \
        round_bf16(np.sin(emb.astype(np.float64)).astype(np.float32))


def apply_rope(x: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """``x*cos + rotate_half(x)*sin`` with each bf16 op rounded (fast.py:141-144)."""
    return round_bf16(round_bf16(x * cos) + round_bf16(rotate_half(x) * sin))


def linear(x: np.ndarray, w_kn: np.ndarray) -> np.ndarray:
    """bf16 output of ``x @ W`` accumulated exactly enough (float64)."""
    return round_bf16((np.asarray(x, np.float64) @ np.asarray(w_kn, np.float64)).astype(np.float32))


def attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float,
              p_bf16: bool = True) -> np.ndarray:
    """GQA decode attention: q ``[H, D]``, k/v ``[Hkv, L, D]`` -> bf16 ``[H, D]``.

    The reference calls ``F.scaled_dot_product_attention`` on bf16 tensors (model.py:183-189,
    fast.py:149-162). torch's fused kernels for that case compute fp32 scores
    ``s = (q . k) * scale``, ``e = exp(s - max s)``, round ``e`` to bf16 for the
    probability-value product and divide by the fp32 sum of the unrounded ``e``. That is
    the default form here. ``p_bf16=False`` gives the exact softmax (no rounding of ``e``).

    Pinned by torch's CPU SDPA on bf16 inputs (equal for single-block lengths), by float64
    brute force with ``p_bf16=False``, and by the special cases of a single position and
    equal scores."""
    h, d = q.shape
    hkv = k.shape[0]
    rep = h // hkv
    out = np.empty((h, d), np.float64)
    for i in range(h):
        kk = k[i // rep].astype(np.float64)
        s = ((kk @ q[i].astype(np.float64)).astype(np.float32) * np.float32(scale)).astype(np.float32)
        e = np.exp((s - s.max()).astype(np.float64)).astype(np.float32)
        p = round_bf16(e) if p_bf16 else e
        out[i] = (p.astype(np.float64) @ v[i // rep].astype(np.float64)) / e.astype(np.float64).sum()
    return round_bf16(out.astype(np.float32))


def silu_mul(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    """``F.silu(g) * u`` on bf16 tensors (fast.py:170-171)."""
    g = np.asarray(g, np.float32)
    sg = round_bf16((g / (np.float32(1.0) + np.exp(-g.astype(np.float64)).astype(np.float32))))
    return round_bf16(sg * np.asarray(u, np.float32))


def decoder_layer(h: np.ndarray, lw: dict, k_cache: np.ndarray, v_cache: np.ndarray, pos: int,
                  cos: np.ndarray, sin: np.ndarray, n_heads: int, n_kv: int, head_dim: int,
                  eps: float = 1e-6):
    """One layer at decode position ``pos`` (model.py:163-197); updates the caches in place.

    ``lw`` holds float32 weights: norms (bf16 values), ``q, k, v, o, gate, up, down`` as
    ``[K, N]`` matrices.  Returns the new residual stream (bf16 values, ``[hidden]``).
    """
    x = rms_norm(h, lw["input_layernorm"], eps)
    q = linear(x, lw["q"]).reshape(n_heads, head_dim)
    k = linear(x, lw["k"]).reshape(n_kv, head_dim)
    v = linear(x, lw["v"]).reshape(n_kv, head_dim)
    q = rms_norm(q, lw["q_norm"], eps)
    k = rms_norm(k, lw["k_norm"], eps)
    q = apply_rope(q, cos[pos], sin[pos])
    k = apply_rope(k, cos[pos], sin[pos])
    k_cache[:, pos] = k
    v_cache[:, pos] = v
    a = attention(q, k_cache[:, :pos + 1], v_cache[:, :pos + 1], 1.0 / np.sqrt(head_dim))
    h = round_bf16(h + linear(a.reshape(-1), lw["o"]))
    x = rms_norm(h, lw["post_attention_layernorm"], eps)
    act = silu_mul(linear(x, lw["gate"]), linear(x, lw["up"]))
    return round_bf16(h + linear(act, lw["down"]))


def embed_sum(ids, tables) -> np.ndarray:
    """Sum of one embedding row per table, left to right, each add a bf16 tensor op
    (model.py:156-161, fast.py:123-128): ``tables[0][ids[0]] + tables[1][ids[1]] + ...``."""
    h = np.asarray(tables[0][int(ids[0])], np.float32)
    for t, i in zip(tables[1:], ids[1:]):
        h = round_bf16(h + np.asarray(t[int(i)], np.float32))
    return h


def bf16_linear_rows(hf: np.ndarray, w: np.ndarray, chunk: int = 8192) -> np.ndarray:
    """``F.linear(hf, W)`` for a bf16 weight ``[N, K]``: float64 products, bf16 out
    (rows taken ``chunk`` at a time, so a long head needs no float64 copy of itself)."""
    x = np.asarray(hf, np.float64)
    out = np.empty(w.shape[0], np.float32)
    for r0 in range(0, w.shape[0], chunk):
        out[r0:r0 + chunk] = (np.asarray(w[r0:r0 + chunk], np.float64) @ x).astype(np.float32)
    return round_bf16(out)


def moss_heads(hf: np.ndarray, head_text, head_audio, head_2way, pad_code: int,
               audio2: bool):
    """The MOSS output heads (fast.py:174-194): text logits ``lt`` (None in the audio2
    variant), audio logits ``la [n_vq, V]`` with column ``pad_code`` set to -inf, and
    the 2-way logits (audio2 only, None otherwise)."""
    la = np.stack([bf16_linear_rows(hf, w) for w in head_audio], 0)
    la[:, pad_code] = -np.inf
    if audio2:
        return None, la, bf16_linear_rows(hf, head_2way)
    return bf16_linear_rows(hf, head_text), la, None


def moss_decode_step(row, pos: int, weights: dict, k_cache, v_cache, cos, sin, n_heads: int,
                     n_kv: int, head_dim: int, pad_code: int, audio2: bool = False,
                     eps: float = 1e-6):
    """One MOSS step (fast.py:123-194): 33-way embedding of ``row``, the layers at
    ``pos``, final norm and heads.  Returns ``(lt, la, hf, two)`` as ``FastMossTTS.step``
    (fast.py:307-325) does, with None for the head the variant skips."""
    h = embed_sum(row, [weights["embed_tokens"]] + list(weights["emb_ext"]))
    for li, lw in enumerate(weights["layers"]):
        h = decoder_layer(h, lw, k_cache[li], v_cache[li], pos, cos, sin, n_heads, n_kv,
                          head_dim, eps)
    hf = rms_norm(h, weights["final_norm"], eps)
    lt, la, two = moss_heads(hf, weights["head"], weights["head_audio"], weights["head_2way"],
                             pad_code, audio2)
    return lt, la, hf, two


def decode_step(token: int, pos: int, weights: dict, k_cache, v_cache, cos, sin, n_heads: int,
                n_kv: int, head_dim: int, eps: float = 1e-6):
    """Whole step (fast.py:123-194 with a single text head): returns
    ``(logits bf16 [vocab], final hidden, greedy token)``."""
    h = np.asarray(weights["embed_tokens"][token], np.float32)
    for li, lw in enumerate(weights["layers"]):
        h = decoder_layer(h, lw, k_cache[li], v_cache[li], pos, cos, sin, n_heads, n_kv,
                          head_dim, eps)
    hf = rms_norm(h, weights["final_norm"], eps)
    logits = bf16_linear_rows(hf, weights["head"])
    return logits, hf, int(np.argmax(logits))
