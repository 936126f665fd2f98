"""Seeded synthetic inputs of the benchmark workloads (oracle; test infrastructure only).

Distributions (the int4 GEMV workloads):
  x        bf16 [M, K] ~ N(0, 1)
  qweight  int32 [K/8, N], every nibble uniform in 0..15
  scales   fp16 [K/g, N] ~ U(0.002, 0.02)
  qzeros   int32 [K/g, N/8], every nibble uniform in 6..9
  g_idx    act-order: perm = permutation(K), g_idx[perm[r]] = r // g
numpy's PCG64 with the given seed; values are the build's own, not the reference's.
"""
from __future__ import annotations

import numpy as np

from . import gptq_ref as G
from .bf16 import bf16_bits_to_f32, f32_to_bf16_bits, f32_to_f16_bits


def rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def random_qweight(r: np.random.Generator, k: int, n: int) -> np.ndarray:
    return r.integers(0, 2**32, size=(k // 8, n), dtype=np.uint64).astype(np.uint32).view(np.int32)


def random_qzeros(r: np.random.Generator, groups: int, n: int, lo: int = 6, hi: int = 9) -> np.ndarray:
    z = r.integers(lo, hi + 1, size=(groups, n), dtype=np.int64).astype(np.uint8)
    return G.pack_qzeros(z)


def random_scales(r: np.random.Generator, groups: int, n: int) -> np.ndarray:
    return f32_to_f16_bits(r.uniform(0.002, 0.02, size=(groups, n)).astype(np.float32))


def random_x_bits(r: np.random.Generator, m: int, k: int) -> np.ndarray:
    return f32_to_bf16_bits(r.standard_normal(size=(m, k)).astype(np.float32))


def gptq_case(k: int, n: int, m: int = 1, group: int = 128, act_order: bool = False,
              seed: int = 1234, with_ref: bool = True, ref_cols=None) -> dict:
    """One AutoGPTQ-layout GEMM case with its float64 reference output.

    ``ref_cols`` (optional index array) limits the reference to those output
    columns (``y_ref`` then has ``len(ref_cols)`` columns).
    """
    r = rng(seed)
    qweight = random_qweight(r, k, n)
    scales = random_scales(r, k // group, n)
    qzeros = random_qzeros(r, k // group, n)
    x_bits = random_x_bits(r, m, k)
    if act_order:
        perm = r.permutation(k)
        g_idx = G.actorder_g_idx(perm, group)
    else:
        g_idx = G.trivial_g_idx(k, group)
    out = dict(qweight=qweight, scales=scales, qzeros=qzeros, x_bits=x_bits, g_idx=g_idx,
               k=k, n=n, m=m, group=group)
    if with_ref:
        x = bf16_bits_to_f32(x_bits)
        if ref_cols is None:
            out["y_ref"] = chunked_gptq_gemm(x, qweight, qzeros, scales, g_idx, group)
        else:
            cols = np.asarray(ref_cols)
            out["y_ref"] = chunked_gptq_gemm(x, qweight[:, cols], None, scales[:, cols], g_idx,
                                             group, zeros_full=G.unpack_qzeros(qzeros)[:, cols])
    return out


def chunked_gptq_gemm(x, qweight, qzeros, scales, g_idx, group, zero_offset=0, chunk=2048,
                      zeros_full=None) -> np.ndarray:
    """float64 ``x @ dequant(W)`` computed over column blocks (bounded memory)."""
    n = qweight.shape[1]
    zf = G.unpack_qzeros(qzeros) if zeros_full is None else zeros_full
    outs = []
    for c0 in range(0, n, chunk):
        c1 = min(n, c0 + chunk)
        q = G.unpack_qweight(np.ascontiguousarray(qweight[:, c0:c1])).astype(np.float32)
        z = zf[:, c0:c1].astype(np.float32) + np.float32(zero_offset)
        s = scales[:, c0:c1].view(np.float16).astype(np.float32)
        gi = np.asarray(g_idx, dtype=np.int64)
        w = (q - z[gi]) * s[gi]
        outs.append(np.asarray(x, np.float64) @ w.astype(np.float64))
    return np.concatenate(outs, axis=1)


def reference_weight(n: int, k: int, scale: float = 0.05, seed: int = 0) -> np.ndarray:
    """A smooth-ish float32 weight ``[N, K]`` (randn times a slow sine ramp)."""
    r = rng(seed)
    w = r.standard_normal(size=(n, k)).astype(np.float32) * np.float32(scale)
    ramp = (1.0 + 0.5 * np.sin(np.arange(k, dtype=np.float32) / np.float32(97.0))).astype(np.float32)
    return bf16_bits_to_f32(f32_to_bf16_bits(w * ramp))


def qsz_case(k: int, n: int, m: int = 1, group: int = 128, seed: int = 1234) -> dict:
    """One reference-contract case: RTN codes + qsz of a bf16 weight, x, reference y."""
    w = reference_weight(n, k, seed=seed)
    q, s, mn = G.rtn_quantize(w, group)
    qsz = G.pack_qsz(s, mn)
    r = rng(seed + 1)
    x_bits = random_x_bits(r, m, k)
    x = bf16_bits_to_f32(x_bits)
    y_ref = G.int4pack_mm(x, q, qsz, group)
    return dict(q=q, qsz=qsz, prepacked=G.prepack_u8(q), x_bits=x_bits, y_ref=y_ref, k=k, n=n,
                m=m, group=group)
