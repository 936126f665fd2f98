"""int4 weight formats and the dequant closed form (oracle; test infrastructure only).

Two weight contracts meet in the hot path:

* the reference's own ``(codes, qsz)`` contract (moss_tts_lite/gptq.py:35-97,
  fast.py:86-101): codes ``q`` uint8 ``[N, K]`` in 0..15, and ``qsz`` bf16
  ``[K/g, N, 2]`` holding ``(scale, zero)`` with ``zero = mn + 8*scale``; the
  weight is ``w[n, k] = (q - 8) * scale + zero`` in float32;
* the AutoGPTQ ``qweight/qzeros/scales/g_idx`` layout the GPTQ linear module
  carries: ``qweight`` int32 ``[K/8, N]`` with code ``k = 8*i + j`` in bits
  ``[4j, 4j+4)`` of ``qweight[i, n]`` (low nibble first), ``qzeros`` int32
  ``[K/g, N/8]`` packed the same way along N, ``scales`` fp16 ``[K/g, N]``,
  ``g_idx`` int32 ``[K]``; ``w[k, n] = (q - (z + zero_offset)) * s`` with the
  group ``g_idx[k]``.

Both are served by one device layout (``qweight [K/8, N]``); the reference's
codes are re-packed into it (``int4pack_from_prepacked``).

Pinning: see the docstring of each function and tests/test_oracle_gptq.py.
"""
from __future__ import annotations

import numpy as np

from .bf16 import bf16_bits_to_f32, f16_bits_to_f32, f32_to_bf16_bits

# ----------------------------------------------------------------------------
# The reference's (codes, qsz) contract
# ----------------------------------------------------------------------------


_FIFTEENTH = np.float32(1.0) / np.float32(15.0)


def group_scales_from_weight(w2d: np.ndarray, group_size: int = 128, divide: str = "device"):
    """Asymmetric per-(row, group) min/max statistics.

    Follows moss_tts_lite/gptq.py:35-45 (also fast.py:88-90): ``s =
    clamp((max - min) / 15.0, min=1e-6)`` in float32. Returns ``(s, mn)``, each
    float32 ``[N, K/g]``.

    torch divides a tensor by a host scalar differently per device. Its GPU kernel
    multiplies by the float32 reciprocal, ``(max - min) * fp32(1/15)``; its CPU kernel
    divides exactly. The reference quantises on the GPU (``--quant`` requires CUDA,
    cli.py:469-471), so ``divide="device"`` is the default; ``divide="cpu"`` gives torch's
    CPU result. Pinned: the CPU form against torch on the CPU; the device form against the
    reference's chain run by torch on the GPU (tests/test_gemm_gpu.py); both by brute force
    (every group's extreme elements reproduce min/max) and the clamp floor.
    """
    if divide not in ("device", "cpu"):
        raise ValueError("divide must be 'device' or 'cpu'")
    w = np.asarray(w2d, dtype=np.float32)
    n, k = w.shape
    if k % group_size:
        raise ValueError(f"K={k} not divisible by group_size={group_size}")
    wg = w.reshape(n, k // group_size, group_size)
    mx = wg.max(-1)
    mn = wg.min(-1)
    span = (mx - mn).astype(np.float32)
    s = (span * _FIFTEENTH) if divide == "device" else (span / np.float32(15.0))
    s = np.maximum(s.astype(np.float32), np.float32(1e-6)).astype(np.float32)
    return s, mn.astype(np.float32)


def rtn_quantize(w2d: np.ndarray, group_size: int = 128, divide: str = "device"):
    """Round-to-nearest int4 group quantisation.

    Follows moss_tts_lite/gptq.py:54-64 (= FastMossTTS._quantize, fast.py:86-92):
    ``q = clamp(round_half_even((w - mn) / s), 0, 15)`` with float32 subtract
    and an exact float32 divide (a tensor by a tensor). ``divide`` picks how ``s`` is
    formed (:func:`group_scales_from_weight`). Returns ``(q uint8 [N, K], s, mn)``.
    Pinned by brute force: each code is the nearest grid point of ``mn + q*s`` measured
    in the same float32 quotient (tests/test_oracle_gptq.py); and against torch on both
    devices.
    """
    w = np.asarray(w2d, dtype=np.float32)
    n, k = w.shape
    g = group_size
    s, mn = group_scales_from_weight(w, g, divide)
    wg = w.reshape(n, k // g, g)
    t = (wg - mn[..., None]) / s[..., None]
    q = np.clip(np.rint(t), 0, 15).astype(np.uint8).reshape(n, k)
    return q, s, mn


def pack_qsz(s: np.ndarray, mn: np.ndarray) -> np.ndarray:
    """``qsz`` half of the reference pack: bf16 bits ``[K/g, N, 2]``.

    Follows moss_tts_lite/gptq.py:73-74,79-85 (fast.py:94-96): the pair
    ``(s, mn + 8*s)`` computed in float32, rounded to bf16 (RNE), transposed to
    group-major.  Pinned against torch's bf16 conversion of the same float32
    pair (tests/test_oracle_gptq.py).
    """
    s = np.asarray(s, dtype=np.float32)
    mn = np.asarray(mn, dtype=np.float32)
    zero = (mn + np.float32(8.0) * s).astype(np.float32)
    pair = np.stack([s, zero], -1)                      # [N, G, 2]
    return np.ascontiguousarray(f32_to_bf16_bits(pair).transpose(1, 0, 2))


def bf16_effective_scale_zero(s: np.ndarray, mn: np.ndarray):
    """Storage-rounded scale and the implied ``min``.

    Follows moss_tts_lite/gptq.py:47-52.  Pinned by the identity
    ``effective_weight(q) == q * s_eff + mn_eff`` for ``q`` in 0..15, which
    holds exactly whenever the products are exact (tests).
    """
    s = np.asarray(s, dtype=np.float32)
    s_eff = bf16_bits_to_f32(f32_to_bf16_bits(s))
    zero = bf16_bits_to_f32(f32_to_bf16_bits((np.asarray(mn, np.float32)
                                               + np.float32(8.0) * s).astype(np.float32)))
    return s_eff, (zero - np.float32(8.0) * s_eff).astype(np.float32)


def effective_weight(q: np.ndarray, qsz: np.ndarray, group_size: int = 128) -> np.ndarray:
    """The dequant closed form of the reference's int4 contract, float32 ``[N, K]``.

    Follows moss_tts_lite/gptq.py:87-97: ``w = (q - 8) * scale + zero`` with
    ``scale, zero`` the bf16 ``qsz`` pair widened to float32.  ``(q-8)*scale``
    is exact in float32 (4-bit integer times 8-bit mantissa), so a fused or an
    unfused multiply-add give the same bits.  Pinned against torch's
    independent CPU int4 kernel ``_weight_int4pack_mm_for_cpu`` (same contract)
    and by the exact special cases q == 8 -> zero and unit steps of ``scale``.
    """
    q = np.asarray(q, dtype=np.uint8)
    n, k = q.shape
    g = group_size
    scale = bf16_bits_to_f32(qsz[:, :, 0]).T          # [N, G]
    zero = bf16_bits_to_f32(qsz[:, :, 1]).T
    qf = q.astype(np.float32).reshape(n, k // g, g)
    w = (qf - np.float32(8.0)) * scale[..., None] + zero[..., None]
    return w.reshape(n, k).astype(np.float32)


def prepack_u8(q: np.ndarray) -> np.ndarray:
    """The reference's nibble pre-pack ``uint8 [N, K/2]``: even ``k`` HIGH.

    Follows moss_tts_lite/gptq.py:76 / fast.py:98:
    ``q[:, 1::2] | (q[:, 0::2] << 4)``.  Pinned by known-answer bytes.
    """
    q = np.asarray(q, dtype=np.uint8)
    return np.ascontiguousarray((q[:, 1::2] & 0xF) | ((q[:, 0::2] & 0xF) << 4)).astype(np.uint8)


def unprepack_u8(p: np.ndarray) -> np.ndarray:
    """Inverse of :func:`prepack_u8` -> codes ``uint8 [N, K]``."""
    p = np.asarray(p, dtype=np.uint8)
    n, kh = p.shape
    q = np.empty((n, 2 * kh), dtype=np.uint8)
    q[:, 0::2] = p >> 4
    q[:, 1::2] = p & 0xF
    return q


# ----------------------------------------------------------------------------
# AutoGPTQ layout (device layout of both contracts)
# ----------------------------------------------------------------------------


def pack_qweight(codes_kn: np.ndarray) -> np.ndarray:
    """codes ``[K, N]`` (0..15) -> ``qweight`` int32 ``[K/8, N]``, low nibble first.

    Bits ``[4j, 4j+4)`` of ``qweight[i, n]`` hold the code of ``k = 8*i + j``.
    Pinned by known-answer words and pack/unpack round trips.
    """
    c = np.asarray(codes_kn, dtype=np.uint32)
    k, n = c.shape
    if k % 8:
        raise ValueError("K must be a multiple of 8")
    c = c.reshape(k // 8, 8, n)
    w = np.zeros((k // 8, n), dtype=np.uint32)
    for j in range(8):
        w |= (c[:, j, :] & np.uint32(0xF)) << np.uint32(4 * j)
    return w.view(np.int32)


def unpack_qweight(qweight: np.ndarray) -> np.ndarray:
    """Inverse of :func:`pack_qweight` -> codes uint8 ``[K, N]``."""
    w = np.ascontiguousarray(qweight).view(np.uint32)
    kq, n = w.shape
    out = np.empty((kq, 8, n), dtype=np.uint8)
    for j in range(8):
        out[:, j, :] = (w >> np.uint32(4 * j)) & np.uint32(0xF)
    return out.reshape(kq * 8, n)


def pack_qzeros(z_gn: np.ndarray) -> np.ndarray:
    """zero points ``[G, N]`` (0..15) -> ``qzeros`` int32 ``[G, N/8]`` (low nibble first along N)."""
    z = np.asarray(z_gn, dtype=np.uint32)
    g, n = z.shape
    if n % 8:
        raise ValueError("N must be a multiple of 8")
    z = z.reshape(g, n // 8, 8)
    w = np.zeros((g, n // 8), dtype=np.uint32)
    for j in range(8):
        w |= (z[:, :, j] & np.uint32(0xF)) << np.uint32(4 * j)
    return w.view(np.int32)


def unpack_qzeros(qzeros: np.ndarray) -> np.ndarray:
    """Inverse of :func:`pack_qzeros` -> uint8 ``[G, N]``."""
    w = np.ascontiguousarray(qzeros).view(np.uint32)
    g, n8 = w.shape
    out = np.empty((g, n8, 8), dtype=np.uint8)
    for j in range(8):
        out[:, :, j] = (w >> np.uint32(4 * j)) & np.uint32(0xF)
    return out.reshape(g, n8 * 8)


def trivial_g_idx(k: int, group_size: int) -> np.ndarray:
    """``g_idx`` of a checkpoint without act-order: ``k // g``."""
    return (np.arange(k, dtype=np.int64) // group_size).astype(np.int32)


def actorder_g_idx(perm: np.ndarray, group_size: int) -> np.ndarray:
    """Act-order ``g_idx``: ``g_idx[perm[r]] = r // g`` for a permutation ``perm``."""
    perm = np.asarray(perm, dtype=np.int64)
    g_idx = np.empty(perm.shape[0], dtype=np.int32)
    g_idx[perm] = (np.arange(perm.shape[0]) // group_size).astype(np.int32)
    return g_idx


def gptq_dequant(qweight, qzeros, scales_f16_bits, g_idx, group_size: int,
                 zero_offset: int = 0) -> np.ndarray:
    """AutoGPTQ dequant closed form, float32 ``[K, N]``.

    ``w[k, n] = (q[k, n] - (z[g_idx[k], n] + zero_offset)) * s[g_idx[k], n]``.
    The product is exact in float32 (5-bit integer times 11-bit mantissa).
    ``g_idx=None`` means ``k // group_size``.  Pinned by brute-force per-element
    evaluation in pure Python on small shapes and by the act-order invariance
    ``gptq_dequant(sorted layout)[perm] == gptq_dequant(original)``.
    """
    q = unpack_qweight(qweight).astype(np.float32)               # [K, N]
    k, n = q.shape
    z = unpack_qzeros(qzeros).astype(np.float32) + np.float32(zero_offset)
    s = f16_bits_to_f32(scales_f16_bits)                         # [G, N]
    gi = trivial_g_idx(k, group_size) if g_idx is None else np.asarray(g_idx, np.int64)
    return ((q - z[gi]) * s[gi]).astype(np.float32)


def actorder_sort(qweight: np.ndarray, g_idx: np.ndarray, group_size: int):
    """Group-contiguous copy of an act-order ``qweight`` plus the gather index.

    ``perm = stable_argsort(g_idx)``; row ``r`` of the sorted code matrix is row
    ``perm[r]`` of the original, so ``x[:, perm] @ W_sorted == x @ W``.  Every
    group must own exactly ``group_size`` channels.  Pinned by the invariance
    stated in :func:`gptq_dequant` (tests).
    """
    g_idx = np.asarray(g_idx, dtype=np.int64)
    k = g_idx.shape[0]
    counts = np.bincount(g_idx, minlength=k // group_size)
    if counts.shape[0] != k // group_size or np.any(counts != group_size):
        raise ValueError("every group must own exactly group_size input channels")
    perm = np.argsort(g_idx, kind="stable").astype(np.int32)
    codes = unpack_qweight(qweight)
    return pack_qweight(codes[perm]), perm


def qweight_from_reference_codes(q_nk: np.ndarray) -> np.ndarray:
    """Reference codes ``uint8 [N, K]`` -> device ``qweight`` int32 ``[K/8, N]``."""
    return pack_qweight(np.ascontiguousarray(np.asarray(q_nk, np.uint8).T))


def strip_layout(qweight: np.ndarray) -> np.ndarray:
    """``qweight [K/8, N]`` words in the build's strip order, flat uint32 ``[N*K/8]``.

    16-byte word l of 1 KB block ``(s * K/128 + b)`` holds, as its 32-bit words j = 0..3,
    the qweight words (row ``16b + 4j + l/16``, column ``16s + l%16``): column strips of 16
    over all of K, one strip a contiguous run.  K % 128 == 0, N % 16 == 0.  Pinned by a
    per-word brute force (tests/test_oracle_gptq.py).
    """
    rows, n = qweight.shape
    w = np.ascontiguousarray(qweight).view(np.uint32).reshape(rows // 16, 4, 4, n // 16, 16)
    return np.ascontiguousarray(w.transpose(3, 0, 2, 4, 1)).reshape(-1)   # s, b, l/16, l%16, j


def strip_layout_inverse(words: np.ndarray, k: int, n: int) -> np.ndarray:
    """Inverse of :func:`strip_layout`: ``qweight [K/8, N]`` (uint32 -> int32)."""
    w = np.ascontiguousarray(words).view(np.uint32).reshape(n // 16, k // 128, 4, 16, 4)
    return np.ascontiguousarray(w.transpose(1, 4, 2, 0, 3)).reshape(k // 8, n).view(np.int32)


def int4pack_from_prepacked(p_u8: np.ndarray) -> np.ndarray:
    """The reference's pre-packed ``uint8 [N, K/2]`` (even k high) -> the packed words the
    build's replacement of ``_convert_weight_to_int4pack`` (called at
    moss_tts_lite/fast.py:97, gptq.py:75) produces: the strip layout of the codes' qweight,
    flat uint32 ``[N*K/8]``.
    """
    return strip_layout(qweight_from_reference_codes(unprepack_u8(p_u8)))


def torch_tile_locate(n, k, K: int, inner_k_tiles: int):
    """(word, nibble) of code ``(n, k)`` in torch's tiled int4 tensor on ROCm.

    The tensor is what ``torch.ops.aten._convert_weight_to_int4pack(pre, T)`` returns on
    a ROCm GPU (int32 ``[N/8, K/(16T), 32, T/2]``), the ``.q`` record of the reference's
    standalone export (moss_tts_lite/export.py:324-334).  Words form 512-word blocks,
    one per (16 columns, 256 channels), the channel block the faster index.  Within a
    block, with ``r = k % 32`` (bits r4..r0) and ``j = (k % 256) // 32``: word
    ``(b * 32 + c) * T/2 + d`` with ``b = 2 * (j // (T/2)) + r3``, ``d = j % (T/2)``,
    ``c = 16 * r2 + n % 16``; nibble ``r1 | r4 << 1 | r0 << 2``.  Pinned against torch
    2.10+rocm7.0's packer on gfx950 (every nibble of separable code patterns, and the
    random-code fixtures in tests/golden).
    """
    n = np.asarray(n, np.int64)
    k = np.asarray(k, np.int64)
    half = inner_k_tiles // 2
    r = k % 32
    j = (k % 256) // 32
    b = 2 * (j // half) + ((r >> 3) & 1)
    c = 16 * ((r >> 2) & 1) + n % 16
    word = (n // 16 * (K // 256) + k // 256) * 512 + (b * 32 + c) * half + j % half
    nib = ((r >> 1) & 1) | (((r >> 4) & 1) << 1) | ((r & 1) << 2)
    return word, nib


def torch_tiles_pack(q_nk: np.ndarray, inner_k_tiles: int) -> np.ndarray:
    """Codes ``uint8 [N, K]`` -> torch's tiled int32 ``[N/8, K/(16T), 32, T/2]`` (ROCm)."""
    q = np.asarray(q_nk, np.uint8)
    n_, k_ = q.shape
    nn, kk = np.meshgrid(np.arange(n_), np.arange(k_), indexing="ij")
    word, nib = torch_tile_locate(nn.ravel(), kk.ravel(), k_, inner_k_tiles)
    out = np.zeros(n_ * k_ // 8, np.uint32)
    np.bitwise_or.at(out, word, q.ravel().astype(np.uint32) << (4 * nib).astype(np.uint32))
    t = inner_k_tiles
    return out.view(np.int32).reshape(n_ // 8, k_ // (16 * t), 32, t // 2)


def torch_tiles_unpack(tiles: np.ndarray, n_: int, k_: int, inner_k_tiles: int) -> np.ndarray:
    """torch's tiled int32 tensor (ROCm) -> codes ``uint8 [N, K]``."""
    w = np.asarray(tiles).reshape(-1).view(np.uint32)
    nn, kk = np.meshgrid(np.arange(n_), np.arange(k_), indexing="ij")
    word, nib = torch_tile_locate(nn, kk, k_, inner_k_tiles)
    return ((w[word] >> (4 * nib).astype(np.uint32)) & 0xF).astype(np.uint8)


def qsz_as_gptq_meta(qsz: np.ndarray):
    """Split reference ``qsz`` bits into float32 ``(scale [G, N], zero [G, N])``."""
    return bf16_bits_to_f32(qsz[:, :, 0]), bf16_bits_to_f32(qsz[:, :, 1])


# ----------------------------------------------------------------------------
# GEMM closed forms
# ----------------------------------------------------------------------------


def gemm_f64(x: np.ndarray, w_kn: np.ndarray) -> np.ndarray:
    """``y = x @ W`` accumulated in float64 (x ``[M, K]``, W ``[K, N]``)."""
    return np.asarray(x, np.float64) @ np.asarray(w_kn, np.float64)


def gptq_gemm(x_f32: np.ndarray, qweight, qzeros, scales_f16_bits, g_idx, group_size,
              zero_offset: int = 0) -> np.ndarray:
    """Reference GEMM of the AutoGPTQ layout: float64 ``x @ dequant(W)``."""
    return gemm_f64(x_f32, gptq_dequant(qweight, qzeros, scales_f16_bits, g_idx,
                                        group_size, zero_offset))


def int4pack_mm(x_f32: np.ndarray, q_nk: np.ndarray, qsz: np.ndarray, group_size: int) -> np.ndarray:
    """Reference GEMM of the (codes, qsz) contract: float64 ``x @ effective_weight.T``.

    This is the CPU path the reference checks its kernel against
    (tests/test_quant.py:104-107).
    """
    return gemm_f64(x_f32, effective_weight(q_nk, qsz, group_size).T)
