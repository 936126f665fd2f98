"""Torch-facing wrappers of the C ABI (device memory and streams come from torch).

Each op takes torch tensors on a HIP device, checks shapes and dtypes the way the
torch ops they replace do (``RuntimeError`` on a bad shape or group size), and
launches on ``torch.cuda.current_stream()``, so the launches are recorded when
the caller is inside ``torch.cuda.graph(...)``.

Replaced reference calls (moss_tts_lite/...):
  ``torch._weight_int4pack_mm``             fast.py:118, gptq.py:582, fast_native.py:169
  ``aten._convert_weight_to_int4pack``      fast.py:97, gptq.py:75
"""
from __future__ import annotations

import os

import torch

from . import _native as N

_MAX_M = 16
_ws_cache: dict = {}


def _ptr(t):
    return None if t is None else ctypes_ptr(t)


def ctypes_ptr(t: torch.Tensor) -> int:
    return t.data_ptr()


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _dev_index(device: torch.device) -> int:
    return device.index if device.index is not None else torch.cuda.current_device()


def reserve_workspace(device, nbytes: int) -> torch.Tensor:
    """Make sure the per-device split-K workspace holds ``nbytes``; return it.

    Call before graph capture: growing allocates.  The buffer starts zeroed and
    every GEMM launch leaves its tile counters at zero again.
    """
    device = torch.device(device)
    key = _dev_index(device)
    ws = _ws_cache.get(key)
    nbytes = max(int(nbytes), 256)
    if ws is None or ws.numel() < nbytes:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("int4 GEMM workspace must be reserved before graph capture")
        nbytes = ((nbytes + 4095) // 4096) * 4096
        ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
        N.check(N.load().mtl_workspace_init(ws.data_ptr(), nbytes, _stream(device)),
                "mtl_workspace_init")
        _ws_cache[key] = ws
    return ws


_pf_ws_cache: dict = {}


def prefill_workspace(device, m: int, k: int, n: int) -> torch.Tensor | None:
    """The per-device K-split workspace of :func:`prefill_gemm` for an ``[m, k] x [k, n]``
    product (grown on demand, outside graph capture); None when no split is needed."""
    nbytes = int(N.load().mtl_w4_gemm_prefill_workspace_bytes(m, k, n))
    if nbytes <= 0:
        return None
    device = torch.device(device)
    key = _dev_index(device)
    ws = _pf_ws_cache.get(key)
    if ws is None or ws.numel() * 4 < nbytes:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("prefill workspace must be reserved before graph capture")
        ws = torch.empty((nbytes + 3) // 4, dtype=torch.float32, device=device)
        _pf_ws_cache[key] = ws
    return ws


def gemm_workspace_bytes(m: int, k: int, n: int, group_size: int) -> int:
    return int(N.load().mtl_gemm_workspace_bytes(min(m, _MAX_M), k, n, group_size))


def _check_x(x: torch.Tensor, k: int) -> torch.Tensor:
    if x.dtype != torch.bfloat16:
        raise RuntimeError(f"expected x to be bfloat16, got {x.dtype}")
    if x.shape[-1] != k:
        raise RuntimeError(f"x has K={x.shape[-1]}, weight expects K={k}")
    if x.device.type != "cuda":
        raise RuntimeError("int4 GEMM runs on a HIP device")
    return x.reshape(-1, k).contiguous()


def w4_gemm(x2: torch.Tensor, qweight: torch.Tensor, meta_format: int, meta0: torch.Tensor,
            qzeros, perm, n: int, group_size: int, zero_offset: int = 0,
            epilogue: int = N.EPI_NONE, resid=None, out: torch.Tensor | None = None,
            out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """General launch over row chunks of at most 16: ``out[M, n or n/2]``."""
    m, k = x2.shape
    dev = x2.device
    ncols = n // 2 if epilogue == N.EPI_SILU_MUL else n
    if out is None:
        out = torch.empty(m, ncols, dtype=out_dtype, device=dev)
    odt = N.OUT_F32 if out.dtype == torch.float32 else N.OUT_BF16
    ws_need = gemm_workspace_bytes(min(m, _MAX_M), k, n, group_size)
    ws = reserve_workspace(dev, ws_need)
    lib = N.load()
    stream = _stream(dev)
    for r0 in range(0, m, _MAX_M):
        r1 = min(m, r0 + _MAX_M)
        rs = None if resid is None else resid[r0:r1]
        st = lib.mtl_w4_gemm_fused(
            x2[r0:r1].data_ptr(), r1 - r0, k, qweight.data_ptr(), meta_format, meta0.data_ptr(),
            _ptr(qzeros), _ptr(perm), n, group_size, zero_offset, epilogue,
            None if rs is None else rs.data_ptr(), out[r0:r1].data_ptr(), odt,
            ws.data_ptr(), ws.numel(), stream)
        N.check(st, "mtl_w4_gemm_fused")
    return out


def gptq_gemm(x: torch.Tensor, qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor,
              group_size: int, perm: torch.Tensor | None = None, zero_offset: int = 0,
              out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """``x[..., K] @ dequant(W)[K, N]`` for the AutoGPTQ layout (fp32 accumulation): the
    ``torch.ops.mtl.gptq_gemm`` operator over ``mtl_gptq_gemm`` (split-K, 16 rows per launch,
    the split partials in a workspace from torch's caching allocator).  ``perm`` is the
    act-order index of :func:`actorder_prepare` for a group-sorted ``qweight``.
    ``RuntimeError`` for a wrong shape, dtype or group size."""
    return torch_ops().gptq_gemm(x, qweight, qzeros, scales, group_size, perm, zero_offset,
                                 out_dtype)


def torch_ops():
    """The torch dispatcher operators of ``libmtl_torch_ops.so`` (``torch.ops.mtl``), loaded
    once after ``libmtl_hip.so``, which they call."""
    global _torch_ops_loaded
    if not _torch_ops_loaded:
        N.load()
        path = N.torch_ops_path()
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is missing: build the libraries first "
                               "(python -c 'import __graft_entry__ as g; g.build()')")
        torch.ops.load_library(path)
        _torch_ops_loaded = True
    return torch.ops.mtl


_torch_ops_loaded = False


def weight_int4pack_mm(x: torch.Tensor, packed: torch.Tensor, q_group_size: int,
                       q_scale_and_zeros: torch.Tensor) -> torch.Tensor:
    """Drop-in for ``torch._weight_int4pack_mm(x, packed, qGroupSize, qScaleAndZeros)``:
    the ``torch.ops.mtl.weight_int4pack_mm`` operator over ``mtl_int4pack_mm``.

    ``x`` bf16 ``[M, K]`` (any M); ``packed`` from :func:`convert_weight_to_int4pack` or
    :func:`int4pack_from_torch_tiles` (torch's 4-D shape, the strip layout inside:
    a concatenation along dim 0 is a concatenation along N, as with torch's tiles);
    ``qScaleAndZeros`` bf16 ``[K/g, N, 2]`` = (scale, zero) with
    ``w = (q - 8) * scale + zero`` (moss_tts_lite/gptq.py:87-97).  Returns bf16 ``[M, N]``.
    M = 1 runs the full-K strip GEMV, 2 to 16 rows the skinny strip GEMM, more
    rows the prompt-length GEMM.  ``RuntimeError`` for a wrong shape, dtype or group size,
    as torch's operator raises.
    """
    return torch_ops().weight_int4pack_mm(x, packed, q_group_size, q_scale_and_zeros)


def convert_weight_to_int4pack(prepacked: torch.Tensor, inner_k_tiles: int = 8) -> torch.Tensor:
    """Drop-in for ``aten._convert_weight_to_int4pack(uint8[N, K/2], innerKTiles)``: the
    ``torch.ops.mtl.convert_weight_to_int4pack`` operator over ``mtl_int4pack_convert``.

    Input is the reference's nibble pre-pack (even k in the high nibble,
    moss_tts_lite/fast.py:98).  Output has torch's shape ``[N/8, K/(16 T), 32, T/2]`` int32
    and holds the strip layout, not torch's tiled bytes: 16-column strips over all
    of K, each one contiguous, so ``torch.cat(..., dim=0)`` of two packed weights is the
    packed concatenation of the weights along N (moss_tts_lite/fast_native.py:158-159).
    K % 256 == 0 and N % 16 == 0.
    """
    return torch_ops().convert_weight_to_int4pack(prepacked, inner_k_tiles)


def int4pack_from_torch_tiles(tiles: torch.Tensor) -> torch.Tensor:
    """torch's tiled int4 tensor -> the strip-layout packed weight (mtl_int4pack_from_torch_tiles),
    in the same ``[N/8, K/(16T), 32, T/2]`` shape.

    ``tiles`` is int32 ``[N/8, K/(16T), 32, T/2]`` as ``aten._convert_weight_to_int4pack(pre,
    T)`` returns it on a ROCm GPU: the ``.q`` records of the reference's standalone export
    (moss_tts_lite/export.py:324-334).  N must be a multiple of 16 and K of 256.
    """
    if tiles.dtype != torch.int32 or tiles.dim() != 4 or tiles.shape[2] != 32:
        raise RuntimeError("expected torch's int32 [N/8, K/(16*T), 32, T/2] int4 tiles")
    t = 2 * tiles.shape[3]
    n, k = tiles.shape[0] * 8, tiles.shape[1] * 16 * t
    if t not in (2, 4, 8):
        raise RuntimeError("innerKTiles must be 2, 4 or 8")
    if n % 16 or k % 256:
        raise RuntimeError(f"N={n} must be a multiple of 16 and K={k} a multiple of 256")
    if tiles.device.type != "cuda":
        raise RuntimeError("int4 tiles must be on the GPU")
    src = tiles.contiguous()
    out = torch.empty_like(src)
    N.check(N.load().mtl_int4pack_from_torch_tiles(src.data_ptr(), n, k, t, out.data_ptr(),
                                                   _stream(src.device)),
            "mtl_int4pack_from_torch_tiles")
    return out


def tile_weights(qweight: torch.Tensor) -> torch.Tensor:
    """Wave-contiguous copy of ``qweight [K/8, N]`` for the decode-step GEMVs
    (``mtl_w4_tile``); N must be a multiple of 64."""
    if qweight.dtype != torch.int32 or qweight.dim() != 2:
        raise RuntimeError("qweight must be int32 [K/8, N]")
    k, n = qweight.shape[0] * 8, qweight.shape[1]
    lib = N.load()
    nbytes = int(lib.mtl_w4_tiled_bytes(k, n))
    if nbytes <= 0:
        raise RuntimeError(f"no tiled layout for K={k}, N={n} (N must be a multiple of 64)")
    src = qweight.contiguous()
    out = torch.empty(nbytes // 4, dtype=torch.int32, device=src.device)
    N.check(lib.mtl_w4_tile(src.data_ptr(), k, n, out.data_ptr(), nbytes, _stream(src.device)),
            "mtl_w4_tile")
    return out


def strip_weights(qweight: torch.Tensor) -> torch.Tensor:
    """Column-strip copy of ``qweight [K/8, N]`` for the full-K strip GEMV
    (``mtl_w4_strip``); N must be a multiple of 16 and K of 256."""
    if qweight.dtype != torch.int32 or qweight.dim() != 2:
        raise RuntimeError("qweight must be int32 [K/8, N]")
    k, n = qweight.shape[0] * 8, qweight.shape[1]
    lib = N.load()
    nbytes = int(lib.mtl_w4_strip_bytes(k, n))
    if nbytes <= 0:
        raise RuntimeError(f"no strip layout for K={k}, N={n} (N % 16 == 0 and K % 256 == 0)")
    src = qweight.contiguous()
    out = torch.empty(nbytes // 4, dtype=torch.int32, device=src.device)
    N.check(lib.mtl_w4_strip(src.data_ptr(), k, n, out.data_ptr(), nbytes, _stream(src.device)),
            "mtl_w4_strip")
    return out


def strip_meta(scales: torch.Tensor, qzeros: torch.Tensor, group_size: int):
    """Strip-ordered copies of ``scales [K/g, N]`` (fp16) and ``qzeros [K/g, N/8]`` for the
    strip GEMV (``mtl_w4_strip_meta``); same sizes as the inputs."""
    if scales.dtype != torch.float16 or qzeros.dtype != torch.int32:
        raise RuntimeError("scales must be float16 and qzeros int32")
    g, n = scales.shape
    k = g * group_size
    sc = torch.empty_like(scales)
    qz = torch.empty_like(qzeros)
    N.check(N.load().mtl_w4_strip_meta(scales.contiguous().data_ptr(), qzeros.contiguous().data_ptr(),
                                       k, n, group_size, sc.data_ptr(), qz.data_ptr(),
                                       _stream(scales.device)), "mtl_w4_strip_meta")
    return sc, qz


def strip_rows_pays(m: int, k: int, n: int, gathered: bool = False) -> bool:
    """Whether the skinny strip GEMM beats the split-K GEMM for ``m`` rows of a ``k x n``
    product on MI355X.  Without the act-order gather it does at every m <= 16 on the four
    decode shapes (measured: q|k|v 6.3-8.3 against 8.7-10.6 us, down 9.6-15.0 against
    14.3-16.7).  With the gather, every workgroup gathers all m * k channels: from x's
    rows held in LDS, which they fit at m * k <= 32768, or else from memory, two bytes per
    load, which pays only on a wide product (n >= 6 k: gate|up).  Measured with the gather:
    q|k|v and o ahead up to m = 8 (q|k|v 9.4 against 12.5 us at m = 8, 20.1 against 14.0 at
    m = 12), gate|up at every m <= 16 (31.3 against 33.7 us at 16), down to m = 4."""
    if m < 1 or m > _MAX_M:
        return False
    return not gathered or m * k <= 32768 or n >= 6 * k


def strip_rows_gemm(x: torch.Tensor, strip_weight: torch.Tensor, qzeros: torch.Tensor,
                    scales: torch.Tensor, n: int, group_size: int, zero_offset: int = 0,
                    out: torch.Tensor | None = None,
                    out_dtype: torch.dtype = torch.bfloat16,
                    perm: torch.Tensor | None = None) -> torch.Tensor:
    """Skinny-batch GEMM over the strip layout (``mtl_w4_gemm_strip_rows_ex``): ``x [M, K]``
    bf16 with M <= 16 rows per launch (longer inputs run in 16-row chunks), AutoGPTQ
    ``scales``/``qzeros``, group 32, 64, 128 or 256; ``perm`` (int32 [K], the act-order
    index of :func:`actorder_prepare`) gathers x's channels into the weight's row order.
    Returns ``[M, n]``."""
    if perm is not None and (perm.dtype != torch.int32 or perm.numel() != x.shape[-1]):
        raise RuntimeError("perm must be int32 [K]")
    return _strip_rows(x, strip_weight, scales, qzeros, n, group_size, zero_offset,
                       N.META_GPTQ, perm, out, out_dtype)


def strip_gemv(x: torch.Tensor, strip_weight: torch.Tensor, strip_scales: torch.Tensor,
               strip_zeros: torch.Tensor, n: int, group_size: int, zero_offset: int = 0,
               perm: torch.Tensor | None = None,
               out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """One row on the full-K strip GEMV (``mtl_w4_gemv_strip``, through the ``mtl::strip_gemv``
    operator): ``x [..., K]`` with one row, the strip copy of a GPTQ linear and its
    strip-ordered metadata (:func:`strip_weights`, :func:`strip_meta`), x gathered through
    ``perm`` (int16 [K]: :func:`actorder_prepare`'s index narrowed, K <= 12288) while
    staging.  Returns ``[..., n]``."""
    return torch_ops().strip_gemv(x, strip_weight, strip_scales, strip_zeros, n, group_size,
                                  zero_offset, perm, out_dtype)


def strip_rows_qsz(x: torch.Tensor, packed: torch.Tensor, qsz: torch.Tensor, group_size: int,
                   out: torch.Tensor | None = None,
                   out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """The skinny-batch strip GEMM on the reference's own records: ``packed`` from
    :func:`convert_weight_to_int4pack` and ``qsz`` bf16 ``[K/g, N, 2]``; ``x [M, K]``."""
    return _strip_rows(x, packed, qsz, None, qsz.shape[1], group_size, 0, N.META_QSZ, None,
                       out, out_dtype)


def _strip_rows(x, strip_weight, meta, qzeros, n, group_size, zero_offset, meta_format, perm,
                out, out_dtype):
    x2 = _check_x(x, x.shape[-1])
    m, k = x2.shape
    if out is None:
        out = torch.empty(m, n, dtype=out_dtype, device=x2.device)
    odt = N.OUT_F32 if out.dtype == torch.float32 else N.OUT_BF16
    lib = N.load()
    stream = _stream(x2.device)
    for r0 in range(0, m, _MAX_M):
        r1 = min(m, r0 + _MAX_M)
        N.check(lib.mtl_w4_gemm_strip_rows_ex(
            x2[r0:r1].data_ptr(), r1 - r0, k, k, _ptr(perm), strip_weight.data_ptr(),
            meta.data_ptr(), _ptr(qzeros), n, group_size, zero_offset, meta_format,
            out[r0:r1].data_ptr(), n, odt, stream),
            "mtl_w4_gemm_strip_rows_ex")
    return out


_PREFILL_EPI = {"none": 0, "residual": 1, "silu_mul": 2}


def prefill_gemm(x: torch.Tensor, strip_weight: torch.Tensor, strip_scales: torch.Tensor,
                 strip_zeros: torch.Tensor, n: int, group_size: int, zero_offset: int = 0,
                 epilogue: str = "none", out: torch.Tensor | None = None,
                 out_dtype: torch.dtype = torch.bfloat16, split: bool = True) -> torch.Tensor:
    """Prompt-length int4 GEMM over the strip layout (``mtl_w4_gemm_prefill``): ``x [M, K]``
    bf16 (any M, channels in the weight's input order) times the strip copy of a linear
    with its strip-ordered metadata.  ``epilogue``: ``"none"`` returns ``[M, n]``
    (``out_dtype``); ``"residual"`` adds into ``out`` (bf16 ``[M, n]``, the residual
    stream) in place; ``"silu_mul"`` returns bf16 ``[M, n/2]`` = SiLU(gate) * up of the
    32-column gate|up interleave.  ``split``: let a small grid split K over workgroups
    (per-device workspace); False runs one pass."""
    if epilogue not in _PREFILL_EPI:
        raise ValueError(f"epilogue must be one of {tuple(_PREFILL_EPI)}")
    x2 = _check_x(x, x.shape[-1])
    m, k = x2.shape
    cols = n // 2 if epilogue == "silu_mul" else n
    if out is None:
        if epilogue == "residual":
            raise RuntimeError("the residual epilogue updates `out` in place")
        out = torch.empty(m, cols, dtype=out_dtype if epilogue == "none" else torch.bfloat16,
                          device=x2.device)
    if out.dim() != 2 or out.shape[0] != m or out.shape[1] < cols or out.stride(1) != 1:
        raise RuntimeError(f"out must be [{m}, >= {cols}] with unit column stride")
    odt = N.OUT_F32 if out.dtype == torch.float32 else N.OUT_BF16
    ws = prefill_workspace(x2.device, m, k, n) if split else None
    N.check(N.load().mtl_w4_gemm_prefill(
        x2.data_ptr(), m, x2.stride(0), k, strip_weight.data_ptr(), strip_scales.data_ptr(),
        strip_zeros.data_ptr(), n, group_size, zero_offset, _PREFILL_EPI[epilogue], odt,
        out.data_ptr(), out.stride(0), None if ws is None else ws.data_ptr(),
        0 if ws is None else ws.numel() * 4, _stream(x2.device)), "mtl_w4_gemm_prefill")
    return out


def prefill_gemm_qsz(x: torch.Tensor, packed: torch.Tensor, qsz: torch.Tensor, group_size: int,
                     epilogue: str = "none", out: torch.Tensor | None = None,
                     out_dtype: torch.dtype = torch.bfloat16, split: bool = True) -> torch.Tensor:
    """:func:`prefill_gemm` on the reference's own contract (``mtl_w4_gemm_prefill_qsz``):
    ``packed`` from :func:`convert_weight_to_int4pack` / :func:`int4pack_from_torch_tiles`,
    ``qsz`` bf16 ``[K/g, N, 2]`` read in place (``w = (q - 8) * scale + zero``)."""
    if epilogue not in _PREFILL_EPI:
        raise ValueError(f"epilogue must be one of {tuple(_PREFILL_EPI)}")
    if qsz.dtype != torch.bfloat16 or qsz.dim() != 3 or qsz.shape[2] != 2:
        raise RuntimeError("qsz must be bfloat16 [K/g, N, 2]")
    k, n = qsz.shape[0] * group_size, qsz.shape[1]
    x2 = _check_x(x, k)
    m = x2.shape[0]
    cols = n // 2 if epilogue == "silu_mul" else n
    if out is None:
        if epilogue == "residual":
            raise RuntimeError("the residual epilogue updates `out` in place")
        out = torch.empty(m, cols, dtype=out_dtype if epilogue == "none" else torch.bfloat16,
                          device=x2.device)
    if out.dim() != 2 or out.shape[0] != m or out.shape[1] < cols or out.stride(1) != 1:
        raise RuntimeError(f"out must be [{m}, >= {cols}] with unit column stride")
    odt = N.OUT_F32 if out.dtype == torch.float32 else N.OUT_BF16
    ws = prefill_workspace(x2.device, m, k, n) if split else None
    N.check(N.load().mtl_w4_gemm_prefill_qsz(
        x2.data_ptr(), m, x2.stride(0), k, packed.data_ptr(), qsz.contiguous().data_ptr(), n,
        group_size, _PREFILL_EPI[epilogue], odt, out.data_ptr(), out.stride(0),
        None if ws is None else ws.data_ptr(), 0 if ws is None else ws.numel() * 4,
        _stream(x2.device)), "mtl_w4_gemm_prefill_qsz")
    return out


def unpack_codes(qweight: torch.Tensor) -> torch.Tensor:
    """``qweight [K/8, N]`` -> codes uint8 ``[K, N]``."""
    k = qweight.shape[0] * 8
    n = qweight.shape[1]
    out = torch.empty(k, n, dtype=torch.uint8, device=qweight.device)
    N.check(N.load().mtl_unpack_codes(qweight.contiguous().data_ptr(), k, n, out.data_ptr(),
                                      _stream(qweight.device)), "mtl_unpack_codes")
    return out


def gptq_dequant(qweight, qzeros, scales, group_size: int, zero_offset: int = 0) -> torch.Tensor:
    """Exact fp32 ``W[K, N]`` of the AutoGPTQ layout (in stored row order)."""
    k = qweight.shape[0] * 8
    n = qweight.shape[1]
    out = torch.empty(k, n, dtype=torch.float32, device=qweight.device)
    N.check(N.load().mtl_gptq_dequant(qweight.contiguous().data_ptr(), qzeros.contiguous().data_ptr(),
                                      scales.contiguous().data_ptr(), k, n, group_size, zero_offset,
                                      out.data_ptr(), _stream(qweight.device)), "mtl_gptq_dequant")
    return out


def qsz_dequant(packed, qsz, group_size: int) -> torch.Tensor:
    """Exact fp32 ``W[K, N]`` of the reference contract (``effective_weight(q, qsz).T``)
    from a packed weight of :func:`convert_weight_to_int4pack`."""
    k, n = qsz.shape[0] * group_size, qsz.shape[1]
    out = torch.empty(k, n, dtype=torch.float32, device=packed.device)
    N.check(N.load().mtl_qsz_dequant(packed.contiguous().data_ptr(), qsz.contiguous().data_ptr(),
                                     k, n, group_size, out.data_ptr(), _stream(packed.device)),
            "mtl_qsz_dequant")
    return out


def actorder_prepare(qweight: torch.Tensor, g_idx: torch.Tensor, group_size: int):
    """Group-contiguous copy of an act-order ``qweight`` and its gather index ``perm``.

    Load-time only (synchronises the stream to validate ``g_idx``).
    """
    k = qweight.shape[0] * 8
    n = qweight.shape[1]
    if g_idx.numel() != k:
        raise RuntimeError(f"g_idx must have K={k} entries")
    dev = qweight.device
    g32 = g_idx.to(device=dev, dtype=torch.int32).contiguous()
    sorted_qw = torch.empty_like(qweight)
    perm = torch.empty(k, dtype=torch.int32, device=dev)
    lib = N.load()
    sb = int(lib.mtl_actorder_scratch_bytes(k))
    scratch = torch.empty(sb, dtype=torch.uint8, device=dev)
    N.check(lib.mtl_gptq_actorder_prepare(qweight.contiguous().data_ptr(), g32.data_ptr(), k, n,
                                          group_size, sorted_qw.data_ptr(), perm.data_ptr(),
                                          scratch.data_ptr(), sb, _stream(dev)),
            "mtl_gptq_actorder_prepare")
    return sorted_qw, perm
