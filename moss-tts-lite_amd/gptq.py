"""GPTQ linear module and the reference's int4 format helpers (torch, device resident).

``GPTQLinear`` carries the AutoGPTQ buffers ``qweight`` int32 ``[K/8, N]``,
``qzeros`` int32 ``[K/g, N/8]``, ``scales`` fp16 ``[K/g, N]`` and ``g_idx`` int32
``[K]`` unchanged; :meth:`GPTQLinear.post_init` builds the device-side group-sorted
copy an act-order checkpoint needs and forward runs the gfx950 int4 GEMV.

The helpers mirror moss_tts_lite/gptq.py:35-97 on torch tensors
(``rtn_quantize``, ``pack_fast``, ``pack_qsz_only``, ``effective_weight``) and
``kernel_linear`` mirrors gptq.py:577-585 on the mtl operator.
"""
from __future__ import annotations

import torch

from . import _native as N
from . import ops

__all__ = ["GPTQLinear", "QszLinear", "fuse_gptq_linears", "fuse_qsz_linears",
           "interleave_qsz_gate_up", "group_scales_from_weight", "rtn_quantize",
           "pack_fast", "pack_qsz_only", "effective_weight", "kernel_linear",
           "interleave_gate_up", "bf16_linear", "W4Dispatch", "load_gptq_state", "LIN_NAMES"]

LIN_NAMES = ("q", "k", "v", "o", "gate", "up", "down")


class GPTQLinear(torch.nn.Module):
    """4-bit GPTQ linear, ``y = x @ dequant(qweight)`` with AutoGPTQ buffers.

    Dequant: ``w[k, n] = (q[k, n] - (z[g_idx[k], n] + zero_offset)) * s[g_idx[k], n]``;
    ``zero_offset`` is 0 for checkpoints storing ``z`` and 1 for ones storing ``z - 1``.
    """

    def __init__(self, in_features: int, out_features: int, group_size: int = 128,
                 bias: bool = False, zero_offset: int = 0, device=None):
        super().__init__()
        if group_size not in (32, 64, 128, 256):
            raise ValueError("group_size must be 32/64/128/256")
        if in_features % group_size or out_features % 8:
            raise ValueError("in_features must divide by group_size and out_features by 8")
        if bias:
            raise ValueError("the int4 decode path has no bias term")
        self.in_features, self.out_features = in_features, out_features
        self.group_size = group_size
        self.zero_offset = int(zero_offset)
        g = in_features // group_size
        self.register_buffer("qweight", torch.zeros(in_features // 8, out_features, dtype=torch.int32, device=device))
        self.register_buffer("qzeros", torch.zeros(g, out_features // 8, dtype=torch.int32, device=device))
        self.register_buffer("scales", torch.zeros(g, out_features, dtype=torch.float16, device=device))
        self.register_buffer("g_idx", (torch.arange(in_features, dtype=torch.int32, device=device)
                                       // group_size).to(torch.int32))
        self._kernel_qweight: torch.Tensor | None = None
        self._perm: torch.Tensor | None = None
        self._tiled: torch.Tensor | None = None
        self._strip: torch.Tensor | None = None
        self._strip_meta: tuple | None = None
        self._strip_only = False
        self._perm16: torch.Tensor | None = None     # the act-order index as int16 (K <= 12288)

    @classmethod
    def from_buffers(cls, qweight, qzeros, scales, g_idx=None, group_size: int = 128,
                     zero_offset: int = 0) -> "GPTQLinear":
        k = qweight.shape[0] * 8
        n = qweight.shape[1]
        m = cls(k, n, group_size, zero_offset=zero_offset, device=qweight.device)
        m.qweight = qweight.contiguous()
        m.qzeros = qzeros.contiguous()
        m.scales = scales.contiguous()
        if g_idx is not None:
            m.g_idx = g_idx.to(device=qweight.device, dtype=torch.int32).contiguous()
        return m

    def is_act_order(self) -> bool:
        trivial = torch.arange(self.in_features, device=self.g_idx.device, dtype=torch.int32) \
            // self.group_size
        return not torch.equal(self.g_idx, trivial)

    @torch.no_grad()
    def post_init(self) -> "GPTQLinear":
        """Build the kernel-side weight: for act-order, the group-sorted copy and gather index."""
        if self._strip_only:
            return self
        if self.is_act_order():
            self._kernel_qweight, self._perm = ops.actorder_prepare(self.qweight, self.g_idx,
                                                                    self.group_size)
        else:
            self._kernel_qweight, self._perm = self.qweight, None
        return self

    def kernel_args(self):
        """``(qweight, qzeros, scales, perm)`` of the AutoGPTQ-layout kernels (the weight
        group-sorted for act-order).  ``RuntimeError`` after :meth:`keep_strip_only`."""
        if self._strip_only:
            raise RuntimeError("this linear keeps only its strip copy (keep_strip_only): "
                               "the AutoGPTQ-layout kernels have no weight to read")
        if self._kernel_qweight is None:
            self.post_init()
        return self._kernel_qweight, self.qzeros, self.scales, self._perm

    @property
    def perm(self) -> torch.Tensor | None:
        """The act-order gather index (int32 ``[K]``: sorted row i is input channel
        ``perm[i]``), or None when the groups are contiguous."""
        if self._kernel_qweight is None and not self._strip_only:
            self.post_init()
        return self._perm

    @torch.no_grad()
    def keep_strip_only(self) -> "GPTQLinear":
        """Keep one resident int4 copy: build the strip copy and its strip-ordered
        metadata, then free the AutoGPTQ ``qweight``, its group-sorted copy and the split-K
        tiled copy.  The linear then serves the strip kernels only (the decode step's strip
        GEMVs, the prompt-length GEMM, :meth:`forward`); ``kernel_args``, ``dequantize``
        and ``reorder_output_columns`` raise ``RuntimeError``."""
        if self._strip_only:
            return self
        self.stream_weight(strip=True)
        self.strip_meta()
        self._kernel_qweight = None
        self._tiled = None
        self.qweight = torch.empty(0, dtype=torch.int32, device=self.scales.device)
        self._strip_only = True
        return self

    def supports_strip(self) -> bool:
        return self.out_features % 16 == 0 and self.in_features % 256 == 0 \
            and self.in_features <= 16384

    def stream_weight(self, strip: bool = False):
        """``(pointer tensor, layout)`` of the weight the decode-step GEMVs stream.

        ``strip=False``: the wave-contiguous tiled copy of the kernel weight (split-K
        GEMV) when N % 64 == 0, else the kernel weight in row layout.  ``strip=True``:
        the column-strip copy for the full-K strip GEMV.  Copies are built once."""
        if strip and self._strip is not None:
            return self._strip, N.LAYOUT_STRIP
        qw = self.kernel_args()[0]
        if strip:
            if not self.supports_strip():
                raise RuntimeError(f"no strip layout for K={self.in_features}, "
                                   f"N={self.out_features}")
            self._strip = ops.strip_weights(qw)
            return self._strip, N.LAYOUT_STRIP
        if self.out_features % 64:
            return qw, N.LAYOUT_ROWS
        if self._tiled is None:
            self._tiled = ops.tile_weights(qw)
        return self._tiled, N.LAYOUT_TILED

    def strip_meta(self):
        """``(scales, qzeros)`` in the strip order the strip GEMV reads (built once)."""
        if self._strip_meta is None:
            self._strip_meta = ops.strip_meta(self.scales, self.qzeros, self.group_size)
        return self._strip_meta

    def drop_original(self) -> None:
        """Free the unsorted ``qweight`` once the sorted copy exists (load-time memory)."""
        if self._perm is not None:
            self.qweight = torch.empty(0, dtype=torch.int32, device=self.qweight.device)

    @torch.no_grad()
    def reorder_output_columns(self, cols: torch.Tensor) -> "GPTQLinear":
        """Permute the output columns in place: new column c is old column ``cols[c]``.

        Used at load time so a producer writes its output directly in the act-order
        input order of its consumer (bitwise neutral per column).
        """
        if self._strip_only:
            raise RuntimeError("reorder_output_columns needs the AutoGPTQ weight "
                               "(freed by keep_strip_only)")
        cols = cols.to(device=self.scales.device, dtype=torch.long)
        if cols.numel() != self.out_features:
            raise ValueError("cols must list every output column once")
        if self._kernel_qweight is None:
            self.post_init()
        self._tiled = self._strip = self._strip_meta = self._perm16 = None
        sorted_separately = self._kernel_qweight is not self.qweight
        self._kernel_qweight = self._kernel_qweight[:, cols].contiguous()
        if sorted_separately and self.qweight.numel():
            self.qweight = self.qweight[:, cols].contiguous()
        elif not sorted_separately:
            self.qweight = self._kernel_qweight
        self.scales = self.scales[:, cols].contiguous()
        self.qzeros = _pack_cols(_unpack_cols(self.qzeros)[:, cols])
        return self

    def forward(self, x: torch.Tensor, out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
        """``x[..., K] @ dequant(W)``.  One row runs on the full-K strip GEMV (x gathered
        through the act-order index while staging), few rows on the skinny strip GEMM where
        it pays (:func:`ops.strip_rows_pays`); both read the strip copy of the weight, built
        once and kept.  The others run on the split-K GEMM over the AutoGPTQ layout (or,
        after :meth:`keep_strip_only`, the prompt-length GEMM over the strip copy).  Calls
        go through the ``torch.ops.mtl`` operators (one dispatcher call, torch's stream and
        allocator)."""
        m = x.numel() // self.in_features if self.in_features else 0
        perm = self.perm
        if m == 1 and self.supports_strip() and (perm is None or self.in_features <= 12288):
            strip = self.stream_weight(strip=True)[0]
            sc, qz = self.strip_meta()
            if perm is not None and self._perm16 is None:
                self._perm16 = perm.to(torch.int16)
            return ops.strip_gemv(x, strip, sc, qz, self.out_features, self.group_size,
                                  self.zero_offset, self._perm16, out_dtype)
        if m and self.supports_strip() and (
                (self._strip_only and m <= 16) or
                ops.strip_rows_pays(m, self.in_features, self.out_features, perm is not None)):
            strip = self.stream_weight(strip=True)[0]
            return ops.torch_ops().strip_rows_gemm(x, strip, self.qzeros, self.scales,
                                                   self.out_features, self.group_size,
                                                   self.zero_offset, perm, out_dtype)
        if self._strip_only:
            # the prompt-length GEMM over the strip copy, x's channels taken into the
            # weight's (group-sorted) row order first
            x2 = x.reshape(-1, self.in_features)
            if perm is not None:
                x2 = x2.index_select(1, perm.long())
            sc, qz = self.strip_meta()
            y = ops.prefill_gemm(x2.contiguous(), self._strip, sc, qz, self.out_features,
                                 self.group_size, self.zero_offset, out_dtype=out_dtype)
            return y.reshape(*x.shape[:-1], self.out_features)
        qw, qz, sc, perm = self.kernel_args()
        return ops.gptq_gemm(x, qw, qz, sc, self.group_size, perm=perm,
                             zero_offset=self.zero_offset, out_dtype=out_dtype)

    def dequantize(self) -> torch.Tensor:
        """Exact fp32 ``W[K, N]`` in the original input-channel order."""
        qw, qz, sc, perm = self.kernel_args()
        w = ops.gptq_dequant(qw, qz, sc, self.group_size, self.zero_offset)
        if perm is None:
            return w
        out = torch.empty_like(w)
        out[perm.long()] = w
        return out


class QszLinear:
    """An int4 linear in the reference's own contract (moss_tts_lite/gptq.py:66-97):
    ``packed`` from :func:`ops.convert_weight_to_int4pack` or
    :func:`ops.int4pack_from_torch_tiles` (the strip layout in torch's 4-D shape) and
    ``qsz`` bf16 ``[K/g, N, 2]`` = (scale, zero), ``w = (q - 8) * scale + zero``.  Its
    groups are contiguous runs of K (no act-order).  The decode step and the prefill run it
    on the strip kernels with the qsz read in place (``MTL_LAYOUT_STRIP_QSZ``).
    """

    zero_offset = 0

    def __init__(self, packed: torch.Tensor, qsz: torch.Tensor, group_size: int):
        if group_size not in (32, 64, 128, 256):
            raise ValueError("group_size must be 32/64/128/256")
        if qsz.dtype != torch.bfloat16 or qsz.dim() != 3 or qsz.shape[2] != 2:
            raise ValueError("qsz must be bfloat16 [K/g, N, 2]")
        self.group_size = group_size
        self.in_features = qsz.shape[0] * group_size
        self.out_features = qsz.shape[1]
        k, n = self.in_features, self.out_features
        if packed.dtype != torch.int32 or packed.numel() * 8 != n * k or packed.shape[0] * 8 != n:
            raise ValueError(f"packed must be the int32 [N/8, ...] packing of N={n}, K={k}")
        if k % 256 or n % 16:
            raise ValueError("the strip kernels need K % 256 == 0 and N % 16 == 0")
        self.packed = packed.contiguous()
        self.qsz = qsz.contiguous()

    def kernel_args(self):
        """``(weight, qzeros, metadata, perm)`` as GPTQLinear's: no zeros, no gather."""
        return self.packed, None, self.qsz, None

    def supports_strip(self) -> bool:
        return self.in_features <= 16384

    def stream_weight(self, strip: bool = True):
        """The packed weight is the strip layout already (``MTL_LAYOUT_STRIP_QSZ``)."""
        return self.packed, N.LAYOUT_STRIP_QSZ

    def strip_meta(self):
        """``(metadata, zeros)`` in the strip kernels' argument order: qsz, none."""
        return self.qsz, None

    perm = None          # contiguous groups: no act-order gather

    def post_init(self) -> "QszLinear":
        return self

    def drop_original(self) -> None:
        pass

    def keep_strip_only(self) -> "QszLinear":
        """The packed weight is the only copy already."""
        return self

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        shp = x.shape
        y = ops.weight_int4pack_mm(x.reshape(-1, shp[-1]), self.packed, self.group_size, self.qsz)
        return y.reshape(*shp[:-1], self.out_features)

    __call__ = forward

    def dequantize(self) -> torch.Tensor:
        """Exact fp32 ``W[K, N]``."""
        return ops.qsz_dequant(self.packed, self.qsz, self.group_size)


def fuse_qsz_linears(parts: list[QszLinear]) -> QszLinear:
    """Concatenate reference-contract linears along N, as fast_native.py:146-161 does
    (``torch.cat(packed, 0)``, ``torch.cat(qsz, 1)``): bitwise neutral per column."""
    g, k = parts[0].group_size, parts[0].in_features
    if any(p.group_size != g or p.in_features != k for p in parts[1:]):
        raise ValueError("fused linears need the same K and group size")
    return QszLinear(torch.cat([p.packed for p in parts], 0), torch.cat([p.qsz for p in parts], 1), g)


def interleave_qsz_gate_up(gate: QszLinear, up: QszLinear, block: int = 32) -> QszLinear:
    """gate and up fused with columns in alternating 32-wide blocks ``[gate 0:32 | up 0:32 |
    gate 32:64 | ...]`` (the layout of the SiLU*up epilogue): whole 16-column strips of the
    packed weights and the matching qsz columns are reordered."""
    n = gate.out_features
    if up.out_features != n or n % block or up.in_features != gate.in_features or \
            up.group_size != gate.group_size:
        raise ValueError("gate and up need the same K, group and N (a multiple of 32)")
    per = block // 16                                   # strips per block
    gp = gate.packed.reshape(n // block, per, -1)
    uq = up.packed.reshape(n // block, per, -1)
    packed = torch.stack([gp, uq], 1).reshape(2 * n // 8, *gate.packed.shape[1:])
    gs = gate.qsz.reshape(gate.qsz.shape[0], n // block, block, 2)
    us = up.qsz.reshape(up.qsz.shape[0], n // block, block, 2)
    qsz = torch.stack([gs, us], 2).reshape(gate.qsz.shape[0], 2 * n, 2)
    return QszLinear(packed, qsz, gate.group_size)


def fuse_gptq_linears(parts: list[GPTQLinear]) -> GPTQLinear:
    """Concatenate GPTQ linears along the output dim (same input, same g_idx).

    Bitwise neutral per output column: each column's K accumulation is untouched
    (the reference fuses (q,k) and (gate,up) the same way, fast_native.py:146-161).
    """
    g = parts[0].group_size
    for p in parts[1:]:
        if p.group_size != g or p.in_features != parts[0].in_features:
            raise ValueError("fused linears need the same K and group size")
        if not torch.equal(p.g_idx, parts[0].g_idx) or p.zero_offset != parts[0].zero_offset:
            raise ValueError("fused linears need the same g_idx and zero convention")
    return GPTQLinear.from_buffers(torch.cat([p.qweight for p in parts], 1),
                                   torch.cat([p.qzeros for p in parts], 1),
                                   torch.cat([p.scales for p in parts], 1), parts[0].g_idx,
                                   g, parts[0].zero_offset)


def interleave_gate_up(gate: GPTQLinear, up: GPTQLinear, block: int = 32) -> GPTQLinear:
    """Fuse gate and up into one linear whose columns alternate 32-wide blocks
    ``[gate 0:32 | up 0:32 | gate 32:64 | ...]``: the layout the SiLU*up epilogue reads."""
    n = gate.out_features
    if up.out_features != n or n % block:
        raise ValueError("gate and up need the same N, a multiple of 32")
    fused = fuse_gptq_linears([gate, up])
    dev = gate.qweight.device
    b = torch.arange(n // block, device=dev)
    cols = torch.stack([b * block, n + b * block], 1).reshape(-1, 1) + torch.arange(block, device=dev)
    cols = cols.reshape(-1)
    zeros = _unpack_cols(fused.qzeros)[:, cols]
    return GPTQLinear.from_buffers(fused.qweight[:, cols].contiguous(), _pack_cols(zeros),
                                   fused.scales[:, cols].contiguous(), fused.g_idx,
                                   fused.group_size, fused.zero_offset)


def _unpack_cols(qzeros: torch.Tensor) -> torch.Tensor:
    z = qzeros.to(torch.int64) & 0xFFFFFFFF
    return torch.stack([(z >> (4 * j)) & 0xF for j in range(8)], -1).reshape(qzeros.shape[0], -1)


def _pack_cols(z: torch.Tensor) -> torch.Tensor:
    z = z.to(torch.int64).reshape(z.shape[0], -1, 8)
    w = torch.zeros(z.shape[:2], dtype=torch.int64, device=z.device)
    for j in range(8):
        w |= (z[..., j] & 0xF) << (4 * j)
    return ((w + 2**31) % 2**32 - 2**31).to(torch.int32)


# ---------------------------------------------------------------------------------
# The reference's (codes, qsz) format helpers (moss_tts_lite/gptq.py:35-97)
# ---------------------------------------------------------------------------------

def group_scales_from_weight(w2d: torch.Tensor, group_size: int = 128):
    """Per-(row, group) ``s = clamp((max - min)/15, 1e-6)`` and ``min`` (gptq.py:35-45)."""
    n, k = w2d.shape
    if k % group_size:
        raise ValueError(f"K={k} not divisible by group_size={group_size}")
    wg = w2d.reshape(n, k // group_size, group_size)
    mx, mn = wg.amax(-1), wg.amin(-1)
    return ((mx - mn) / 15.0).clamp(min=1e-6), mn


def rtn_quantize(w2d: torch.Tensor, group_size: int = 128):
    """Round-to-nearest codes ``uint8 [N, K]`` plus ``(s, mn)`` (gptq.py:54-64)."""
    w = w2d.float()
    n, k = w.shape
    s, mn = group_scales_from_weight(w, group_size)
    wg = w.reshape(n, k // group_size, group_size)
    q = ((wg - mn.unsqueeze(-1)) / s.unsqueeze(-1)).round().clamp(0, 15).to(torch.uint8)
    return q.reshape(n, k), s, mn


def pack_qsz_only(s: torch.Tensor, mn: torch.Tensor, group_size: int = 128) -> torch.Tensor:
    """``qsz`` bf16 ``[K/g, N, 2]`` = (scale, mn + 8 scale) (gptq.py:79-85)."""
    del group_size
    return torch.stack([s, mn + 8.0 * s], -1).bfloat16().transpose(0, 1).contiguous()


def pack_fast(q: torch.Tensor, s: torch.Tensor, mn: torch.Tensor, inner_k_tiles: int = 8):
    """``(packed, qsz)`` for :func:`ops.weight_int4pack_mm` (gptq.py:66-77): the same
    nibble pre-pack as the reference, converted to the strip layout."""
    q = q.to(torch.uint8).contiguous()
    qsz = pack_qsz_only(s, mn)
    pre = (q[:, 1::2] | (q[:, 0::2] << 4)).contiguous()
    return ops.convert_weight_to_int4pack(pre, inner_k_tiles), qsz


def effective_weight(q: torch.Tensor, qsz: torch.Tensor, group_size: int = 128,
                     dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """``w = (q - 8) * scale + zero`` (gptq.py:87-97)."""
    n, k = q.shape
    scale = qsz[:, :, 0].t().to(dtype)
    zero = qsz[:, :, 1].t().to(dtype)
    qf = q.to(dtype).reshape(n, k // group_size, group_size)
    return ((qf - 8.0) * scale.unsqueeze(-1) + zero.unsqueeze(-1)).reshape(n, k)


def kernel_linear(x: torch.Tensor, packed: torch.Tensor, g: int, qsz: torch.Tensor,
                  out_dtype: torch.dtype) -> torch.Tensor:
    """int4 GEMM shaped like ``F.linear`` (gptq.py:577-585)."""
    shp = x.shape
    out = ops.weight_int4pack_mm(x.reshape(-1, shp[-1]), packed, g, qsz)
    if out.dtype != out_dtype:
        out = out.to(out_dtype)
    return out.reshape(*shp[:-1], qsz.shape[1])


def bf16_linear(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """``F.linear(x, W)`` for a bf16 weight ``[N, K]`` on the gfx950 bf16 GEMV (one
    launch per row of ``x``): the path of linears kept in bf16 (gptq.py:689-693)."""
    if w.dtype != torch.bfloat16 or w.dim() != 2:
        raise RuntimeError("weight must be bfloat16 [N, K]")
    n, k = w.shape
    shp = x.shape
    if shp[-1] != k:
        raise RuntimeError(f"x has {shp[-1]} features, weight expects {k}")
    x2 = x.reshape(-1, k).to(torch.bfloat16).contiguous()
    w = w.contiguous()
    out = torch.empty(x2.shape[0], n, dtype=torch.bfloat16, device=x.device)
    lib = N.load()
    stream = torch.cuda.current_stream(x.device).cuda_stream
    for r in range(x2.shape[0]):
        N.check(lib.mtl_bf16_gemv(x2[r].data_ptr(), w.data_ptr(), n, k, out[r].data_ptr(), 0, 0,
                                  stream), "mtl_bf16_gemv")
    return out.reshape(*shp[:-1], n)


_GROUP_SIZES = (32, 64, 128, 256)


def _layer_linear(key: str) -> tuple[int, str]:
    """``"3:down"`` -> ``(3, "down")``: how the reference's metadata names one linear."""
    layer, _, linear = key.partition(":")
    return int(layer), linear


def split_keeps(bf16_keep) -> tuple[set, set]:
    """The reference's bf16-keep list (gptq.py:645-650) as two sets: whole layers (plain
    layer indices) and single linears (``(layer, name)`` pairs)."""
    layers, linears = set(), set()
    for item in bf16_keep:
        if isinstance(item, (tuple, list)):
            linears.add((int(item[0]), str(item[1])))
        else:
            layers.add(int(item))
    return layers, linears


class W4Dispatch:
    """The reference's per-linear int4 dispatch on the mtl kernels.

    Mirrors ``FastMossTTS._quantize/_linear`` (moss_tts_lite/fast.py:73-121) and
    ``GptqMossTTS._quantize/_linear`` (gptq.py:641-697):
    - ``qlayers[li]`` maps each quantised linear name to ``(packed, qsz)``, with ``packed``
      in the strip ``[K/8, N]`` layout (:func:`ops.convert_weight_to_int4pack`);
      ``qlayers[li]`` is None for a layer with nothing quantised;
    - ``group_size_map[li][name]`` holds each linear's group size (``w4_group_size``
      unless ``group_size_map`` overrides it);
    - linears in ``bf16_keep`` stay bf16 and run :func:`bf16_linear`: a layer index keeps
      the whole layer, a ``(li, name)`` pair one linear.

    Without ``state``, every other linear of ``layers`` is quantised round-to-nearest
    (fast.py:86-101). With ``state``, every linear that is not kept must have a record in
    it, or ``KeyError`` is raised, as the reference's ``state[li][name]`` lookup does. A
    record holds either the GPTQ state's unpacked codes (``{"q", "qsz"}``,
    :func:`load_gptq_state`) or the standalone export's torch tiles (``{"packed", "qsz"}``,
    :func:`moss_tts_lite_amd.export.read_standalone`). A record's linear need not be in
    ``layers``; it is placed on ``device`` then. Quantised bf16 weights are dropped from
    ``layers``.
    """

    def __init__(self, layers: list, w4_group_size: int = 128, bf16_keep=(),
                 group_size_map: dict | None = None, state: dict | None = None,
                 device="cuda"):
        overrides = {(int(li), str(name)): int(g) for (li, name), g in (group_size_map or {}).items()}
        for where, g in [("w4_group_size", w4_group_size)] + list(overrides.items()):
            if g not in _GROUP_SIZES:
                raise ValueError(f"group size {g} ({where}) is not one of {_GROUP_SIZES}")
        self.layers = layers
        self.w4_group_size = w4_group_size
        self._keep_layers, self._keep_linears = split_keeps(bf16_keep)
        self.group_size_map = {li: {name: overrides.get((li, name), w4_group_size)
                                    for name in LIN_NAMES} for li in range(len(layers))}
        self._device = torch.device(device)
        self.qlayers = [self._install(li, state) for li in range(len(layers))]

    def is_kept(self, li: int, name: str) -> bool:
        return li in self._keep_layers or (li, name) in self._keep_linears

    def _install(self, li: int, state: dict | None):
        if li in self._keep_layers:
            return None
        weights = self.layers[li]
        installed = {}
        for name in LIN_NAMES:
            if (li, name) in self._keep_linears:
                continue
            g = self.group_size_map[li][name]
            if state is None:
                if name not in weights:
                    continue
                codes, s, mn = rtn_quantize(weights[name], g)
                installed[name] = pack_fast(codes, s, mn)
            else:
                try:
                    rec = state[li][name]
                except KeyError:
                    raise KeyError(f"the GPTQ state has no record for layer {li} {name}, "
                                   "which is not kept in bf16") from None
                dev = weights[name].device if name in weights else self._device
                installed[name] = self._from_record(rec, dev)
            weights.pop(name, None)
        return installed or None

    @staticmethod
    def _from_record(rec: dict, dev) -> tuple:
        qsz = rec["qsz"].to(device=dev, dtype=torch.bfloat16).contiguous()
        if "q" in rec:        # calibrated codes [N, K] (gptq.py:504-509)
            codes = rec["q"].to(device=dev, dtype=torch.uint8)
            prepacked = (codes[:, 1::2] | (codes[:, 0::2] << 4)).contiguous()
            return ops.convert_weight_to_int4pack(prepacked, 8), qsz
        # torch's int4 tiles as stored by the export (export.py:712-734)
        return ops.int4pack_from_torch_tiles(rec["packed"].to(dev)), qsz

    def _linear(self, x: torch.Tensor, li: int, name: str) -> torch.Tensor:
        """``F.linear``-shaped projection ``x[..., K] -> [..., N]`` in the active mode."""
        qd = self.qlayers[li]
        if qd is None or name not in qd:
            return bf16_linear(x, self.layers[li][name])
        packed, qsz = qd[name]
        return kernel_linear(x, packed, self.group_size_map[li][name], qsz, torch.bfloat16)


def load_gptq_state(path: str):
    """``(state, group_size_map, bf16_keep)`` of an offline GPTQ state file and the
    ``<path>.meta.json`` beside it (the format of gptq.py:608-626).

    The weights load with ``torch.load(weights_only=True)`` and the metadata with json, so
    nothing in either file runs. The metadata is required: a state's group sizes and bf16
    keeps cannot be recovered from its tensors (``FileNotFoundError`` without it).
    """
    import json
    import os

    meta_path = f"{path}.meta.json"
    if not os.path.isfile(meta_path):
        raise FileNotFoundError(f"{meta_path} is missing; it records the state's per-linear "
                                "group sizes and bf16 keeps")
    state = torch.load(path, map_location="cpu", weights_only=True)
    with open(meta_path, encoding="utf-8") as fh:
        meta = json.load(fh)
    gmap = {_layer_linear(k): int(g) for k, g in (meta.get("group_size_map") or {}).items()}
    keep: list = [_layer_linear(k) for k in (meta.get("bf16_linears") or [])]
    keep.extend(int(layer) for layer in (meta.get("bf16_layers") or []))
    return state, gmap, keep
