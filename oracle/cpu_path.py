"""The reference's CPU path for one int4 linear, in torch ops on the CPU (oracle; test
infrastructure and the bench's CPU baseline only).

``linear_fp32`` restates tests/test_quant.py:104-107 with moss_tts_lite/gptq.py:87-97:
dequantise the codes with ``effective_weight`` (``(q - 8) * scale + zero`` in fp32) and
multiply, ``x.float() @ W.T``. ``pack_for_cpu`` / ``int4pack_mm_cpu`` wrap torch's own CPU
int4 operator pair (``aten._convert_weight_to_int4pack_for_cpu``,
``aten._weight_int4pack_mm_for_cpu``). That pair takes the same ``(scale, zero)`` bf16
``[K/g, N, 2]`` contract as the reference's GPU operator.

Pinned by tests/test_oracle_cpu_path.py against the float64 closed form
(``oracle.gptq_ref.int4pack_mm``).
"""
from __future__ import annotations

import torch


def effective_weight(q: torch.Tensor, qsz: torch.Tensor, group_size: int) -> torch.Tensor:
    """fp32 ``[N, K]`` weight of codes ``q [N, K]`` (0..15) and bf16 ``qsz [K/g, N, 2]``:
    ``(q - 8) * scale + zero`` per (column, group) (gptq.py:87-97)."""
    n, k = q.shape
    scale = qsz[:, :, 0].t().float().unsqueeze(-1)
    zero = qsz[:, :, 1].t().float().unsqueeze(-1)
    w = (q.float() - 8.0).reshape(n, k // group_size, group_size) * scale + zero
    return w.reshape(n, k)


def linear_fp32(x: torch.Tensor, q: torch.Tensor, qsz: torch.Tensor, group_size: int) -> torch.Tensor:
    """The reference's CPU int4 linear: ``x.float() @ effective_weight(q, qsz).T``, fp32
    ``[M, N]`` (tests/test_quant.py:104-107)."""
    return x.float() @ effective_weight(q, qsz, group_size).t()


def pack_for_cpu(q: torch.Tensor, inner_k_tiles: int = 8) -> torch.Tensor:
    """torch's CPU int4 packing of codes ``q [N, K]`` (0..15)."""
    return torch.ops.aten._convert_weight_to_int4pack_for_cpu(q.to(torch.int32).contiguous(),
                                                              inner_k_tiles)


def int4pack_mm_cpu(x: torch.Tensor, packed: torch.Tensor, group_size: int,
                    qsz: torch.Tensor) -> torch.Tensor:
    """torch's CPU int4 GEMM on the same contract: bf16 ``[M, N]``."""
    return torch.ops.aten._weight_int4pack_mm_for_cpu(x.to(torch.bfloat16).contiguous(), packed,
                                                      group_size, qsz.contiguous())
