"""Host-side assembly of the reference's ``(packed, qsz)`` records into backbone linears
(moss-tts-lite_amd/gptq.py: QszLinear, fuse_qsz_linears, interleave_qsz_gate_up), checked
against the strip layout's definition in the oracle (``gptq_ref.strip_layout``): no
kernel runs."""
import numpy as np
import pytest
import torch

from oracle import gptq_ref as G

K, GROUP = 256, 128


def _packed(qw):
    """The packed tensor of a ``[K/8, N]`` qweight: its strip words in torch's 4-D shape
    ``[N/8, K/128, 32, 4]`` (inner_k_tiles 8)."""
    k, n = qw.shape[0] * 8, qw.shape[1]
    words = G.strip_layout(qw).view(np.int32)
    return torch.from_numpy(words.copy()).reshape(n // 8, k // 128, 32, 4)


def _linear(n, seed):
    from moss_tts_lite_amd.gptq import QszLinear

    r = np.random.default_rng(seed)
    qw = r.integers(-2**31, 2**31, (K // 8, n), dtype=np.int64).astype(np.int32)
    qsz = torch.from_numpy(r.standard_normal((K // GROUP, n, 2)).astype(np.float32)).bfloat16()
    return qw, qsz, QszLinear(_packed(qw), qsz, GROUP)


def test_fuse_is_concatenation_along_n():
    from moss_tts_lite_amd.gptq import fuse_qsz_linears

    parts = [_linear(n, s) for s, n in enumerate((64, 16, 16))]
    fused = fuse_qsz_linears([p[2] for p in parts])
    qw = np.concatenate([p[0] for p in parts], 1)
    assert fused.out_features == 96 and fused.in_features == K
    assert torch.equal(fused.packed, _packed(qw))
    assert torch.equal(fused.qsz, torch.cat([p[1] for p in parts], 1))
    assert fused.kernel_args()[3] is None and fused.strip_meta()[1] is None


def test_gate_up_interleave_is_the_32_column_block_order():
    from moss_tts_lite_amd.gptq import interleave_qsz_gate_up

    n = 96
    qg, sg, gate = _linear(n, 10)
    qu, su, up = _linear(n, 11)
    gu = interleave_qsz_gate_up(gate, up)
    # fused column 64*b + c is gate column 32*b + c, and 64*b + 32 + c is up's
    cols = [(src, 32 * b + c) for b in range(n // 32) for src in (0, 1) for c in range(32)]
    qw = np.stack([(qg, qu)[src][:, c] for src, c in cols], 1)
    qsz = torch.stack([(sg, su)[src][:, c] for src, c in cols], 1)
    assert torch.equal(gu.packed, _packed(qw))
    assert torch.equal(gu.qsz, qsz)
    with pytest.raises(ValueError):
        interleave_qsz_gate_up(gate, _linear(64, 12)[2])


def test_qsz_linear_rejects_bad_shapes():
    from moss_tts_lite_amd.gptq import QszLinear

    qw, qsz, _ = _linear(32, 3)
    with pytest.raises(ValueError):
        QszLinear(_packed(qw), qsz, 16)                      # group size
    with pytest.raises(ValueError):
        QszLinear(_packed(qw), qsz.float(), GROUP)           # qsz dtype
    with pytest.raises(ValueError):
        QszLinear(_packed(qw)[:2], qsz, GROUP)               # packed of another N
    with pytest.raises(ValueError):
        QszLinear(_packed(qw), qsz[:, :16], GROUP)           # qsz of another N
