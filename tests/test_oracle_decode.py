"""Pins the oracle's decode-step math (CPU): RMSNorm, RoPE, attention, SiLU*up.

Checks come from independent implementations (torch's CPU ops), float64 closed forms
and exact invariants, so a dropped term, a wrong sign or a transposed operand fails.
"""
import numpy as np
import torch
import torch.nn.functional as F

from oracle import decode_ref as D
from oracle.bf16 import round_bf16


def _bf(r, shape, std=1.0):
    return round_bf16((r.standard_normal(shape) * std).astype(np.float32))


def test_rms_norm_matches_torch_bf16_chain_within_one_ulp():
    r = np.random.default_rng(0)
    x = _bf(r, (16, 4096), 3.0)
    w = round_bf16((1 + 0.1 * r.standard_normal(4096)).astype(np.float32))
    ours = D.rms_norm(x, w)
    tx, tw = torch.from_numpy(x).bfloat16(), torch.from_numpy(w).bfloat16()
    xf = tx.float()
    ref = (tw * (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)).bfloat16()).float().numpy()
    ulp = np.abs(ref) * 2.0 ** -7 + 1e-30
    assert np.all(np.abs(ours - ref) <= ulp)
    # and against torch's fused rms_norm (no intermediate rounding): close, not equal
    fused = F.rms_norm(xf, (4096,), tw.float(), 1e-6).numpy()
    assert np.abs(ours - fused).max() <= 2 * (np.abs(fused).max() * 2.0 ** -8)


def test_rms_norm_invariants():
    r = np.random.default_rng(1)
    x = _bf(r, (4, 256))
    w = np.ones(256, np.float32)
    # exact scale invariance for power-of-two scaling
    assert np.array_equal(D.rms_norm(x, w), D.rms_norm(x * np.float32(8.0), w))
    # a constant vector normalises to +-1 (up to eps)
    c = np.full((1, 128), 0.5, np.float32)
    assert np.allclose(D.rms_norm(c, np.ones(128, np.float32)), 1.0, atol=2 ** -7)


def test_rope_tables_match_float64_trig():
    cos, sin = D.rope_tables(2048, 128, 1e6)
    i = np.arange(0, 128, 2, dtype=np.float64)
    inv = 1.0 / (1e6 ** (i / 128))
    ang = np.outer(np.arange(2048, dtype=np.float64), np.concatenate([inv, inv]))
    # within one bf16 ulp of the exact values (the fp32 argument rounding moves them)
    assert np.all(np.abs(cos - np.cos(ang)) <= 2.0 ** -8 + 1e-3 * (ang / 2048))
    assert np.all(np.abs(sin - np.sin(ang)) <= 2.0 ** -8 + 1e-3 * (ang / 2048))
    # position 0: cos = 1, sin = 0 exactly; the two halves are duplicated
    assert np.all(cos[0] == 1.0) and np.all(sin[0] == 0.0)
    assert np.array_equal(cos[:, :64], cos[:, 64:])


def test_rope_rotation_properties():
    r = np.random.default_rng(2)
    x = _bf(r, (8, 128))
    cos, sin = D.rope_tables(100, 128)
    assert np.array_equal(D.apply_rope(x, cos[0], sin[0]), x)   # identity at position 0
    y = D.apply_rope(x, cos[57], sin[57])
    # each (i, i+64) pair is rotated: pair norms preserved up to bf16 rounding
    n0 = x[:, :64] ** 2 + x[:, 64:] ** 2
    n1 = y[:, :64] ** 2 + y[:, 64:] ** 2
    assert np.allclose(n1, n0, rtol=3e-2, atol=1e-3)
    # sign convention: rotate_half(x) = cat(-x2, x1)
    assert np.array_equal(D.rotate_half(np.arange(4.0)), np.array([-2.0, -3.0, 0.0, 1.0]))


def test_attention_matches_torch_sdpa():
    r = np.random.default_rng(3)
    q = _bf(r, (8, 128))
    k = _bf(r, (2, 37, 128))
    v = _bf(r, (2, 37, 128))
    tq = torch.from_numpy(q).view(1, 8, 1, 128)
    tk = torch.from_numpy(k).repeat_interleave(4, 0).view(1, 8, 37, 128)
    tv = torch.from_numpy(v).repeat_interleave(4, 0).view(1, 8, 37, 128)
    # the flash form: torch's CPU SDPA on the bf16 tensors, up to rare flips of one
    # probability's bf16 rounding (fp32 score sums in another order); the exact softmax
    # is three times further away
    ours = D.attention(q, k, v, 1 / np.sqrt(128))
    got = F.scaled_dot_product_attention(tq.bfloat16(), tk.bfloat16(), tv.bfloat16())
    got = got.view(8, 128).float().numpy()
    flash_err = np.linalg.norm(ours - got) / np.linalg.norm(got)
    exact_err = np.linalg.norm(D.attention(q, k, v, 1 / np.sqrt(128), p_bf16=False) - got) \
        / np.linalg.norm(got)
    assert flash_err < 1.5e-3 and exact_err > 2 * flash_err, (flash_err, exact_err)
    # single kv head, 4 query heads (the reference's ratio): equal bit for bit
    q4, k1, v1 = q[:4], k[:1, :6], v[:1, :6]
    got4 = F.scaled_dot_product_attention(
        torch.from_numpy(q4).bfloat16().view(1, 4, 1, 128),
        torch.from_numpy(k1).bfloat16().repeat_interleave(4, 0).view(1, 4, 6, 128),
        torch.from_numpy(v1).bfloat16().repeat_interleave(4, 0).view(1, 4, 6, 128))
    np.testing.assert_array_equal(D.attention(q4, k1, v1, 1 / np.sqrt(128)),
                                  got4.view(4, 128).float().numpy())
    # the exact form: float64 SDPA, to the final bf16 rounding
    exact = D.attention(q, k, v, 1 / np.sqrt(128), p_bf16=False)
    ref = F.scaled_dot_product_attention(tq.double(), tk.double(), tv.double()).view(8, 128).float().numpy()
    assert np.all(np.abs(exact - ref) <= np.abs(ref) * 2.0 ** -8 + 1e-6)
    # the two forms differ by the bf16 rounding of the probabilities only
    assert 2e-4 < np.linalg.norm(ours - exact) / np.linalg.norm(exact) < 5e-3


def test_attention_special_cases():
    v = np.arange(3 * 128, dtype=np.float32).reshape(1, 3, 128) / 64
    k = np.zeros((1, 3, 128), np.float32)
    q = np.ones((1, 128), np.float32)
    # equal scores -> plain mean of the values
    assert np.allclose(D.attention(q, k, v, 1.0), round_bf16(v.mean(1)))
    # one position -> that value row
    assert np.array_equal(D.attention(q, k[:, :1], v[:, :1], 1.0), round_bf16(v[:, 0]))


def test_silu_mul_matches_torch():
    r = np.random.default_rng(4)
    g, u = _bf(r, 4096, 3.0), _bf(r, 4096)
    tg, tu = torch.from_numpy(g).bfloat16(), torch.from_numpy(u).bfloat16()
    ref = (F.silu(tg) * tu).float().numpy()
    ours = D.silu_mul(g, u)
    assert np.all(np.abs(ours - ref) <= np.abs(ref) * 2.0 ** -7 + 1e-30)


def test_embed_sum_matches_torch_bf16_adds():
    # the reference's 33-way embedding: F.embedding per table, bf16 adds left to right
    r = np.random.default_rng(5)
    tables = [_bf(r, (50, 64))] + [_bf(r, (9, 64)) for _ in range(4)]
    ids = [7, 3, 8, 0, 5]
    tt = [torch.from_numpy(t).bfloat16() for t in tables]
    h = F.embedding(torch.tensor([ids[0]]), tt[0])
    for t, i in zip(tt[1:], ids[1:]):
        h = h + F.embedding(torch.tensor([i]), t)
    assert np.array_equal(D.embed_sum(ids, tables), h[0].float().numpy())


def test_moss_heads_layout_and_pad():
    r = np.random.default_rng(6)
    hf = _bf(r, 64)
    text = _bf(r, (300, 64), 0.02)
    audio = _bf(r, (3, 17, 64), 0.02)
    two_ids = [250, 260]
    lt, la, two = D.moss_heads(hf, text, audio, text[two_ids], pad_code=16, audio2=False)
    assert two is None and la.shape == (3, 17) and lt.shape == (300,)
    assert np.all(np.isneginf(la[:, 16])) and np.all(np.isfinite(la[:, :16]))
    ref = (torch.from_numpy(audio).double() @ torch.from_numpy(hf).double()).float()
    assert np.array_equal(la[:, :16], ref.bfloat16().float().numpy()[:, :16])
    lt2, la2, two2 = D.moss_heads(hf, text, audio, text[two_ids], pad_code=16, audio2=True)
    assert lt2 is None and np.array_equal(la2, la)
    # the 2-way head is the text head's rows at the two slot ids (model.py head_2way)
    assert np.array_equal(two2, lt[two_ids])
