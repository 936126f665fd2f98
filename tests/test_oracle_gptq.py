"""Pins the oracle's int4 formats and dequant closed forms.

Each check is chosen so that a plausible slip in the oracle fails it: brute force
on tiny inputs, known-answer words, torch's independent CPU int4 kernel, and the
exact special cases of the closed forms.  Nothing here retypes a formula as its
own check.
"""
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import gptq_ref as G
from oracle import synth
from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits


# ---------------------------------------------------------------- nibble orders

def test_qweight_known_answer_low_nibble_first():
    codes = np.arange(1, 9, dtype=np.uint8).reshape(8, 1)          # k = 0..7 -> 1..8
    w = G.pack_qweight(codes)
    assert w.shape == (1, 1)
    assert w.view(np.uint32)[0, 0] == 0x87654321


def test_qzeros_known_answer_along_n():
    z = np.array([[9, 8, 7, 6, 5, 4, 3, 2]], dtype=np.uint8)
    assert G.pack_qzeros(z).view(np.uint32)[0, 0] == 0x23456789


def test_reference_prepack_even_k_high_nibble():
    q = np.array([[0xA, 0x3, 0x1, 0xF]], dtype=np.uint8)
    assert G.prepack_u8(q).tolist() == [[0xA3, 0x1F]]


@pytest.mark.parametrize("k,n", [(8, 8), (64, 24), (256, 40), (512, 48)])
def test_pack_round_trips(k, n):
    r = np.random.default_rng(k + n)
    codes = r.integers(0, 16, size=(k, n)).astype(np.uint8)
    assert np.array_equal(G.unpack_qweight(G.pack_qweight(codes)), codes)
    z = r.integers(0, 16, size=(k // 8, n)).astype(np.uint8)
    assert np.array_equal(G.unpack_qzeros(G.pack_qzeros(z)), z)
    qn = codes.T.copy()
    assert np.array_equal(G.unprepack_u8(G.prepack_u8(qn)), qn)
    # reference pre-pack -> the drop-in's strip layout keeps every (n, k) code
    if k % 128 == 0 and n % 16 == 0:
        words = G.int4pack_from_prepacked(G.prepack_u8(qn))
        assert np.array_equal(G.unpack_qweight(G.strip_layout_inverse(words, k, n)), codes)


def test_strip_layout_brute_force():
    # every 32-bit word lands where the layout's formula puts it
    k, n = 256, 48
    qw = np.arange(k // 8 * n, dtype=np.uint32).reshape(k // 8, n).view(np.int32)
    words = G.strip_layout(qw)
    kb = k // 128
    for r in range(k // 8):
        for c in range(n):
            s_, b, rr = c // 16, r // 16, r % 16
            lane, j = 16 * (rr % 4) + c % 16, rr // 4
            assert words[((s_ * kb + b) * 64 + lane) * 4 + j] == qw[r, c].view(np.uint32)
    assert np.array_equal(G.strip_layout_inverse(words, k, n), qw)
    # a strip is one contiguous run: column 0..15 over all of K come first
    assert set(words[:k // 8 * 16].tolist()) == set(qw[:, :16].view(np.uint32).reshape(-1).tolist())


def test_pack_brute_force_bits():
    r = np.random.default_rng(3)
    codes = r.integers(0, 16, size=(16, 5)).astype(np.uint8)
    w = G.pack_qweight(codes).view(np.uint32)
    for k in range(16):
        for n in range(5):
            assert (int(w[k // 8, n]) >> (4 * (k % 8))) & 0xF == codes[k, n]


# ---------------------------------------------------------------- RTN + qsz

def test_rtn_brute_force_nearest_grid_point():
    r = np.random.default_rng(11)
    w = (r.standard_normal((6, 64)) * 0.05).astype(np.float32)
    w = bf16_bits_to_f32(f32_to_bf16_bits(w))
    q, s, mn = G.rtn_quantize(w, 32)
    for n in range(6):
        for k in range(64):
            g = k // 32
            t = float(np.float32(np.float32(w[n, k]) - mn[n, g]) / np.float32(s[n, g]))
            cands = sorted(range(16), key=lambda c: (abs(t - c), c % 2))   # ties -> even
            assert q[n, k] == cands[0], (n, k, t)
    # the group extremes land on the grid ends
    wg = w.reshape(6, 2, 32)
    for n in range(6):
        for g in range(2):
            assert q[n, g * 32 + int(np.argmin(wg[n, g]))] == 0
            assert q[n, g * 32 + int(np.argmax(wg[n, g]))] == 15


def _torch_rtn(w: torch.Tensor, g: int):
    """The reference's RTN chain (gptq.py:35-64) in torch ops, on ``w``'s device."""
    n, k = w.shape
    wg = w.float().reshape(n, k // g, g)
    mx, mn = wg.amax(-1), wg.amin(-1)
    s = ((mx - mn) / 15.0).clamp(min=1e-6)
    q = ((wg - mn.unsqueeze(-1)) / s.unsqueeze(-1)).round().clamp(0, 15).to(torch.uint8)
    return q.reshape(n, k), s, mn


def test_rtn_cpu_form_matches_torch_on_cpu():
    # torch's CPU kernel divides the span by 15 exactly: the oracle's "cpu" form, bit for bit
    r = np.random.default_rng(12)
    w = bf16_bits_to_f32(f32_to_bf16_bits((r.standard_normal((64, 512)) * 0.05).astype(np.float32)))
    q, s, mn = G.rtn_quantize(w, 128, divide="cpu")
    tq, ts, tm = _torch_rtn(torch.from_numpy(w), 128)
    assert np.array_equal(s, ts.numpy()) and np.array_equal(mn, tm.numpy())
    assert np.array_equal(q, tq.numpy())


def test_rtn_device_form_is_the_reciprocal_product():
    # the device form (the default): span * fp32(1/15), which differs from the exact
    # quotient by one float32 ulp in many groups (so the two forms are distinguishable)
    r = np.random.default_rng(13)
    w = (r.standard_normal((64, 512)) * 0.05).astype(np.float32)
    s_dev, mn = G.group_scales_from_weight(w, 128)
    s_cpu, _ = G.group_scales_from_weight(w, 128, divide="cpu")
    wg = w.reshape(64, 4, 128)
    span = (wg.max(-1) - wg.min(-1)).astype(np.float32)
    assert np.array_equal(s_dev, (span * (np.float32(1.0) / np.float32(15.0))).astype(np.float32))
    assert np.array_equal(s_cpu, (span / np.float32(15.0)).astype(np.float32))
    ulps = np.abs(s_dev.view(np.int32).astype(np.int64) - s_cpu.view(np.int32))
    assert ulps.max() == 1 and 0.2 < (ulps == 1).mean() < 0.9


def test_rtn_scale_floor():
    w = np.zeros((2, 64), dtype=np.float32)
    q, s, mn = G.rtn_quantize(w, 32)
    assert np.all(s == np.float32(1e-6)) and np.all(q == 0) and np.all(mn == 0)


def test_qsz_rounding_matches_torch():
    r = np.random.default_rng(5)
    s = r.uniform(1e-4, 1e-2, size=(7, 4)).astype(np.float32)
    mn = (-r.uniform(0, 0.3, size=(7, 4))).astype(np.float32)
    qsz = G.pack_qsz(s, mn)
    ts, tm = torch.from_numpy(s), torch.from_numpy(mn)
    ref = torch.stack([ts, tm + 8.0 * ts], -1).bfloat16().transpose(0, 1).contiguous()
    assert np.array_equal(qsz, ref.view(torch.int16).numpy().view(np.uint16))


# ---------------------------------------------------------------- dequant closed forms

def test_effective_weight_special_cases():
    r = np.random.default_rng(9)
    n, k, g = 4, 64, 32
    s = r.uniform(1e-3, 1e-2, size=(n, k // g)).astype(np.float32)
    mn = (-r.uniform(0, 0.1, size=(n, k // g))).astype(np.float32)
    qsz = G.pack_qsz(s, mn)
    scale = bf16_bits_to_f32(qsz[:, :, 0]).T
    zero = bf16_bits_to_f32(qsz[:, :, 1]).T
    # q == 8 gives the stored zero exactly; each code step adds exactly one scale
    w8 = G.effective_weight(np.full((n, k), 8, np.uint8), qsz, g).reshape(n, k // g, g)
    assert np.array_equal(w8, np.broadcast_to(zero[..., None], w8.shape))
    for q in range(16):
        wq = G.effective_weight(np.full((n, k), q, np.uint8), qsz, g).reshape(n, k // g, g)
        exact = (np.float64(q) - 8.0) * scale.astype(np.float64) + zero.astype(np.float64)
        assert np.allclose(wq[..., 0], exact, rtol=0, atol=np.abs(exact).max() * 2 ** -23)
    # storage-rounded scale/min reproduce the same grid
    s_eff, mn_eff = G.bf16_effective_scale_zero(s, mn)
    assert np.array_equal(s_eff, scale.astype(np.float32))


def test_effective_weight_matches_torch_cpu_int4_kernel():
    # torch's own CPU int4 op uses the same (scale, zero) contract independently.
    n, k, g = 64, 512, 128
    w = synth.reference_weight(n, k, seed=3)
    q, s, mn = G.rtn_quantize(w, g)
    qsz = G.pack_qsz(s, mn)
    r = np.random.default_rng(4)
    x = bf16_bits_to_f32(f32_to_bf16_bits(r.standard_normal((4, k)).astype(np.float32)))
    ours = G.int4pack_mm(x, q, qsz, g)
    tq = torch.from_numpy(q.astype(np.int32))
    packed = torch.ops.aten._convert_weight_to_int4pack_for_cpu(tq, 1)
    tqsz = torch.from_numpy(qsz.view(np.int16)).view(torch.bfloat16)
    tx = torch.from_numpy(x).bfloat16()
    theirs = torch.ops.aten._weight_int4pack_mm_for_cpu(tx, packed, g, tqsz).float().numpy()
    rel = np.linalg.norm(theirs - ours) / np.linalg.norm(ours)
    assert rel < 5e-3, rel
    # a transposed operand or a dropped zero term is far outside this band
    bad = G.int4pack_mm(x, q, np.stack([qsz[..., 0], qsz[..., 0]], -1), g)
    assert np.linalg.norm(theirs - bad) / np.linalg.norm(bad) > 0.1


def test_gptq_dequant_brute_force():
    r = np.random.default_rng(21)
    k, n, g = 64, 16, 32
    codes = r.integers(0, 16, size=(k, n)).astype(np.uint8)
    z = r.integers(0, 16, size=(k // g, n)).astype(np.uint8)
    s = r.uniform(0.002, 0.02, size=(k // g, n)).astype(np.float16)
    perm = r.permutation(k)
    g_idx = G.actorder_g_idx(perm, g)
    for zo in (0, 1):
        w = G.gptq_dequant(G.pack_qweight(codes), G.pack_qzeros(z), s.view(np.uint16), g_idx, g, zo)
        for kk in range(k):
            for nn in range(n):
                gg = int(g_idx[kk])
                want = (int(codes[kk, nn]) - int(z[gg, nn]) - zo) * float(s[gg, nn])
                assert w[kk, nn] == np.float32(want)


def test_actorder_g_idx_definition():
    perm = np.array([3, 0, 2, 1, 7, 5, 6, 4])
    gi = G.actorder_g_idx(perm, 4)
    assert gi.tolist() == [0, 0, 0, 0, 1, 1, 1, 1]
    # g_idx[perm[r]] == r // 4
    assert all(gi[perm[r]] == r // 4 for r in range(8))


def test_actorder_sort_invariance():
    case = synth.gptq_case(k=512, n=64, m=3, group=128, act_order=True, seed=5)
    qs, perm = G.actorder_sort(case["qweight"], case["g_idx"], 128)
    # sorted channel r is original channel perm[r]; its group is r // 128
    w_orig = G.gptq_dequant(case["qweight"], case["qzeros"], case["scales"], case["g_idx"], 128)
    w_sorted = G.gptq_dequant(qs, case["qzeros"], case["scales"], None, 128)
    assert np.array_equal(w_sorted, w_orig[perm])
    x = bf16_bits_to_f32(case["x_bits"])
    assert np.allclose(G.gemm_f64(x[:, perm], w_sorted), case["y_ref"], rtol=1e-12, atol=1e-9)


def test_actorder_sort_rejects_uneven_groups():
    g_idx = np.array([0] * 9 + [1] * 7, dtype=np.int32)
    qw = np.zeros((2, 8), dtype=np.int32)
    with pytest.raises(ValueError):
        G.actorder_sort(qw, g_idx, 8)


def test_gptq_gemm_against_float64_brute_force():
    case = synth.gptq_case(k=64, n=8, m=2, group=32, act_order=True, seed=8)
    x = bf16_bits_to_f32(case["x_bits"]).astype(np.float64)
    codes = G.unpack_qweight(case["qweight"])
    z = G.unpack_qzeros(case["qzeros"])
    s = case["scales"].view(np.float16).astype(np.float64)
    for m in range(2):
        for n in range(8):
            acc = 0.0
            for k in range(64):
                gg = case["g_idx"][k]
                acc += x[m, k] * (int(codes[k, n]) - int(z[gg, n])) * s[gg, n]
            assert abs(acc - case["y_ref"][m, n]) <= 1e-9 * max(1.0, abs(acc))


# -- torch's tiled int4 tensor (the standalone export's `.q`, export.py:324-334) ---------

_TILE_FIXTURES = Path(__file__).parent / "golden" / "int4pack_fixtures.npz"


def _tile_cases():
    z = np.load(_TILE_FIXTURES, allow_pickle=False)
    for key in sorted(z.files):
        if key.startswith("pre_"):
            tag = key[4:]
            n, k = map(int, tag.split("_t")[0].split("x"))
            yield tag, n, k, int(tag.split("_t")[1]), G.unprepack_u8(z[key]), z["packed_" + tag]


def test_torch_tiles_fixture_provenance():
    z = np.load(_TILE_FIXTURES, allow_pickle=False)
    assert "rocm" in str(z["torch_version"])
    assert {t for t, *_ in _tile_cases()} == {"64x512_t2", "64x512_t4", "64x512_t8", "48x256_t8"}


@pytest.mark.parametrize("case", list(_tile_cases()), ids=lambda c: c[0])
def test_torch_tiles_match_torch_rocm_packer(case):
    # torch's own packer output (tests/golden) decodes to the codes it was given, and the
    # restatement re-packs them to the same words
    tag, n, k, t, codes, packed = case
    assert packed.shape == (n // 8, k // (16 * t), 32, t // 2) and packed.dtype == np.int32
    np.testing.assert_array_equal(G.torch_tiles_unpack(packed, n, k, t), codes)
    np.testing.assert_array_equal(G.torch_tiles_pack(codes, t), packed)


def test_torch_tile_locate_is_a_bijection():
    for n, k, t in ((64, 512, 2), (32, 1024, 4), (48, 768, 8)):
        nn, kk = np.meshgrid(np.arange(n), np.arange(k), indexing="ij")
        word, nib = G.torch_tile_locate(nn.ravel(), kk.ravel(), k, t)
        slots = np.sort(word * 8 + nib)
        np.testing.assert_array_equal(slots, np.arange(n * k))


def test_torch_int4pack_mm_fixture_matches_closed_form():
    # y from torch._weight_int4pack_mm on ROCm (tests/golden) == x @ effective_weight^T:
    # pins the qsz contract (q - 8) * scale + zero together with the tile layout
    z = np.load(_TILE_FIXTURES, allow_pickle=False)
    m, n, k, g, t = (int(v) for v in z["mm_meta"])
    codes = G.unprepack_u8(z["mm_pre"])
    qsz = z["mm_qsz_bits"].view(np.uint16)
    x = bf16_bits_to_f32(z["mm_x_bits"].view(np.uint16))
    y_torch = bf16_bits_to_f32(z["mm_y_bits"].view(np.uint16)).astype(np.float64)
    w = G.effective_weight(codes, qsz, g)
    y = G.gemm_f64(x, w.T)
    rel = np.linalg.norm(y - y_torch) / np.linalg.norm(y)
    assert rel < 1e-2, rel
    # a transposed group order of the metadata does not pass
    w_bad = G.effective_weight(codes, qsz[::-1].copy(), g)
    assert np.linalg.norm(G.gemm_f64(x, w_bad.T) - y_torch) / np.linalg.norm(y) > 5e-2


def test_torch_tile_fixtures_reject_plausible_mistakes():
    # each variant of the tile formula with one plausible slip (nibble bits swapped, the
    # column half-select dropped, the channel-block order transposed) misreads torch's tiles
    tag, n, k, t, codes, packed = next(c for c in _tile_cases() if c[0] == "64x512_t8")
    w = packed.reshape(-1).view(np.uint32)
    nn, kk = np.meshgrid(np.arange(n), np.arange(k), indexing="ij")
    half = t // 2

    def read(word, nib):
        return ((w[word] >> (4 * nib).astype(np.uint32)) & 0xF).astype(np.uint8)

    r, j = kk % 32, (kk % 256) // 32
    b = 2 * (j // half) + ((r >> 3) & 1)
    c = 16 * ((r >> 2) & 1) + nn % 16
    good_nib = ((r >> 1) & 1) | (((r >> 4) & 1) << 1) | ((r & 1) << 2)
    block = nn // 16 * (k // 256) + kk // 256
    word = block * 512 + (b * 32 + c) * half + j % half
    np.testing.assert_array_equal(read(word, good_nib), codes)
    slips = {
        "nibble bits r0/r1 swapped": (word, (r & 1) | (((r >> 4) & 1) << 1) | (((r >> 1) & 1) << 2)),
        "column half-select dropped": (block * 512 + (b * 32 + nn % 16) * half + j % half, good_nib),
        "block order transposed": ((kk // 256 * (n // 16) + nn // 16) * 512
                                   + (b * 32 + c) * half + j % half, good_nib),
    }
    for name, (wd, nb) in slips.items():
        assert (read(wd, nb) != codes).mean() > 0.25, name      # and fails exact equality
