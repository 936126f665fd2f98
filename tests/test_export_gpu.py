"""GPU parity of the standalone-export ingestion (moss_tts_lite/export.py:324-334, 691-769)
and of the drop-in int4 operators against torch's own ROCm packer and int4 GEMM.

The export's ``.q`` records are torch's tiled int4 tensors.  Bars: the converted
``[K/8, N]`` words bit-exact against the mtl packer of the same codes (torch's tiles
from the committed fixtures and from torch's packer run live at the model's shapes); the
int4 GEMM on an ingested export within rel-L2 1e-2 of ``torch._weight_int4pack_mm`` on
the export's own tiles (the reference's kernel) and of the oracle's float64 product.
"""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from moss_tts_lite_amd import export as E
from moss_tts_lite_amd import ops
from moss_tts_lite_amd.gptq import W4Dispatch
from oracle import gptq_ref as G
from oracle.bf16 import bf16_bits_to_f32

pytestmark = pytest.mark.gpu

FIX = Path(__file__).parent / "golden" / "int4pack_fixtures.npz"


def _prepack(codes: torch.Tensor) -> torch.Tensor:
    c = codes.to(torch.int32)
    return (c[:, 1::2] | (c[:, 0::2] << 4)).to(torch.uint8).contiguous()


def rel_l2(got, ref):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    return float(np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30))


def test_fixture_tiles_convert_bitwise(dev):
    z = np.load(FIX, allow_pickle=False)
    for key in sorted(k for k in z.files if k.startswith("pre_")):
        tag = key[4:]
        t = int(tag.split("_t")[1])
        print("case", tag, flush=True)
        pre = torch.from_numpy(z[key]).to(dev)
        tiles = torch.from_numpy(z["packed_" + tag]).to(dev)
        got = ops.int4pack_from_torch_tiles(tiles)
        want = ops.convert_weight_to_int4pack(pre, t)
        assert torch.equal(got, want), tag
        # and against the oracle's packer of the codes
        codes = G.unprepack_u8(z[key])
        assert np.array_equal(got.cpu().numpy().reshape(-1).view(np.uint32),
                              G.strip_layout(G.qweight_from_reference_codes(codes))), tag


@pytest.mark.parametrize("n,k,t", [(4096, 4096, 8), (6144, 4096, 8), (4096, 12288, 8),
                                   (24576, 4096, 8), (1024, 4096, 2), (2048, 2048, 4),
                                   (48, 256, 8)])
def test_live_torch_tiles_convert_bitwise(dev, n, k, t):
    print("shape", n, k, t, flush=True)
    g = torch.Generator(device="cpu").manual_seed(n * 7 + k + t)
    codes = torch.randint(0, 16, (n, k), generator=g, dtype=torch.int32).to(dev)
    pre = _prepack(codes)
    tiles = torch.ops.aten._convert_weight_to_int4pack(pre, t)
    assert tuple(tiles.shape) == (n // 8, k // (16 * t), 32, t // 2)
    assert torch.equal(ops.int4pack_from_torch_tiles(tiles), ops.convert_weight_to_int4pack(pre, t))


def test_from_torch_tiles_rejects_bad_input(dev):
    with pytest.raises(RuntimeError):
        ops.int4pack_from_torch_tiles(torch.zeros(8, 4, 32, 4, dtype=torch.int64, device=dev))
    with pytest.raises(RuntimeError):      # N = 56 is not a multiple of 16
        ops.int4pack_from_torch_tiles(torch.zeros(7, 4, 32, 4, dtype=torch.int32, device=dev))
    with pytest.raises(RuntimeError):      # K = 128 is not a multiple of 256
        ops.int4pack_from_torch_tiles(torch.zeros(8, 1, 32, 4, dtype=torch.int32, device=dev))


def test_ingested_export_matches_torch_int4pack_mm(dev, tmp_path):
    from safetensors.torch import save_file
    rng = np.random.default_rng(7)
    shapes = {"o": (512, 1024, 128), "down": (256, 2048, 32)}     # name: (N, K, g)
    recs, ref = {}, {}
    for name, (n, k, g) in shapes.items():
        codes = rng.integers(0, 16, size=(n, k), dtype=np.uint8)
        sc = rng.uniform(0.002, 0.02, size=(k // g, n)).astype(np.float32)
        zr = rng.uniform(-0.1, 0.1, size=(k // g, n)).astype(np.float32)
        qsz = torch.stack([torch.from_numpy(sc), torch.from_numpy(zr)], 2).to(torch.bfloat16)
        tiles = torch.ops.aten._convert_weight_to_int4pack(
            _prepack(torch.from_numpy(codes).to(dev)), 8)
        recs[f"layers.0.{name}.q"] = tiles.cpu().contiguous()
        recs[f"layers.0.{name}.qsz"] = qsz.contiguous()
        ref[name] = (codes, qsz, tiles, g)
    recs["layers.0.self_attn.v_proj.weight"] = torch.zeros(64, 1024, dtype=torch.bfloat16)
    save_file(recs, str(tmp_path / E.Q_FILE))
    (tmp_path / E.META_FILE).write_text(json.dumps({
        "format": E.FORMAT_TAG, "preset_name": "p", "weight_file": {"name": E.Q_FILE},
        "presets": {"p": {"group_size_map": {"0:o": 128, "0:down": 32}, "bf16_linears": []}},
        "quantization": {"method": "gptq", "inner_k_tiles": 8},
        "tool": {"torch": torch.__version__}}))     # the tiles come from this ROCm torch
    meta, weights, state, gmap, keep = E.read_standalone(str(tmp_path))
    # the linears without a record must be kept in bf16 (else the state is incomplete)
    with pytest.raises(KeyError):
        W4Dispatch([{}], w4_group_size=128, bf16_keep=keep, group_size_map=gmap, state=state,
                   device=dev)
    keep = keep + [(0, n) for n in ("q", "k", "v", "gate", "up")]
    disp = W4Dispatch([{}], w4_group_size=128, bf16_keep=keep, group_size_map=gmap,
                      state=state, device=dev)
    for name, (codes, qsz, tiles, g) in ref.items():
        n, k, _ = shapes[name]
        print("linear", name, n, k, g, flush=True)
        x = torch.randn(5, k, generator=torch.Generator().manual_seed(k)).to(torch.bfloat16).to(dev)
        y = disp._linear(x, 0, name).float().cpu().numpy()
        y_torch = torch._weight_int4pack_mm(x, tiles, g, qsz.to(dev)).float().cpu().numpy()
        xb = bf16_bits_to_f32(x.view(torch.int16).cpu().numpy().view(np.uint16))
        y_ref = G.gemm_f64(xb, G.effective_weight(codes, qsz.view(torch.int16).numpy().view(np.uint16), g).T)
        assert rel_l2(y, y_torch) < 1e-2, (name, rel_l2(y, y_torch))
        assert rel_l2(y, y_ref) < 1e-2, (name, rel_l2(y, y_ref))


@pytest.mark.parametrize("m,k,n,g", [(1, 4096, 4096, 128), (1, 4096, 24576, 128),
                                     (1, 12288, 4096, 128), (16, 4096, 6144, 128),
                                     (3, 4096, 4096, 32), (5, 2048, 1024, 64),
                                     (2, 4096, 2048, 256)])
def test_drop_in_matches_torch_int4_operators(dev, m, k, n, g):
    # the reference's two operators on ROCm (fast.py:97-99, 118): torch's packer + int4 GEMM,
    # against the mtl drop-ins on the same pre-pack bytes, qsz and x
    print("shape", m, k, n, g, flush=True)
    gen = torch.Generator().manual_seed(m * 131 + k + n + g)
    codes = torch.randint(0, 16, (n, k), generator=gen, dtype=torch.int32)
    pre = _prepack(codes).to(dev)
    sc = torch.rand(k // g, n, generator=gen) * 0.02 + 0.002
    zr = torch.rand(k // g, n, generator=gen) * 0.2 - 0.1
    qsz = torch.stack([sc, zr], 2).to(torch.bfloat16).to(dev).contiguous()
    x = torch.randn(m, k, generator=gen).to(torch.bfloat16).to(dev)
    y_torch = torch._weight_int4pack_mm(x, torch.ops.aten._convert_weight_to_int4pack(pre, 8), g, qsz)
    y = ops.weight_int4pack_mm(x, ops.convert_weight_to_int4pack(pre, 8), g, qsz)
    assert y.dtype == y_torch.dtype == torch.bfloat16 and y.shape == y_torch.shape
    r = rel_l2(y.float().cpu().numpy(), y_torch.float().cpu().numpy())
    assert r < 1e-2, r


def test_reference_gptq_state_file(dev, tmp_path):
    # A GPTQ state as the reference's calibration writes it (gptq.py:504-509): per linear the
    # torch-packed tiles of pack_fast (gptq.py:66-77, here torch's ROCm packer), qsz, the
    # codes q [N, K] and the scale/zero; saved with torch.save beside its .meta.json
    # (gptq.py:608-626).  Loading it must rebuild the mtl layout from q: the record's
    # "packed" holds torch's tiles, which the mtl kernels do not read.
    from moss_tts_lite_amd.gptq import load_gptq_state
    rng = np.random.default_rng(11)
    shapes = {"q": (512, 1024, 128), "down": (256, 2048, 32)}     # name: (N, K, g)
    state, ref = {0: {}}, {}
    for name, (n, k, g) in shapes.items():
        codes = rng.integers(0, 16, size=(n, k), dtype=np.uint8)
        sc = rng.uniform(0.002, 0.02, size=(n, k // g)).astype(np.float32)
        mn = rng.uniform(-0.1, 0.0, size=(n, k // g)).astype(np.float32)
        qsz = torch.stack([torch.from_numpy(sc), torch.from_numpy(mn + 8 * sc)], -1)
        qsz = qsz.to(torch.bfloat16).transpose(0, 1).contiguous()           # [K/g, N, 2]
        tiles = torch.ops.aten._convert_weight_to_int4pack(
            _prepack(torch.from_numpy(codes).to(dev)), 8).cpu()
        state[0][name] = {"packed": tiles, "qsz": qsz, "q": torch.from_numpy(codes),
                          "scale": torch.from_numpy(sc), "zero": torch.from_numpy(mn),
                          "shape": (n, k)}
        ref[name] = (codes, qsz, tiles, g)
    path = tmp_path / "w4.pt"
    torch.save(state, str(path))
    keep = [f"0:{n}" for n in ("k", "v", "o", "gate", "up")]
    (tmp_path / "w4.pt.meta.json").write_text(json.dumps(
        {"group_size_map": {"0:q": 128, "0:down": 32}, "bf16_linears": keep}))
    st, gmap, kept = load_gptq_state(str(path))
    disp = W4Dispatch([{}], w4_group_size=128, bf16_keep=kept, group_size_map=gmap, state=st,
                      device=dev)
    for name, (codes, qsz, tiles, g) in ref.items():
        n, k, _ = shapes[name]
        print("linear", name, n, k, g, flush=True)
        packed, _ = disp.qlayers[0][name]
        assert tuple(packed.shape) == tuple(tiles.shape)
        assert not torch.equal(packed.cpu(), tiles)       # rebuilt from q, not torch's tiles
        assert torch.equal(packed, ops.convert_weight_to_int4pack(
            _prepack(torch.from_numpy(codes).to(dev)), 8))
        x = torch.randn(3, k, generator=torch.Generator().manual_seed(k)).to(torch.bfloat16).to(dev)
        y = disp._linear(x, 0, name).float().cpu().numpy()
        y_torch = torch._weight_int4pack_mm(x, tiles.to(dev), g, qsz.to(dev)).float().cpu().numpy()
        xb = bf16_bits_to_f32(x.view(torch.int16).cpu().numpy().view(np.uint16))
        y_ref = G.gemm_f64(xb, G.effective_weight(codes, qsz.view(torch.int16).numpy().view(np.uint16), g).T)
        assert rel_l2(y, y_ref) < 1e-2, (name, rel_l2(y, y_ref))
        assert rel_l2(y, y_torch) < 1e-2, (name, rel_l2(y, y_torch))
