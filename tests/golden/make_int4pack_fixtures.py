"""Known-answer vectors of torch's int4 packer and int4 GEMM on a ROCm GPU.

The reference's standalone export stores each int4 linear as the int32 tensor that
``torch.ops.aten._convert_weight_to_int4pack(pre, inner_k_tiles)`` returns
(moss_tts_lite/export.py:324-334, quantization note at export.py:409-417), where
``pre`` is the nibble pre-pack ``q[:, 1::2] | q[:, 0::2] << 4`` of the codes
(moss_tts_lite/gptq.py:76, fast.py:98).  That tiled layout is torch's own, so this
script runs torch's packer (and ``torch._weight_int4pack_mm``) on a ROCm GPU over
known codes and writes what they return:

- ``int4pack_patterns_<N>x<K>_t<T>.npz`` (analysis, not committed): the packed result
  of seven separable code patterns (nibbles 0..2 of n, nibbles 0..3 of k), so that
  every output nibble names its (n, k);
- ``int4pack_fixtures.npz`` (committed beside this script): random codes (as the
  reference's uint8 pre-pack ``[N, K/2]``) and torch's packed tensor for several
  (N, K, inner_k_tiles), plus one ``_weight_int4pack_mm`` case (x, pre-pack, qsz, y)
  with ``y`` from torch's kernel.

Usage: ``python tests/golden/make_int4pack_fixtures.py OUT_DIR`` on a machine whose
torch has a ROCm GPU.
"""
import os
import sys

import numpy as np
import torch

CASES = [(64, 512, 2), (64, 512, 4), (64, 512, 8), (48, 256, 8)]
PATTERN_SHAPES = [(64, 512, 2), (64, 512, 4), (64, 512, 8), (256, 4096, 8), (128, 1024, 4)]


def prepack(codes: torch.Tensor) -> torch.Tensor:
    """uint8 [N, K/2]: even k in the high nibble (gptq.py:76, fast.py:98)."""
    return (codes[:, 1::2] | (codes[:, 0::2] << 4)).to(torch.uint8)


def pack(codes: np.ndarray, tiles: int) -> np.ndarray:
    pre = prepack(torch.from_numpy(codes.astype(np.int32)).cuda())
    out = torch.ops.aten._convert_weight_to_int4pack(pre.contiguous(), tiles)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def main(out_dir: str) -> int:
    os.makedirs(out_dir, exist_ok=True)
    print("torch", torch.__version__, "hip", torch.version.hip,
          torch.cuda.get_device_name(0), flush=True)
    for n, k, t in PATTERN_SHAPES:
        nn = np.arange(n)[:, None] + np.zeros((1, k), np.int64)
        kk = np.arange(k)[None, :] + np.zeros((n, 1), np.int64)
        pats = {"n0": nn & 15, "n1": (nn >> 4) & 15, "n2": (nn >> 8) & 15,
                "k0": kk & 15, "k1": (kk >> 4) & 15, "k2": (kk >> 8) & 15, "k3": (kk >> 12) & 15}
        try:
            res = {name: pack(c, t) for name, c in pats.items()}
        except RuntimeError as e:
            print(f"patterns {n}x{k} t{t}: {e}".splitlines()[0], flush=True)
            continue
        shape = next(iter(res.values())).shape
        np.savez_compressed(os.path.join(out_dir, f"int4pack_patterns_{n}x{k}_t{t}.npz"), **res)
        print(f"patterns {n}x{k} t{t}: packed {shape} {next(iter(res.values())).dtype}", flush=True)

    rng = np.random.default_rng(20261202)
    fx = {}
    for n, k, t in CASES:
        codes = rng.integers(0, 16, size=(n, k), dtype=np.uint8)
        try:
            packed = pack(codes, t)
        except RuntimeError as e:
            print(f"case {n}x{k} t{t}: {e}".splitlines()[0], flush=True)
            continue
        tag = f"{n}x{k}_t{t}"
        fx[f"pre_{tag}"] = prepack(torch.from_numpy(codes.astype(np.int32))).numpy()
        fx[f"packed_{tag}"] = packed
        print(f"case {tag}: packed {packed.shape}", flush=True)

    # torch._weight_int4pack_mm(x, packed, group, qsz): qsz [K/g, N, 2] bf16 = (scale, zero)
    m, n, k, g, t = 3, 64, 512, 128, 8
    codes = rng.integers(0, 16, size=(n, k), dtype=np.uint8)
    scale = torch.from_numpy(rng.uniform(0.002, 0.02, size=(k // g, n)).astype(np.float32))
    zero = torch.from_numpy(rng.uniform(-0.1, 0.1, size=(k // g, n)).astype(np.float32))
    qsz = torch.stack([scale, zero], dim=2).to(torch.bfloat16).cuda().contiguous()
    x = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).to(torch.bfloat16).cuda()
    packed = torch.from_numpy(pack(codes, t)).cuda()
    try:
        y = torch._weight_int4pack_mm(x, packed, g, qsz)
        torch.cuda.synchronize()
        fx["mm_x_bits"] = x.view(torch.int16).cpu().numpy()
        fx["mm_pre"] = prepack(torch.from_numpy(codes.astype(np.int32))).numpy()
        fx["mm_qsz_bits"] = qsz.view(torch.int16).cpu().numpy()
        fx["mm_y_bits"] = y.view(torch.int16).cpu().numpy()
        fx["mm_meta"] = np.array([m, n, k, g, t], np.int64)
        print(f"mm case: y {tuple(y.shape)} {y.dtype}", flush=True)
    except RuntimeError as e:
        print(f"mm case: {e}".splitlines()[0], flush=True)
    fx["torch_version"] = np.array(torch.__version__)
    fx["device"] = np.array(torch.cuda.get_device_name(0))
    np.savez_compressed(os.path.join(out_dir, "int4pack_fixtures.npz"), **fx)
    print("wrote", os.path.join(out_dir, "int4pack_fixtures.npz"), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1] if len(sys.argv) > 1 else "."))
