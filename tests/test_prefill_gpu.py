"""GPU parity of the prefill path: the prompt-length int4 GEMM over the strip layout.

Bars as for the decode GEMMs: fp32 output within rel-L2 1e-3 of the oracle's float64
product, bf16 output within 1e-2; the residual epilogue bit for bit against a numpy
restatement of bf16(bf16(y) + h) on the fp32 result, SiLU*up within 1 bf16 ulp of
bf16(silu(bf16 g) * bf16 u) (float32 libm differences).
"""
import numpy as np
import pytest
import torch

from moss_tts_lite_amd import ops
from oracle import synth
from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits
from tests.test_gemm_gpu import TOL_BF16, TOL_F32, rel_l2, t_bf16, t_f16, t_i32

pytestmark = pytest.mark.gpu


def strip_linear(case, dev):
    qw = ops.strip_weights(t_i32(case["qweight"], dev))
    sc, qz = ops.strip_meta(t_f16(case["scales"], dev), t_i32(case["qzeros"], dev), case["group"])
    return qw, sc, qz


def run_prefill(case, dev, epilogue="none", out=None, out_dtype=torch.float32, x=None,
                split=True):
    qw, sc, qz = strip_linear(case, dev)
    x = t_bf16(case["x_bits"], dev) if x is None else x
    y = ops.prefill_gemm(x, qw, sc, qz, case["n"], case["group"], epilogue=epilogue, out=out,
                         out_dtype=out_dtype, split=split)
    torch.cuda.synchronize()
    return y


@pytest.mark.parametrize("group,k,n,m", [
    (128, 4096, 1024, 256),     # prompt-length q|k|v / o shaped
    (128, 12288, 256, 33),      # down's K
    (128, 768, 384, 64),        # K / 128 = 6: the 2-block ring
    (256, 2048, 640, 129),      # g = 256: groups span two blocks
    (64, 1024, 256, 70),
    (32, 1024, 128, 65),
    (128, 512, 128, 1),         # one row
])
def test_prefill_gemm_matches_oracle(dev, group, k, n, m):
    case = synth.gptq_case(k=k, n=n, m=m, group=group, act_order=False, seed=group + k + n + m)
    y = run_prefill(case, dev).cpu().numpy()
    err = rel_l2(y, case["y_ref"])
    print(f"prefill g{group} {k}x{n} M={m} rel_l2={err:.2e} "
          f"ws={ops.N.load().mtl_w4_gemm_prefill_workspace_bytes(m, k, n)}")
    assert err < TOL_F32 and np.isfinite(y).all()
    # one pass (no K split) agrees to fp32 rounding
    y1 = run_prefill(case, dev, split=False).cpu().numpy()
    assert rel_l2(y1, case["y_ref"]) < TOL_F32 and rel_l2(y1, y) < 1e-5
    yb = run_prefill(case, dev, out_dtype=torch.bfloat16).float().cpu().numpy()
    assert rel_l2(yb, case["y_ref"]) < TOL_BF16
    # the bf16 output is the fp32 result rounded
    assert np.array_equal(f32_to_bf16_bits(y), f32_to_bf16_bits(yb))


def test_prefill_gemm_gate_up_prompt(dev):
    # the 4096 x 24576 gate|up projection at a 256-token prompt, sampled columns
    cols = np.arange(0, 24576, 97)
    case = synth.gptq_case(k=4096, n=24576, m=256, group=128, seed=5, ref_cols=cols)
    y = run_prefill(case, dev).cpu().numpy()
    err = rel_l2(y[:, cols], case["y_ref"])
    print(f"prefill gate_up M=256 rel_l2={err:.2e}")
    assert err < TOL_F32


def test_prefill_rows_are_independent(dev):
    # each row's products are its own: rows of a batch equal the same rows run alone,
    # bit for bit, and repeated launches agree
    case = synth.gptq_case(k=1024, n=512, m=100, group=128, seed=8)
    y = run_prefill(case, dev).cpu().numpy()
    assert np.array_equal(y, run_prefill(case, dev).cpu().numpy())
    for r0, r1 in ((0, 1), (63, 65), (97, 100)):
        part = dict(case, m=r1 - r0, x_bits=case["x_bits"][r0:r1])
        assert np.array_equal(run_prefill(part, dev).cpu().numpy(), y[r0:r1])


def test_prefill_gemm_strided_rows(dev):
    # x rows ldx apart (a column slice of a wider buffer) and y rows ldy apart
    case = synth.gptq_case(k=1024, n=256, m=40, group=128, seed=9)
    xw = torch.zeros(40, 1024 + 64, dtype=torch.bfloat16, device=dev)
    xw[:, :1024] = t_bf16(case["x_bits"], dev)
    qw, sc, qz = strip_linear(case, dev)
    from moss_tts_lite_amd import _native as N
    out = torch.full((40, 384), 7.0, dtype=torch.float32, device=dev)
    ws = ops.prefill_workspace(dev, 40, 1024, 256)
    assert ws is not None                        # a 2 x 1 grid splits K
    N.check(N.load().mtl_w4_gemm_prefill(
        xw.data_ptr(), 40, xw.stride(0), 1024, qw.data_ptr(), sc.data_ptr(), qz.data_ptr(), 256,
        128, 0, 0, N.OUT_F32, out.data_ptr(), out.stride(0), ws.data_ptr(), ws.numel() * 4,
        torch.cuda.current_stream().cuda_stream), "prefill strided")
    torch.cuda.synchronize()
    o = out.cpu().numpy()
    assert rel_l2(o[:, :256], case["y_ref"]) < TOL_F32
    assert (o[:, 256:] == 7.0).all()


@pytest.mark.parametrize("split", [True, False])
def test_prefill_residual_epilogue(dev, split):
    # the epilogue in the GEMM (one pass) or in the split-sum launch
    case = synth.gptq_case(k=1024, n=512, m=77, group=128, seed=10)
    y = run_prefill(case, dev, split=split).cpu().numpy()
    r = np.random.default_rng(11)
    h_bits = f32_to_bf16_bits(r.standard_normal((77, 512)).astype(np.float32))
    h = t_bf16(h_bits, dev)
    run_prefill(case, dev, epilogue="residual", out=h, split=split)
    rb = lambda v: bf16_bits_to_f32(f32_to_bf16_bits(np.asarray(v, np.float32)))  # noqa: E731
    ref = f32_to_bf16_bits((rb(y) + bf16_bits_to_f32(h_bits)).astype(np.float32))
    assert np.array_equal(h.view(torch.int16).cpu().numpy().view(np.uint16), ref)


@pytest.mark.parametrize("split", [True, False])
def test_prefill_silu_mul_epilogue(dev, split):
    # gate|up interleaved in 32-column blocks; act column 32 b + i = silu(gate) * up
    case = synth.gptq_case(k=1024, n=512, m=50, group=128, seed=12)
    y = run_prefill(case, dev, split=split).cpu().numpy()
    act = run_prefill(case, dev, epilogue="silu_mul", split=split)
    assert act.shape == (50, 256)
    j = np.arange(256)
    gcol = (j // 32) * 64 + j % 32
    rb = lambda v: bf16_bits_to_f32(f32_to_bf16_bits(np.asarray(v, np.float32)))  # noqa: E731
    g = rb(y[:, gcol])
    sg = rb(g / (np.float32(1) + np.exp(-g)))
    ref = f32_to_bf16_bits((sg * rb(y[:, gcol + 32])).astype(np.float32))
    got = act.view(torch.int16).cpu().numpy().view(np.uint16)
    ulps = np.abs(got.astype(np.int32) - ref.astype(np.int32))
    assert ulps.max() <= 1 and np.mean(ulps == 0) > 0.99
