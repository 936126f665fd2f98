"""GPU parity of the int4 GEMV / skinny GEMM and its load-time utilities.

Bars: bit-exact for unpacked codes, packed layouts, act-order index and dequantised
weights; GEMM output within rel-L2 1e-3 (fp32 output, fp32 accumulation) and 1e-2
(bf16 output) of the oracle's float64 product -- the reference's own kernel gate is
rel < 5e-3 at bf16 (tests/test_quant.py:96-119), which the bf16 cases also meet.
"""
import numpy as np
import pytest
import torch

from moss_tts_lite_amd import _native as N
from moss_tts_lite_amd import ops
from oracle import gptq_ref as G
from oracle import synth
from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits

pytestmark = pytest.mark.gpu

TOL_F32 = 1e-3
TOL_BF16 = 1e-2


def t_i32(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int32)).to(dev)


def t_bf16(bits, dev):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).to(dev)


def t_f16(bits, dev):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.float16)).to(dev)


def rel_l2(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30))


def run_gptq(case, dev, act_order, out_dtype=torch.float32, zero_offset=0):
    qw = t_i32(case["qweight"], dev)
    qz = t_i32(case["qzeros"], dev)
    sc = t_f16(case["scales"], dev)
    x = t_bf16(case["x_bits"], dev)
    perm = None
    if act_order:
        qw, perm = ops.actorder_prepare(qw, torch.from_numpy(case["g_idx"]).to(dev), case["group"])
    y = ops.gptq_gemm(x, qw, qz, sc, case["group"], perm=perm, zero_offset=zero_offset,
                      out_dtype=out_dtype)
    torch.cuda.synchronize()
    return y.float().cpu().numpy()


# ------------------------------------------------------------------ bit-exact utilities

def test_unpack_codes_bit_exact(dev):
    r = np.random.default_rng(1)
    qw = synth.random_qweight(r, 512, 264)
    got = ops.unpack_codes(t_i32(qw, dev)).cpu().numpy()
    assert np.array_equal(got, G.unpack_qweight(qw))


@pytest.mark.parametrize("group", [32, 64, 128, 256])
@pytest.mark.parametrize("zero_offset", [0, 1])
def test_gptq_dequant_bit_exact(dev, group, zero_offset):
    case = synth.gptq_case(k=1024, n=136, group=group, seed=group + zero_offset, with_ref=False)
    got = ops.gptq_dequant(t_i32(case["qweight"], dev), t_i32(case["qzeros"], dev),
                           t_f16(case["scales"], dev), group, zero_offset).cpu().numpy()
    ref = G.gptq_dequant(case["qweight"], case["qzeros"], case["scales"], None, group, zero_offset)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("group", [32, 128])
def test_qsz_dequant_bit_exact(dev, group):
    case = synth.qsz_case(k=512, n=96, group=group, seed=group)
    packed = t_i32(G.int4pack_from_prepacked(G.prepack_u8(case["q"])).view(np.int32), dev)
    got = ops.qsz_dequant(packed, t_bf16(case["qsz"], dev), group).cpu().numpy()
    ref = G.effective_weight(case["q"], case["qsz"], group).T
    assert np.array_equal(got.view(np.uint32), np.ascontiguousarray(ref).view(np.uint32))


def test_int4pack_convert_bit_exact(dev):
    r = np.random.default_rng(2)
    q = r.integers(0, 16, size=(208, 512)).astype(np.uint8)      # [N, K]
    pre = G.prepack_u8(q)
    got = ops.convert_weight_to_int4pack(torch.from_numpy(pre).to(dev), 8)
    assert tuple(got.shape) == (208 // 8, 512 // 128, 32, 4) and got.dtype == torch.int32
    words = got.cpu().numpy().reshape(-1).view(np.uint32)
    assert np.array_equal(words, G.int4pack_from_prepacked(pre))
    assert np.array_equal(G.unpack_qweight(G.strip_layout_inverse(words, 512, 208)), q.T)
    # torch's shape for other inner_k_tiles, the same words inside
    for t in (2, 4):
        other = ops.convert_weight_to_int4pack(torch.from_numpy(pre).to(dev), t)
        assert tuple(other.shape) == (26, 512 // (16 * t), 32, t // 2)
        assert torch.equal(other.reshape(-1), got.reshape(-1))
    with pytest.raises(RuntimeError):
        ops.convert_weight_to_int4pack(torch.from_numpy(G.prepack_u8(q[:200])).to(dev), 8)


def test_actorder_prepare_bit_exact(dev):
    case = synth.gptq_case(k=2048, n=264, group=128, act_order=True, seed=3, with_ref=False)
    qs, perm = ops.actorder_prepare(t_i32(case["qweight"], dev),
                                    torch.from_numpy(case["g_idx"]).to(dev), 128)
    ref_qs, ref_perm = G.actorder_sort(case["qweight"], case["g_idx"], 128)
    assert np.array_equal(perm.cpu().numpy(), ref_perm)
    assert np.array_equal(qs.cpu().numpy(), ref_qs)


def test_actorder_prepare_rejects_uneven_groups(dev):
    g_idx = torch.tensor([0] * 160 + [1] * 96, dtype=torch.int32, device=dev)
    qw = torch.zeros(32, 8, dtype=torch.int32, device=dev)
    with pytest.raises(N.MtlError):
        ops.actorder_prepare(qw, g_idx, 128)


# ------------------------------------------------------------------ GEMM parity

@pytest.mark.parametrize("m", [1, 2, 3, 4, 8, 16])
@pytest.mark.parametrize("act_order", [False, True])
def test_gptq_gemm_rows(dev, m, act_order):
    case = synth.gptq_case(k=1024, n=768, m=m, group=128, act_order=act_order, seed=10 + m)
    y = run_gptq(case, dev, act_order)
    err = rel_l2(y, case["y_ref"])
    print(f"gptq M={m} act={act_order} rel_l2={err:.2e}")
    assert err < TOL_F32


@pytest.mark.parametrize("group", [32, 64, 128, 256])
def test_gptq_gemm_groups(dev, group):
    case = synth.gptq_case(k=2048, n=512, m=2, group=group, act_order=True, seed=group)
    for odt, tol in ((torch.float32, TOL_F32), (torch.bfloat16, TOL_BF16)):
        err = rel_l2(run_gptq(case, dev, True, out_dtype=odt), case["y_ref"])
        print(f"gptq g={group} {odt} rel_l2={err:.2e}")
        assert err < tol


@pytest.mark.parametrize("group,k,n", [(32, 1024, 520), (64, 2048, 768), (128, 4096, 1032),
                                      (256, 4608, 264)])
@pytest.mark.parametrize("m", [1, 5])
def test_group_layouts_ragged(dev, group, k, n, m):
    # every row-quads-per-group variant, M = 1 (broadcast A) and M > 1 (padded A), with
    # and without act-order, N not a multiple of the 256-column tile, K not a multiple
    # of the 512-channel split
    for act in (False, True):
        case = synth.gptq_case(k=k, n=n, m=m, group=group, act_order=act, seed=m + group + k)
        err = rel_l2(run_gptq(case, dev, act), case["y_ref"])
        print(f"g={group} K={k} N={n} M={m} act={act} rel_l2={err:.2e}")
        assert err < TOL_F32


@pytest.mark.parametrize("k,n", [(32, 8), (96, 24), (256, 264), (640, 1000), (12288, 264)])
def test_gptq_gemm_ragged_shapes(dev, k, n):
    group = 32
    case = synth.gptq_case(k=k, n=n, m=3, group=group, act_order=False, seed=k + n)
    err = rel_l2(run_gptq(case, dev, False), case["y_ref"])
    print(f"gptq K={k} N={n} rel_l2={err:.2e}")
    assert err < TOL_F32


def test_gptq_zero_offset_v1_checkpoints(dev):
    case = synth.gptq_case(k=512, n=256, m=1, group=128, seed=77, with_ref=False)
    x = bf16_bits_to_f32(case["x_bits"])
    ref = synth.chunked_gptq_gemm(x, case["qweight"], case["qzeros"], case["scales"],
                                  case["g_idx"], 128, zero_offset=1)
    err = rel_l2(run_gptq(case, dev, False, zero_offset=1), ref)
    assert err < TOL_F32


@pytest.mark.parametrize("name,k,n", [("qkv", 4096, 6144), ("o", 4096, 4096),
                                      ("gate_up", 4096, 24576), ("down", 12288, 4096)])
def test_gptq_gemm_full_size_actorder(dev, name, k, n):
    cols = np.random.default_rng(0).choice(n, size=512, replace=False)
    cols.sort()
    case = synth.gptq_case(k=k, n=n, m=1, group=128, act_order=True, seed=1234, ref_cols=cols)
    y = run_gptq(case, dev, True)
    err = rel_l2(y[:, cols], case["y_ref"])
    print(f"{name} K={k} N={n} act-order rel_l2={err:.2e} (512 sampled columns)")
    assert err < TOL_F32
    assert np.isfinite(y).all()


@pytest.mark.parametrize("m", [1, 2, 4, 8, 16])
def test_gate_up_skinny_batch(dev, m):
    cols = np.arange(0, 24576, 48)
    case = synth.gptq_case(k=4096, n=24576, m=m, group=128, act_order=False, seed=99 + m,
                           ref_cols=cols)
    y = run_gptq(case, dev, False)
    err = rel_l2(y[:, cols], case["y_ref"])
    print(f"gate_up M={m} rel_l2={err:.2e}")
    assert err < TOL_F32


def run_strip_rows(case, dev, out_dtype=torch.float32, zero_offset=0):
    qw = ops.strip_weights(t_i32(case["qweight"], dev))
    y = ops.strip_rows_gemm(t_bf16(case["x_bits"], dev), qw, t_i32(case["qzeros"], dev),
                            t_f16(case["scales"], dev), case["n"], case["group"],
                            zero_offset=zero_offset, out_dtype=out_dtype)
    torch.cuda.synchronize()
    return y.float().cpu().numpy()


@pytest.mark.parametrize("m", [1, 2, 3, 8, 16, 21])
def test_strip_rows_gate_up_skinny_batch(dev, m):
    # the full-K strip GEMM on the 4096 x 24576 projection: every row against float64
    # (M = 21 runs as a 16-row and a 5-row launch)
    cols = np.arange(0, 24576, 48)
    case = synth.gptq_case(k=4096, n=24576, m=m, group=128, act_order=False, seed=199 + m,
                           ref_cols=cols)
    y = run_strip_rows(case, dev)
    err = rel_l2(y[:, cols], case["y_ref"])
    print(f"strip rows gate_up M={m} rel_l2={err:.2e}")
    assert err < TOL_F32 and np.isfinite(y).all()
    if 1 < m <= 16:   # one launch: its last row equals the same row alone, bit for bit
        one = dict(case, m=1, x_bits=case["x_bits"][m - 1:m])
        assert np.array_equal(run_strip_rows(one, dev)[0], y[m - 1])


@pytest.mark.parametrize("group,k,n,m", [(128, 1024, 528, 5), (256, 4096, 6144, 16),
                                         (128, 768, 4096, 7), (256, 512, 96, 2),
                                         (32, 1024, 528, 5), (64, 2048, 1536, 16),
                                         (32, 256, 64, 1), (64, 768, 4096, 3)])
def test_strip_rows_shapes(dev, group, k, n, m):
    case = synth.gptq_case(k=k, n=n, m=m, group=group, act_order=False, seed=group + k + n + m)
    y = run_strip_rows(case, dev)
    err = rel_l2(y, case["y_ref"])
    print(f"strip rows g{group} {k}x{n} M={m} rel_l2={err:.2e}")
    assert err < TOL_F32
    yb = run_strip_rows(case, dev, out_dtype=torch.bfloat16, zero_offset=0)
    assert rel_l2(yb, case["y_ref"]) < TOL_BF16
    # repeatable bit for bit, and row r of a batch equals the same row alone (rows do not
    # interact: the same strips, slices and summation order)
    assert np.array_equal(y, run_strip_rows(case, dev))
    one = dict(case, m=1, x_bits=case["x_bits"][m - 1:m])
    assert np.array_equal(run_strip_rows(one, dev)[0], y[m - 1])


@pytest.mark.parametrize("group", [32, 64])
def test_strip_rows_gate_up_small_groups(dev, group):
    # g 32 / 64 on the gate|up projection at 16 rows: 4 / 2 groups per 1 KB block, and at
    # g 32 x, its group sums and the slice tiles fill the 160 KB of LDS
    cols = np.arange(0, 24576, 96)
    case = synth.gptq_case(k=4096, n=24576, m=16, group=group, act_order=False,
                           seed=group + 5, ref_cols=cols)
    y = run_strip_rows(case, dev)
    err = rel_l2(y[:, cols], case["y_ref"])
    print(f"strip rows gate_up g{group} M=16 rel_l2={err:.2e}")
    assert err < TOL_F32 and np.isfinite(y).all()


@pytest.mark.parametrize("group,k,n,m", [(128, 12288, 4096, 16), (32, 12288, 4096, 16),
                                         (256, 8192, 1024, 9), (64, 6144, 512, 2),
                                         (128, 12288, 1024, 1)])
def test_strip_rows_k_phases(dev, group, k, n, m):
    # K beyond what one LDS tile of x holds runs in phases (the down projection's 12288 at
    # 16 rows: three of 4096); every row against float64, and each row of the batch equals
    # the same row run alone (phases keep the summation order per row)
    cols = np.arange(0, n, 7)
    case = synth.gptq_case(k=k, n=n, m=m, group=group, act_order=False, seed=group + k + m,
                           ref_cols=cols)
    y = run_strip_rows(case, dev)
    err = rel_l2(y[:, cols], case["y_ref"])
    print(f"strip rows phases g{group} {k}x{n} M={m} rel_l2={err:.2e}")
    assert err < TOL_F32 and np.isfinite(y).all()
    one = dict(case, m=1, x_bits=case["x_bits"][m - 1:m])
    assert np.array_equal(run_strip_rows(one, dev)[0], y[m - 1])


@pytest.mark.parametrize("group,k,n,m", [(128, 4096, 6144, 8), (32, 2048, 1024, 3),
                                         (128, 12288, 4096, 4), (256, 4096, 512, 16),
                                         (128, 12288, 4096, 1), (128, 4096, 24576, 16)])
def test_strip_rows_act_order(dev, group, k, n, m):
    # act-order weights: the group-sorted copy in the strip layout, x gathered through the
    # act-order index while staging (from x's rows held in LDS where M * K fits beside the
    # tile, else from memory); against float64 on the original (unsorted) weight
    cols = np.arange(0, n, 5)
    case = synth.gptq_case(k=k, n=n, m=m, group=group, act_order=True, seed=3 * group + k + m,
                           ref_cols=cols)
    qws, perm = ops.actorder_prepare(t_i32(case["qweight"], dev), t_i32(case["g_idx"], dev), group)
    args = (ops.strip_weights(qws), t_i32(case["qzeros"], dev), t_f16(case["scales"], dev), n,
            group)
    y = ops.strip_rows_gemm(t_bf16(case["x_bits"], dev), *args, out_dtype=torch.float32,
                            perm=perm).cpu().numpy()
    err = rel_l2(y[:, cols], case["y_ref"])
    print(f"strip rows act-order g{group} {k}x{n} M={m} rel_l2={err:.2e}")
    assert err < TOL_F32
    # the last row alone (x in LDS) is the same row of the batch bit for bit (at M = 16,
    # gathered from memory): the same channels in the same order
    one = ops.strip_rows_gemm(t_bf16(case["x_bits"][m - 1:m], dev), *args,
                              out_dtype=torch.float32, perm=perm).cpu().numpy()
    assert np.array_equal(one[0], y[m - 1])


@pytest.mark.parametrize("group,k,n,m", [(128, 4096, 1024, 16), (32, 4096, 512, 5),
                                         (64, 12288, 256, 16), (256, 2048, 768, 2)])
def test_strip_rows_qsz(dev, group, k, n, m):
    # the reference's (packed, qsz) records: the group adds s * (A - 136 X) + zero * X
    case = synth.qsz_case(k=k, n=n, m=m, group=group, seed=group + m)
    packed = ops.convert_weight_to_int4pack(torch.from_numpy(case["prepacked"]).to(dev), 8)
    y = ops.strip_rows_qsz(t_bf16(case["x_bits"], dev), packed, t_bf16(case["qsz"], dev), group,
                           out_dtype=torch.float32)
    err = rel_l2(y.cpu().numpy(), case["y_ref"])
    print(f"strip rows qsz g{group} {k}x{n} M={m} rel_l2={err:.2e}")
    assert err < TOL_F32


@pytest.mark.parametrize("act_order", [False, True])
@pytest.mark.parametrize("k,n", [(4096, 6144), (2048, 2048)])
def test_gptq_linear_forward_routes(dev, act_order, k, n):
    # the module's forward over 1..21 rows crosses from the skinny strip GEMM to the split-K
    # GEMM (ops.strip_rows_pays); every row count against float64 of the original weight
    from moss_tts_lite_amd.gptq import GPTQLinear
    case = synth.gptq_case(k=k, n=n, m=21, group=128, act_order=act_order, seed=k + n + act_order)
    lin = GPTQLinear.from_buffers(t_i32(case["qweight"], dev), t_i32(case["qzeros"], dev),
                                  t_f16(case["scales"], dev),
                                  t_i32(case["g_idx"], dev) if act_order else None, 128)
    x = t_bf16(case["x_bits"], dev)
    routes = []
    for m in (1, 2, 3, 4, 8, 16, 21):
        routes.append(ops.strip_rows_pays(m, k, n, act_order))
        y = lin(x[:m], out_dtype=torch.float32).cpu().numpy()
        assert rel_l2(y, case["y_ref"][:m]) < TOL_F32, m
    assert any(routes) and not all(routes)


@pytest.mark.parametrize("act_order", [False, True])
def test_gptq_linear_strip_only_forward(dev, act_order):
    # keep_strip_only frees the AutoGPTQ copies: up to 16 rows run on the skinny strip GEMM
    # (the same launches as before, bit for bit), more rows on the prompt-length GEMM over
    # the strip copy (x gathered into the sorted row order); every row count against float64
    from moss_tts_lite_amd.gptq import GPTQLinear
    k, n = 2048, 1024
    case = synth.gptq_case(k=k, n=n, m=40, group=128, act_order=act_order, seed=k + act_order)
    lin = GPTQLinear.from_buffers(t_i32(case["qweight"], dev), t_i32(case["qzeros"], dev),
                                  t_f16(case["scales"], dev),
                                  t_i32(case["g_idx"], dev) if act_order else None, 128)
    x = t_bf16(case["x_bits"], dev)
    rows = (1, 5, 16, 40)
    ref = {m: lin(x[:m], out_dtype=torch.float32) for m in rows}
    lin.keep_strip_only()
    assert lin.qweight.numel() == 0 and lin._kernel_qweight is None and lin._tiled is None
    for m in rows:
        y = lin(x[:m], out_dtype=torch.float32)
        assert rel_l2(y.cpu().numpy(), case["y_ref"][:m]) < TOL_F32, m
        if m == 1 or ops.strip_rows_pays(m, k, n, act_order):
            assert torch.equal(y, ref[m]), m
    with pytest.raises(RuntimeError, match="strip copy"):
        lin.kernel_args()


@pytest.mark.parametrize("group,k,n", [(128, 4096, 24576), (128, 12288, 4096), (32, 4096, 1024),
                                       (64, 2048, 768), (256, 4096, 512), (128, 4096, 6144)])
def test_gemv_strip_act_order_gather(dev, group, k, n):
    # mtl_w4_gemv_strip: x in the checkpoint's channel order, gathered through perm from the
    # LDS copy while staging, gives the same bits as x taken into the sorted row order
    # beforehand and gathered through the identity (the same launch, the same sums), in
    # bf16 and fp32, and the float64 product of the original weight; so does the launch
    # without perm on the sorted x (its own launch shape: within fp32 rounding)
    lib = N.load()
    case = synth.gptq_case(k=k, n=n, m=1, group=group, act_order=True, seed=group + k + n)
    qws, perm = ops.actorder_prepare(t_i32(case["qweight"], dev), t_i32(case["g_idx"], dev), group)
    strip = ops.strip_weights(qws)
    sc, qz = ops.strip_meta(t_f16(case["scales"], dev), t_i32(case["qzeros"], dev), group)
    x = t_bf16(case["x_bits"], dev)[0].contiguous()
    xs = x[perm.long()].contiguous()
    perm16 = perm.to(torch.int16)
    ident16 = torch.arange(k, dtype=torch.int16, device=dev)
    st = torch.cuda.current_stream().cuda_stream
    for odt, dt in ((N.OUT_F32, torch.float32), (N.OUT_BF16, torch.bfloat16)):
        y = torch.full((n,), float("nan"), dtype=dt, device=dev)
        ys = torch.full((n,), float("nan"), dtype=dt, device=dev)
        N.check(lib.mtl_w4_gemv_strip(x.data_ptr(), k, perm16.data_ptr(), strip.data_ptr(),
                                      sc.data_ptr(), qz.data_ptr(), n, group, 0, odt,
                                      y.data_ptr(), st), "gather")
        yn = torch.full((n,), float("nan"), dtype=dt, device=dev)
        N.check(lib.mtl_w4_gemv_strip(xs.data_ptr(), k, ident16.data_ptr(), strip.data_ptr(),
                                      sc.data_ptr(), qz.data_ptr(), n, group, 0, odt,
                                      ys.data_ptr(), st), "sorted x, identity")
        N.check(lib.mtl_w4_gemv_strip(xs.data_ptr(), k, None, strip.data_ptr(), sc.data_ptr(),
                                      qz.data_ptr(), n, group, 0, odt, yn.data_ptr(), st),
                "sorted x, no gather")
        torch.cuda.synchronize()
        assert torch.equal(y, ys), dt
        tol = TOL_F32 if dt == torch.float32 else TOL_BF16
        for out in (y, yn):
            err = rel_l2(out.float().cpu().numpy(), case["y_ref"][0])
            print(f"gemv strip g{group} {k}x{n} {dt} rel_l2={err:.2e}")
            assert err < tol


def test_strip_rows_matches_strip_gemv_at_m1(dev):
    # at M = 1 the skinny kernel and the decode GEMV run different launch shapes; both
    # agree with float64 and with each other within fp32 rounding
    case = synth.gptq_case(k=4096, n=1024, m=1, group=128, seed=77)
    y = run_strip_rows(case, dev)[0]
    ys = _strip_partials(N.load(), case, dev, "bf16", x=t_bf16(case["x_bits"], dev)).cpu().numpy()
    assert rel_l2(y, case["y_ref"][0]) < TOL_F32 and rel_l2(y, ys) < 1e-5


def test_strip_rows_validation(dev):
    lib = N.load()
    st = torch.cuda.current_stream().cuda_stream
    x = torch.zeros(16, 8192, dtype=torch.bfloat16, device=dev)
    w = torch.zeros(8192 * 64 // 8, dtype=torch.int32, device=dev)
    sc = torch.zeros(8192 // 32 * 64, dtype=torch.float16, device=dev)
    qz = torch.zeros(8192 // 32 * 8, dtype=torch.int32, device=dev)
    y = torch.zeros(16, 64, dtype=torch.float32, device=dev)
    call = lambda m, k, g, n=64: lib.mtl_w4_gemm_strip_rows(  # noqa: E731
        x.data_ptr(), m, 8192, k, w.data_ptr(), sc.data_ptr(), qz.data_ptr(), n, g, 0,
        y.data_ptr(), 64, N.OUT_F32, st)
    assert call(4, 4096, 32) == 0                      # g 32 and 64 run here too
    assert call(4, 8192, 128) == 0                     # K in phases
    assert call(4, 4096, 48) == N.MTL_ERR_GROUP
    assert call(17, 4096, 128) == N.MTL_ERR_SHAPE
    assert call(4, 4096, 128, n=72) == N.MTL_ERR_SHAPE
    assert call(4, 4096, 128, n=1 << 20) == N.MTL_ERR_SHAPE   # N * K / 2 reaches 2^31
    ex = lambda fmt, perm, zo: lib.mtl_w4_gemm_strip_rows_ex(  # noqa: E731
        x.data_ptr(), 4, 8192, 4096, perm, w.data_ptr(), sc.data_ptr(), qz.data_ptr(), 64, 128,
        zo, fmt, y.data_ptr(), 64, N.OUT_F32, st)
    assert ex(2, None, 0) == N.MTL_ERR_INVALID_ARG            # no such metadata format
    assert ex(N.META_QSZ, None, 1) == N.MTL_ERR_INVALID_ARG   # qsz has no zero offset
    assert ex(N.META_QSZ, w.data_ptr(), 0) == N.MTL_ERR_INVALID_ARG   # nor an act-order index
    torch.cuda.synchronize()


# ------------------------------------------------------------------ reference contract

@pytest.mark.parametrize("n,k,m", [(512, 512, 8), (1024, 4096, 8), (4096, 4096, 1)])
def test_int4pack_mm_matches_effective_weight(dev, n, k, m):
    # Mirrors the reference's G2 gate (tests/test_quant.py:96-119): kernel vs
    # x.float() @ effective_weight(q, qsz).T, rel < 5e-3.
    case = synth.qsz_case(k=k, n=n, m=m, group=128, seed=n)
    packed = ops.convert_weight_to_int4pack(torch.from_numpy(case["prepacked"]).to(dev), 8)
    y = ops.weight_int4pack_mm(t_bf16(case["x_bits"], dev), packed, 128, t_bf16(case["qsz"], dev))
    assert y.dtype == torch.bfloat16 and tuple(y.shape) == (m, n)
    err = rel_l2(y.float().cpu().numpy(), case["y_ref"])
    print(f"int4pack_mm N={n} K={k} M={m} rel_l2={err:.2e}")
    assert err < 5e-3


def _qsz_weights(r, n, k, g):
    """Reference-contract operands: codes [N, K], qsz bits [K/g, N, 2] (scale, zero)."""
    q = r.integers(0, 16, (n, k), dtype=np.uint8)
    qsz = f32_to_bf16_bits(np.stack([r.uniform(0.002, 0.02, (k // g, n)),
                                     r.uniform(-0.1, 0.1, (k // g, n))], -1).astype(np.float32))
    return q, qsz


@pytest.mark.parametrize("m,k,n,g", [(1, 4096, 24576, 128), (1, 12288, 4096, 32),
                                     (1, 4096, 6144, 64), (1, 2048, 1024, 256),
                                     (1, 16384, 512, 128), (5, 4096, 4096, 128),
                                     (64, 2048, 1024, 32), (3, 1024, 208, 128),
                                     (300, 1024, 256, 256)])
def test_int4pack_mm_paths_match_oracle(dev, m, k, n, g):
    # the drop-in's three paths on the reference's own metadata (qsz read in place): M = 1
    # strip GEMV, M > 1 prompt-length GEMM, and per-row strip GEMVs when N % 128 != 0;
    # against the float64 closed form x @ effective_weight(q, qsz).T on sampled columns
    print("int4pack_mm path", m, k, n, g, flush=True)
    r = np.random.default_rng(m * 7 + k + n + g)
    q, qsz = _qsz_weights(r, n, k, g)
    xb = f32_to_bf16_bits(r.standard_normal((m, k)).astype(np.float32))
    packed = ops.convert_weight_to_int4pack(torch.from_numpy(G.prepack_u8(q)).to(dev), 8)
    y = ops.weight_int4pack_mm(t_bf16(xb, dev), packed, g, t_bf16(qsz, dev))
    assert y.dtype == torch.bfloat16 and tuple(y.shape) == (m, n)
    cols = np.sort(r.choice(n, min(n, 1024), replace=False))
    ref = G.int4pack_mm(bf16_bits_to_f32(xb), q[cols], np.ascontiguousarray(qsz[:, cols]), g)
    err = rel_l2(y.float().cpu().numpy()[:, cols], ref)
    print(f"  rel_l2={err:.2e}")
    assert err < TOL_BF16


def test_int4pack_dim0_concat_is_concat_along_n(dev):
    # moss_tts_lite/fast_native.py:146-161 fuses linears with torch.cat(packed, dim=0) and
    # torch.cat(qsz, dim=1): the concatenated packed words are the packing of the
    # concatenated weights, and the M = 1 GEMM on them is the separate GEMMs side by side
    r = np.random.default_rng(77)
    k, g = 4096, 128
    parts = [_qsz_weights(r, n, k, g) for n in (4096, 1024)]
    packed = [ops.convert_weight_to_int4pack(torch.from_numpy(G.prepack_u8(q)).to(dev), 8)
              for q, _ in parts]
    fused_q = np.concatenate([q for q, _ in parts], 0)
    fused = ops.convert_weight_to_int4pack(torch.from_numpy(G.prepack_u8(fused_q)).to(dev), 8)
    cat = torch.cat(packed, dim=0)
    assert torch.equal(cat, fused)
    qszs = [t_bf16(z, dev) for _, z in parts]
    x = t_bf16(f32_to_bf16_bits(r.standard_normal((1, k)).astype(np.float32)), dev)
    y_fused = ops.weight_int4pack_mm(x, cat, g, torch.cat(qszs, dim=1))
    y_parts = torch.cat([ops.weight_int4pack_mm(x, p, g, z) for p, z in zip(packed, qszs)], 1)
    assert torch.equal(y_fused, y_parts)


def test_int4pack_mm_graph_replay(dev):
    # the drop-in operator under capture at M = 1 (strip GEMV), 8 (skinny strip GEMM) and 40
    # (prompt-length GEMM, its K-split workspace allocated inside the capture), replayed
    # with eager work in between
    r = np.random.default_rng(5)
    k, n, g = 4096, 6144, 128
    q, qsz = _qsz_weights(r, n, k, g)
    packed = ops.convert_weight_to_int4pack(torch.from_numpy(G.prepack_u8(q)).to(dev), 8)
    tq = t_bf16(qsz, dev)
    xs = [t_bf16(f32_to_bf16_bits(r.standard_normal((m, k)).astype(np.float32)), dev)
          for m in (1, 8, 40)]
    eager = [ops.weight_int4pack_mm(x, packed, g, tq) for x in xs]
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = [ops.weight_int4pack_mm(x, packed, g, tq) for x in xs]
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        for a, b in zip(outs, eager):
            assert torch.equal(a, b)
        ops.weight_int4pack_mm(xs[1], packed, g, tq)                 # eager work between


@pytest.mark.parametrize("epilogue", ["none", "residual", "silu_mul"])
@pytest.mark.parametrize("g", [32, 128, 256])
def test_prefill_gemm_qsz_epilogues(dev, epilogue, g):
    # the prompt-length GEMM on the reference's metadata with each epilogue, vs the oracle:
    # residual h = bf16(bf16(acc) + h); silu_mul over 32-column gate|up blocks
    r = np.random.default_rng(g + len(epilogue))
    m, k, n = 37, 2048, 1024
    q, qsz = _qsz_weights(r, n, k, g)
    xb = f32_to_bf16_bits(r.standard_normal((m, k)).astype(np.float32))
    packed = ops.convert_weight_to_int4pack(torch.from_numpy(G.prepack_u8(q)).to(dev), 8)
    acc = G.int4pack_mm(bf16_bits_to_f32(xb), q, qsz, g).astype(np.float32)
    x = t_bf16(xb, dev)
    if epilogue == "none":
        got = ops.prefill_gemm_qsz(x, packed, t_bf16(qsz, dev), g).float().cpu().numpy()
        ref = bf16_bits_to_f32(f32_to_bf16_bits(acc))
    elif epilogue == "residual":
        hb = f32_to_bf16_bits(r.standard_normal((m, n)).astype(np.float32))
        h = t_bf16(hb, dev)
        ops.prefill_gemm_qsz(x, packed, t_bf16(qsz, dev), g, epilogue="residual", out=h)
        got = h.float().cpu().numpy()
        ref = bf16_bits_to_f32(f32_to_bf16_bits(bf16_bits_to_f32(f32_to_bf16_bits(acc))
                                                + bf16_bits_to_f32(hb)))
    else:
        got = ops.prefill_gemm_qsz(x, packed, t_bf16(qsz, dev), g,
                                   epilogue="silu_mul").float().cpu().numpy()
        j = np.arange(n // 2)
        gate = bf16_bits_to_f32(f32_to_bf16_bits(acc[:, (j // 32) * 64 + j % 32]))
        up = bf16_bits_to_f32(f32_to_bf16_bits(acc[:, (j // 32) * 64 + j % 32 + 32]))
        sg = bf16_bits_to_f32(f32_to_bf16_bits(gate / (1.0 + np.exp(-gate))))
        ref = bf16_bits_to_f32(f32_to_bf16_bits(sg * up))
    err = rel_l2(got, ref)
    print(f"prefill qsz {epilogue} g={g}: rel_l2={err:.2e}")
    assert err < TOL_BF16


def test_int4pack_group_sizes_like_g9(dev):
    # reference G9 (tests/test_quant.py:427-457): 32..256 accepted, 16 rejected
    case = synth.qsz_case(k=4096, n=256, m=4, group=128, seed=1)
    packed = ops.convert_weight_to_int4pack(torch.from_numpy(case["prepacked"]).to(dev), 8)
    x = t_bf16(case["x_bits"], dev)
    w = synth.reference_weight(256, 4096, seed=1)
    for g in (32, 64, 128, 256):
        q, s, mn = G.rtn_quantize(w, g)
        qsz = G.pack_qsz(s, mn)
        pk = ops.convert_weight_to_int4pack(torch.from_numpy(G.prepack_u8(q)).to(dev), 8)
        y = ops.weight_int4pack_mm(x, pk, g, t_bf16(qsz, dev)).float().cpu().numpy()
        ref = G.int4pack_mm(bf16_bits_to_f32(case["x_bits"]), q, qsz, g)
        assert rel_l2(y, ref) < 5e-3
    q, s, mn = G.rtn_quantize(w, 16)
    with pytest.raises(RuntimeError):
        ops.weight_int4pack_mm(x, packed, 16, t_bf16(G.pack_qsz(s, mn), dev))


# ------------------------------------------------------------------ fused epilogues

def test_residual_epilogue(dev):
    case = synth.qsz_case(k=1024, n=512, m=1, group=128, seed=5)
    packed = t_i32(G.qweight_from_reference_codes(case["q"]), dev)      # [K/8, N] rows
    x = t_bf16(case["x_bits"], dev).reshape(1, -1)
    resid_bits = f32_to_bf16_bits(np.random.default_rng(6).standard_normal((1, 512)).astype(np.float32))
    resid = t_bf16(resid_bits, dev)
    y = ops.w4_gemm(x, packed, N.META_QSZ, t_bf16(case["qsz"], dev), None, None, 512, 128,
                    epilogue=N.EPI_RESIDUAL, resid=resid)
    # h + linear(x): the linear output is rounded to bf16, then added in fp32 and rounded
    lin = bf16_bits_to_f32(f32_to_bf16_bits(case["y_ref"].astype(np.float32)))
    ref = bf16_bits_to_f32(f32_to_bf16_bits(lin + bf16_bits_to_f32(resid_bits)))
    got = y.float().cpu().numpy()
    assert rel_l2(got, ref) < TOL_BF16
    # in place (y aliases the residual), as the decode step uses it
    y2 = ops.w4_gemm(x, packed, N.META_QSZ, t_bf16(case["qsz"], dev), None, None, 512, 128,
                     epilogue=N.EPI_RESIDUAL, resid=resid, out=resid)
    assert torch.equal(y2, y)


def test_silu_mul_epilogue(dev):
    k, inter = 1024, 256
    case = synth.gptq_case(k=k, n=2 * inter, m=2, group=128, seed=12)
    # interleave gate/up columns in blocks of 32 as the fused layout requires
    order = np.concatenate([np.r_[b * 32:(b + 1) * 32, inter + b * 32:inter + (b + 1) * 32]
                            for b in range(inter // 32)])
    qw = case["qweight"][:, order]
    sc = case["scales"][:, order]
    z = G.unpack_qzeros(case["qzeros"])[:, order]
    qz = G.pack_qzeros(z)
    x = t_bf16(case["x_bits"], dev)
    y = ops.w4_gemm(x, t_i32(qw, dev), N.META_GPTQ, t_f16(sc, dev), t_i32(qz, dev), None,
                    2 * inter, 128, epilogue=N.EPI_SILU_MUL)
    assert tuple(y.shape) == (2, inter)
    yr = case["y_ref"].astype(np.float32)
    g = bf16_bits_to_f32(f32_to_bf16_bits(yr[:, :inter]))
    u = bf16_bits_to_f32(f32_to_bf16_bits(yr[:, inter:]))
    sg = bf16_bits_to_f32(f32_to_bf16_bits(g / (1.0 + np.exp(-g))))
    ref = bf16_bits_to_f32(f32_to_bf16_bits(sg * u))
    err = rel_l2(y.float().cpu().numpy(), ref)
    print(f"silu_mul rel_l2={err:.2e}")
    assert err < TOL_BF16


# ------------------------------------------------------------------ determinism + graphs

def test_deterministic_and_graph_replay(dev):
    case = synth.gptq_case(k=4096, n=24576, m=1, group=128, act_order=True, seed=4, with_ref=False)
    qw, perm = ops.actorder_prepare(t_i32(case["qweight"], dev),
                                    torch.from_numpy(case["g_idx"]).to(dev), 128)
    qz, sc = t_i32(case["qzeros"], dev), t_f16(case["scales"], dev)
    x = t_bf16(case["x_bits"], dev)
    y0 = ops.gptq_gemm(x, qw, qz, sc, 128, perm=perm)
    y1 = ops.gptq_gemm(x, qw, qz, sc, 128, perm=perm)
    assert torch.equal(y0, y1)
    out = torch.empty_like(y0)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ops.w4_gemm(x.reshape(1, -1), qw, N.META_GPTQ, sc, qz, perm, 24576, 128, out=out)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ops.w4_gemm(x.reshape(1, -1), qw, N.META_GPTQ, sc, qz, perm, 24576, 128, out=out)
    for i in range(3):
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, y0), f"replay {i}"
        ops.gptq_gemm(x, qw, qz, sc, 128, perm=perm)   # eager work between replays


def test_module_operators_match_c_entries(dev):
    # torch.ops.mtl.gptq_gemm / strip_rows_gemm (the GPTQ module's eager path) run the C
    # entries' kernels: the same bits, [..., K] in and [..., N] out, 16 rows per launch, and
    # graph capture (the split partials then come from the graph's pool)
    case = synth.gptq_case(k=4096, n=6144, m=21, group=128, act_order=True, seed=21,
                           with_ref=False)
    qws, perm = ops.actorder_prepare(t_i32(case["qweight"], dev),
                                     torch.from_numpy(case["g_idx"]).to(dev), 128)
    qz, sc = t_i32(case["qzeros"], dev), t_f16(case["scales"], dev)
    x = t_bf16(case["x_bits"], dev)
    mtl = ops.torch_ops()
    y_op = mtl.gptq_gemm(x.view(3, 7, 4096), qws, qz, sc, 128, perm, 0, torch.float32)
    y_c = ops.w4_gemm(x, qws, N.META_GPTQ, sc, qz, perm, 6144, 128, out_dtype=torch.float32)
    assert tuple(y_op.shape) == (3, 7, 6144) and torch.equal(y_op.reshape(21, 6144), y_c)
    strip = ops.strip_weights(qws)
    s_op = mtl.strip_rows_gemm(x, strip, qz, sc, 6144, 128, 0, perm, torch.float32)
    s_c = ops.strip_rows_gemm(x, strip, qz, sc, 6144, 128, perm=perm, out_dtype=torch.float32)
    assert torch.equal(s_op, s_c)
    x1 = x[:1]
    eager = mtl.gptq_gemm(x1, qws, qz, sc, 128, perm)
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        mtl.gptq_gemm(x1, qws, qz, sc, 128, perm)
    torch.cuda.current_stream().wait_stream(s)
    with torch.cuda.graph(g):
        out = mtl.gptq_gemm(x1, qws, qz, sc, 128, perm)
    for i in range(3):
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"
        mtl.gptq_gemm(x, qws, qz, sc, 128, perm)       # eager work between replays


# ------------------------------------------------------------------ per-linear dispatch

def test_w4_dispatch_modes(dev):
    # FastMossTTS/GptqMossTTS-style dispatch (fast.py:107-121, gptq.py:689-697): RTN int4
    # at the default group, a per-linear group override, bf16-kept linears and layers.
    # Every reference value comes from the oracle: its RTN codes and qsz of the same bf16
    # weights, the packed words of its restatement of the layout, its dequant.
    from moss_tts_lite_amd.gptq import LIN_NAMES, W4Dispatch
    r = np.random.default_rng(0)
    shapes = {"q": (512, 256), "k": (128, 256), "v": (128, 256), "o": (256, 512),
              "gate": (512, 256), "up": (512, 256), "down": (256, 512)}
    def layer():
        return {n: torch.from_numpy((r.standard_normal(s) * 0.05).astype(np.float32))
                .to(dev).bfloat16() for n, s in shapes.items()}
    layers = [layer() for _ in range(3)]
    orig = [{n: w.float().cpu().numpy() for n, w in lyr.items()} for lyr in layers]
    disp = W4Dispatch(layers, w4_group_size=128, bf16_keep=[2, (1, "down")],
                      group_size_map={(0, "o"): 32, (1, "q"): 64})
    assert disp.qlayers[2] is None and "down" not in disp.qlayers[1]
    assert disp.group_size_map[0]["o"] == 32 and disp.group_size_map[0]["q"] == 128
    x = torch.from_numpy(r.standard_normal((3, 512)).astype(np.float32)).to(dev).bfloat16()
    for li in range(3):
        for name in LIN_NAMES:
            k = shapes[name][1]
            xi = x[:, :k]
            got = disp._linear(xi.reshape(1, 3, k), li, name).float().cpu().numpy()[0]
            xf = xi.float().cpu().numpy().astype(np.float64)
            if disp.qlayers[li] is None or name not in disp.qlayers[li]:
                ref = xf @ orig[li][name].astype(np.float64).T          # bf16 kept
            else:
                g = disp.group_size_map[li][name]
                codes, sc, mn = G.rtn_quantize(orig[li][name], g)
                qsz_o = G.pack_qsz(sc, mn)
                packed, qsz = disp.qlayers[li][name]
                np.testing.assert_array_equal(qsz.view(torch.int16).cpu().numpy().view(np.uint16),
                                              qsz_o)
                np.testing.assert_array_equal(packed.cpu().numpy().reshape(-1).view(np.uint32),
                                              G.int4pack_from_prepacked(G.prepack_u8(codes)))
                ref = xf @ G.effective_weight(codes, qsz_o, g).astype(np.float64).T
            err = rel_l2(got, ref)
            assert err < TOL_BF16, (li, name, err)


@pytest.mark.parametrize("group", [32, 128])
def test_product_rtn_and_qsz_match_oracle(dev, group):
    # gptq.rtn_quantize / pack_qsz_only on the device == the oracle's (gptq.py:35-85) bit for
    # bit: codes, fp32 scale and min, bf16 qsz. The weights include a constant group (the
    # 1e-6 scale floor), a group whose values sit on exact half-steps of the grid (ties to
    # even) and a wide-range group.
    from moss_tts_lite_amd.gptq import pack_qsz_only, rtn_quantize
    r = np.random.default_rng(group)
    n, k = 96, 1024
    w = (r.standard_normal((n, k)) * 0.05).astype(np.float32)
    w[0, :group] = 0.125                                   # constant group
    # min 0, max 15/16: scale exactly 1/16, and the values k/32 land on exact half-steps
    # for odd k (bf16 holds them exactly), so the rounding of ties decides those codes
    w[1, :group] = (np.arange(group) % 31) * 2.0 ** -5
    w[2, :group] *= 100.0                                  # wide range
    wb = torch.from_numpy(w).to(dev).bfloat16()
    w32 = wb.float().cpu().numpy()
    q, sc, mn = rtn_quantize(wb, group)
    qo, so, mno = G.rtn_quantize(w32, group)          # the device form of the span / 15
    # the reference's chain in torch ops on this device (gptq.py:35-64) pins that form
    from tests.test_oracle_gptq import _torch_rtn
    tq, ts, tm = _torch_rtn(wb, group)
    np.testing.assert_array_equal(ts.cpu().numpy(), so)
    np.testing.assert_array_equal(tq.cpu().numpy(), qo)
    np.testing.assert_array_equal(sc.cpu().numpy(), so)
    np.testing.assert_array_equal(mn.cpu().numpy(), mno)
    np.testing.assert_array_equal(q.cpu().numpy(), qo)
    assert float(so[0, 0]) == np.float32(1e-6)
    qsz = pack_qsz_only(sc, mn, group)
    np.testing.assert_array_equal(qsz.view(torch.int16).cpu().numpy().view(np.uint16),
                                  G.pack_qsz(so, mno))


# ------------------------------------------------------------------ tiled weight stream

def _tile_np(qweight: np.ndarray) -> np.ndarray:
    """The documented layout: word l of block ((s*N/64 + cg)*16 + q) = row 64s+4q+l/16,
    columns 64cg+4(l%16)..+3; rows past K/8 zero."""
    rows, n = qweight.shape
    splits = (rows + 63) // 64
    pad = np.zeros((splits * 64, n), np.uint32)
    pad[:rows] = qweight.view(np.uint32)
    t = pad.reshape(splits, 16, 4, n // 64, 16, 4)       # s, q, l/16, cg, l%16, word
    return np.ascontiguousarray(t.transpose(0, 3, 1, 2, 4, 5)).reshape(-1)


@pytest.mark.parametrize("k,n", [(1024, 128), (4608, 320)])
def test_tile_layout_bit_exact(dev, k, n):
    qw = synth.random_qweight(synth.rng(k + n), k, n)
    out = ops.tile_weights(t_i32(qw, dev)).cpu().numpy().view(np.uint32)
    assert np.array_equal(out, _tile_np(qw))


@pytest.mark.parametrize("k,n,src", [(4096, 24576, "norm"), (12288, 4096, "silu"),
                                     (4096, 6144, "norm"), (4096, 4096, "bf16"),
                                     (4608, 320, "bf16")])
def test_tiled_stream_equals_row_stream(dev, k, n, src):
    # same arithmetic, only the weight addresses differ: partials bit for bit
    import ctypes
    lib = N.load()
    case = synth.gptq_case(k=k, n=n, m=1, group=128, seed=k + n, with_ref=False)
    qw, qz, sc = t_i32(case["qweight"], dev), t_i32(case["qzeros"], dev), t_f16(case["scales"], dev)
    tiled = ops.tile_weights(qw)
    r = np.random.default_rng(5)
    S = int(lib.mtl_w4_gemm_splits(k, n))
    st = torch.cuda.current_stream().cuda_stream
    outs = []
    for w, layout in ((qw, N.LAYOUT_ROWS), (tiled, N.LAYOUT_TILED)):
        part = torch.zeros(S * n, dtype=torch.float32, device=dev)
        if src == "norm":
            h = t_bf16(f32_to_bf16_bits(r.standard_normal(k).astype(np.float32)), dev) if not outs else h
            wn = t_bf16(f32_to_bf16_bits(np.ones(k, np.float32)), dev) if not outs else wn
            slots = torch.ones(1024, dtype=torch.float32, device=dev) * 16.0   # sum = k
            N.check(lib.mtl_w4_gemm_norm_partials(h.data_ptr(), wn.data_ptr(), slots.data_ptr(),
                                                  ctypes.c_float(1e-6), k, w.data_ptr(), sc.data_ptr(),
                                                  qz.data_ptr(), n, 128, 0, layout, part.data_ptr(),
                                                  part.numel() * 4, st), "norm partials")
        elif src == "silu":
            xp = torch.from_numpy(r.standard_normal((8, 2 * k)).astype(np.float32)).to(dev) if not outs else xp
            N.check(lib.mtl_w4_gemm_partials(None, xp.data_ptr(), 8, 2 * k, 1, k, w.data_ptr(),
                                             sc.data_ptr(), qz.data_ptr(), None, n, 128, 0, layout,
                                             part.data_ptr(), part.numel() * 4, st), "silu partials")
        else:
            x = t_bf16(case["x_bits"], dev)
            N.check(lib.mtl_w4_gemm_partials(x.data_ptr(), None, 0, 0, 1, k, w.data_ptr(),
                                             sc.data_ptr(), qz.data_ptr(), None, n, 128, 0, layout,
                                             part.data_ptr(), part.numel() * 4, st), "partials")
        outs.append(part)
    assert torch.equal(outs[0], outs[1])


# ------------------------------------------------------------------ full-K strip GEMV

def _strip_np(qweight: np.ndarray) -> np.ndarray:
    """The documented layout: 16-byte word l of 1 KB block (s*K/128 + b) holds the words
    (row 16b + 4j + l/16, column 16s + l%16), j = 0..3."""
    rows, n = qweight.shape
    w = qweight.view(np.uint32).reshape(rows // 16, 4, 4, n // 16, 16)   # b, j, l/16, s, l%16
    return np.ascontiguousarray(w.transpose(3, 0, 2, 4, 1)).reshape(-1)


@pytest.mark.parametrize("k,n", [(1024, 128), (4608, 336)])
def test_strip_layout_bit_exact(dev, k, n):
    qw = synth.random_qweight(synth.rng(k + n + 1), k, n)
    out = ops.strip_weights(t_i32(qw, dev)).cpu().numpy().view(np.uint32)
    assert np.array_equal(out, _strip_np(qw))


def _strip_meta_np(scales_bits, qzeros, k, n, g):
    """The strip order of the group metadata, restated: per strip and 128-channel block
    (block pair at g = 256) the scales of each column contiguously, and the zero nibbles
    of each column packed in column order."""
    z = np.stack([(qzeros.view(np.uint32) >> (4 * j)) & 0xF for j in range(8)], -1)
    z = z.reshape(k // g, n)
    pair = g == 256
    mb = 1 if pair else 128 // g
    krec = k // 256 if pair else k // 128
    sc_out, z_nib = [], []
    for s_ in range(n // 16):
        for i in range(krec):
            grp = [i] if pair else [i * mb + m for m in range(mb)]
            for c in range(16):
                col = 16 * s_ + c
                sc_out += [scales_bits[gg, col] for gg in grp]
                z_nib += [z[gg, col] for gg in grp]
    z_nib = np.array(z_nib, np.uint32)
    packed = (z_nib[0::2] | (z_nib[1::2] << 4)).astype(np.uint8)
    return np.array(sc_out, np.uint16), packed


@pytest.mark.parametrize("group", [32, 64, 128, 256])
def test_strip_meta_layout_bit_exact(dev, group):
    k, n = 1024, 96
    case = synth.gptq_case(k=k, n=n, m=1, group=group, seed=group, with_ref=False)
    sc, qz = ops.strip_meta(t_f16(case["scales"], dev), t_i32(case["qzeros"], dev), group)
    ref_sc, ref_z = _strip_meta_np(case["scales"].view(np.uint16), case["qzeros"], k, n, group)
    assert np.array_equal(sc.cpu().numpy().view(np.uint16).reshape(-1), ref_sc)
    assert np.array_equal(qz.cpu().numpy().view(np.uint8).reshape(-1), ref_z)


def _strip_partials(lib, case, dev, src, x=None, xp=None, h=None, wn=None, slots=None, geom=None):
    """One strip launch through the partials (or norm-partials) entry: fp32 [N]; with
    ``geom`` (a dict of mtl_strip_geometry fields) through its ``_geom`` twin."""
    import ctypes
    k, n, g = case["k"], case["n"], case["group"]
    qw = ops.strip_weights(t_i32(case["qweight"], dev))
    sc, qz = ops.strip_meta(t_f16(case["scales"], dev), t_i32(case["qzeros"], dev), case["group"])
    y = torch.full((n,), float("nan"), dtype=torch.float32, device=dev)
    st = torch.cuda.current_stream().cuda_stream
    extra = () if geom is None else (N.strip_geometry(**geom),)
    if src == "norm":
        fn = lib.mtl_w4_gemm_norm_partials if geom is None else lib.mtl_w4_gemm_norm_partials_geom
        N.check(fn(h.data_ptr(), wn.data_ptr(), slots.data_ptr(), ctypes.c_float(1e-6), k,
                   qw.data_ptr(), sc.data_ptr(), qz.data_ptr(), n, g, 0, N.LAYOUT_STRIP,
                   y.data_ptr(), y.numel() * 4, *extra, st), "strip norm")
    else:
        fn = lib.mtl_w4_gemm_partials if geom is None else lib.mtl_w4_gemm_partials_geom
        N.check(fn(None if x is None else x.data_ptr(), None if xp is None else xp.data_ptr(),
                   0 if xp is None else xp.shape[0], 0 if xp is None else 2 * k,
                   1, k, qw.data_ptr(), sc.data_ptr(), qz.data_ptr(), None, n,
                   g, 0, N.LAYOUT_STRIP, y.data_ptr(), y.numel() * 4, *extra, st),
                "strip partials")
    torch.cuda.synchronize()
    return y


@pytest.mark.parametrize("group,k,n", [(32, 1024, 528), (64, 2048, 768), (128, 4096, 6144),
                                       (128, 12288, 4096), (256, 4096, 4112), (128, 512, 1024)])
def test_strip_gemv_matches_oracle(dev, group, k, n):
    lib = N.load()
    case = synth.gptq_case(k=k, n=n, m=1, group=group, seed=group + k + n)
    y = _strip_partials(lib, case, dev, "bf16", x=t_bf16(case["x_bits"], dev))
    err = rel_l2(y.cpu().numpy(), case["y_ref"][0])
    print(f"strip g{group} {k}x{n} rel_l2={err:.2e}")
    assert err < TOL_F32
    # repeatable bit for bit
    assert torch.equal(y, _strip_partials(lib, case, dev, "bf16", x=t_bf16(case["x_bits"], dev)))


def test_strip_norm_staging_matches_oracle(dev):
    from oracle import decode_ref as D
    from tests._decode_case import slots16
    lib = N.load()
    k, n = 4096, 6144
    case = synth.gptq_case(k=k, n=n, m=1, group=128, seed=77, with_ref=False)
    r = np.random.default_rng(78)
    hf = bf16_bits_to_f32(f32_to_bf16_bits(r.standard_normal(k).astype(np.float32)))
    wf = bf16_bits_to_f32(f32_to_bf16_bits((1 + 0.1 * r.standard_normal(k)).astype(np.float32)))
    h, wn = t_bf16(f32_to_bf16_bits(hf), dev), t_bf16(f32_to_bf16_bits(wf), dev)
    slots = torch.from_numpy(slots16(hf)).to(dev)
    y = _strip_partials(lib, case, dev, "norm", h=h, wn=wn, slots=slots)
    x = D.rms_norm(hf, wf)
    ref = G.gptq_gemm(x[None], case["qweight"], case["qzeros"], case["scales"], case["g_idx"], 128)[0]
    err = rel_l2(y.cpu().numpy(), ref)
    print(f"strip norm-staged rel_l2={err:.2e}")
    assert err < TOL_F32


@pytest.mark.parametrize("fmt,group,n,bn", [("gptq", 128, 6144, 1024), ("gptq", 32, 5120, 1024),
                                            ("qsz", 32, 5120, 1024), ("qsz", 32, 12288, 12288),
                                            ("rows", 128, 4096, 37)])
def test_norm_partials_bf16_one_launch(dev, fmt, group, n, bn):
    # the RMSNorm-staged int4 GEMV and a bf16-kept projection of the same h in one entry
    # (the MOSS step's q|k + v_proj, gate + up_proj): the same bits as the two entries,
    # whether it runs as one launch (strip layouts) or as the two (the split-K layout)
    import ctypes
    from tests._decode_case import slots16
    lib = N.load()
    k = 4096
    r = np.random.default_rng(group + n + bn)
    hf = bf16_bits_to_f32(f32_to_bf16_bits(r.standard_normal(k).astype(np.float32)))
    wf = bf16_bits_to_f32(f32_to_bf16_bits((1 + 0.1 * r.standard_normal(k)).astype(np.float32)))
    h, wn = t_bf16(f32_to_bf16_bits(hf), dev), t_bf16(f32_to_bf16_bits(wf), dev)
    w2 = t_bf16(f32_to_bf16_bits((1 + 0.1 * r.standard_normal(k)).astype(np.float32)), dev)
    slots = torch.from_numpy(slots16(hf)).to(dev)
    bw = t_bf16(f32_to_bf16_bits((r.standard_normal((bn, k)) * 0.05).astype(np.float32)), dev)
    if fmt == "qsz":
        q, qsz = _qsz_weights(r, n, k, group)
        qw = ops.convert_weight_to_int4pack(torch.from_numpy(G.prepack_u8(q)).to(dev), 8)
        meta, qz, layout = t_bf16(qsz, dev), None, N.LAYOUT_STRIP_QSZ
    else:
        case = synth.gptq_case(k=k, n=n, m=1, group=group, seed=n + bn, with_ref=False)
        qw, qz = t_i32(case["qweight"], dev), t_i32(case["qzeros"], dev)
        meta, layout = t_f16(case["scales"], dev), N.LAYOUT_ROWS
        if fmt == "gptq":
            qw = ops.strip_weights(qw)
            meta, qz = ops.strip_meta(meta, qz, group)
            layout = N.LAYOUT_STRIP
    ws = int(lib.mtl_w4_gemm_splits(k, n)) * n if layout == N.LAYOUT_ROWS else n
    st = torch.cuda.current_stream().cuda_stream
    eps = ctypes.c_float(1e-6)
    p = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    y1 = torch.full((ws,), float("nan"), dtype=torch.float32, device=dev)
    b1 = torch.full((bn,), float("nan"), dtype=torch.float32, device=dev)
    N.check(lib.mtl_w4_gemm_norm_partials(h.data_ptr(), wn.data_ptr(), slots.data_ptr(), eps, k,
                                          qw.data_ptr(), meta.data_ptr(), p(qz), n, group, 0,
                                          layout, y1.data_ptr(), ws * 4, st), "norm partials")
    N.check(lib.mtl_bf16_gemv_norm(h.data_ptr(), w2.data_ptr(), slots.data_ptr(), eps,
                                   bw.data_ptr(), bn, k, b1.data_ptr(), st), "bf16 rows")
    y2, b2 = torch.full_like(y1, float("nan")), torch.full_like(b1, float("nan"))
    N.check(lib.mtl_w4_gemm_norm_partials_bf16(h.data_ptr(), wn.data_ptr(), slots.data_ptr(), eps,
                                               k, qw.data_ptr(), meta.data_ptr(), p(qz), n, group,
                                               0, layout, y2.data_ptr(), ws * 4, h.data_ptr(),
                                               w2.data_ptr(), bw.data_ptr(), bn, b2.data_ptr(),
                                               st), "one launch")
    torch.cuda.synchronize()
    assert torch.equal(y1, y2) and torch.equal(b1, b2)
    assert torch.isfinite(y2).all() and torch.isfinite(b2).all()


@pytest.mark.parametrize("xsplits", [1, 8])
def test_strip_silu_staging_matches_split_k(dev, xsplits):
    # same SiLU*up staging (bitwise equal x) as the split-K GEMV; only the fp32 summation
    # order of the product differs
    import ctypes  # noqa: F401
    lib = N.load()
    k, n = 12288, 4096
    case = synth.gptq_case(k=k, n=n, m=1, group=128, seed=91, with_ref=False)
    r = np.random.default_rng(92)
    xp = torch.from_numpy((r.standard_normal((xsplits, 2 * k)) * 0.5).astype(np.float32)).to(dev)
    y = _strip_partials(lib, case, dev, "silu", xp=xp)
    qw, qz, sc = t_i32(case["qweight"], dev), t_i32(case["qzeros"], dev), t_f16(case["scales"], dev)
    S = int(lib.mtl_w4_gemm_splits(k, n))
    part = torch.zeros(S * n, dtype=torch.float32, device=dev)
    N.check(lib.mtl_w4_gemm_partials(None, xp.data_ptr(), xsplits, 2 * k, 1, k, qw.data_ptr(),
                                     sc.data_ptr(), qz.data_ptr(), None, n, 128, 0, N.LAYOUT_ROWS,
                                     part.data_ptr(), part.numel() * 4,
                                     torch.cuda.current_stream().cuda_stream), "split-k silu")
    ref = part.view(S, n).double().sum(0).cpu().numpy()
    err = rel_l2(y.cpu().numpy(), ref)
    print(f"strip silu xsplits={xsplits} vs split-K rel_l2={err:.2e}")
    assert err < 1e-5


@pytest.mark.parametrize("src", ["bf16", "silu"])
def test_strip_residual_epilogue(dev, src):
    # h = bf16(bf16(y) + h) with y the strip GEMV's own sums (store path), the scattered
    # copy and the per-16-column slots, bit for bit; equal to the store path followed by
    # mtl_residual_add over that single split
    from tests._decode_case import slots16
    lib = N.load()
    k, n = (4096, 4096) if src == "bf16" else (12288, 4096)
    case = synth.gptq_case(k=k, n=n, m=1, group=128, seed=5 + k, with_ref=False)
    r = np.random.default_rng(6)
    x = xp = None
    if src == "bf16":
        x = t_bf16(case["x_bits"], dev)
    else:
        xp = torch.from_numpy((r.standard_normal((1, 2 * k)) * 0.5).astype(np.float32)).to(dev)
    y = _strip_partials(lib, case, dev, src, x=x, xp=xp)
    h0f = bf16_bits_to_f32(f32_to_bf16_bits(r.standard_normal(n).astype(np.float32)))
    scatter = torch.from_numpy(r.permutation(n).astype(np.int32)).to(dev)
    qw = ops.strip_weights(t_i32(case["qweight"], dev))
    sc, qz = ops.strip_meta(t_f16(case["scales"], dev), t_i32(case["qzeros"], dev), case["group"])
    st = torch.cuda.current_stream().cuda_stream
    for rep in range(2):
        h = t_bf16(f32_to_bf16_bits(h0f), dev)
        h_ord = torch.zeros(n, dtype=torch.bfloat16, device=dev)
        slots = torch.zeros(1024, dtype=torch.float32, device=dev)
        N.check(lib.mtl_w4_gemm_residual(None if x is None else x.data_ptr(),
                                         None if xp is None else xp.data_ptr(),
                                         0 if xp is None else 1, 0 if xp is None else 2 * k, k,
                                         qw.data_ptr(), sc.data_ptr(), qz.data_ptr(), n, 128, 0,
                                         N.LAYOUT_STRIP, h.data_ptr(), scatter.data_ptr(),
                                         h_ord.data_ptr(), slots.data_ptr(), None, 0, st),
                "strip residual")
        torch.cuda.synchronize()
        yv = y.cpu().numpy()
        hv = bf16_bits_to_f32(f32_to_bf16_bits(
            bf16_bits_to_f32(f32_to_bf16_bits(yv)) + h0f))
        got = h.view(torch.int16).cpu().numpy().view(np.uint16)
        assert np.array_equal(got, f32_to_bf16_bits(hv)), f"rep {rep}"
        ho = np.empty(n, np.uint16)
        ho[scatter.cpu().numpy()] = f32_to_bf16_bits(hv)
        assert np.array_equal(h_ord.view(torch.int16).cpu().numpy().view(np.uint16), ho)
        assert np.array_equal(slots[:n // 16].cpu().numpy(), slots16(hv))
    # the same through mtl_residual_add over the store path's single split
    h2 = t_bf16(f32_to_bf16_bits(h0f), dev)
    o2 = torch.zeros(n, dtype=torch.bfloat16, device=dev)
    s2 = torch.zeros(1024, dtype=torch.float32, device=dev)
    N.check(lib.mtl_residual_add(y.data_ptr(), 1, h2.data_ptr(), scatter.data_ptr(), o2.data_ptr(),
                                 s2.data_ptr(), n, st), "residual_add")
    torch.cuda.synchronize()
    assert torch.equal(h2, h) and torch.equal(o2, h_ord) and torch.equal(s2, slots)


@pytest.mark.parametrize("k,n,nb,rings", [(4096, 1024, 8, (2, 4, 8)), (4096, 1024, 16, (4, 8, 16)),
                                           (12288, 512, 8, (2, 4, 8))])
def test_strip_ring_depth_is_bitwise_neutral(dev, k, n, nb, rings):
    # the load ring (blocks in flight per wave) changes when loads are issued, not the
    # arithmetic: every ring gives the automatic ring's outputs bit for bit
    lib = N.load()
    case = synth.gptq_case(k=k, n=n, m=1, group=128, seed=k + n + nb)
    x = t_bf16(case["x_bits"], dev)
    outs = [_strip_partials(lib, case, dev, "bf16", x=x, geom=dict(nb=nb, ring=r)) for r in rings]
    assert rel_l2(outs[0].cpu().numpy(), case["y_ref"][0]) < TOL_F32
    for o in outs[1:]:
        assert torch.equal(outs[0], o)
    if nb == 8:        # the automatic geometry is one of them
        assert torch.equal(outs[0], _strip_partials(lib, case, dev, "bf16", x=x))


def test_strip_blocks_per_wave_geometry(dev):
    # every launch shape of the strip GEMV computes the same product (rounding aside)
    lib = N.load()
    case = synth.gptq_case(k=4096, n=1024, m=1, group=128, seed=3)
    x = t_bf16(case["x_bits"], dev)
    outs = {nb: _strip_partials(lib, case, dev, "bf16", x=x,
                                geom=None if nb == 0 else dict(nb=nb)).cpu().numpy()
            for nb in (0, 2, 4, 8)}
    for nb, y in outs.items():
        assert rel_l2(y, case["y_ref"][0]) < TOL_F32, nb
    assert np.array_equal(outs[0], outs[8])     # automatic choice for K = 4096


@pytest.mark.parametrize("n,ct,nb", [(2048, 0, 0), (3072, 6, 16)])
def test_strip_norm_silu_epilogue(dev, n, ct, nb):
    # gate|up with RMSNorm staging and the SiLU*up epilogue (one gate|up strip pair per
    # workgroup by default, three with ct = 6): act equals bf16(silu(bf16 g) * bf16 u) of
    # the strip sums taken with the same K slicing (8 blocks per wave for K = 4096 by
    # default, 16 with three pairs), up to the hardware SiLU's rare bf16 neighbour
    # (tests/_decode_case.silu_mul_check), and the float64 oracle within the bf16 bar
    import ctypes
    from oracle import decode_ref as D
    from tests._decode_case import silu_mul_check, slots16
    lib = N.load()
    k = 4096
    case = synth.gptq_case(k=k, n=n, m=1, group=128, seed=123, with_ref=False)
    r = np.random.default_rng(124)
    hf = bf16_bits_to_f32(f32_to_bf16_bits(r.standard_normal(k).astype(np.float32)))
    wf = bf16_bits_to_f32(f32_to_bf16_bits((1 + 0.1 * r.standard_normal(k)).astype(np.float32)))
    h, wn = t_bf16(f32_to_bf16_bits(hf), dev), t_bf16(f32_to_bf16_bits(wf), dev)
    slots = torch.from_numpy(slots16(hf)).to(dev)
    qw = ops.strip_weights(t_i32(case["qweight"], dev))
    sc, qz = ops.strip_meta(t_f16(case["scales"], dev), t_i32(case["qzeros"], dev), case["group"])
    act = torch.zeros(n // 2, dtype=torch.bfloat16, device=dev)
    st = torch.cuda.current_stream().cuda_stream
    assert lib.mtl_w4_gemm_norm_silu(h.data_ptr(), wn.data_ptr(), slots.data_ptr(),
                                     ctypes.c_float(1e-6), k, qw.data_ptr(), sc.data_ptr(),
                                     qz.data_ptr(), n, 128, 0, N.LAYOUT_ROWS, act.data_ptr(),
                                     st) == N.MTL_ERR_UNSUPPORTED
    N.check(lib.mtl_w4_gemm_norm_silu_geom(h.data_ptr(), wn.data_ptr(), slots.data_ptr(),
                                           ctypes.c_float(1e-6), k, qw.data_ptr(), sc.data_ptr(),
                                           qz.data_ptr(), n, 128, 0, N.LAYOUT_STRIP, act.data_ptr(),
                                           N.strip_geometry(ct=ct, nb=nb), st), "norm silu")
    y = _strip_partials(lib, case, dev, "norm", h=h, wn=wn, slots=slots,
                        geom=dict(nb=nb)).cpu().numpy()
    j = np.arange(n // 2)
    gcol = (j // 32) * 64 + j % 32
    got_bits = act.view(torch.int16).cpu().numpy().view(np.uint16)
    same, near = silu_mul_check(got_bits, y[gcol], y[gcol + 32])
    assert near and same > 0.99, same
    x = D.rms_norm(hf, wf)
    y64 = G.gptq_gemm(x[None], case["qweight"], case["qzeros"], case["scales"], case["g_idx"], 128)[0]
    g64, u64 = y64[gcol], y64[gcol + 32]
    ref = g64 / (1 + np.exp(-g64)) * u64
    err = rel_l2(bf16_bits_to_f32(got_bits), ref)
    print(f"strip norm+silu rel_l2={err:.2e}")
    assert err < TOL_BF16
