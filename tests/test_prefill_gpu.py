"""GPU parity of the prefill path: the prompt-length int4 GEMM over the strip layout.

Bars as for the decode GEMMs: fp32 output within rel-L2 1e-3 of the oracle's float64
product, bf16 output within 1e-2; the residual epilogue bit for bit against a numpy
restatement of bf16(bf16(y) + h) on the fp32 result, SiLU*up within 1 bf16 ulp of
bf16(silu(bf16 g) * bf16 u) (float32 libm differences).
"""
import os

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
    from tests._decode_case import silu_mul_check
    got = act.view(torch.int16).cpu().numpy().view(np.uint16)
    same, near = silu_mul_check(got, y[:, gcol], y[:, gcol + 32])
    assert near and same > 0.99, same


# ---------------------------------------------------------------- prompt-row kernels
import ctypes  # noqa: E402

from moss_tts_lite_amd import _native as N  # noqa: E402
from oracle import decode_ref as D  # noqa: E402
from oracle.bf16 import round_bf16  # noqa: E402


def tb(a, dev):
    return torch.from_numpy(f32_to_bf16_bits(np.asarray(a, np.float32)).view(np.int16)).view(torch.bfloat16).to(dev)


def fb(t):
    return t.float().cpu().numpy()


def stream():
    return torch.cuda.current_stream().cuda_stream


@pytest.fixture(scope="module")
def lib():
    return N.load()


def test_rmsnorm_gather_rows_match_rmsnorm(dev, lib):
    # each row bit for bit the single-row RMSNorm kernel's result, gathered by the perm
    r = np.random.default_rng(20)
    rows, n = 5, 4096
    x = round_bf16((3 * r.standard_normal((rows, n))).astype(np.float32))
    w = round_bf16((1 + 0.1 * r.standard_normal(n)).astype(np.float32))
    perm = r.permutation(n).astype(np.int32)
    tx, tw = tb(x, dev), tb(w, dev)
    ref = torch.empty_like(tx)
    N.check(lib.mtl_rmsnorm(tx.data_ptr(), tw.data_ptr(), ref.data_ptr(), rows, n,
                            ctypes.c_float(1e-6), stream()), "rmsnorm")
    tp = torch.from_numpy(perm).to(dev)
    out = torch.zeros(rows, n + 64, dtype=torch.bfloat16, device=dev)
    N.check(lib.mtl_rmsnorm_gather(tx.data_ptr(), n, tw.data_ptr(), tp.data_ptr(), out.data_ptr(),
                                   n + 64, rows, n, ctypes.c_float(1e-6), stream()), "gather")
    assert torch.equal(out[:, :n], ref[:, tp.long()]) and not out[:, n:].any()
    plain = torch.empty_like(tx)
    N.check(lib.mtl_rmsnorm_gather(tx.data_ptr(), n, tw.data_ptr(), None, plain.data_ptr(), n,
                                   rows, n, ctypes.c_float(1e-6), stream()), "plain")
    assert torch.equal(plain, ref)


def test_embed_rows_match_embed_sum(dev, lib):
    r = np.random.default_rng(21)
    tabs = [round_bf16(r.standard_normal((v, 256)).astype(np.float32)) for v in (50, 7, 9)]
    tt = [tb(t, dev) for t in tabs]
    ptrs = torch.tensor([t.data_ptr() for t in tt], dtype=torch.int64, device=dev)
    vocabs = torch.tensor([50, 7, 9], dtype=torch.int64, device=dev)
    ids = torch.tensor([[3, 6, 0], [49, 2, 99], [0, 0, 8], [7, -1, 1]], dtype=torch.int64, device=dev)
    out = torch.empty(4, 256, dtype=torch.bfloat16, device=dev)
    N.check(lib.mtl_embed_rows(ids.data_ptr(), 4, 3, ptrs.data_ptr(), vocabs.data_ptr(), 256,
                               out.data_ptr(), stream()), "embed rows")
    for i in range(4):
        one = torch.empty(256, dtype=torch.bfloat16, device=dev)
        N.check(lib.mtl_embed_sum(ids[i].data_ptr(), 3, ptrs.data_ptr(), vocabs.data_ptr(), 256,
                                  one.data_ptr(), stream()), "embed")
        assert torch.equal(out[i], one)


def test_qk_norm_rope_rows_match_decode_kernel(dev, lib):
    # rows at positions pos0 .. pos0 + L - 1: q out, K/V cache rows bit for bit the
    # single-position kernel's
    r = np.random.default_rng(22)
    H, Hkv, S, L, pos0 = 8, 2, 96, 21, 30
    ld = (H + 2 * Hkv) * 128
    qkv = round_bf16((2 * r.standard_normal((L, ld))).astype(np.float32))
    qn = round_bf16((1 + 0.1 * r.standard_normal(128)).astype(np.float32))
    kn = round_bf16((1 + 0.1 * r.standard_normal(128)).astype(np.float32))
    ocos, osin = D.rope_tables(S, 128)
    cos, sin = tb(ocos, dev), tb(osin, dev)
    tq, tqn, tkn = tb(qkv, dev), tb(qn, dev), tb(kn, dev)
    kc = torch.zeros(Hkv, S, 128, dtype=torch.bfloat16, device=dev)
    vc, kc1, vc1 = torch.zeros_like(kc), torch.zeros_like(kc), torch.zeros_like(kc)
    q_out = torch.zeros(L, H * 128, dtype=torch.bfloat16, device=dev)
    eps = ctypes.c_float(1e-6)
    N.check(lib.mtl_qk_norm_rope_kv_rows(tq.data_ptr(), ld, L, pos0, tqn.data_ptr(), tkn.data_ptr(),
                                         cos.data_ptr(), sin.data_ptr(), q_out.data_ptr(),
                                         kc.data_ptr(), vc.data_ptr(), H, Hkv, 128, S, eps,
                                         stream()), "rows")
    q1 = torch.zeros(H * 128, dtype=torch.bfloat16, device=dev)
    for i in range(L):
        tpos = torch.tensor([pos0 + i], dtype=torch.int64, device=dev)
        N.check(lib.mtl_qk_norm_rope_kv(tq[i].data_ptr(), tqn.data_ptr(), tkn.data_ptr(),
                                        cos.data_ptr(), sin.data_ptr(), tpos.data_ptr(),
                                        q1.data_ptr(), kc1.data_ptr(), vc1.data_ptr(), H, Hkv, 128,
                                        S, eps, stream()), "one")
        assert torch.equal(q_out[i], q1)
    assert torch.equal(kc, kc1) and torch.equal(vc, vc1)
    assert lib.mtl_qk_norm_rope_kv_rows(tq.data_ptr(), ld, L, S - L + 1, tqn.data_ptr(),
                                        tkn.data_ptr(), cos.data_ptr(), sin.data_ptr(),
                                        q_out.data_ptr(), kc.data_ptr(), vc.data_ptr(), H, Hkv,
                                        128, S, eps, stream()) == N.MTL_ERR_SHAPE


@pytest.mark.parametrize("H,Hkv,L,pos0", [(32, 8, 70, 0), (4, 2, 33, 0), (16, 2, 17, 5),
                                          (8, 8, 1, 0), (32, 8, 200, 40)])
def test_prefill_attention_matches_oracle(dev, lib, H, Hkv, L, pos0):
    # causal GQA attention of every row against float64 softmax attention over [0, pos]
    r = np.random.default_rng(H + L + pos0)
    S = pos0 + L + 8
    kc = round_bf16(r.standard_normal((Hkv, S, 128)).astype(np.float32))
    vc = round_bf16(r.standard_normal((Hkv, S, 128)).astype(np.float32))
    q = round_bf16((0.5 * r.standard_normal((L, H, 128))).astype(np.float32))
    perm = r.permutation(H * 128).astype(np.int32)
    tk, tv, tq = tb(kc, dev), tb(vc, dev), tb(q.reshape(L, H * 128), dev)
    tidx = torch.from_numpy(perm).to(dev)
    out = torch.zeros(L, H * 128, dtype=torch.bfloat16, device=dev)
    scale = 1 / np.sqrt(128)
    N.check(lib.mtl_prefill_attention(tq.data_ptr(), tk.data_ptr(), tv.data_ptr(), L, pos0,
                                      out.data_ptr(), H * 128, tidx.data_ptr(), H, Hkv, 128, S,
                                      ctypes.c_float(scale), stream()), "prefill attention")
    got = fb(out)[:, perm].reshape(L, H, 128)       # value c went to column perm[c]
    errs = []
    for i in range(L):
        n = pos0 + i + 1
        errs.append(rel_l2(got[i], D.attention(q[i], kc[:, :n], vc[:, :n], scale)))
    print(f"prefill attention H={H} Hkv={Hkv} L={L} pos0={pos0} max rel_l2={max(errs):.2e}")
    assert max(errs) < 1e-2


def test_prefill_attention_agrees_with_decode_attention(dev, lib):
    # row i equals the decode kernel at position pos0 + i to bf16 rounding
    r = np.random.default_rng(23)
    H, Hkv, S, L = 32, 8, 160, 40
    kc = round_bf16(r.standard_normal((Hkv, S, 128)).astype(np.float32))
    vc = round_bf16(r.standard_normal((Hkv, S, 128)).astype(np.float32))
    q = round_bf16(r.standard_normal((L, H * 128)).astype(np.float32))
    tk, tv, tq = tb(kc, dev), tb(vc, dev), tb(q, dev)
    out = torch.zeros(L, H * 128, dtype=torch.bfloat16, device=dev)
    scale = ctypes.c_float(1 / np.sqrt(128))
    N.check(lib.mtl_prefill_attention(tq.data_ptr(), tk.data_ptr(), tv.data_ptr(), L, 100,
                                      out.data_ptr(), H * 128, None, H, Hkv, 128, S, scale,
                                      stream()), "prefill attention")
    ws = torch.zeros(int(lib.mtl_decode_attention_workspace_bytes(H, 128)), dtype=torch.uint8, device=dev)
    one = torch.empty(H * 128, dtype=torch.bfloat16, device=dev)
    for i in (0, 17, 39):
        tpos = torch.tensor([100 + i], dtype=torch.int64, device=dev)
        N.check(lib.mtl_decode_attention(tq[i].data_ptr(), tk.data_ptr(), tv.data_ptr(),
                                         tpos.data_ptr(), one.data_ptr(), None, H, Hkv, 128, S,
                                         scale, ws.data_ptr(), ws.numel(), stream()), "decode")
        assert rel_l2(fb(out[i]), fb(one)) < 1e-2


# ------------------------------------------------------------------ the whole prefill
def _oracle_prompt(ow, cfg, prompt, model):
    cos, sin = D.rope_tables(cfg.max_seq, 128)
    okc = np.zeros((cfg.n_layers, cfg.n_kv_heads, cfg.max_seq, 128), np.float32)
    ovc = okc.copy()
    for p, t in enumerate(prompt):
        lg, hf, tok = D.decode_step(t, p, ow, okc, ovc, cos, sin, cfg.n_heads, cfg.n_kv_heads, 128)
    return lg, hf, tok, okc, ovc


@pytest.mark.parametrize("v_keep,L", [(False, 37), (False, 1), (True, 23)])
def test_prefill_matches_oracle_and_stepwise(dev, v_keep, L):
    # the batched prompt against the oracle's token-by-token decode of the same prompt:
    # last-row logits, final hidden state and every K/V cache row within the bf16 bar;
    # the device's own stepwise prefill lands on the same caches within that bar too
    from moss_tts_lite_amd.fast import FastDecoder
    from tests._decode_case import build_case, small_config
    cfg = small_config()
    model, ow = build_case(cfg, seed=41 + L, dev=dev, v_keep=v_keep)
    dec = FastDecoder(model)
    prompt = np.random.default_rng(L).integers(0, cfg.vocab, L)
    lg, hf, tok, okc, ovc = _oracle_prompt(ow, cfg, prompt, model)
    dec.prefill(torch.from_numpy(prompt))
    torch.cuda.synchronize()
    errs = {"logits": rel_l2(fb(dec.logits), lg), "h_final": rel_l2(fb(dec.h_final), hf),
            "k": rel_l2(fb(model.k_cache)[:, :, :L], okc[:, :, :L]),
            "v": rel_l2(fb(model.v_cache)[:, :, :L], ovc[:, :, :L])}
    print(f"prefill L={L} v_keep={v_keep} " + " ".join(f"{k}={v:.2e}" for k, v in errs.items()))
    assert max(errs.values()) < 1e-2
    assert int(dec.pos.item()) == L
    srt = np.sort(lg)
    if srt[-1] - srt[-2] > 0.05:
        assert int(dec.ids.item()) == tok
    assert not fb(model.k_cache)[:, :, L:].any()
    kb, vb = model.k_cache.clone(), model.v_cache.clone()
    dec.prefill_stepwise(torch.from_numpy(prompt))
    assert rel_l2(fb(kb), fb(model.k_cache)) < 1e-2 and rel_l2(fb(vb), fb(model.v_cache)) < 1e-2


def test_prefill_then_graph_decode(dev):
    # decode steps after the batched prefill: graph replays equal eager steps bit for bit
    # and the greedy trajectory follows the oracle's where its margin allows
    from moss_tts_lite_amd.fast import FastDecoder
    from tests._decode_case import build_case, small_config
    cfg = small_config()
    model, ow = build_case(cfg, seed=47, dev=dev)
    dec = FastDecoder(model)
    prompt = np.random.default_rng(5).integers(0, cfg.vocab, 29)
    lg, hf, tok, okc, ovc = _oracle_prompt(ow, cfg, prompt, model)
    cos, sin = D.rope_tables(cfg.max_seq, 128)
    dec.prefill(torch.from_numpy(prompt))
    eager = []
    for i in range(4):
        assert int(dec.ids.item()) == tok or np.sort(lg)[-1] - np.sort(lg)[-2] <= 0.05
        dec.ids.fill_(tok)                       # teacher-forced on the oracle's tokens
        dec.run_step()
        eager.append(dec.logits.clone())
        lg, hf, tok = D.decode_step(tok, len(prompt) + i, ow, okc, ovc, cos, sin, cfg.n_heads,
                                    cfg.n_kv_heads, 128)
        assert rel_l2(fb(eager[-1]), lg) < 1e-2
    toks = []
    _, _, t0, okc2, ovc2 = _oracle_prompt(ow, cfg, prompt, model)
    dec.prefill(torch.from_numpy(prompt))
    dec.capture()
    tok = t0
    for i in range(4):
        dec.ids.fill_(tok)
        dec.graph.replay()
        assert torch.equal(dec.logits, eager[i])
        toks.append(tok)
        _, _, tok = D.decode_step(tok, len(prompt) + i, ow, okc2, ovc2, cos, sin, cfg.n_heads,
                                  cfg.n_kv_heads, 128)


@pytest.mark.parametrize("group", [32, 256])
def test_prefill_group_sizes_match_oracle(dev, group):
    # the presets' g32 (and g256) linears through the whole prefill
    from moss_tts_lite_amd.fast import FastDecoder
    from tests._decode_case import build_case, small_config
    cfg = small_config(group_size=group)
    model, ow = build_case(cfg, seed=50 + group, dev=dev)
    dec = FastDecoder(model)
    prompt = np.random.default_rng(group).integers(0, cfg.vocab, 45)
    lg, hf, tok, okc, ovc = _oracle_prompt(ow, cfg, prompt, model)
    dec.prefill(torch.from_numpy(prompt))
    torch.cuda.synchronize()
    errs = [rel_l2(fb(dec.logits), lg), rel_l2(fb(model.k_cache)[:, :, :45], okc[:, :, :45]),
            rel_l2(fb(model.v_cache)[:, :, :45], ovc[:, :, :45])]
    print(f"prefill g{group}: " + " ".join(f"{e:.2e}" for e in errs))
    assert max(errs) < 1e-2


def test_prefill_in_chunks_continues_the_cache(dev):
    # prefill_rows from pos0 > 0 continues a cache: two chunks land where one pass does
    from moss_tts_lite_amd.fast import FastDecoder
    from tests._decode_case import build_case, small_config
    cfg = small_config()
    model, ow = build_case(cfg, seed=60, dev=dev)
    dec = FastDecoder(model)
    prompt = torch.from_numpy(np.random.default_rng(60).integers(0, cfg.vocab, 50))
    model.reset_cache()
    h_one = dec.prefill_rows(prompt.reshape(-1, 1)).clone()
    k_one, v_one = model.k_cache.clone(), model.v_cache.clone()
    model.reset_cache()
    h_a = dec.prefill_rows(prompt[:21].reshape(-1, 1)).clone()
    h_b = dec.prefill_rows(prompt[21:].reshape(-1, 1), pos0=21).clone()
    torch.cuda.synchronize()
    # the first chunk's rows are the same computation; the second attends to the first's
    # cache rows, written bit for bit alike
    assert torch.equal(h_a, h_one[:21])
    assert torch.equal(model.k_cache[:, :, :21], k_one[:, :, :21])
    assert rel_l2(fb(h_b), fb(h_one[21:])) < 1e-2
    assert rel_l2(fb(model.k_cache), fb(k_one)) < 1e-2 and rel_l2(fb(model.v_cache), fb(v_one)) < 1e-2
    with pytest.raises(ValueError):
        dec.prefill_rows(prompt.reshape(-1, 1), pos0=cfg.max_seq - 10)


def test_moss_prefill_matches_stepwise(dev):
    # MOSS rows (1 + n_vq embedding tables): the batched prompt and the step-per-row prompt
    # give the same final hidden state and caches to the bf16 bar, and both leave pos = L
    from moss_tts_lite_amd.fast import FastMossDecoder
    from tests._decode_case import build_case, small_config
    cfg = small_config(vocab=2000, n_vq=4, audio_vocab=1025, audio_pad_code=1024,
                       two_way_ids=(1500, 1777))
    model, ow = build_case(cfg, seed=61, dev=dev)
    dec = FastMossDecoder(model)
    r = np.random.default_rng(61)
    rows = np.concatenate([r.integers(0, cfg.vocab, (19, 1)), r.integers(0, 1025, (19, cfg.n_vq))], 1)
    hb = dec.prefill(torch.from_numpy(rows)).clone()
    kb, vb = model.k_cache.clone(), model.v_cache.clone()
    assert int(dec.pos.item()) == 19
    hs = dec.prefill_stepwise(torch.from_numpy(rows)).clone()
    assert int(dec.pos.item()) == 19
    assert rel_l2(fb(hb), fb(hs)) < 1e-2
    assert rel_l2(fb(kb), fb(model.k_cache)) < 1e-2 and rel_l2(fb(vb), fb(model.v_cache)) < 1e-2


def _meta_weights(meta, m, k, n, dev, seed, group=128):
    """Strip weight, meta and zeros of a random [k, n] int4 linear in either format."""
    if meta == "gptq":
        case = synth.gptq_case(k=k, n=n, m=1, group=group, act_order=False, seed=seed,
                               ref_cols=np.arange(1))
        qw, sc, qz = strip_linear(case, dev)
        return qw, sc, qz, N.META_GPTQ
    from oracle import gptq_ref as G
    from tests.test_gemm_gpu import _qsz_weights
    q, qsz = _qsz_weights(np.random.default_rng(seed), n, k, group)
    packed = ops.convert_weight_to_int4pack(torch.from_numpy(G.prepack_u8(q)).to(dev), 8)
    return packed, t_bf16(qsz, dev), None, N.META_QSZ


@pytest.mark.parametrize("meta", ["gptq", "qsz"])
@pytest.mark.parametrize("m,k,n,splits", [(77, 1024, 512, 4), (256, 4096, 4096, 4),
                                          (33, 12288, 4096, 8), (1, 2048, 1024, 8),
                                          (2048, 1024, 4096, 1)])
def test_residual_rmsnorm_gather_matches_two_launches(dev, lib, meta, m, k, n, splits):
    # the GEMM's split partials, then one launch for the split sum, the residual add and
    # the gathered RMSNorm: bit for bit the GEMM's residual launch followed by
    # mtl_rmsnorm_gather (h and the norm); with one split the partials are the sums
    print("residual+norm", meta, m, k, n, flush=True)
    qw, meta_t, qz, fmt = _meta_weights(meta, m, k, n, dev, seed=m + k + n)
    r = np.random.default_rng(m + n)
    x = tb(r.standard_normal((m, k)), dev)
    h0 = tb(3 * r.standard_normal((m, n)), dev)
    w = tb(1 + 0.1 * r.standard_normal(n), dev)
    perm = torch.from_numpy(r.permutation(n).astype(np.int32)).to(dev)
    eps = ctypes.c_float(1e-6)
    h_a = h0.clone()
    if meta == "gptq":
        ops.prefill_gemm(x, qw, meta_t, qz, n, 128, epilogue="residual", out=h_a)
    else:
        ops.prefill_gemm_qsz(x, qw, meta_t.reshape(k // 128, n, 2), 128, epilogue="residual",
                             out=h_a)
    out_a = torch.empty_like(h0)
    N.check(lib.mtl_rmsnorm_gather(h_a.data_ptr(), n, w.data_ptr(), perm.data_ptr(),
                                   out_a.data_ptr(), n, m, n, eps, stream()), "norm")
    nbytes = int(lib.mtl_w4_gemm_prefill_partials_bytes(m, k, n))
    assert nbytes == splits * m * n * 4
    part = torch.empty(nbytes // 4, dtype=torch.float32, device=dev)
    # one float short of the splits' partials is refused before any launch
    assert lib.mtl_w4_gemm_prefill_partials(
        x.data_ptr(), None, m, k, k, qw.data_ptr(), meta_t.data_ptr(),
        None if qz is None else qz.data_ptr(), n, 128, 0, fmt, part.data_ptr(), nbytes - 4,
        stream()) == N.MTL_ERR_WORKSPACE
    N.check(lib.mtl_w4_gemm_prefill_partials(
        x.data_ptr(), None, m, k, k, qw.data_ptr(), meta_t.data_ptr(),
        None if qz is None else qz.data_ptr(), n, 128, 0, fmt, part.data_ptr(), nbytes,
        stream()), "partials")
    h_b = h0.clone()
    out_b = torch.zeros(m, n + 64, dtype=torch.bfloat16, device=dev)
    N.check(lib.mtl_residual_rmsnorm_gather(part.data_ptr(), splits, nbytes, h_b.data_ptr(),
                                            n, w.data_ptr(), perm.data_ptr(), out_b.data_ptr(),
                                            n + 64, None, m, n, eps, stream()), "residual norm")
    torch.cuda.synchronize()
    assert torch.equal(h_a, h_b) and not torch.equal(h_a, h0)
    assert torch.equal(out_a, out_b[:, :n]) and not out_b[:, n:].any()
    args = (w.data_ptr(), None, out_b.data_ptr(), n + 64, None, m, n, eps, stream())
    assert lib.mtl_residual_rmsnorm_gather(part.data_ptr(), splits, nbytes, h_b.data_ptr(), n,
                                           w.data_ptr(), None, h_b.data_ptr(), n, None, m, n,
                                           eps, stream()) == N.MTL_ERR_INVALID_ARG   # out is h
    assert lib.mtl_residual_rmsnorm_gather(part.data_ptr(), splits, nbytes - 4, h_b.data_ptr(),
                                           n, *args) == N.MTL_ERR_WORKSPACE


@pytest.mark.parametrize("m,part_heads", [(77, 48), (256, 48), (1, 48), (40, 40)])
def test_qk_norm_rope_partials_match_two_launches(dev, lib, m, part_heads):
    # the q|k|v GEMM's split partials summed inside the q/k norm + RoPE + KV write launch:
    # q, the K and V cache rows bit for bit those of the GEMM's split-sum launch followed by
    # mtl_qk_norm_rope_kv_rows; with 40 of 48 heads in the partials the v heads come from a
    # bf16 buffer (a kept v_proj)
    print("qk norm partials", m, part_heads, flush=True)
    H, Hkv, D, S, k, pos0 = 32, 8, 128, 512, 1024, 17
    cols, pcols = (H + 2 * Hkv) * D, part_heads * D
    qw, sc, qz, fmt = _meta_weights("gptq", m, k, pcols, dev, seed=m + pcols)
    r = np.random.default_rng(m)
    x = tb(r.standard_normal((m, k)), dev)
    qn, kn = tb(1 + 0.1 * r.standard_normal(D), dev), tb(1 + 0.1 * r.standard_normal(D), dev)
    from moss_tts_lite_amd.model import rope_tables
    cos, sin = rope_tables(S, D, 1e6, dev)
    qkv = torch.zeros(m, cols, dtype=torch.bfloat16, device=dev)
    if pcols < cols:
        qkv[:, pcols:] = tb(r.standard_normal((m, cols - pcols)), dev)
    ops.prefill_gemm(x, qw, sc, qz, pcols, 128, out=qkv[:, :pcols])
    eps = ctypes.c_float(1e-6)
    outs = []
    for fused in (False, True):
        q = torch.zeros(m, H * D, dtype=torch.bfloat16, device=dev)
        kc = torch.zeros(Hkv, S, D, dtype=torch.bfloat16, device=dev)
        vc = torch.zeros_like(kc)
        tail = (qn.data_ptr(), kn.data_ptr(), cos.data_ptr(), sin.data_ptr(), q.data_ptr(),
                kc.data_ptr(), vc.data_ptr(), H, Hkv, D, S, eps, stream())
        if fused:
            nbytes = int(lib.mtl_w4_gemm_prefill_partials_bytes(m, k, pcols))
            part = torch.empty(nbytes // 4, dtype=torch.float32, device=dev)
            N.check(lib.mtl_w4_gemm_prefill_partials(
                x.data_ptr(), None, m, k, k, qw.data_ptr(), sc.data_ptr(), qz.data_ptr(), pcols,
                128, 0, fmt, part.data_ptr(), nbytes, stream()), "partials")
            splits = nbytes // (m * pcols * 4)
            v_src = qkv.data_ptr() if pcols < cols else None
            N.check(lib.mtl_qk_norm_rope_kv_rows_partials(
                part.data_ptr(), splits, nbytes, pcols, v_src, cols, m, pos0, *tail), "fused")
            assert lib.mtl_qk_norm_rope_kv_rows_partials(
                part.data_ptr(), splits, nbytes - 4, pcols, v_src, cols, m, pos0,
                *tail) == N.MTL_ERR_WORKSPACE
        else:
            N.check(lib.mtl_qk_norm_rope_kv_rows(qkv.data_ptr(), cols, m, pos0, *tail), "rows")
        torch.cuda.synchronize()
        outs.append((q, kc, vc))
    (q1, k1, v1), (q2, k2, v2) = outs
    assert torch.equal(q1, q2) and torch.equal(k1, k2) and torch.equal(v1, v2)
    assert q1.any() and k1[:, pos0:pos0 + m].any() and v1[:, pos0:pos0 + m].any()


@pytest.mark.parametrize("meta,group", [("gptq", 128), ("gptq", 32), ("gptq", 256),
                                        ("qsz", 32), ("qsz", 64), ("qsz", 128)])
@pytest.mark.parametrize("m", [1, 77, 256])
def test_staged_x_matches_plain_x(dev, lib, meta, group, m):
    # the norm's output staged for the GEMM (pair order, 32-channel sums): un-paired it is
    # the natural output, its sums are the rows' group sums, and the GEMM on it gives the
    # bits of the GEMM on the natural rows with the plain, SiLU*up and partials epilogues
    print("staged x", meta, group, m, flush=True)
    k, n = 1024, 512
    qw, meta_t, qz, fmt = _meta_weights(meta, m, k, n, dev, seed=group + m, group=group)
    r = np.random.default_rng(group * 7 + m)
    h = tb(3 * r.standard_normal((m, k)), dev)
    w = tb(1 + 0.1 * r.standard_normal(k), dev)
    perm = torch.from_numpy(r.permutation(k).astype(np.int32)).to(dev) if meta == "gptq" else None
    pp = None if perm is None else perm.data_ptr()
    eps = ctypes.c_float(1e-6)
    x_nat = torch.empty(m, k, dtype=torch.bfloat16, device=dev)
    x_st = torch.empty_like(x_nat)
    sums = torch.empty(m, k // 32, dtype=torch.float32, device=dev)
    N.check(lib.mtl_rmsnorm_gather(h.data_ptr(), k, w.data_ptr(), pp, x_nat.data_ptr(), k, m, k,
                                   eps, stream()), "norm")
    N.check(lib.mtl_rmsnorm_gather_staged(h.data_ptr(), k, w.data_ptr(), pp, x_st.data_ptr(), k,
                                          sums.data_ptr(), m, k, eps, stream()), "staged norm")
    torch.cuda.synchronize()
    unpaired = x_st.view(m, k // 8, 8)[:, :, [0, 2, 4, 6, 1, 3, 5, 7]].reshape(m, k)
    assert torch.equal(unpaired, x_nat)
    ref = x_nat.float().view(m, k // 32, 32).sum(-1)
    assert torch.allclose(sums, ref, rtol=1e-5, atol=1e-4)
    zp = None if qz is None else qz.data_ptr()
    ws = ops.prefill_workspace(dev, m, k, n)
    wsp, wsb = (None, 0) if ws is None else (ws.data_ptr(), ws.numel() * 4)

    def plain(epi, y, odt, ldy):
        if meta == "gptq":
            return lib.mtl_w4_gemm_prefill(x_nat.data_ptr(), m, k, k, qw.data_ptr(),
                                           meta_t.data_ptr(), zp, n, group, 0, epi, odt,
                                           y.data_ptr(), ldy, wsp, wsb, stream())
        return lib.mtl_w4_gemm_prefill_qsz(x_nat.data_ptr(), m, k, k, qw.data_ptr(),
                                           meta_t.data_ptr(), n, group, epi, odt, y.data_ptr(),
                                           ldy, wsp, wsb, stream())

    def staged(epi, y, odt, ldy):
        return lib.mtl_w4_gemm_prefill_staged(x_st.data_ptr(), sums.data_ptr(), m, k, k,
                                              qw.data_ptr(), meta_t.data_ptr(), zp, n, group, 0,
                                              fmt, epi, odt, y.data_ptr(), ldy, wsp, wsb,
                                              stream())
    for epi, odt, cols, dt in ((N.EPI_NONE, N.OUT_F32, n, torch.float32),
                               (N.EPI_SILU_MUL, N.OUT_BF16, n // 2, torch.bfloat16)):
        ya = torch.zeros(m, cols, dtype=dt, device=dev)
        yb = torch.ones(m, cols, dtype=dt, device=dev)
        N.check(plain(epi, ya, odt, cols), "plain")
        N.check(staged(epi, yb, odt, cols), "staged")
        torch.cuda.synchronize()
        assert torch.equal(ya, yb), epi
    nbytes = int(lib.mtl_w4_gemm_prefill_partials_bytes(m, k, n))
    pa = torch.zeros(nbytes // 4, dtype=torch.float32, device=dev)
    pb = torch.ones_like(pa)
    for buf, xp, sp in ((pa, x_nat, None), (pb, x_st, sums.data_ptr())):
        N.check(lib.mtl_w4_gemm_prefill_partials(
            xp.data_ptr(), sp, m, k, k, qw.data_ptr(), meta_t.data_ptr(), zp, n, group, 0, fmt,
            buf.data_ptr(), nbytes, stream()), "partials")
    torch.cuda.synchronize()
    assert torch.equal(pa, pb)


def _prefill_both_ways(dec, model, rows_ids):
    # fused split sums on staged x, then on x the GEMMs stage themselves, then neither: the
    # last two returned (the first checked against the second here)
    out = []
    for fuse, stage in ((True, True), (True, False), (False, False)):
        model.k_cache.zero_()
        model.v_cache.zero_()
        dec.fuse_split_sums, dec.stage_prefill_x = fuse, stage
        h = dec.prefill_rows(rows_ids).clone()
        torch.cuda.synchronize()
        out.append((h, model.k_cache.clone(), model.v_cache.clone()))
    dec.fuse_split_sums, dec.stage_prefill_x = True, True
    assert all(torch.equal(a, b) for a, b in zip(out[0], out[1]))
    return out[1:]


@pytest.mark.parametrize("v_keep,L", [(False, 37), (True, 70), (False, 1)])
def test_prefill_rows_fused_residual_norm_is_bitwise(dev, v_keep, L):
    # prefill_rows with the o/down residual adds fused into the next norms leaves the same
    # residual stream and K/V caches, bit for bit, as the GEMMs' own residual launches
    from moss_tts_lite_amd.fast import FastDecoder
    from tests._decode_case import build_case, small_config
    cfg = small_config(n_layers=3)
    model, _ = build_case(cfg, seed=90 + L, dev=dev, v_keep=v_keep)
    dec = FastDecoder(model)
    prompt = torch.from_numpy(np.random.default_rng(L).integers(0, cfg.vocab, (L, 1)))
    (h1, k1, v1), (h2, k2, v2) = _prefill_both_ways(dec, model, prompt)
    assert torch.equal(h1, h2) and torch.equal(k1, k2) and torch.equal(v1, v2)
    assert k1[:, :, :L].any()


def test_moss_prefill_rows_fused_residual_norm_is_bitwise(dev):
    # the same on the reference's (codes, qsz) records with v_proj and up_proj kept bf16
    from moss_tts_lite_amd.fast import FastMossDecoder
    from tests import _moss_tiny as T
    model = T.dispatch_backbone(T.generate(T.SEED, False), dev, max_seq=64,
                                keep=[(0, "v"), (1, "v"), (0, "up")])
    dec = FastMossDecoder(model)
    assert dec.up_keep[0] and dec.v_keep[0]
    fix = np.load(os.path.join(os.path.dirname(__file__), "golden", "moss_step_fixtures.npz"))
    rows = torch.from_numpy(fix["rows"][:int(fix["prompt_rows"])])
    (h1, k1, v1), (h2, k2, v2) = _prefill_both_ways(dec, model, rows)
    assert torch.equal(h1, h2) and torch.equal(k1, k2) and torch.equal(v1, v2)
