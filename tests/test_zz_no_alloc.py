"""mtl_gptq_gemm_noalloc (split-K scratch in a static device array, no allocation) against
mtl_gptq_gemm with a caller-owned workspace, through the C ABI.

Bar: bit for bit (the same kernels and split plan). Two shapes run in a row, the second
smaller, so the second call reuses an array that holds the first call's partials; the
first shape also runs twice. A shape whose workspace exceeds the array is refused with
MTL_ERR_WORKSPACE before any launch. In a fresh process whose first call of the entry is
made under graph capture, every replay of the graph gives the workspace entry's bits.
"""
import os
import subprocess
import sys

import numpy as np
import pytest
import torch

from moss_tts_lite_amd import _native as N
from moss_tts_lite_amd import ops
from oracle import synth

pytestmark = pytest.mark.gpu


def _operands(dev, m, k, n, group, act_order, seed):
    case = synth.gptq_case(k=k, n=n, m=m, group=group, act_order=act_order, seed=seed,
                           with_ref=False)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    qw, qz = t(case["qweight"]), t(case["qzeros"])
    sc = t(case["scales"].view(np.float16))
    x = t(case["x_bits"].view(np.int16)).view(torch.bfloat16)
    perm = None
    if act_order:
        qw, perm = ops.actorder_prepare(qw, t(case["g_idx"]), group)
    return x, qw, qz, sc, perm


def test_noalloc_gemm_matches_workspace_gemm(dev):
    lib = N.load()
    stream = torch.cuda.current_stream().cuda_stream
    p = lambda v: None if v is None else v.data_ptr()  # noqa: E731
    cases = [(16, 4096, 24576, 128, True, 1), (3, 1024, 512, 32, False, 2)]
    for m, k, n, group, act, seed in cases:
        print(f"noalloc case M={m} K={k} N={n} g={group} act_order={act}", flush=True)
        x, qw, qz, sc, perm = _operands(dev, m, k, n, group, act, seed)
        nbytes = int(lib.mtl_gemm_workspace_bytes(m, k, n, group))
        assert 0 < nbytes <= N.NOALLOC_SCRATCH_BYTES
        ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        N.check(lib.mtl_workspace_init(ws.data_ptr(), nbytes, stream), "workspace init")
        for out_dtype, odt in ((torch.bfloat16, N.OUT_BF16), (torch.float32, N.OUT_F32)):
            y_ref = torch.empty(m, n, dtype=out_dtype, device=dev)
            N.check(lib.mtl_gptq_gemm(x.data_ptr(), m, k, qw.data_ptr(), qz.data_ptr(),
                                      sc.data_ptr(), p(perm), n, group, 0, y_ref.data_ptr(),
                                      odt, ws.data_ptr(), nbytes, stream), "mtl_gptq_gemm")
            for rep in range(2):
                y = torch.full((m, n), float("nan"), dtype=out_dtype, device=dev)
                N.check(lib.mtl_gptq_gemm_noalloc(x.data_ptr(), m, k, qw.data_ptr(),
                                                  qz.data_ptr(), sc.data_ptr(), p(perm), n,
                                                  group, 0, y.data_ptr(), odt, stream),
                        "mtl_gptq_gemm_noalloc")
                torch.cuda.synchronize()
                assert torch.equal(y, y_ref), (m, k, n, out_dtype, rep)


def test_noalloc_gemm_refuses_oversized_workspace(dev):
    lib = N.load()
    m, k, n, group = 16, 12288, 24576, 128
    assert lib.mtl_gemm_workspace_bytes(m, k, n, group) > N.NOALLOC_SCRATCH_BYTES
    x = torch.zeros(m, k, dtype=torch.bfloat16, device=dev)
    qw = torch.zeros(k // 8, n, dtype=torch.int32, device=dev)
    qz = torch.zeros(k // group, n // 8, dtype=torch.int32, device=dev)
    sc = torch.zeros(k // group, n, dtype=torch.float16, device=dev)
    y = torch.zeros(m, n, dtype=torch.bfloat16, device=dev)
    st = lib.mtl_gptq_gemm_noalloc(x.data_ptr(), m, k, qw.data_ptr(), qz.data_ptr(),
                                   sc.data_ptr(), None, n, group, 0, y.data_ptr(), N.OUT_BF16,
                                   torch.cuda.current_stream().cuda_stream)
    assert st == N.MTL_ERR_WORKSPACE
    assert not y.any()


_FIRST_CALL_CAPTURED = r"""
import sys
sys.path.insert(0, sys.argv[1])
import __graft_entry__
__graft_entry__.import_package()
import torch
from moss_tts_lite_amd import _native as N
from tests.test_zz_no_alloc import _operands

dev = torch.device("cuda:0")
lib = N.load()
m, k, n, group = 4, 4096, 6144, 128
print(f"noalloc first call under capture: M={m} K={k} N={n} g={group}", flush=True)
x, qw, qz, sc, perm = _operands(dev, m, k, n, group, True, 3)
nbytes = int(lib.mtl_gemm_workspace_bytes(m, k, n, group))
ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
y_ref = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
stream = torch.cuda.current_stream().cuda_stream
N.check(lib.mtl_gptq_gemm(x.data_ptr(), m, k, qw.data_ptr(), qz.data_ptr(), sc.data_ptr(),
                          perm.data_ptr(), n, group, 0, y_ref.data_ptr(), N.OUT_BF16,
                          ws.data_ptr(), nbytes, stream), "mtl_gptq_gemm")
torch.cuda.synchronize()
y = torch.zeros(m, n, dtype=torch.bfloat16, device=dev)
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g):
    s = torch.cuda.current_stream().cuda_stream
    N.check(lib.mtl_gptq_gemm_noalloc(x.data_ptr(), m, k, qw.data_ptr(), qz.data_ptr(),
                                      sc.data_ptr(), perm.data_ptr(), n, group, 0, y.data_ptr(),
                                      N.OUT_BF16, s), "mtl_gptq_gemm_noalloc (captured)")
torch.cuda.synchronize()
for rep in range(3):
    y.fill_(float("nan"))                 # eager work between the replays
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(y, y_ref), rep
print("replays equal", flush=True)
"""


def test_noalloc_first_call_under_capture(dev):
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", _FIRST_CALL_CAPTURED, root], capture_output=True,
                       text=True, timeout=300)
    print(r.stdout[-2000:], r.stderr[-2000:])
    assert r.returncode == 0
    assert "replays equal" in r.stdout
