"""The C-ABI library loads, exports every symbol the headers declare, and rejects bad
arguments with the documented status codes before touching a device (CPU only)."""
import ctypes

import pytest

from moss_tts_lite_amd import _native as N


@pytest.fixture(scope="module")
def lib():
    return N.load()


def test_every_header_symbol_is_exported(lib):
    names = N.header_symbols()
    assert len(names) >= 10
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_every_header_symbol_has_a_signature():
    # ctypes without argtypes would pass Python ints as 32-bit C ints (truncated pointers)
    missing = [n for n in N.header_symbols() if n not in N._SIGNATURES]
    assert not missing, missing


def test_every_bound_symbol_is_declared():
    declared = set(N.header_symbols())
    undeclared = [n for n in N._SIGNATURES if n not in declared]
    assert not undeclared, undeclared


def test_no_process_wide_tuning_state(lib):
    # launch shapes travel as arguments (mtl_strip_geometry), never as library state
    names = set(N.header_symbols()) | set(N._SIGNATURES)
    assert not [n for n in names if n.startswith("mtl_tune_")]
    assert not hasattr(lib, "mtl_tune_set_strip_nb")


def test_status_strings(lib):
    assert lib.mtl_status_string(0) == b"ok"
    assert lib.mtl_status_string(N.MTL_ERR_GROUP) == b"unsupported group size"
    assert lib.mtl_abi_version() == 1


def test_workspace_bytes(lib):
    # 16 KB tile counters + split partials: one split per 512 input channels, M x N fp32
    assert lib.mtl_gemm_workspace_bytes(1, 4096, 24576, 128) == 16384 + 8 * 24576 * 4
    assert lib.mtl_gemm_workspace_bytes(3, 12288, 4096, 128) == 16384 + 24 * 3 * 4096 * 4
    assert lib.mtl_gemm_workspace_bytes(0, 4096, 4096, 128) == 0
    assert lib.mtl_gemm_workspace_bytes(17, 4096, 4096, 128) == 0


FAKE = ctypes.c_void_p(0x1000)   # never dereferenced: every call below fails validation


@pytest.mark.parametrize("group,expect", [(16, N.MTL_ERR_GROUP), (96, N.MTL_ERR_GROUP),
                                          (512, N.MTL_ERR_GROUP)])
def test_gemm_rejects_group_sizes(lib, group, expect):
    st = lib.mtl_gptq_gemm(FAKE, 1, 4096, FAKE, FAKE, FAKE, None, 4096, group, 0, FAKE, 0,
                           None, 0, None)
    assert st == expect


def test_gemm_rejects_bad_shapes(lib):
    args = lambda m, k, n: lib.mtl_gptq_gemm(FAKE, m, k, FAKE, FAKE, FAKE, None, n, 128, 0,  # noqa: E731
                                             FAKE, 0, None, 0, None)
    assert args(0, 4096, 4096) == N.MTL_ERR_SHAPE
    assert args(17, 4096, 4096) == N.MTL_ERR_SHAPE
    assert args(1, 4000, 4096) == N.MTL_ERR_SHAPE     # K not a multiple of the group
    assert args(1, 4096, 4100) == N.MTL_ERR_SHAPE     # N not a multiple of 8


def test_gemm_rejects_null_and_misaligned(lib):
    assert lib.mtl_gptq_gemm(None, 1, 4096, FAKE, FAKE, FAKE, None, 4096, 128, 0, FAKE, 0,
                             None, 0, None) == N.MTL_ERR_INVALID_ARG
    odd = ctypes.c_void_p(0x1008)
    assert lib.mtl_gptq_gemm(FAKE, 1, 4096, odd, FAKE, FAKE, None, 4096, 128, 0, FAKE, 0,
                             None, 0, None) == N.MTL_ERR_ALIGN


def test_gemm_needs_workspace_for_split_k(lib):
    # 4096 x 24576 splits K across workgroups, so a missing workspace is an error
    st = lib.mtl_gptq_gemm(FAKE, 1, 4096, FAKE, FAKE, FAKE, None, 24576, 128, 0, FAKE, 0,
                           None, 0, None)
    assert st == N.MTL_ERR_WORKSPACE


def test_fused_epilogue_validation(lib):
    st = lib.mtl_w4_gemm_fused(FAKE, 1, 4096, FAKE, N.META_QSZ, FAKE, None, None, 4128, 128, 0,
                               N.EPI_SILU_MUL, None, FAKE, 0, None, 0, None)
    assert st == N.MTL_ERR_SHAPE        # SiLU*up pairs need N % 64 == 0
    st = lib.mtl_w4_gemm_fused(FAKE, 1, 4096, FAKE, N.META_QSZ, FAKE, None, None, 4096, 128, 0,
                               N.EPI_RESIDUAL, None, FAKE, 0, None, 0, None)
    assert st == N.MTL_ERR_INVALID_ARG  # residual epilogue without a residual
    st = lib.mtl_w4_gemm_fused(FAKE, 1, 4096, FAKE, N.META_QSZ, FAKE, None, FAKE, 4096, 128, 0,
                               N.EPI_NONE, None, FAKE, 0, None, 0, None)
    assert st == N.MTL_ERR_INVALID_ARG  # act-order gather is a GPTQ-meta feature


def test_decode_entry_validation(lib):
    import ctypes as C
    eps = C.c_float(1e-6)
    assert lib.mtl_rmsnorm(FAKE, FAKE, FAKE, 1, 4100, eps, None) == N.MTL_ERR_SHAPE
    assert lib.mtl_rmsnorm(None, FAKE, FAKE, 1, 4096, eps, None) == N.MTL_ERR_INVALID_ARG
    assert lib.mtl_qk_norm_rope_kv(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 32, 8, 64,
                                   64, eps, None) == N.MTL_ERR_UNSUPPORTED
    assert lib.mtl_qk_norm_rope_kv(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 32, 6, 128,
                                   64, eps, None) == N.MTL_ERR_SHAPE
    assert lib.mtl_decode_attention_workspace_bytes(32, 128) == 1024 + 32 * 64 * 132 * 4
    assert lib.mtl_decode_attention(FAKE, FAKE, FAKE, FAKE, FAKE, None, 32, 8, 128, 2048,
                                    C.c_float(0.1), None, 0, None) == N.MTL_ERR_WORKSPACE
    # 128 kv heads would reach the placement word at byte 1016 of the counter area
    assert lib.mtl_decode_attention(FAKE, FAKE, FAKE, FAKE, FAKE, None, 128, 128, 128, 2048,
                                    C.c_float(0.1), FAKE, 1 << 30, None) == N.MTL_ERR_SHAPE
    assert lib.mtl_decode_attention_set_handoff(2) == N.MTL_ERR_INVALID_ARG
    assert lib.mtl_decode_attention_set_handoff(1) == N.MTL_OK
    assert lib.mtl_residual_rmsnorm(None, 0, FAKE, FAKE, FAKE, FAKE, None, 4098, eps,
                                    None) == N.MTL_ERR_SHAPE
    assert lib.mtl_residual_rmsnorm(FAKE, 0, FAKE, FAKE, FAKE, FAKE, None, 4096, eps,
                                    None) == N.MTL_ERR_SHAPE
    assert lib.mtl_w4_gemm_splits(4096, 24576) == 8 and lib.mtl_w4_gemm_splits(12288, 4096) == 24
    # partials entry: x and xpart are exclusive; the gate|up source needs M = 1
    assert lib.mtl_w4_gemm_partials(FAKE, FAKE, 8, 8192, 1, 4096, FAKE, FAKE, FAKE, None, 4096,
                                    128, 0, 0, FAKE, 1 << 30, None) == N.MTL_ERR_INVALID_ARG
    assert lib.mtl_w4_gemm_partials(None, FAKE, 8, 8192, 2, 4096, FAKE, FAKE, FAKE, None, 4096,
                                    128, 0, 0, FAKE, 1 << 30, None) == N.MTL_ERR_UNSUPPORTED
    # the tiled layout needs N % 64 == 0, M = 1 and no gather index
    assert lib.mtl_w4_gemm_partials(FAKE, None, 0, 0, 1, 4096, FAKE, FAKE, FAKE, None, 4104,
                                    128, 0, 1, FAKE, 1 << 30, None) == N.MTL_ERR_SHAPE
    assert lib.mtl_w4_gemm_partials(FAKE, None, 0, 0, 1, 4096, FAKE, FAKE, FAKE, None, 4096,
                                    128, 0, 4, FAKE, 1 << 30, None) == N.MTL_ERR_INVALID_ARG
    assert lib.mtl_w4_tiled_bytes(4096, 24576) == 8 * 384 * 16 * 1024
    assert lib.mtl_w4_tiled_bytes(4096, 24600) == 0
    # the strip layout needs N % 16 == 0, K % 256 == 0 (K <= 16384), M = 1, no gather index
    strip = N.LAYOUT_STRIP
    part = lambda m, k, n, perm=None: lib.mtl_w4_gemm_partials(  # noqa: E731
        FAKE, None, 0, 0, m, k, FAKE, FAKE, FAKE, perm, n, 128, 0, strip, FAKE, 1 << 30, None)
    assert part(1, 4096, 4104) == N.MTL_ERR_SHAPE
    assert part(1, 4224, 4096) == N.MTL_ERR_SHAPE
    assert part(1, 32768, 4096) == N.MTL_ERR_SHAPE
    assert part(2, 4096, 4096) == N.MTL_ERR_SHAPE
    assert part(1, 4096, 4096, FAKE) == N.MTL_ERR_SHAPE
    # the same shapes with the reference's qsz (layout STRIP_QSZ, qzeros unused)
    qpart = lambda m, k, n: lib.mtl_w4_gemm_partials(  # noqa: E731
        FAKE, None, 0, 0, m, k, FAKE, FAKE, None, None, n, 128, 0, N.LAYOUT_STRIP_QSZ, FAKE,
        1 << 30, None)
    assert qpart(1, 4096, 4104) == N.MTL_ERR_SHAPE
    assert qpart(1, 4224, 4096) == N.MTL_ERR_SHAPE
    assert qpart(2, 4096, 4096) == N.MTL_ERR_SHAPE
    # GPTQ strip metadata still needs its zeros
    assert lib.mtl_w4_gemm_partials(FAKE, None, 0, 0, 1, 4096, FAKE, FAKE, None, None, 4096, 128,
                                    0, strip, FAKE, 1 << 30, None) == N.MTL_ERR_INVALID_ARG
    assert lib.mtl_w4_gemm_partials(FAKE, None, 0, 0, 1, 4096, FAKE, FAKE, FAKE, None, 4096, 128,
                                    0, strip, FAKE, 4096 * 4 - 4, None) == N.MTL_ERR_WORKSPACE
    assert lib.mtl_w4_strip_bytes(4096, 24576) == 4096 * 24576 // 2
    assert lib.mtl_w4_strip_bytes(4096, 24584) == 0 and lib.mtl_w4_strip_bytes(4224, 4096) == 0
    assert lib.mtl_w4_strip(FAKE, 4096, 24584, FAKE, 1 << 30, None) == N.MTL_ERR_SHAPE
    assert lib.mtl_w4_strip(FAKE, 4096, 4096, FAKE, 100, None) == N.MTL_ERR_WORKSPACE
    # explicit launch geometries are validated before any launch
    geo = lambda **kw: lib.mtl_w4_gemm_partials_geom(  # noqa: E731
        FAKE, None, 0, 0, 1, 4096, FAKE, FAKE, FAKE, None, 4096, 128, 0, strip, FAKE, 1 << 30,
        N.strip_geometry(**kw), None)
    assert geo(nb=3) == N.MTL_ERR_SHAPE             # 32 blocks do not split into 3s
    assert geo(ct=2) == N.MTL_ERR_UNSUPPORTED       # the plain store serves one strip
    assert geo(nb=4, ring=2) == N.MTL_ERR_UNSUPPORTED
    assert geo(nb=2, ring=4) == N.MTL_ERR_UNSUPPORTED
    assert geo(xcd_order=2) == N.MTL_ERR_INVALID_ARG
    assert lib.mtl_w4_gemm_partials_geom(FAKE, None, 0, 0, 1, 4096, FAKE, FAKE, FAKE, None, 4096,
                                         128, 0, N.LAYOUT_ROWS, FAKE, 1 << 30,
                                         N.strip_geometry(nb=8), None) == N.MTL_ERR_UNSUPPORTED
    silu = lambda **kw: lib.mtl_w4_gemm_norm_silu_geom(  # noqa: E731
        FAKE, FAKE, FAKE, ctypes.c_float(1e-6), 4096, FAKE, FAKE, FAKE, 24576, 128, 0, strip,
        FAKE, N.strip_geometry(**kw), None)
    assert silu(ct=4) == N.MTL_ERR_UNSUPPORTED     # gate|up pairs: 2 or 6 strips
    assert silu(ct=6, nb=8) == N.MTL_ERR_SHAPE      # 4 slices x 6 strips: 24 waves
    assert silu(ct=2, nb=8, ring=16) == N.MTL_ERR_UNSUPPORTED
    assert lib.mtl_bf16_gemv_argmax(FAKE, FAKE, 100, 4100, None, None, FAKE, 1 << 20,
                                    None) == N.MTL_ERR_SHAPE
    assert lib.mtl_advance_position(None, None) == N.MTL_ERR_INVALID_ARG


def test_prefill_gemm_validation(lib):
    pf = lambda m, k, n, g=128, epi=0, odt=0, ldx=None, ldy=None, x=FAKE, y=FAKE: \
        lib.mtl_w4_gemm_prefill(x, m, k if ldx is None else ldx, k, FAKE, FAKE, FAKE, n, g, 0,  # noqa: E731
                                epi, odt, y, n if ldy is None else ldy, None, 0, None)
    assert pf(0, 4096, 4096) == N.MTL_ERR_SHAPE
    assert pf(256, 4224, 4096) == N.MTL_ERR_SHAPE          # K % 256
    assert pf(256, 4096, 4112) == N.MTL_ERR_SHAPE          # N % 128
    assert pf(256, 4096, 4096, ldx=4000) == N.MTL_ERR_SHAPE
    assert pf(256, 4096, 4096, g=96) == N.MTL_ERR_GROUP
    assert pf(256, 4096, 4096, epi=3) == N.MTL_ERR_INVALID_ARG
    assert pf(256, 4096, 4096, epi=1, odt=1) == N.MTL_ERR_INVALID_ARG   # residual is bf16
    assert pf(256, 4096, 4096, ldx=4100) == N.MTL_ERR_ALIGN              # 16-byte rows
    assert pf(256, 4096, 4096, x=None) == N.MTL_ERR_INVALID_ARG
    assert pf(256, 4096, 4096, y=ctypes.c_void_p(0x1001)) == N.MTL_ERR_ALIGN
    # SiLU*up writes N/2 columns per row
    assert pf(256, 4096, 4096, epi=2, ldy=2047) == N.MTL_ERR_SHAPE
    # K splits only where the grid is small: 4096 x 24576 at 256 rows fills the CUs
    assert lib.mtl_w4_gemm_prefill_workspace_bytes(256, 4096, 24576) == 0
    ws = lib.mtl_w4_gemm_prefill_workspace_bytes(256, 4096, 4096)
    assert ws > 0 and ws % (256 * 4096 * 4) == 0
    assert lib.mtl_w4_gemm_prefill_workspace_bytes(256, 4100, 4096) == 0


def test_prefill_partials_validation(lib):
    # the split partials of a residual GEMM: their bytes (one plane when the grid fills the
    # CUs), the metadata format, and a buffer short of the splits' planes
    assert lib.mtl_w4_gemm_prefill_partials_bytes(2048, 1024, 4096) == 2048 * 4096 * 4
    pb = lib.mtl_w4_gemm_prefill_partials_bytes(256, 4096, 4096)
    assert pb > 256 * 4096 * 4 and pb % (256 * 4096 * 4) == 0
    assert lib.mtl_w4_gemm_prefill_partials_bytes(256, 4100, 4096) == 0
    pp = lambda fmt=N.META_GPTQ, zeros=FAKE, part=FAKE, nbytes=pb, xs=None: \
        lib.mtl_w4_gemm_prefill_partials(FAKE, xs, 256, 4096, 4096, FAKE, FAKE, zeros,  # noqa: E731
                                         4096, 128, 0, fmt, part, nbytes, None)
    assert pp(fmt=2) == N.MTL_ERR_INVALID_ARG
    assert pp(zeros=None) == N.MTL_ERR_INVALID_ARG          # GPTQ metadata has zeros
    assert pp(part=None) == N.MTL_ERR_INVALID_ARG
    assert pp(nbytes=pb - 4) == N.MTL_ERR_WORKSPACE
    assert pp(fmt=N.META_QSZ, zeros=None, nbytes=pb - 4) == N.MTL_ERR_WORKSPACE
    assert pp(xs=ctypes.c_void_p(0x1008)) == N.MTL_ERR_ALIGN   # staged sums: 16-byte rows
    assert pp(xs=FAKE, nbytes=pb - 4) == N.MTL_ERR_WORKSPACE
    # the split sum + residual + RMSNorm: splits, the partials' bytes, out distinct from h
    eps = ctypes.c_float(1e-6)
    rn = lambda splits=4, nbytes=4 * 16 * 4096 * 4, h=FAKE, out=ctypes.c_void_p(0x2000), \
        ldo=4096, sums=None, n=4096: lib.mtl_residual_rmsnorm_gather(  # noqa: E731
            FAKE, splits, nbytes, h, n, FAKE, None, out, ldo, sums, 16, n, eps, None)
    assert rn(splits=0) == N.MTL_ERR_SHAPE
    assert rn(nbytes=4 * 16 * 4096 * 4 - 4) == N.MTL_ERR_WORKSPACE
    assert rn(ldo=4000) == N.MTL_ERR_SHAPE
    assert rn(h=ctypes.c_void_p(0x1008)) == N.MTL_ERR_ALIGN
    assert rn(out=FAKE) == N.MTL_ERR_INVALID_ARG            # h is updated in place
    assert rn(h=None) == N.MTL_ERR_INVALID_ARG
    assert rn(splits=9) == N.MTL_ERR_SHAPE                  # at most 8 splits
    assert rn(sums=FAKE, n=4080, ldo=4080) == N.MTL_ERR_SHAPE   # staged: n % 32
    assert rn(sums=ctypes.c_void_p(0x1002)) == N.MTL_ERR_ALIGN
    # the norm staged for the GEMM: n % 32, the sums buffer, a 16-byte gather
    sg = lambda n=4096, sums=FAKE, gather=None: lib.mtl_rmsnorm_gather_staged(  # noqa: E731
        FAKE, n, FAKE, gather, ctypes.c_void_p(0x2000), n, sums, 16, n, eps, None)
    assert sg(n=4080) == N.MTL_ERR_SHAPE
    assert sg(sums=None) == N.MTL_ERR_INVALID_ARG
    assert sg(gather=ctypes.c_void_p(0x1008)) == N.MTL_ERR_ALIGN
    # the GEMM on staged x: plain and SiLU*up epilogues only, the sums required
    gs = lambda epi=0, xs=FAKE, fmt=N.META_GPTQ: lib.mtl_w4_gemm_prefill_staged(  # noqa: E731
        FAKE, xs, 256, 4096, 4096, FAKE, FAKE, FAKE, 4096, 128, 0, fmt, epi, 0, FAKE, 4096,
        None, 0, None)
    assert gs(epi=1) == N.MTL_ERR_INVALID_ARG               # the residual takes plain x
    assert gs(xs=None) == N.MTL_ERR_INVALID_ARG
    assert gs(fmt=2) == N.MTL_ERR_INVALID_ARG
    assert gs(xs=ctypes.c_void_p(0x1008)) == N.MTL_ERR_ALIGN
    # the q|k|v split partials into the q/k norm + RoPE launch: the partial columns cover
    # whole heads, the heads past them need the bf16 buffer, and the partials' bytes
    qk = lambda splits=2, nbytes=2 * 16 * 6144 * 4, pcols=6144, qkv=None, ldq=6144: \
        lib.mtl_qk_norm_rope_kv_rows_partials(FAKE, splits, nbytes, pcols, qkv, ldq, 16, 0,  # noqa: E731
                                              FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 32, 8,
                                              128, 2048, eps, None)
    assert qk(pcols=6100) == N.MTL_ERR_SHAPE
    assert qk(pcols=6272) == N.MTL_ERR_SHAPE
    assert qk(splits=0) == N.MTL_ERR_SHAPE
    assert qk(pcols=5120) == N.MTL_ERR_INVALID_ARG          # v heads need qkv
    assert qk(pcols=5120, qkv=FAKE, ldq=6000) == N.MTL_ERR_SHAPE
    assert qk(nbytes=2 * 16 * 6144 * 4 - 4) == N.MTL_ERR_WORKSPACE


def test_gemv_strip_validation(lib):
    gv = lambda k, n, g=128, perm=None, odt=0, x=FAKE, y=FAKE, w=FAKE: lib.mtl_w4_gemv_strip(  # noqa: E731
        x, k, perm, w, FAKE, FAKE, n, g, 0, odt, y, None)
    assert gv(4096, 4096, x=None) == N.MTL_ERR_INVALID_ARG
    assert gv(4096, 4096, w=None) == N.MTL_ERR_INVALID_ARG
    assert gv(4096, 4096, odt=2) == N.MTL_ERR_INVALID_ARG
    assert gv(4096, 4096, g=96) == N.MTL_ERR_GROUP
    assert gv(4224, 4096) == N.MTL_ERR_SHAPE             # K % 256
    assert gv(4096, 4104) == N.MTL_ERR_SHAPE             # N % 16
    assert gv(32768, 512) == N.MTL_ERR_SHAPE             # K <= 16384
    assert gv(16384, 512, perm=FAKE) == N.MTL_ERR_SHAPE  # the gather keeps x in LDS: K <= 12288
    assert gv(4096, 4096, perm=ctypes.c_void_p(0x1008)) == N.MTL_ERR_ALIGN
    assert gv(4096, 4096, x=ctypes.c_void_p(0x1008)) == N.MTL_ERR_ALIGN
    assert gv(4096, 4096, odt=1, y=ctypes.c_void_p(0x1008)) == N.MTL_ERR_ALIGN   # fp32: 16 B


def test_prefill_row_entry_validation(lib):
    eps = ctypes.c_float(1e-6)
    sc = ctypes.c_float(0.088)
    # embedding rows
    assert lib.mtl_embed_rows(None, 4, 1, FAKE, FAKE, 4096, FAKE, None) == N.MTL_ERR_INVALID_ARG
    assert lib.mtl_embed_rows(FAKE, 0, 1, FAKE, FAKE, 4096, FAKE, None) == N.MTL_ERR_SHAPE
    assert lib.mtl_embed_rows(FAKE, 4, 0, FAKE, FAKE, 4096, FAKE, None) == N.MTL_ERR_SHAPE
    # RMSNorm + gather: n % 8, n <= 16384, row pitches, alignment, in place only with one pitch
    ng = lambda x, ldx, out, ldo, rows, n: lib.mtl_rmsnorm_gather(  # noqa: E731
        x, ldx, FAKE, None, out, ldo, rows, n, eps, None)
    assert ng(FAKE, 4100, FAKE, 4100, 4, 4100) == N.MTL_ERR_SHAPE
    assert ng(FAKE, 32768, FAKE, 32768, 4, 32768) == N.MTL_ERR_SHAPE
    assert ng(FAKE, 4000, FAKE, 4096, 4, 4096) == N.MTL_ERR_SHAPE
    assert ng(FAKE, 4096, FAKE, 4096, 0, 4096) == N.MTL_ERR_SHAPE
    assert ng(ctypes.c_void_p(0x1008), 4096, FAKE, 4096, 4, 4096) == N.MTL_ERR_ALIGN
    assert ng(FAKE, 4096, FAKE, 4104, 4, 4096) == N.MTL_ERR_INVALID_ARG
    assert ng(None, 4096, FAKE, 4096, 4, 4096) == N.MTL_ERR_INVALID_ARG
    # q/k norm + RoPE rows: head_dim 128, rows inside the cache, the q|k|v row pitch
    qk = lambda ldq, rows, pos0, hd=128, S=2048: lib.mtl_qk_norm_rope_kv_rows(  # noqa: E731
        FAKE, ldq, rows, pos0, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 32, 8, hd, S, eps, None)
    assert qk(6144, 16, 0, hd=64) == N.MTL_ERR_UNSUPPORTED
    assert qk(6144, 16, 2040) == N.MTL_ERR_SHAPE
    assert qk(6000, 16, 0) == N.MTL_ERR_SHAPE
    assert qk(6144, 16, -1) == N.MTL_ERR_SHAPE
    # causal attention: GQA ratio <= 8, rows inside the cache, out pitch
    at = lambda rows, pos0, H=32, Hkv=8, ldo=4096, S=2048: lib.mtl_prefill_attention(  # noqa: E731
        FAKE, FAKE, FAKE, rows, pos0, FAKE, ldo, None, H, Hkv, 128, S, sc, None)
    assert at(16, 0, H=32, Hkv=2) == N.MTL_ERR_SHAPE
    assert at(16, 0, H=32, Hkv=6) == N.MTL_ERR_SHAPE
    assert at(16, 2040) == N.MTL_ERR_SHAPE
    assert at(0, 0) == N.MTL_ERR_SHAPE
    assert at(16, 0, ldo=4000) == N.MTL_ERR_SHAPE
    assert lib.mtl_prefill_attention(FAKE, FAKE, FAKE, 16, 0, FAKE, 4096, None, 32, 8, 64, 2048,
                                     sc, None) == N.MTL_ERR_UNSUPPORTED
    assert lib.mtl_prefill_attention(ctypes.c_void_p(0x1008), FAKE, FAKE, 16, 0, FAKE, 4096, None,
                                     32, 8, 128, 2048, sc, None) == N.MTL_ERR_ALIGN


def test_converter_validation(lib):
    assert lib.mtl_int4pack_convert(FAKE, 64, 64, 3, FAKE, None) == N.MTL_ERR_INVALID_ARG
    assert lib.mtl_int4pack_convert(FAKE, 56, 512, 8, FAKE, None) == N.MTL_ERR_SHAPE   # N % 16
    assert lib.mtl_int4pack_convert(FAKE, 64, 384, 8, FAKE, None) == N.MTL_ERR_SHAPE   # K % 256
    mm = lib.mtl_int4pack_mm
    assert mm(None, 1, 512, FAKE, 128, FAKE, 64, FAKE, None, 0, None) == N.MTL_ERR_INVALID_ARG
    assert mm(FAKE, 1, 512, FAKE, 16, FAKE, 64, FAKE, None, 0, None) == N.MTL_ERR_GROUP
    assert mm(FAKE, 1, 384, FAKE, 128, FAKE, 64, FAKE, None, 0, None) == N.MTL_ERR_SHAPE
    assert mm(FAKE, 1, 512, FAKE, 128, FAKE, 56, FAKE, None, 0, None) == N.MTL_ERR_SHAPE
    assert mm(FAKE, 0, 512, FAKE, 128, FAKE, 64, FAKE, None, 0, None) == N.MTL_ERR_SHAPE
    assert mm(FAKE, 1, 512, FAKE, 128, FAKE, 64, ctypes.c_void_p(0x1004), None, 0,
              None) == N.MTL_ERR_ALIGN
    assert lib.mtl_int4pack_mm_workspace_bytes(1, 4096, 4096) == 0
    tt = lib.mtl_int4pack_from_torch_tiles
    assert tt(None, 64, 512, 8, FAKE, None) == N.MTL_ERR_INVALID_ARG
    assert tt(FAKE, 64, 512, 6, FAKE, None) == N.MTL_ERR_INVALID_ARG
    assert tt(FAKE, 56, 512, 8, FAKE, None) == N.MTL_ERR_SHAPE      # N % 16
    assert tt(FAKE, 64, 384, 8, FAKE, None) == N.MTL_ERR_SHAPE      # K % 256
    assert tt(ctypes.c_void_p(0x1002), 64, 512, 8, FAKE, None) == N.MTL_ERR_ALIGN


def test_load_gptq_state_safe_loader(tmp_path):
    # the reference's offline GPTQ state layout (gptq.py:504-509) + meta json (gptq.py:608-626)
    import json
    import torch
    from moss_tts_lite_amd.gptq import load_gptq_state
    state = {0: {"q": {"q": torch.zeros(8, 256, dtype=torch.uint8),
                       "qsz": torch.zeros(2, 8, 2, dtype=torch.bfloat16)}}}
    p = tmp_path / "state.pt"
    torch.save(state, p)
    with pytest.raises(FileNotFoundError):
        load_gptq_state(str(p))
    (tmp_path / "state.pt.meta.json").write_text(json.dumps(
        {"group_size_map": {"0:q": 32}, "bf16_linears": ["1:down"], "bf16_layers": [3]}))
    st, gmap, keep = load_gptq_state(str(p))
    assert gmap == {(0, "q"): 32} and keep == [(1, "down"), 3]
    assert torch.equal(st[0]["q"]["q"], state[0]["q"]["q"])


def test_w4_dispatch_incomplete_state_raises():
    # with a GPTQ state, a linear that is neither kept in bf16 nor recorded is an error
    # (the reference indexes state[li][name], gptq.py:675), not a silent round-to-nearest
    import torch
    from moss_tts_lite_amd.gptq import W4Dispatch
    layers = [{"q": torch.zeros(8, 256, dtype=torch.bfloat16)}]
    with pytest.raises(KeyError, match="layer 0 q"):
        W4Dispatch(layers, state={0: {}}, device="cpu")
    with pytest.raises(KeyError, match="layer 0 q"):
        W4Dispatch(layers, state={}, device="cpu")
    # a kept layer needs no record and installs nothing
    assert W4Dispatch(layers, bf16_keep=[0], state={}, device="cpu").qlayers == [None]
    with pytest.raises(ValueError):
        W4Dispatch(layers, w4_group_size=16)


def test_step_position_and_id_checks():
    # the decoders' host checks (moss_tts_lite/model.py:_check_ids raises for ids and
    # lengths that do not fit)
    import torch
    from moss_tts_lite_amd.fast import _check_ids, _check_pos
    _check_ids(torch.tensor([[0, 1024], [8191, 0]]), [8192, 1025])
    for bad in ([[8192, 0]], [[0, 1025]], [[-1, 0]]):
        with pytest.raises(ValueError, match="outside its embedding table"):
            _check_ids(torch.tensor(bad), [8192, 1025])
    assert _check_pos(63, 64) == 63
    for bad in (64, -1):
        with pytest.raises(ValueError, match="outside the KV cache"):
            _check_pos(bad, 64)


def test_torch_operators_registered():
    # the dispatcher operators over the C ABI load on the CPU and report shapes through
    # their meta kernels; bad arguments raise RuntimeError as torch's operators do
    import torch
    from moss_tts_lite_amd import ops
    mtl = ops.torch_ops()
    x = torch.empty(3, 4096, dtype=torch.bfloat16, device="meta")
    packed = torch.empty(64, 32, 32, 4, dtype=torch.int32, device="meta")
    qsz = torch.empty(32, 512, 2, dtype=torch.bfloat16, device="meta")
    assert tuple(mtl.weight_int4pack_mm(x, packed, 128, qsz).shape) == (3, 512)
    with pytest.raises(RuntimeError):
        mtl.weight_int4pack_mm(x.float(), packed, 128, qsz)
    with pytest.raises(RuntimeError):
        mtl.weight_int4pack_mm(x, packed, 16, torch.empty(256, 512, 2, dtype=torch.bfloat16,
                                                          device="meta"))
    with pytest.raises(RuntimeError):
        mtl.weight_int4pack_mm(x[:, :2048], packed, 128, qsz)
    pre = torch.empty(512, 2048, dtype=torch.uint8, device="meta")
    assert tuple(mtl.convert_weight_to_int4pack(pre, 8).shape) == (64, 32, 32, 4)
    sw = torch.empty(4096 * 512 // 8, dtype=torch.int32, device="meta")
    ssc = torch.empty(32, 512, dtype=torch.float16, device="meta")
    szr = torch.empty(32, 64, dtype=torch.int32, device="meta")
    assert tuple(mtl.strip_gemv(x[:1], sw, ssc, szr, 512, 128).shape) == (1, 512)
    with pytest.raises(RuntimeError):
        mtl.convert_weight_to_int4pack(pre, 3)
    # the GPTQ module's operators over the AutoGPTQ tensors: [..., K] in, [..., N] out
    x3 = torch.empty(2, 3, 4096, dtype=torch.bfloat16, device="meta")
    qw = torch.empty(512, 1024, dtype=torch.int32, device="meta")
    qz = torch.empty(32, 128, dtype=torch.int32, device="meta")
    sc = torch.empty(32, 1024, dtype=torch.float16, device="meta")
    y = mtl.gptq_gemm(x3, qw, qz, sc, 128)
    assert tuple(y.shape) == (2, 3, 1024) and y.dtype == torch.bfloat16
    assert mtl.gptq_gemm(x3, qw, qz, sc, 128, out_dtype=torch.float32).dtype == torch.float32
    with pytest.raises(RuntimeError):
        mtl.gptq_gemm(x3, qw, qz, sc, 64)                     # scales of g128
    with pytest.raises(RuntimeError):
        mtl.gptq_gemm(x3, qw, qz, sc.float(), 128)
    strip = torch.empty(4096 * 1024 // 8, dtype=torch.int32, device="meta")
    assert tuple(mtl.strip_rows_gemm(x3, strip, qz, sc, 1024, 128).shape) == (2, 3, 1024)
    with pytest.raises(RuntimeError):
        mtl.strip_rows_gemm(x3, strip, qz, sc, 1024, 96)
