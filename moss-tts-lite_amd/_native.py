"""ctypes binding of ``libmtl_hip.so`` (the C ABI in ``include/*.h``).

The library is loaded after ``torch`` so that it binds to torch's HIP runtime
(``libamdhip64`` resolves by soname to the copy torch already mapped); the
loader checks that exactly one HIP runtime is mapped in the process.  There is
no fallback: if the library is missing or was built for another ABI, every op
raises.
"""
from __future__ import annotations

import ctypes
import os
import re

from . import build as _build

_c_void_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32

# name -> (restype, argtypes)
_SIGNATURES = {
    # mtl_gptq.h
    "mtl_status_string": (ctypes.c_char_p, [_i32]),
    "mtl_abi_version": (_i32, []),
    "mtl_gemm_workspace_bytes": (_i64, [_i64, _i64, _i64, _i32]),
    "mtl_workspace_init": (_i32, [_c_void_p, _i64, _c_void_p]),
    "mtl_gptq_gemm": (_i32, [_c_void_p, _i64, _i64, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                             _i64, _i32, _i32, _c_void_p, _i32, _c_void_p, _i64, _c_void_p]),
    "mtl_gptq_gemm_noalloc": (_i32, [_c_void_p, _i64, _i64, _c_void_p, _c_void_p, _c_void_p,
                                     _c_void_p, _i64, _i32, _i32, _c_void_p, _i32, _c_void_p]),
    "mtl_actorder_scratch_bytes": (_i64, [_i64]),
    "mtl_gptq_actorder_prepare": (_i32, [_c_void_p, _c_void_p, _i64, _i64, _i32, _c_void_p,
                                         _c_void_p, _c_void_p, _i64, _c_void_p]),
    "mtl_int4pack_mm": (_i32, [_c_void_p, _i64, _i64, _c_void_p, _i32, _c_void_p, _i64,
                               _c_void_p, _c_void_p, _i64, _c_void_p]),
    "mtl_int4pack_convert": (_i32, [_c_void_p, _i64, _i64, _i32, _c_void_p, _c_void_p]),
    "mtl_int4pack_from_torch_tiles": (_i32, [_c_void_p, _i64, _i64, _i32, _c_void_p, _c_void_p]),
    "mtl_unpack_codes": (_i32, [_c_void_p, _i64, _i64, _c_void_p, _c_void_p]),
    "mtl_gptq_dequant": (_i32, [_c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i32, _i32,
                                _c_void_p, _c_void_p]),
    "mtl_qsz_dequant": (_i32, [_c_void_p, _c_void_p, _i64, _i64, _i32, _c_void_p, _c_void_p]),
    "mtl_w4_gemm_fused": (_i32, [_c_void_p, _i64, _i64, _c_void_p, _i32, _c_void_p, _c_void_p,
                                 _c_void_p, _i64, _i32, _i32, _i32, _c_void_p, _c_void_p, _i32,
                                 _c_void_p, _i64, _c_void_p]),
    # mtl_decode.h
    "mtl_rmsnorm": (_i32, [_c_void_p, _c_void_p, _c_void_p, _i64, _i64, ctypes.c_float, _c_void_p]),
    "mtl_embed_sum": (_i32, [_c_void_p, _i32, _c_void_p, _c_void_p, _i64, _c_void_p, _c_void_p]),
    "mtl_embed_sum_stats": (_i32, [_c_void_p, _i32, _c_void_p, _c_void_p, _i64, _c_void_p,
                                   _c_void_p, _c_void_p, _c_void_p, _c_void_p]),
    "mtl_qk_norm_rope_kv": (_i32, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                   _c_void_p, _c_void_p, _c_void_p, _i32, _i32, _i32, _i64,
                                   ctypes.c_float, _c_void_p]),
    "mtl_decode_attention_workspace_bytes": (_i64, [_i32, _i32]),
    "mtl_decode_attention_set_handoff": (_i32, [_i32]),
    "mtl_decode_attention": (_i32, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                    _i32, _i32, _i32, _i64, ctypes.c_float, _c_void_p, _i64,
                                    _c_void_p]),
    "mtl_qk_norm_rope_kv_partials": (_i32, [_c_void_p, _i32, _c_void_p, _c_void_p, _c_void_p,
                                            _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                            _i32, _i32, _i32, _i64, ctypes.c_float, _c_void_p]),
    "mtl_residual_rmsnorm": (_i32, [_c_void_p, _i32, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                    _c_void_p, _i64, ctypes.c_float, _c_void_p]),
    "mtl_head_workspace_bytes": (_i64, [_i64]),
    "mtl_bf16_gemv_argmax": (_i32, [_c_void_p, _c_void_p, _i64, _i64, _c_void_p, _c_void_p,
                                    _c_void_p, _i64, _c_void_p]),
    "mtl_advance_position": (_i32, [_c_void_p, _c_void_p]),
    "mtl_silu_mul_f32": (_i32, [_c_void_p, _c_void_p, _c_void_p, _i64, _c_void_p]),
    "mtl_bf16_gemv_norm": (_i32, [_c_void_p, _c_void_p, _c_void_p, ctypes.c_float, _c_void_p, _i64,
                                  _i64, _c_void_p, _c_void_p]),
    "mtl_bf16_gemv": (_i32, [_c_void_p, _c_void_p, _i64, _i64, _c_void_p, _i64, _i64, _c_void_p]),
    "mtl_residual_add": (_i32, [_c_void_p, _i32, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64,
                                _c_void_p]),
    "mtl_decode_attention_fused": (_i32, [_c_void_p, _i32, _c_void_p, _c_void_p, _c_void_p,
                                          _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                          _c_void_p, _i32, _i32, _i32, _i64, ctypes.c_float,
                                          ctypes.c_float, _c_void_p, _i64, _c_void_p]),
    "mtl_bf16_gemv_argmax_norm": (_i32, [_c_void_p, _c_void_p, _c_void_p, ctypes.c_float,
                                         _c_void_p, _i64, _i64, _c_void_p, _c_void_p, _c_void_p,
                                         _i64, _c_void_p]),
    "mtl_bf16_gemv_argmax_norm_advance": (_i32, [_c_void_p, _c_void_p, _c_void_p,
                                                 ctypes.c_float, _c_void_p, _i64, _i64,
                                                 _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                                 _i64, _c_void_p]),
    # tuning knobs (not part of the headers)
    "mtl_w4_gemm_splits": (_i32, [_i64, _i64]),
    "mtl_w4_gemm_partials": (_i32, [_c_void_p, _c_void_p, _i32, _i64, _i64, _i64, _c_void_p,
                                    _c_void_p, _c_void_p, _c_void_p, _i64, _i32, _i32, _i32,
                                    _c_void_p, _i64, _c_void_p]),
    "mtl_w4_gemm_residual": (_i32, [_c_void_p, _c_void_p, _i32, _i64, _i64, _c_void_p, _c_void_p,
                                    _c_void_p, _i64, _i32, _i32, _i32, _c_void_p, _c_void_p,
                                    _c_void_p, _c_void_p, _c_void_p, _i64, _c_void_p]),
    "mtl_w4_gemm_norm_partials": (_i32, [_c_void_p, _c_void_p, _c_void_p, ctypes.c_float, _i64,
                                         _c_void_p, _c_void_p, _c_void_p, _i64, _i32, _i32, _i32,
                                         _c_void_p, _i64, _c_void_p]),
    "mtl_w4_gemm_norm_partials_bf16": (_i32, [_c_void_p, _c_void_p, _c_void_p, ctypes.c_float,
                                              _i64, _c_void_p, _c_void_p, _c_void_p, _i64, _i32,
                                              _i32, _i32, _c_void_p, _i64, _c_void_p, _c_void_p,
                                              _c_void_p, _i64, _c_void_p, _c_void_p]),
    "mtl_w4_gemm_strip_rows": (_i32, [_c_void_p, _i64, _i64, _i64, _c_void_p, _c_void_p, _c_void_p,
                                      _i64, _i32, _i32, _c_void_p, _i64, _i32, _c_void_p]),
    "mtl_w4_gemm_strip_rows_ex": (_i32, [_c_void_p, _i64, _i64, _i64, _c_void_p, _c_void_p,
                                         _c_void_p, _c_void_p, _i64, _i32, _i32, _i32,
                                         _c_void_p, _i64, _i32, _c_void_p]),
    "mtl_w4_gemv_strip": (_i32, [_c_void_p, _i64, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                 _i64, _i32, _i32, _i32, _c_void_p, _c_void_p]),
    "mtl_w4_gemm_prefill": (_i32, [_c_void_p, _i64, _i64, _i64, _c_void_p, _c_void_p, _c_void_p,
                                   _i64, _i32, _i32, _i32, _i32, _c_void_p, _i64, _c_void_p,
                                   _i64, _c_void_p]),
    "mtl_w4_gemm_prefill_workspace_bytes": (_i64, [_i64, _i64, _i64]),
    "mtl_w4_gemm_prefill_partials_bytes": (_i64, [_i64, _i64, _i64]),
    "mtl_w4_gemm_prefill_partials": (_i32, [_c_void_p, _c_void_p, _i64, _i64, _i64, _c_void_p,
                                            _c_void_p, _c_void_p, _i64, _i32, _i32, _i32,
                                            _c_void_p, _i64, _c_void_p]),
    "mtl_w4_gemm_prefill_staged": (_i32, [_c_void_p, _c_void_p, _i64, _i64, _i64, _c_void_p,
                                          _c_void_p, _c_void_p, _i64, _i32, _i32, _i32, _i32,
                                          _i32, _c_void_p, _i64, _c_void_p, _i64, _c_void_p]),
    "mtl_qk_norm_rope_kv_rows_partials": (_i32, [_c_void_p, _i32, _i64, _i64, _c_void_p, _i64,
                                                 _i64, _i64, _c_void_p, _c_void_p, _c_void_p,
                                                 _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                                 _i32, _i32, _i32, _i64, ctypes.c_float,
                                                 _c_void_p]),
    "mtl_residual_rmsnorm_gather": (_i32, [_c_void_p, _i32, _i64, _c_void_p, _i64, _c_void_p,
                                           _c_void_p, _c_void_p, _i64, _c_void_p, _i64, _i64,
                                           ctypes.c_float, _c_void_p]),
    "mtl_rmsnorm_gather_staged": (_i32, [_c_void_p, _i64, _c_void_p, _c_void_p, _c_void_p, _i64,
                                         _c_void_p, _i64, _i64, ctypes.c_float, _c_void_p]),
    "mtl_w4_gemm_prefill_qsz": (_i32, [_c_void_p, _i64, _i64, _i64, _c_void_p, _c_void_p, _i64,
                                       _i32, _i32, _i32, _c_void_p, _i64, _c_void_p, _i64,
                                       _c_void_p]),
    "mtl_int4pack_mm_workspace_bytes": (_i64, [_i64, _i64, _i64]),
    "mtl_embed_rows": (_i32, [_c_void_p, _i64, _i32, _c_void_p, _c_void_p, _i64, _c_void_p,
                              _c_void_p]),
    "mtl_rmsnorm_gather": (_i32, [_c_void_p, _i64, _c_void_p, _c_void_p, _c_void_p, _i64, _i64,
                                  _i64, ctypes.c_float, _c_void_p]),
    "mtl_qk_norm_rope_kv_rows": (_i32, [_c_void_p, _i64, _i64, _i64, _c_void_p, _c_void_p,
                                        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                        _i32, _i32, _i32, _i64, ctypes.c_float, _c_void_p]),
    "mtl_prefill_attention": (_i32, [_c_void_p, _c_void_p, _c_void_p, _i64, _i64, _c_void_p, _i64,
                                     _c_void_p, _i32, _i32, _i32, _i64, ctypes.c_float,
                                     _c_void_p]),
    "mtl_w4_gemm_norm_silu": (_i32, [_c_void_p, _c_void_p, _c_void_p, ctypes.c_float, _i64,
                                     _c_void_p, _c_void_p, _c_void_p, _i64, _i32, _i32, _i32,
                                     _c_void_p, _c_void_p]),
    "mtl_w4_gemm_partials_geom": (_i32, [_c_void_p, _c_void_p, _i32, _i64, _i64, _i64, _c_void_p,
                                         _c_void_p, _c_void_p, _c_void_p, _i64, _i32, _i32, _i32,
                                         _c_void_p, _i64, _c_void_p, _c_void_p]),
    "mtl_w4_gemm_norm_partials_geom": (_i32, [_c_void_p, _c_void_p, _c_void_p, ctypes.c_float,
                                              _i64, _c_void_p, _c_void_p, _c_void_p, _i64, _i32,
                                              _i32, _i32, _c_void_p, _i64, _c_void_p, _c_void_p]),
    "mtl_w4_gemm_residual_geom": (_i32, [_c_void_p, _c_void_p, _i32, _i64, _i64, _c_void_p,
                                         _c_void_p, _c_void_p, _i64, _i32, _i32, _i32, _c_void_p,
                                         _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64,
                                         _c_void_p, _c_void_p]),
    "mtl_w4_gemm_norm_silu_geom": (_i32, [_c_void_p, _c_void_p, _c_void_p, ctypes.c_float, _i64,
                                          _c_void_p, _c_void_p, _c_void_p, _i64, _i32, _i32, _i32,
                                          _c_void_p, _c_void_p, _c_void_p]),
    "mtl_w4_tiled_bytes": (_i64, [_i64, _i64]),
    "mtl_w4_tile": (_i32, [_c_void_p, _i64, _i64, _c_void_p, _i64, _c_void_p]),
    "mtl_w4_strip_bytes": (_i64, [_i64, _i64]),
    "mtl_w4_strip_meta": (_i32, [_c_void_p, _c_void_p, _i64, _i64, _i32, _c_void_p, _c_void_p,
                                 _c_void_p]),
    "mtl_w4_strip": (_i32, [_c_void_p, _i64, _i64, _c_void_p, _i64, _c_void_p]),
}

class StripGeometry(ctypes.Structure):
    """``mtl_strip_geometry``: the strip GEMV's launch shape (0 = automatic per field)."""
    _fields_ = [("strips_per_wg", ctypes.c_int32), ("blocks_per_wave", ctypes.c_int32),
                ("ring", ctypes.c_int32), ("xcd_order", ctypes.c_int32)]


def strip_geometry(ct: int = 0, nb: int = 0, ring: int = 0, xcd_order: int = 0):
    """A ``mtl_strip_geometry`` passed by reference to the ``*_geom`` entries."""
    return ctypes.byref(StripGeometry(ct, nb, ring, xcd_order))


NOALLOC_SCRATCH_BYTES = 16 << 20      # MTL_NOALLOC_SCRATCH_BYTES
MTL_OK = 0
MTL_ERR_INVALID_ARG = -1
MTL_ERR_SHAPE = -2
MTL_ERR_GROUP = -3
MTL_ERR_ALIGN = -4
MTL_ERR_WORKSPACE = -5
MTL_ERR_LAUNCH = -6
MTL_ERR_UNSUPPORTED = -7

OUT_BF16, OUT_F32 = 0, 1
LAYOUT_ROWS, LAYOUT_TILED, LAYOUT_STRIP, LAYOUT_STRIP_QSZ = 0, 1, 2, 3
XPART_HALVES = 1 << 30                # MTL_XPART_HALVES, OR'ed into mtl_w4_gemm_residual's xsplits
EPI_NONE, EPI_RESIDUAL, EPI_SILU_MUL = 0, 1, 2
META_GPTQ, META_QSZ = 0, 1

_lib = None


class MtlError(RuntimeError):
    """A non-zero status returned by the C ABI."""

    def __init__(self, status: int, what: str):
        self.status = status
        super().__init__(f"{what}: {status_string(status)} (status {status})")


def lib_path() -> str:
    return _build.LIB_PATH


def torch_ops_path() -> str:
    """The torch operator library built beside the C library (libmtl_torch_ops.so)."""
    return _build.TORCH_OPS_PATH


def header_symbols() -> list[str]:
    """Every function name declared in ``include/*.h``."""
    inc = os.path.join(_build.ROOT, "include")
    names = []
    for fn in sorted(os.listdir(inc)):
        if not fn.endswith(".h"):
            continue
        text = open(os.path.join(inc, fn)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names += re.findall(r"^\s*(?:const\s+)?[A-Za-z_][A-Za-z0-9_]*\s*\*?\s*(mtl_[A-Za-z0-9_]+)\s*\(",
                            text, flags=re.M)
    return names


def _hip_runtimes_mapped() -> list[str]:
    try:
        with open("/proc/self/maps") as f:
            return sorted({ln.split()[-1] for ln in f if "libamdhip64" in ln})
    except OSError:
        return []


def load(path: str | None = None):
    """Load the library once (after torch) and attach the ctypes signatures."""
    global _lib
    if _lib is not None:
        return _lib
    import torch  # noqa: F401  (maps torch's HIP runtime first)

    p = path or lib_path()
    if not os.path.exists(p):
        raise RuntimeError(
            f"{p} is missing: build the gfx950 HIP library first "
            "(python -c 'import __graft_entry__ as g; g.build()')")
    lib = ctypes.CDLL(p)
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.mtl_abi_version() != 1:
        raise RuntimeError(f"{p}: unexpected ABI version {lib.mtl_abi_version()}")
    runtimes = _hip_runtimes_mapped()
    if len(runtimes) > 1:
        raise RuntimeError(f"more than one HIP runtime mapped: {runtimes}")
    _lib = lib
    return lib


def status_string(status: int) -> str:
    try:
        return load().mtl_status_string(status).decode()
    except Exception:  # noqa: BLE001  (message only)
        return "unknown"


def check(status: int, what: str) -> None:
    if status != MTL_OK:
        raise MtlError(status, what)
