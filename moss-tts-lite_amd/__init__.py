"""MI355X (gfx950) int4 GPTQ decode hot path of moss-tts-lite.

Import name: ``moss_tts_lite_amd`` (the directory name carries hyphens, so it is
loaded by path; see ``__graft_entry__.import_package``).

Modules
-------
``_native``  ctypes binding of ``libmtl_hip.so`` (C ABI in ``include/``)
``ops``      torch-facing int4 GEMM / pack / dequant ops
``gptq``     the GPTQ linear module and the reference's format helpers
``build``    the hipcc recipe of ``libmtl_hip.so``
"""
__version__ = "0.1.0"
