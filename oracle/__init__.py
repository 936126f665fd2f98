"""CPU oracle for the int4 GPTQ decode hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the arithmetic of the reference's int4 path
(moss_tts_lite/gptq.py, fast.py, fast_native.py, model.py) so that the HIP
kernels can be checked against it.  Only ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` may import it, and only as the
checker or the timed CPU baseline.  The product path (``moss-tts-lite_amd``)
never imports, calls or falls back to anything in here.

Modules
-------
``bf16``        bit-exact float32 <-> bfloat16 conversions (round-to-nearest-even).
``gptq_ref``    quantisation formats: RTN, qsz packing, the dequant closed form,
                AutoGPTQ ``qweight/qzeros/scales/g_idx`` pack/unpack, act-order.
``decode_ref``  one batch-1 decode step of the Qwen3-shaped backbone (RMSNorm,
                q/k norm, RoPE, KV write, GQA attention, SwiGLU, head).
``synth``       seeded synthetic inputs for the benchmark configurations.

Pinning status of every function is stated in its docstring; the tests under
``tests/test_oracle_*.py`` hold the checks that pin them.
"""
