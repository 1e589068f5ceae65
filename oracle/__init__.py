"""CPU oracle for the W3 packed-LUT batch-1 decode path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg
may import, call, link or execute anything under ``oracle/``, and only as the
checker (or the timed CPU baseline), never as the thing measured on the GPU or
shipped.  The product package ``marlin_style_fluxbin_amd`` never imports it.

Contents
--------
``w3``         numpy restatement of the reference's GPTQ int3 packing, the planar
               ``[G,3,O,16]`` layout, dequantize-then-matmul and the two grouped
               matvec semantics (``gptq_deployment.py``), extended with the
               per-group zero-points and fp16 scales the benchmark configs use.
``norms``      numpy restatement of Qwen3 RMSNorm, per-head q/k RMSNorm and RoPE
               (``fused_modules.py`` + HF ``modeling_qwen3``).
``two_base``   numpy closed form of the two-base binary-basis GEMV (config 4).
``bf16``       bit-exact bfloat16 rounding helpers used by all of the above.
``kernel_order.c``  plain C restatement of the reference kernel's fp32 LUT
               order (``csrc/lut8_unsigned.cuh:13-27``, ``csrc/w3_lut.cu:57-123``).
``ref_lut_driver.cpp`` + ``Makefile``  compile the reference's own LUT header
               where it lies under ``/root/reference`` into ``oracle/_ref/`` so the
               C restatement can be checked against it.

How each function is pinned (golden vectors, closed forms, library routines)
is stated in its docstring; the tests in ``tests/test_oracle_*.py`` run the pins.
"""
