"""CPU oracle for the W4A16 hot path. TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the arithmetic of torch2iron's W4A16
reference path so that the HIP kernels can be checked against it.  Only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only as what results are compared against
or as the timed CPU baseline.  The product path (``torch2iron_amd``) never imports it and fails
loudly when its HIP library is missing.

Modules
-------
``oracle.w4a16``  numpy: AutoGPTQ nibble unpack, zero-point convention,
                  exact fp32 dequantisation, fp64/fp32 linear.
``oracle.qwen3``  torch-CPU: RMSNorm, RoPE, GQA decode attention, SwiGLU,
                  the fused decode layer and a batched greedy Qwen3 model.
"""
