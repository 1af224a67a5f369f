"""CPU oracle for the W8A16 quantized linear -- TEST INFRASTRUCTURE ONLY.

Nothing in the product (``rhinoforge_amd``) imports, links or runs this
package.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may use it, and only as the checker.

Contents (every function cites the reference file:line it restates, paths
relative to the RhinoForge source tree):

* ``w8a16.quantize_linear_per_channel`` -- python/rpu_backend/quant/_common.py:10-36
* ``w8a16.dequantize_linear_per_channel`` -- quant/_common.py:39-41
* ``w8a16.dequantize_fp32_then_fp16`` -- adapters/qwen3.py:617-621
* ``w8a16.cpu_path`` -- adapters/qwen3.py:623 and src/ops/rpu_linear.cpp:133-163
* ``w8a16.oracle_fp64`` -- quant/verify_qwen3_w8a16.py:185-197 (f64 form)
* ``w8a16.check_tolerance`` -- the BASELINE parity bar (max error against
  the CPU path relative to its rms, cosine against the fp64 oracle)
* ``w8a16.normal`` / ``make_weight`` / ``make_activation`` -- the portable
  seeded input generator (SplitMix64 + Box-Muller); not a reference algorithm
* ``w4a16.quantize_int4_per_channel`` -- quant/int4_pack.py:21-23
* ``w4a16.quantize_int4_group_wise`` -- quant/int4_pgrp_pack.py:33-60
* ``w4a16.dequantize_int4`` -- quant/int4_pgrp_pack.py:63-70
* ``w4a16.cpu_path`` / ``oracle_fp64`` -- the int4 forms of the two above
* ``w4a16.pack_index`` / ``pack_reference`` -- the TILE16X128_I4 layout
  definition of include/w8a16.h (this build's own layout, which replaces the
  reference's RPU swizzles, runtime/weights.py:150-203)

The reference's 8-core partition and swizzles (runtime/weights.py:97-203)
are not restated: this build replaces them with its own packed layouts,
whose definitions are pinned instead.

How each function is pinned (closed forms, the reference's own KAT, library
routines, brute force) is listed in the headers of ``w8a16.py`` and
``w4a16.py``.
"""
