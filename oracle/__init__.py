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
* ``w8a16.get_linear_partition`` / ``tp_col_swizzle`` / ``tp_row_swizzle``
  -- python/rpu_backend/runtime/weights.py:97-203
* ``gen`` -- the portable seeded input generator (SplitMix64 + Box-Muller);
  not a reference algorithm.

How each function is pinned (closed forms, the reference's own KAT, library
routines, brute force) is listed in the header of ``w8a16.py``.
"""
