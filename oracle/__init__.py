"""CPU oracle for the int4/int8 quantized matrix-product path.

TEST INFRASTRUCTURE ONLY. Nothing in the shipped package imports this
module. Only ``tests/``, ``__graft_entry__.smoke()`` and the CPU-baseline leg
of ``bench.py`` use it, and only as the checker (or the timed CPU baseline),
never as the thing measured or shipped.

``q4_oracle`` restates, in numpy, the reference engine's quantizer
(``src/vk_engine.py:125-159``), the shaders' arithmetic (``vk/*.comp``) and
the reference's own numpy dequant+matmul checks (``benchmarks/*.py``).
Every function cites the reference file:line it follows. The checks that pin
each function (known answers, closed forms, exhaustive tables, brute force)
live in ``tests/test_oracle.py``.
"""
