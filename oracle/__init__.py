"""CPU oracle for the weight-only quantized Linear hot path.

TEST INFRASTRUCTURE ONLY. Nothing in the product (``infinitemodel_amd``) imports this package;
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
use it, and there only as the checker or the timed CPU comparator, never as the measured or
shipped path.

Contents
--------
``oracle.quant``   numpy restatement of the reference packers, dequant and
                   dequantize-then-matmul (bit-level bf16/fp16 rounding emulation).
``oracle.moe``     the reference MoE semantics (OLMoE eager experts loop, fused T==1 gather)
                   and the routing generator used by the benchmark configs.
``oracle.cpu_path`` the reference's CPU dispatch (torch tinygemm int4 + naive dequant+matmul),
                   used as the timed CPU baseline.

Parity pins (what fixes each function besides its own listing) are documented in each
module's docstring; every function here is pinned by at least one independent check in
``tests/test_oracle.py``.
"""
