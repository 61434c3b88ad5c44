"""infinitemodel_amd: MI355X-native (gfx950) weight-only quantized Linear hot path.

A drop-in for the quantized-Linear family of InfiniteModel's ``worker_quant.py``
(``QuantLinear4`` / ``QuantLinear2`` / ``QuantLinear`` / ``Packed4Tensor3D`` + the fused-MoE
experts forward) and for the ``_shards/<quant>/`` packers of ``shard_compile.py``, backed by
hand-written HIP kernels in ``libimq.so`` (see ``include/imq.h``).
"""
__version__ = "0.1.0"
