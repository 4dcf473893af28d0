"""MI355X (gfx950) quantized matrix-product path behind the reference's operator API.

The compute path is libstark_qmm.so (HIP kernels + C ABI, include/stark_qmm.h);
``stark_amd.qmm`` is the Python mirror of the reference's MatmulKernel /
mapped_many / MoE interfaces over that ABI.
"""
