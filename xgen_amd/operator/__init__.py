"""Modules and functions with the reference's x_base.operator surface for the
W8A8 linear path (h3_fp8, h3_fp8_quant, h3_abs_peak, matmul, npu_fusion.nq2,
npu_fusion.runtime), backed by the xgen_amd HIP kernels."""
