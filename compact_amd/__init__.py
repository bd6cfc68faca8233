"""compact_amd: the FlashFFN v3 hot path of SDMuhsin/CompAct, MI355X-native.

A LLaMA-style SwiGLU FFN whose backward cache is int4/int8 per-group absmax
codes of h_gate/h_up, computed by hand-written gfx950 HIP kernels behind the C
ABI in include/compact_amd.h (libcompact_amd.so, loaded with ctypes).  The
Python API mirrors the reference's src/flashffn.py.
"""

from .kernels import (  # noqa: F401
    _V3_COUNTERS, v3_reset_counters,
    silu_mul, swiglu_backward, swiglu_backward_glu, silu_mul_quant, dequant_swiglu_backward,
    v3_quantize_group_absmax, v3_dequantize_group_absmax,
    triton_silu_mul, triton_swiglu_backward, triton_swiglu_backward_glu,
    triton_silu_mul_quant, triton_dequant_swiglu_backward,
    outlier_select, outlier_select_pair, v3_quantize_outlier, v3_dequantize_outlier,
    silu_mul_quant_outlier, dequant_swiglu_backward_outlier, dora_scale, col_dot_div, dora_col_norm,
    topk_abs, topk_scatter,
)
from .flashffn import (  # noqa: F401
    FlashFFNv3Function, FlashFFNv3, make_v3_forward, _v3_extract_proj, _v3_proj_kind,
    FlashFFNv3AdapterFunction, make_v3_adapter_forward, _v3_extract_proj_adapter,
    _v3_dora_col_norm, FlashFFNFunction, FlashFFN, StandardFFN,
)
