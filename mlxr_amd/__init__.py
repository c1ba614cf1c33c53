"""mlxr_amd -- MI355X (gfx950) quantized matmul path for MLXR (q_gemm_dequant)."""
from .qgemm import (F16, F32, BF16, PATH_AUTO, PATH_GEMV, PATH_MFMA, PackedWeight, QGemmError,  # noqa: F401
                    QuantType, compute_quantized_weight_size, dequantize, get_bytes_per_weight,
                    get_default_group_size, gguf_size, lib, MlpWorkspace, mlp_workspace_size, pack_weights, packed_size, q_gemm_dequant,
                    quant_type_name, q_gemm_dequant_grouped, q_gemm_mlp, q_gemm_swiglu, synth_act, synth_gguf,
                    workspace_size, auto_path)
from .layers import MLP, Linear, swiglu  # noqa: E402,F401
