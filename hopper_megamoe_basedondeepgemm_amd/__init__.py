"""MI355X (gfx950) MegaMoE: the fused decode MoE layer of the DeepGEMM MegaMoE fork,
re-built on CDNA4 matrix cores behind the same Python entry points.

Exports mirror deep_gemm/__init__.py:84-110 for the MegaMoE path plus the packers."""
from . import _lib
from .mega import (FusedSymmBuffer, get_fused_symm_buffer_for_mega_moe,
                   transform_mxfp4_weights_for_mega_moe_fused, transform_qoq_weights_for_mega_moe_fused,
                   transform_weights_for_mega_moe,
                   fable_router_quant_topk_frontend, fable_frontend_keys, mxfp4_mega_moe_fused, mxfp4_mega_moe_split,
                   mxfp4_mega_moe_from_bf16, qoq_mega_moe_fused, qoq_mega_moe_split,
                   transform_nvfp4_weights_for_mega_moe_fused, fp4_fp4_mega_moe, nvfp4_mega_moe,
                   transform_qoq_int4_weights_for_mega_moe_sm90, SymmBuffer, get_symm_buffer_for_mega_moe,
                   get_mxfp4_mega_moe_sm90_block_n, transform_mxfp4_weights_for_mega_moe_sm90, mxfp4_mega_moe,
                   int4_mega_moe, FE_PATH_WMMA, FE_PATH_SWAPAB, FE_PATH_CC, fable_frontend_path,
                   fable_frontend_router_ctas, fable_frontend_workspace_bytes, fable_frontend_workspace,
                   fable_router_weight_fragment_layout, fable_frontend_stamps, get_nvfp4_mega_moe_sm90_block_n,
                   get_nvfp4_mega_moe_sm90_weight_layout)
from . import quantization_mxfp4, quantization_mxfp4_fused, quantization_nvfp4, quantization_qoq_fused
from .utils import per_token_cast_to_fp4, per_token_cast_to_fp8, ceil_div, align
from . import checkpoint
from .checkpoint import (mxfp4_checkpoint_to_mega_moe, nvfp4_checkpoint_to_mega_moe, mega_moe_to_mxfp4_checkpoint,
                         mega_moe_to_nvfp4_checkpoint, untransform_mxfp4_weights_for_mega_moe_fused,
                         untransform_nvfp4_weights_for_mega_moe_fused)

__all__ = [
    "FusedSymmBuffer", "get_fused_symm_buffer_for_mega_moe", "transform_mxfp4_weights_for_mega_moe_fused",
    "transform_qoq_weights_for_mega_moe_fused",
    "transform_weights_for_mega_moe", "fable_router_quant_topk_frontend", "fable_frontend_keys",
    "mxfp4_mega_moe_fused",
    "mxfp4_mega_moe_split", "mxfp4_mega_moe_from_bf16", "qoq_mega_moe_fused", "qoq_mega_moe_split",
    "transform_nvfp4_weights_for_mega_moe_fused", "fp4_fp4_mega_moe", "nvfp4_mega_moe",
    "transform_qoq_int4_weights_for_mega_moe_sm90", "quantization_mxfp4", "quantization_mxfp4_fused",
    "quantization_nvfp4",
    "quantization_qoq_fused", "per_token_cast_to_fp4", "per_token_cast_to_fp8", "ceil_div", "align",
    "SymmBuffer", "get_symm_buffer_for_mega_moe", "get_mxfp4_mega_moe_sm90_block_n",
    "transform_mxfp4_weights_for_mega_moe_sm90", "mxfp4_mega_moe", "int4_mega_moe",
    "FE_PATH_WMMA", "FE_PATH_SWAPAB", "FE_PATH_CC", "fable_frontend_path", "fable_frontend_router_ctas",
    "fable_frontend_workspace_bytes", "fable_frontend_workspace", "fable_router_weight_fragment_layout",
    "checkpoint", "mxfp4_checkpoint_to_mega_moe", "nvfp4_checkpoint_to_mega_moe", "mega_moe_to_mxfp4_checkpoint",
    "mega_moe_to_nvfp4_checkpoint", "untransform_mxfp4_weights_for_mega_moe_fused",
    "untransform_nvfp4_weights_for_mega_moe_fused", "fable_frontend_stamps", "get_nvfp4_mega_moe_sm90_block_n",
    "get_nvfp4_mega_moe_sm90_weight_layout",
]
