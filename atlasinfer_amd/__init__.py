"""atlasinfer_amd -- MI355X (gfx950) implementation of AtlasInfer's adaptive
hybrid FP8/FP16 weight quantization path.

    atlasinfer_amd.quant.adaptive_quantizer   quantize / dequantize / QuantizedTensor
    atlasinfer_amd.integration.atlas_wrappers QuantizedLinear
    atlasinfer_amd.integration.model_modifier apply_atlas_quantization_to_model

The same modules are importable under the reference's names
(atlasinfer_core.quant.adaptive_quantizer, integration.atlas_wrappers,
integration.model_modifier).  Kernels live in libatlasinfer_amd.so
(csrc/*.hip, C ABI in include/atlasinfer_amd.h), built by
``python -m atlasinfer_amd.build``.
"""
