"""Export of fine-tuned quantized models (export/__init__.py of the
reference): the merged fp16 weights, built on the GPU from the quantized
buffers."""
from rocm_qlora.export.gguf_export import merge_and_export_fp16

__all__ = ["merge_and_export_fp16"]
