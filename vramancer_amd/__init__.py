"""vramancer_amd — MI355X-native paged-attention decode over a quantized KV
cache, a drop-in for VRAMancer's core/paged_attention_cuda.py,
core/kv_quantizer.py and core/turboquant_cuda.py.

Modules:
  paged_attention_cuda  paged_attention_decode / _q4 (split-K gfx950 kernels)
  kv_quant              int8 / fp8-e4m3 pools: quantize-on-append, page writes
  kv_quantizer          KVCacheCompressor (TurboQuant) on the GPU
  turboquant_cuda       CUDATurboQuantOps surface of the TurboQuant kernels
  build                 builds libvrm_paged.so with hipcc for gfx950
"""
__version__ = "0.1.0"
