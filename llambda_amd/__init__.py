"""llambda_amd -- an MI355X (gfx950) backend for llambda's quantized decode
hot path: the Q4_K / Q6_K dequant-fused GEMV and the routed-MoE feed-forward
of qwen3next and nemotron_h_moe, behind llambda's accelerator-backend
protocol.

Modules:
  native       ctypes bindings of libllambda_hip.so (the C ABI)
  hip_backend  projection sessions and the :hip backend descriptor
  moe          routed-MoE layer sessions
  accelerator  the backend descriptor protocol
  projection   the tensor-indexed binding store with runtime fallback
  ggml         type tags and block geometry
  synthetic    seeded GGUF-layout test tensors
  build        compiles the library (hipcc, gfx950)
"""
__version__ = "0.1.0"
