"""MI355X (gfx950) fused causal attention with the Python API of the cuTile reference.

attention.fused.fused.fused_attention            causal MHA forward
attention.gqa.fused_gqa.fused_gqa_attention      causal GQA/MQA forward
attention.backward.fused_backward.fused_attention_autograd   forward + recompute backward

All three call hand-written HIP kernels in libfa.so through ctypes (attention._lib).
"""
