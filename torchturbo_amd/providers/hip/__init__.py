"""HIP (gfx950) providers: ``kind=CUSTOM``, ``devices=(CUDA,)``, priority 200.

PyTorch-ROCm reports the GPU as ``cuda``; priority 200 ranks these providers
above every reference CUDA provider (TransformerEngine at 100, grouped_gemm
at 0; ``src/torchturbo/ops/providers/cuda/*.py``).
"""

PRIORITY = 200
