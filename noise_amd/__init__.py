"""MI355X-native population-perturbed forward of the Noise 37.7M GPT (EGGROLL path).

Host side in PyTorch-ROCm; compute in hand-written gfx950 HIP kernels behind the C ABI of
`libnoise_hip.so` (declared in include/noise_hip.h).
"""
from .model import GPT, GPTConfig, make_model  # noqa: F401
