"""qwen3-tts per-frame token loop on MI355X (gfx950).

Python side of the package: hyperparameters, synthetic weights, the ctypes
binding of the device C ABI (include/q3t_dev.h) and the host driver that
mirrors TTSTransformer::generate (src/tts_transformer.cpp:3007-3371).
"""
from .config import Config, full_06b, tiny  # noqa: F401
