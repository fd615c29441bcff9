"""MI355X-native `hip` backend for the Lykuro inference engine.

The compute path is hand-written gfx950 HIP (engine_amd/csrc/kernels) behind
the C ABI of include/lykuro_hip.h; the host model (QwenHipModel,
engine_amd/csrc/host) implements the engine's GenerativeModel interface in
C++20. This package only binds those libraries for Python callers (tests,
bench): PyTorch is used for device memory and streams, nothing else.
"""
from .lib import LykError, kernels  # noqa: F401
