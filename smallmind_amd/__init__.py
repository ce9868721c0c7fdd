"""smallmind_amd -- MI355X (gfx950) backend for SmallMind's quantized transformer forward path.

Layers (see include/smx.h for the C-ABI the reference's C# code would bind):
  quantization  IWeightTensor mirror (GpuWeightTensor) + dequant / quantize / norm / RoPE /
                softmax / attention / activation operators
  model         GpuTransformerModel (TransformerModel.Forward + KV cache) and
                GpuInferenceSession (prefill + greedy decode on the device)
  synthetic     seeded workloads of the benchmark configurations

All compute runs in libsmx.so; importing fails if it has not been built.
"""
from . import _lib

_lib.load()

from .model import GpuContext, GpuInferenceSession, GpuTransformerModel, ModelConfig  # noqa: E402
from .quantization import GgufTensorType, GpuWeightTensor, SmxError  # noqa: E402

__all__ = ["GpuContext", "GpuInferenceSession", "GpuTransformerModel", "ModelConfig",
           "GgufTensorType", "GpuWeightTensor", "SmxError"]
