"""800h fake quantization for training on ROCm GPUs: the HIP counterpart of the reference's train.py:82-100, 238-242.

The reference trains with straight-through 800h K / V (patch_for_training): the forward value of the quantized
layers' keys and values is what the cache would hold after a quantize -> dequantize round trip, the gradient passes
straight through. Its fake_quant_k / fake_quant_v are torch expressions; here they are one HIP launch each
(kv800_hip_fake_quant_k / _v), with the same signatures and values:

  fake_quant_k(x)     x (..., G, 256, C) float32 (groups of 256 tokens on dim -2) -> float32, bit-identical to
                      train.py:82-89 and, after the bf16 cast, to the quantizer's K round trip;
  fake_quant_v(v, H)  v (..., 4, 128) float32 -> float32, the V of the quantizer's round trip (train.py:92-100;
                      H must be the normalized 128-point Hadamard, the only one the format uses);
  ste(x, fq)          forward fq(x), gradient identity (train.py:238-242).

The reference's patch_for_training resolves fake_quant_k / fake_quant_v as module globals at call time, so on ROCm a
caller swaps these in (`lfm3_kv800.train.fake_quant_k = lfm3_kv800_amd.train.fake_quant_k`, the same for _v).
Tensors must be on a ROCm device: there is no CPU path.
"""
import torch

from . import kv800, kv800_hip

__all__ = ["fake_quant_k", "fake_quant_v", "ste", "hadamard"]

hadamard = kv800.hadamard


def fake_quant_k(x):
    """x (..., G, 256, C) float32 pre-RoPE keys -> dequantized 800h keys (float32), per (group, channel): 2-bit codes,
    fp8 lo and scale (hi - lo) / 3 (train.py:82-89)."""
    return kv800_hip.fake_quant_k(x)


def fake_quant_v(v, H=None):
    """v (..., 4, 128) float32 values -> dequantized 800h values (float32): per-head Hadamard, one bit per dim over each
    pair of heads, fp8 lo and scale hi - lo, rotated back (train.py:92-100)."""
    if H is not None and tuple(H.shape) != (128, 128):
        raise ValueError(f"H must be the 128 x 128 normalized Hadamard, got shape {tuple(H.shape)}")
    return kv800_hip.fake_quant_v(v)


def ste(x, fq):
    """Forward value exactly fq(x); gradient straight through (identity), as train.py:238-242."""
    with torch.no_grad():
        y = fq(x)
    return y + (x - x.detach())
