"""Writes tests/golden/quantize_golden.npz: the bytes the reference quantizer (kv800.py:56-76, evaluated by
torch_statement.quantize on CPU torch) produces for seeded bf16 K / V inputs. The inputs are not stored: tests
regenerate them with case_inputs() and check them against the stored SHA-256.

    python tests/golden/make_golden.py

Cases (inputs from numpy's legacy RandomState, float32 normals rounded to bf16):
  parity : 2 sub-blocks, K = N(0,1) + 3 N(0,1) per-channel offset, V = N(0,1)  (tests/test_parity.py:85-86 shape)
  outlier: 2 sub-blocks, K, V = N(0,1) with 1 % of the elements x 8              (config C2)
  edge   : 1 sub-block with constant channels (hi == lo), tiny and large magnitudes near fp8 boundaries, and
           V rows whose Hadamard transform is constant (all-equal V)
  scaled : 4 sub-blocks, K, V = 4 N(0,1) (SHA-256 of each 51,200-byte block only)."""
import hashlib
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
import torch_statement as ts  # noqa: E402


def bf16_bits(x):
    u = np.ascontiguousarray(x, np.float32).view(np.uint32)
    return ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)


def as_bf16(bits):
    return torch.from_numpy(bits.astype(np.int16)).view(torch.bfloat16)


def case_inputs(name):
    shape = (256, 4, 128)
    if name == "parity":
        rng = np.random.RandomState(1001)
        k = rng.standard_normal((2,) + shape).astype(np.float32) + 3 * rng.standard_normal((1, 1, 4, 128)).astype(np.float32)
        v = rng.standard_normal((2,) + shape).astype(np.float32)
    elif name == "outlier":
        rng = np.random.RandomState(1002)
        k = rng.standard_normal((2,) + shape).astype(np.float32)
        v = rng.standard_normal((2,) + shape).astype(np.float32)
        k[rng.random_sample(k.shape) < 0.01] *= 8
        v[rng.random_sample(v.shape) < 0.01] *= 8
    elif name == "edge":
        rng = np.random.RandomState(1003)
        k = rng.standard_normal((1,) + shape).astype(np.float32)
        v = rng.standard_normal((1,) + shape).astype(np.float32)
        k[0, :, 0, :8] = 0.75                                       # constant channels: hi == lo
        k[0, :, 1, :16] *= 1e-3                                     # tiny ranges: fp8 subnormal scales
        k[0, :, 2, :16] *= 60.0                                     # large ranges near the fp8 top
        k[0, :, 3, 100:] = np.float32(0.015625) * rng.randint(-3, 4, size=(256, 28))   # exact fp8 grid values
        v[0, :16] = 0.5                                             # all-equal V rows
        v[0, 16:32, 1] *= 1e-4
    else:
        rng = np.random.RandomState(1004)
        k = 4 * rng.standard_normal((4,) + shape).astype(np.float32)
        v = 4 * rng.standard_normal((4,) + shape).astype(np.float32)
    return bf16_bits(k), bf16_bits(v)


def input_digest(kb, vb):
    """SHA-256 of the regenerated inputs: a drift check of the seeded generator."""
    return hashlib.sha256(kb.tobytes() + vb.tobytes()).hexdigest()


def main():
    data = {}
    for name in ("parity", "outlier", "edge", "scaled"):
        kb, vb = case_inputs(name)
        out = ts.quantize(as_bf16(kb), as_bf16(vb)).numpy()
        data[f"{name}_input_sha256"] = np.array(input_digest(kb, vb))
        if name == "scaled":
            data[f"{name}_sha256"] = np.array([hashlib.sha256(out[m].tobytes()).hexdigest() for m in range(out.shape[0])])
        else:
            data[f"{name}_out"] = out
    path = os.path.join(HERE, "quantize_golden.npz")
    np.savez_compressed(path, **data)
    print(path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
