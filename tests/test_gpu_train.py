"""Training fake quantization on an MI355X (lfm3-kv800_amd/train.py, the HIP counterpart of train.py:82-100, 238-242),
checked against the CPU oracle and against the HIP quantizer's own round trip (tests/test_train_hook.py:92-106)."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"


def say(*a):
    print("[gpu-train]", *a, flush=True)


def _inputs(oracle, seed, G=3):
    rng = np.random.RandomState(seed)
    k = rng.standard_normal((G, 256, 4, 128)) * rng.rand(1, 1, 4, 128) * 4 + 0.3
    v = rng.standard_normal((G, 256, 4, 128)) * 2
    return oracle.f32_to_bf16(k.astype(np.float32)), oracle.f32_to_bf16(v.astype(np.float32))


def test_fake_quant_k_vs_oracle(hip, oracle):
    """float32 inputs that are not bf16 values, an odd channel count, a constant channel and outliers: bit-exact."""
    from lfm3_kv800_amd import train as kt
    rng = np.random.RandomState(11)
    x = (rng.standard_normal((5, 256, 300)) * rng.rand(1, 1, 300) * 5).astype(np.float32)
    x[0, :, 7] = 1.25
    x[2, ::13, 40] *= 50
    say("fake_quant_k", x.shape)
    got = kt.fake_quant_k(torch.from_numpy(x).to(DEV)).cpu().numpy()
    assert np.array_equal(got, oracle.fake_quant_k(x))


def test_fake_quant_v_vs_oracle(hip, oracle):
    from lfm3_kv800_amd import train as kt
    rng = np.random.RandomState(12)
    v = (rng.standard_normal((2, 333, 4, 128)) * 3).astype(np.float32)   # token count not a multiple of the tiling
    say("fake_quant_v", v.shape)
    got = kt.fake_quant_v(torch.from_numpy(v).to(DEV), kt.hadamard(128)).cpu().numpy()
    assert np.array_equal(got, oracle.fake_quant_v(v))


def test_fake_quant_equals_hip_round_trip(hip, oracle):
    """tests/test_train_hook.py:92-101 on the GPU: fake_quant_k cast to bf16 equals the K of the HIP quantizer's
    dequantize(quantize(k, v)); fake_quant_v matches its V within the reference's atol 1e-5 (bit for bit here)."""
    from lfm3_kv800_amd import train as kt
    kb, vb = _inputs(oracle, 13)
    k = torch.from_numpy(kb.view(np.int16)).view(torch.bfloat16).to(DEV)
    v = torch.from_numpy(vb.view(np.int16)).view(torch.bfloat16).to(DEV)
    kr, vr = hip.dequantize_blocks(hip.quantize_blocks(k, v))
    say("round trip", tuple(k.shape))
    kq = kt.fake_quant_k(k.float().reshape(3, 256, 512)).reshape(3, 256, 4, 128).to(torch.bfloat16)
    assert torch.equal(kq, kr)
    vq = kt.fake_quant_v(v.float())
    assert torch.allclose(vq, vr, atol=1e-5, rtol=0)
    assert torch.equal(vq, vr)


def test_ste_gradient(hip, oracle):
    """Forward value fq(x), gradient identity (train.py:238-242)."""
    from lfm3_kv800_amd import train as kt
    x = torch.randn(2, 256, 512, device=DEV, requires_grad=True)
    y = kt.ste(x, kt.fake_quant_k)
    assert torch.equal(y.detach(), kt.fake_quant_k(x.detach()))
    g = torch.randn_like(y)
    y.backward(g)
    assert torch.equal(x.grad, g)
