"""Host logic of the product package on the CPU: backend selection and its failure modes (the product path raises
instead of falling back), the Paged descriptor, hadamard, and the import contract of the HIP binding."""
import os

import pytest
import torch

import lfm3_kv800_amd.kv800 as kv
import lfm3_kv800_amd.kv800_hip as kh


@pytest.fixture(autouse=True)
def _reset():
    kv.set_backend(None)
    yield
    kv.set_backend(None)


def test_hadamard_matches_sylvester():
    import torch_statement as ts
    H = kv.hadamard(128)
    assert torch.equal(H.view(torch.int32), ts.sylvester().view(torch.int32))
    assert torch.allclose(H @ H, torch.eye(128), atol=1e-6)


def test_flat_view():
    t = torch.arange(24).view(4, 6)[1:]
    f = kv.flat(t)
    assert f.shape == (18,) and int(f[0]) == 6 and int(f[-1]) == 23


def test_cpu_decode_raises_no_fallback():
    q = torch.zeros(1, 16, 128, dtype=torch.bfloat16)
    P = kv.Paged(epool=torch.zeros(1, dtype=torch.bfloat16), N=torch.ones(1, dtype=torch.int32))
    with pytest.raises(RuntimeError, match="no 800h decode backend"):
        kv.decode(P, q, None, None, None)


@pytest.mark.parametrize("name", ["torch", "triton", "sycl"])
def test_reference_backends_are_not_in_this_build(name):
    kv.set_backend(name)
    with pytest.raises(RuntimeError, match="not part of the MI355X build"):
        kv._SEL.backend_for("cuda")


def test_unknown_backend_rejected():
    kv.set_backend("hip")
    with pytest.raises(ValueError):
        kv.set_backend("cuda-graphs")
    assert kv._SEL.wanted() == "hip"           # the rejected name left the setting as it was


def test_env_backend(monkeypatch):
    monkeypatch.setenv("LFM3KV_BACKEND", "hip")
    assert kv._SEL.wanted() == "hip"
    why = kv._SEL.refusal("hip", "cpu")
    assert why is not None and "ROCm" in why
    with pytest.raises(RuntimeError, match="was requested"):
        kv._SEL.backend_for("cpu")


def test_hip_ops_raises_importerror_without_gpu():
    if torch.cuda.is_available():
        pytest.skip("GPU present")
    with pytest.raises(ImportError):
        kh.ops()


def test_paged_slots():
    P = kv.Paged(N=1, win=256)
    assert P.N == 1 and P.win == 256 and P.qpool is None


def test_plan_rules():
    assert kh.plan(8, 0) == (0, 1)
    assert kh.plan(64, 127, spb=16) == (8, 16)
    ns, spb = kh.plan(64, 127, target=1024)            # the reference's rule: spb = ceil(nqmax * B * 4 / target)
    assert spb == 32 and ns == 4


def test_ranges_helper():
    """vllm_cache._ranges: the concatenated key / position ranges the prefill rows assemble on the host."""
    from lfm3_kv800_amd import vllm_cache as vc
    got = vc._ranges([5, 0, 100, 7], [3, 0, 2, 1])
    assert got.tolist() == [5, 6, 7, 100, 101, 7]
    assert vc._ranges([], []).tolist() == []
    assert vc._ranges([3], [0]).tolist() == []


def test_host_to_device_on_cpu():
    """kv800_hip.host_to_device: lists, numpy arrays and tensors become tensors of the asked dtype on the device (on
    the CPU here; on a GPU the copy goes through pinned memory, asynchronously)."""
    import numpy as np
    dev = torch.device("cpu")
    a = kh.host_to_device([3, 1, 2], torch.int32, dev)
    assert a.dtype == torch.int32 and a.tolist() == [3, 1, 2]
    b = kh.host_to_device(np.arange(4, dtype=np.int64), torch.int64, dev)
    assert b.dtype == torch.int64 and b.tolist() == [0, 1, 2, 3]
    c = kh.host_to_device(torch.tensor([7, 8], dtype=torch.int64), torch.int32, dev)
    assert c.dtype == torch.int32 and c.tolist() == [7, 8]
    assert kh.host_to_device([], torch.int64, dev).numel() == 0
