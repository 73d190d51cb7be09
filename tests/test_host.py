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
        kv._resolve("cuda")


def test_unknown_backend_rejected():
    with pytest.raises(ValueError):
        kv.set_backend("cuda-graphs")


def test_env_backend(monkeypatch):
    monkeypatch.setenv("LFM3KV_BACKEND", "hip")
    assert kv._requested() == "hip"
    ok, why = kv._available("hip", "cpu")
    assert not ok and "ROCm" in why


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


def test_prefill_window_rows_on_host(oracle):
    """The window-layer extend rows (vllm_cache.prefill_window_rows) are host-side gathers + torch attention; the GPU
    test's cases run here on CPU tensors against the same float64 restatement."""
    import test_gpu_prefill as tp
    old = tp.DEV
    tp.DEV = "cpu"
    try:
        tp.test_prefill_window_rows(None, oracle)
    finally:
        tp.DEV = old
