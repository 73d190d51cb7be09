"""kv800_hip_decode_noalloc (the decode without a workspace argument, its partials in the library's static per-device
scratch) against kv800_hip_decode_sized with a caller workspace: bit-identical outputs, through the C ABI, on two calls
in a row (the second with fewer rows and shorter sequences, so stale scratch contents from the first would show),
with and without a prebuilt rope pair table, on a quantized and a window layer; oversized calls are rejected on the host."""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def say(*a):
    print("[no-alloc]", *a, flush=True)


def _layer(oracle, seed, lens, win):
    import test_gpu_parity as G
    rng = np.random.RandomState(seed)
    K = [oracle.randn_bf16(rng, (n, 4, 128), offset=rng.standard_normal((1, 4, 128))) for n in lens]
    V = [oracle.randn_bf16(rng, (n, 4, 128)) for n in lens]
    q = oracle.randn_bf16(rng, (len(lens), 16, 128), scale=1.5)
    case = oracle.build_paged(lambda b, p0, p1: (K[b][p0:p1], V[b][p0:p1]), lens, win=win, ebs=128, shuffle_seed=seed)
    return G.upload(case), G.to_dev_bf16(q)


def _both(hip, oracle, P, q, cos, sin, with_table, spb):
    """(workspace entry output, no-alloc entry output) for one layer."""
    L = hip.ops()
    B = q.shape[0]
    s, qbytes, eelems, selems = hip.paged_struct(P, B)
    cs2 = hip.rope_pairs(cos, sin) if with_table and s.nqmax else None
    rows = cos.shape[0]
    if not s.nqmax:
        wsb = int(L.kv800_hip_decode_workspace(B, 0, 0))
    elif spb > 0:
        wsb = int(L.kv800_hip_decode_workspace(B, -(-s.nqmax // spb), 0 if cs2 is not None else s.nqmax * 256))
    else:
        G = -spb if spb < 0 else hip.plan_balanced(B, s.nqmax)
        wsb = int(L.kv800_hip_decode_workspace_balanced(B, G, 0 if cs2 is not None else s.nqmax * 256))
    ws = torch.empty(wsb, dtype=torch.uint8, device=DEV)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    P_ = lambda t: ctypes.c_void_p(t.data_ptr()) if t is not None else None
    ref = torch.empty(B, 16, 128, dtype=torch.bfloat16, device=DEV)
    out = torch.full((B, 16, 128), float("nan"), dtype=torch.bfloat16, device=DEV)
    assert L.kv800_hip_decode_sized(ctypes.byref(s), P_(q), B, P_(cos), P_(sin), rows, P_(cs2), qbytes, eelems, selems,
                                    P_(ref), P_(ws), wsb, spb, st) == 0, L.kv800_hip_last_error()
    rc = L.kv800_hip_decode_noalloc(ctypes.byref(s), P_(q), B, P_(cos), P_(sin), rows, P_(cs2), qbytes, eelems,
                                    selems, P_(out), spb, st)
    assert rc == 0, L.kv800_hip_last_error()
    torch.cuda.synchronize()
    return ref, out


@pytest.mark.parametrize("with_table", [True, False])
def test_noalloc_matches_workspace_entry(hip, oracle, with_table):
    cos, sin = (torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).to(DEV)
                for a in oracle.rope_tables(5200))
    calls = [  # (seed, lengths, window, spb): a larger call first, then a smaller one on the same scratch
        (11, [5000, 1, 700, 3000, 383, 4100, 1500], 0, 0),
        (12, [900, 2400, 385], 0, 0),
        (13, [3000, 777, 5000, 260], 0, 3),
        (14, [1500, 260, 3], 256, 0),
    ]
    for seed, lens, win, spb in calls:
        say("call", seed, "rows", len(lens), "win", win, "spb", spb, "table", with_table)
        P, q = _layer(oracle, seed, lens, win)
        ref, out = _both(hip, oracle, P, q, cos, sin, with_table, spb)
        assert torch.isfinite(ref.float()).all()
        assert torch.equal(ref.view(torch.int16), out.view(torch.int16)), (seed, (ref.float() - out.float()).abs().max())


def test_noalloc_rejects_oversized_call(hip):
    L = hip.ops()
    s = hip.Paged()
    s.nqmax, s.win = 127, 0
    B = 20000                                     # far more partials than the scratch holds
    rc = L.kv800_hip_decode_noalloc(ctypes.byref(s), None, B, None, None, 32768, None, 0, 0, 0, None, 0, None)
    assert rc == -1
    msg = L.kv800_hip_last_error().decode()
    say("rejected:", msg)
    assert "scratch" in msg
