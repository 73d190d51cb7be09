"""ctypes binding of the engine loop's fused elementwise kernels (include/lfm3_model.h, in libkv800_hip.so).

Each function takes bf16 CUDA tensors, allocates its outputs with torch and launches on the current stream; like
kv800_hip, there is no fallback: without the library or a GPU the first call raises ImportError."""
import ctypes

import torch

from . import kv800_hip

_VP, _I64, _I32, _F32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float
SIGNATURES = {
    "lfm3_hip_add_rmsnorm": (_I32, [_VP, _VP, _VP, _VP, _F32, _I64, _I64, _VP, _VP, _VP]),
    "lfm3_hip_silu_mul": (_I32, [_VP, _I64, _I64, _VP, _VP]),
    "lfm3_hip_qkv_post": (_I32, [_VP, _I64, _VP, _VP, _VP, _VP, _I64, _VP, _F32, _I64, _VP, _VP, _VP, _VP, _VP]),
    "lfm3_hip_conv_step": (_I32, [_VP, _I64, _VP, _VP, _I64, _I64, _VP, _VP]),
    "lfm3_hip_gate_mul": (_I32, [_VP, _VP, _I64, _I64, _VP, _VP]),
    "lfm3_hip_argmax": (_I32, [_VP, _I64, _I64, _I64, _VP, _VP]),
}
_BOUND = {}


def _lib():
    L = kv800_hip.ops()
    if id(L) not in _BOUND:
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype, fn.argtypes = res, args
        _BOUND.clear()
        _BOUND[id(L)] = True
    return L


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _stream(t):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _bf16(t, name):
    if t.dtype != torch.bfloat16 or t.device.type != "cuda":
        raise TypeError(f"{name} must be a bf16 CUDA tensor, got {t.dtype} on {t.device}")
    return t.contiguous()


def add_rmsnorm(h, x, w_post, w_next, eps):
    """(x + bf16(rms(h) w_post), bf16(rms(that) w_next)) for (R, 2048) rows; h None: (x, bf16(rms(x) w_next));
    w_next None: the second output is None."""
    L = _lib()
    x = _bf16(x, "x")
    R, H = x.shape
    xo = torch.empty_like(x) if h is not None else x
    no = torch.empty_like(x) if w_next is not None else None
    kv800_hip._check(L.lfm3_hip_add_rmsnorm(_ptr(_bf16(h, "h") if h is not None else None), _ptr(x),
                                            _ptr(w_post if h is not None else None), _ptr(w_next), float(eps), R, H,
                                            _ptr(xo if h is not None else None), _ptr(no), _stream(x)))
    return xo, no


def silu_mul(gu):
    """(R, 2F) [g | u] -> (R, F) bf16(bf16(silu(g)) u)."""
    L = _lib()
    gu = _bf16(gu, "gu")
    R, F2 = gu.shape
    out = torch.empty(R, F2 // 2, dtype=torch.bfloat16, device=gu.device)
    kv800_hip._check(L.lfm3_hip_silu_mul(_ptr(gu), R, F2 // 2, _ptr(out), _stream(gu)))
    return out


def qkv_post(qkv, q_w, k_w, cos_t, sin_t, pos, eps):
    """qkv (R, >= 3072) rows [q 16x128 | k 4x128 | v 4x128 | ...] -> q_rot (R, 16, 128), k_pre, k_rot, v (R, 4, 128);
    cos_t / sin_t (P, 64) bf16 per frequency, pos (R,) int64."""
    L = _lib()
    if qkv.stride(-1) != 1:
        raise ValueError("qkv rows must be contiguous")
    R = qkv.shape[0]
    dev = qkv.device
    q = torch.empty(R, 16, 128, dtype=torch.bfloat16, device=dev)
    kp, kr, v = (torch.empty(R, 4, 128, dtype=torch.bfloat16, device=dev) for _ in range(3))
    kv800_hip._check(L.lfm3_hip_qkv_post(_ptr(qkv), qkv.stride(0), _ptr(q_w), _ptr(k_w), _ptr(cos_t), _ptr(sin_t),
                                         cos_t.shape[0], _ptr(pos), float(eps), R, _ptr(q), _ptr(kp), _ptr(kr),
                                         _ptr(v), _stream(qkv)))
    return q, kp, kr, v


def conv_step(bcx, conv_w, state):
    """Short-conv decode step: bcx (R, >= 3H) rows [B | C | x], conv_w (H, 7), state (R, H, 6) updated in place ->
    (R, H)."""
    L = _lib()
    if bcx.stride(-1) != 1 or not state.is_contiguous():
        raise ValueError("bcx rows and the state must be contiguous")
    R, H = state.shape[0], state.shape[1]
    out = torch.empty(R, H, dtype=torch.bfloat16, device=bcx.device)
    kv800_hip._check(L.lfm3_hip_conv_step(_ptr(bcx), bcx.stride(0), _ptr(conv_w.contiguous()), _ptr(state), R, H,
                                          _ptr(out), _stream(bcx)))
    return out


def gate_mul(o, g):
    """o (R, 16, 128) times bf16(sigmoid(g)) per head; g (R, >= 16) with contiguous rows (a column slice is fine)."""
    L = _lib()
    o = _bf16(o, "o")
    out = torch.empty_like(o)
    kv800_hip._check(L.lfm3_hip_gate_mul(_ptr(o), _ptr(g), g.stride(0), o.shape[0], _ptr(out), _stream(o)))
    return out


def argmax(x):
    """(R, V) bf16 -> (R,) int64 index of each row's largest value (torch.argmax(-1) of the same values)."""
    L = _lib()
    x = _bf16(x, "x")
    R, V = x.shape
    out = torch.empty(R, dtype=torch.int64, device=x.device)
    kv800_hip._check(L.lfm3_hip_argmax(_ptr(x), R, V, x.stride(0), _ptr(out), _stream(x)))
    return out
