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
    "lfm3_hip_shuffle_weight": (_I32, [_VP, _I64, _I64, _I64, _VP, _VP]),
    "lfm3_hip_linear": (_I32, [_VP, _I64, _VP, _I64, _I64, _I64, _VP, _I64, _I32, _VP, _I32, _VP]),
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


def _same(t, name, dtype, like, shape=None):
    """t must have `dtype`, live on like's device and (when given) have `shape`; returns it contiguous."""
    if t.dtype != dtype or t.device != like.device:
        raise TypeError(f"{name} must be {dtype} on {like.device}, got {t.dtype} on {t.device}")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} must be {tuple(shape)}, got {tuple(t.shape)}")
    return t.contiguous()


def add_rmsnorm(h, x, w_post, w_next, eps):
    """(x + bf16(rms(h) w_post), bf16(rms(that) w_next)) for (R, 2048) rows; h None: (x, bf16(rms(x) w_next));
    w_next None: the second output is None."""
    L = _lib()
    x = _bf16(x, "x")
    if x.dim() != 2 or x.shape[1] != 2048:
        raise ValueError(f"x must be (R, 2048), got {tuple(x.shape)}")
    R, H = x.shape
    if h is not None:
        h = _same(h, "h", torch.bfloat16, x, x.shape)
        w_post = _same(w_post, "w_post", torch.bfloat16, x, (H,))
    if w_next is not None:
        w_next = _same(w_next, "w_next", torch.bfloat16, x, (H,))
    xo = torch.empty_like(x) if h is not None else x
    no = torch.empty_like(x) if w_next is not None else None
    kv800_hip._check(L.lfm3_hip_add_rmsnorm(_ptr(h), _ptr(x),
                                            _ptr(w_post if h is not None else None), _ptr(w_next), float(eps), R, H,
                                            _ptr(xo if h is not None else None), _ptr(no), _stream(x)))
    return xo, no


def silu_mul(gu):
    """(R, 2F) [g | u] -> (R, F) bf16(bf16(silu(g)) u)."""
    L = _lib()
    gu = _bf16(gu, "gu")
    if gu.dim() != 2 or gu.shape[1] % 16:
        raise ValueError(f"gu must be (R, 2F) with F a multiple of 8, got {tuple(gu.shape)}")
    R, F2 = gu.shape
    out = torch.empty(R, F2 // 2, dtype=torch.bfloat16, device=gu.device)
    kv800_hip._check(L.lfm3_hip_silu_mul(_ptr(gu), R, F2 // 2, _ptr(out), _stream(gu)))
    return out


def qkv_post(qkv, q_w, k_w, cos_t, sin_t, pos, eps):
    """qkv (R, >= 3072) rows [q 16x128 | k 4x128 | v 4x128 | ...] -> q_rot (R, 16, 128), k_pre, k_rot, v (R, 4, 128);
    cos_t / sin_t (P, 64) bf16 per frequency, pos (R,) int64."""
    L = _lib()
    if qkv.dtype != torch.bfloat16 or qkv.device.type != "cuda" or qkv.dim() != 2 or qkv.shape[1] < 3072:
        raise TypeError(f"qkv must be a bf16 CUDA tensor (R, >= 3072), got {qkv.dtype} {tuple(qkv.shape)}")
    if qkv.stride(-1) != 1:
        raise ValueError("qkv rows must be contiguous")
    R = qkv.shape[0]
    dev = qkv.device
    q_w = _same(q_w, "q_w", torch.bfloat16, qkv, (128,))
    k_w = _same(k_w, "k_w", torch.bfloat16, qkv, (128,))
    cos_t = _same(cos_t, "cos_t", torch.bfloat16, qkv)
    sin_t = _same(sin_t, "sin_t", torch.bfloat16, qkv, cos_t.shape)
    if cos_t.dim() != 2 or cos_t.shape[1] != 64:
        raise ValueError(f"cos_t / sin_t must be (P, 64), got {tuple(cos_t.shape)}")
    pos = _same(pos, "pos", torch.int64, qkv, (R,))
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
    if bcx.dtype != torch.bfloat16 or bcx.device.type != "cuda" or bcx.dim() != 2:
        raise TypeError(f"bcx must be a bf16 CUDA tensor (R, >= 3H), got {bcx.dtype} {tuple(bcx.shape)}")
    if state.dtype != torch.bfloat16 or state.device != bcx.device or state.dim() != 3 or state.shape[2] != 6:
        raise TypeError(f"state must be bf16 (R, H, 6) on {bcx.device}, got {state.dtype} {tuple(state.shape)}")
    if bcx.stride(-1) != 1 or not state.is_contiguous():
        raise ValueError("bcx rows and the state must be contiguous")
    R, H = state.shape[0], state.shape[1]
    if bcx.shape[0] != R or bcx.shape[1] < 3 * H:
        raise ValueError(f"bcx must be ({R}, >= {3 * H}), got {tuple(bcx.shape)}")
    conv_w = _same(conv_w, "conv_w", torch.bfloat16, bcx, (H, 7))
    out = torch.empty(R, H, dtype=torch.bfloat16, device=bcx.device)
    kv800_hip._check(L.lfm3_hip_conv_step(_ptr(bcx), bcx.stride(0), _ptr(conv_w), _ptr(state), R, H,
                                          _ptr(out), _stream(bcx)))
    return out


def gate_mul(o, g):
    """o (R, 16, 128) times bf16(sigmoid(g)) per head; g (R, >= 16) with contiguous rows (a column slice is fine)."""
    L = _lib()
    o = _bf16(o, "o")
    if o.dim() != 3 or o.shape[1:] != (16, 128):
        raise ValueError(f"o must be (R, 16, 128), got {tuple(o.shape)}")
    if g.dtype != torch.bfloat16 or g.device != o.device or g.dim() != 2 or g.shape[0] != o.shape[0] \
            or g.shape[1] < 16 or g.stride(-1) != 1:
        raise ValueError(f"g must be bf16 (R, >= 16) with contiguous rows on {o.device}")
    out = torch.empty_like(o)
    kv800_hip._check(L.lfm3_hip_gate_mul(_ptr(o), _ptr(g), g.stride(0), o.shape[0], _ptr(out), _stream(o)))
    return out


def argmax(x):
    """(R, V) bf16 -> (R,) int64 index of each row's largest value (torch.argmax(-1) of the same values)."""
    L = _lib()
    x = _bf16(x, "x")
    if x.dim() != 2:
        raise ValueError(f"x must be (R, V), got {tuple(x.shape)}")
    R, V = x.shape
    out = torch.empty(R, dtype=torch.int64, device=x.device)
    kv800_hip._check(L.lfm3_hip_argmax(_ptr(x), R, V, x.stride(0), _ptr(out), _stream(x)))
    return out


class PackedWeight:
    """A (N, K) bf16 weight in the MFMA operand order of lfm3_hip_linear, padded to Npad = ceil(N / 128) 128 columns
    (zeros); n, k the logical shape. glu: w is a [g | u] (2F, K) gate / up pair (F a multiple of 64) whose rows are
    regrouped as [64 g rows | the matching 64 u rows] so that linear() returns bf16(bf16(silu(g)) u), (R, F)."""

    def __init__(self, w, glu=False):
        L = _lib()
        w = _bf16(w, "w")
        if w.dim() != 2 or w.shape[1] % 64:
            raise ValueError(f"w must be (N, K) with K a multiple of 64, got {tuple(w.shape)}")
        self.n, self.k = w.shape
        self.glu = bool(glu)
        if self.glu:
            if self.n % 128:
                raise ValueError(f"a [g | u] weight needs 2F a multiple of 128, got {self.n}")
            w = w.view(2, self.n // 128, 64, self.k).transpose(0, 1).contiguous().view(self.n, self.k)
        self.npad = (self.n + 127) // 128 * 128
        self.data = torch.empty(self.npad * self.k, dtype=torch.bfloat16, device=w.device)
        kv800_hip._check(L.lfm3_hip_shuffle_weight(_ptr(w), self.n, self.k, self.npad, _ptr(self.data), _stream(w)))


def linear(x, pw, split=1, out=None, work=None):
    """(R, K) bf16 . W^T -> (R, Npad) bf16 (columns >= pw.n are zero), or (R, n / 2) silu(g) u for a glu weight;
    out / work optional preallocated buffers."""
    L = _lib()
    if x.dtype != torch.bfloat16 or x.device.type != "cuda" or x.dim() != 2 or x.shape[1] != pw.k \
            or x.stride(-1) != 1 or x.stride(0) % 8:
        raise ValueError(f"x must be bf16 (R, {pw.k}) with contiguous rows, got {x.dtype} {tuple(x.shape)}")
    if x.device != pw.data.device:
        raise ValueError("x and the weight must be on one device")
    if pw.glu and split != 1:
        raise ValueError("a glu product takes no K split")
    R = x.shape[0]
    width = pw.npad // 2 if pw.glu else pw.npad
    if out is None:
        out = torch.empty(R, width, dtype=torch.bfloat16, device=x.device)
    elif out.dtype != torch.bfloat16 or out.device != x.device or out.dim() != 2 or out.shape[0] != R \
            or out.shape[1] < width or out.stride(-1) != 1 or out.stride(0) % 8:
        raise ValueError(f"out must be bf16 ({R}, >= {width}) with contiguous rows")
    if split > 1:
        need = split * R * pw.npad
        if work is None or work.dtype != torch.float32 or work.device != x.device or work.numel() < need:
            work = torch.empty(need, dtype=torch.float32, device=x.device)
    kv800_hip._check(L.lfm3_hip_linear(_ptr(x), x.stride(0), _ptr(pw.data), R, pw.npad, pw.k, _ptr(out),
                                       out.stride(0), int(split), _ptr(work if split > 1 else None), int(pw.glu),
                                       _stream(x)))
    return out
