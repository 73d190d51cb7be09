"""HIP backend of kv800.decode / quantize_blocks / dequantize_blocks / flush for MI355X (gfx950).

Binds the C ABI of _lib/libkv800_hip.so (include/kv800_hip.h) with ctypes: no torch C++ extension, so the library
is independent of the torch build. Load contract, as the reference's SYCL loader (kv800_sycl.py:68-91): the first
call to ops() loads the library; any failure (no ROCm torch, no GPU, library missing or not loadable) raises
ImportError, which kv800 reports as "backend not available". There is no fallback inside this module: every entry
point either runs the HIP kernels or raises.

Tensors are passed by data_ptr(); launches go on torch's current stream of the tensors' device. Extents of every
pool (from its data_ptr to the end of its storage) are passed to the bounds-checked entry points."""
import ctypes
import math
import os
from collections import OrderedDict

import numpy as np

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "_lib", "libkv800_hip.so")
SOURCE = None        # how the library was obtained (for the backend log line)
_L = None
_ERR = None

BLK, LAG, NSINK, SUB = 256, 128, 4, 51200
LOG2E = 1.4426950408889634


class Paged(ctypes.Structure):
    """kv800_paged_t (include/kv800_hip.h)."""
    _fields_ = [("qpool", ctypes.c_void_p), ("boff", ctypes.c_void_p), ("boff_stride", ctypes.c_int64),
                ("epool", ctypes.c_void_p), ("eoff", ctypes.c_void_p), ("eoff_stride", ctypes.c_int64),
                ("ebs", ctypes.c_int64), ("e_hs", ctypes.c_int64), ("e_ts", ctypes.c_int64), ("e_v", ctypes.c_int64),
                ("sk", ctypes.c_void_p), ("sv", ctypes.c_void_p), ("skoff", ctypes.c_void_p), ("svoff", ctypes.c_void_p),
                ("N", ctypes.c_void_p), ("NQ", ctypes.c_void_p), ("nqmax", ctypes.c_int64), ("win", ctypes.c_int64)]


# exported symbol -> (restype, argtypes); the ABI check in tests compares this list with include/kv800_hip.h
_VP, _I64, _I32, _F32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float
SIGNATURES = {
    "kv800_hip_version": (_I32, []),
    "kv800_hip_last_error": (ctypes.c_char_p, []),
    "kv800_hip_read_probe": (_I32, [_VP, _I64, _VP, _I64, _VP]),
    "kv800_hip_quantize_blocks": (_I32, [_VP, _VP, _I64, _VP, _VP]),
    "kv800_hip_flush": (_I32, [_VP, _VP, _I64, _I64, _I64, _I64, _I64, _VP, _VP, _I64, _I64, _I64, _VP, _VP, _I64, _I64,
                               _VP]),
    "kv800_hip_dequantize_blocks": (_I32, [_VP, _I64, _VP, _VP, _VP]),
    "kv800_hip_rope_table": (_I32, [_VP, _VP, _I64, _VP, _VP]),
    "kv800_hip_decode_quant": (_I32, [_VP, _VP, _VP, _I64, _VP, _VP, _VP, _VP, _VP, _I64, _I64, _I64, _F32, _VP]),
    "kv800_hip_decode_exact": (_I32, [ctypes.POINTER(Paged), _VP, _VP, _VP, _VP, _VP, _VP, _I64, _I64, _F32, _VP]),
    "kv800_hip_decode_merge": (_I32, [_VP, _VP, _VP, _I64, _I64, _VP, _VP]),
    "kv800_hip_plan": (_I32, [_I64, _I64, ctypes.POINTER(_I64), ctypes.POINTER(_I64)]),
    "kv800_hip_decode_workspace": (_I64, [_I64, _I64, _I64]),
    "kv800_hip_plan_balanced": (_I32, [_I64, _I64, ctypes.POINTER(_I64)]),
    "kv800_hip_decode_workspace_balanced": (_I64, [_I64, _I64, _I64]),
    "kv800_hip_decode": (_I32, [ctypes.POINTER(Paged), _VP, _I64, _VP, _VP, _VP, _VP, _VP, _I64, _I64, _VP]),
    "kv800_hip_decode_quant_sized": (_I32, [_VP, _VP, _I64, _VP, _I64, _VP, _VP, _I64, _VP, _VP, _VP, _I64, _I64, _I64,
                                            _F32, _VP]),
    "kv800_hip_decode_exact_sized": (_I32, [ctypes.POINTER(Paged), _VP, _VP, _VP, _I64, _I64, _I64, _VP, _VP, _VP, _I64,
                                            _I64, _F32, _VP]),
    "kv800_hip_decode_sized": (_I32, [ctypes.POINTER(Paged), _VP, _I64, _VP, _VP, _I64, _VP, _I64, _I64, _I64, _VP, _VP,
                                      _I64, _I64, _VP]),
    "kv800_hip_write_exact": (_I32, [_VP, _I64, _I64, _I64, _I64, _I64, _VP, _VP, _VP, _I64, _VP, _VP, _VP, _VP, _VP,
                                     _VP]),
    "kv800_hip_decode_tables": (_I32, [_VP, _I64, _I64, _I64, _VP, _I64, _I64, _VP, _VP, _VP]),
    "kv800_hip_step_tables": (_I32, [_VP, _I64, _I64, _I64, _VP, _I64, _I64, _I64, _VP, _VP, _VP, _VP, _VP, _VP, _I64,
                                     _I64, _VP]),
    "kv800_hip_page_offsets": (_I32, [_VP, _I64, _I64, _I64, _I64, _I64, _VP, _VP]),
    "kv800_hip_step_meta": (_I32, [_VP, _I64, _I64, _VP, _I64, _I64, _VP, _VP, _VP, _VP]),
    "kv800_hip_history": (_I32, [ctypes.POINTER(Paged), _I64, _I64, _VP, _VP, _I64, _I64, _I64, _VP, _VP, _VP, _VP]),
    "kv800_hip_rope_rows": (_I32, [_VP, _VP, _I64, _VP, _VP, _I64, _VP, _VP]),
    "kv800_hip_prefill": (_I32, [_VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _I64, _I64, _I64, _I64, _VP, _VP]),
    "kv800_hip_prefill_split": (_I32, [_VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _I64, _I64, _I64, _I64, _I64, _I64,
                                        _VP, _I64, _VP, _VP]),
    "kv800_hip_fake_quant_k": (_I32, [_VP, _I64, _I64, _VP, _VP]),
    "kv800_hip_flush_latency": (_I32, [_VP, _VP, _I64, _I64, _I64, _I64, _I64, _VP, _VP, _I64, _I64, _I64, _VP, _VP,
                                       _I64, _I64, _VP]),
    "kv800_hip_fake_quant_v": (_I32, [_VP, _I64, _VP, _VP]),
    "kv800_hip_decode_noalloc": (_I32, [ctypes.POINTER(Paged), _VP, _I64, _VP, _VP, _I64, _VP, _I64, _I64, _I64, _VP,
                                        _I64, _VP]),
}


def load_library(path=LIB):
    """ctypes handle of the library with every signature set (no GPU needed; used by the ABI tests too)."""
    if not os.path.isfile(path):
        raise ImportError(f"{path} is not built (run __graft_entry__.build() or python lfm3-kv800_amd/build.py)")
    try:
        L = ctypes.CDLL(path)
    except OSError as e:
        raise ImportError(f"loading {path} failed: {e}") from e
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(L, name)
        fn.restype, fn.argtypes = res, args
    return L


def ops():
    """The loaded library; raises ImportError when the HIP backend cannot run in this process."""
    global _L, _ERR, SOURCE
    if _L is not None:
        return _L
    if _ERR is not None:
        raise ImportError(_ERR)
    if getattr(torch.version, "hip", None) is None:
        _ERR = "this torch is not a ROCm build"
        raise ImportError(_ERR)
    if not torch.cuda.is_available():
        _ERR = "torch sees no ROCm GPU"
        raise ImportError(_ERR)
    try:
        _L = load_library()
    except ImportError as e:
        _ERR = str(e)
        raise
    SOURCE = f"{LIB} (ABI {_L.kv800_hip_version()})"
    return _L


def _check(rc):
    if rc != 0:
        raise RuntimeError(f"kv800 HIP: {ops().kv800_hip_last_error().decode(errors='replace')} (status {rc})")


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _stream(dev):
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def _extent(t):
    """Elements from t's first element to the end of its storage (what the kernels may address from data_ptr)."""
    return t.untyped_storage().nbytes() // t.element_size() - t.storage_offset()


def host_to_device(x, dtype, dev):
    """A host sequence or array as a tensor on dev: through pinned memory and an asynchronous copy on the current
    stream on a GPU (a pageable copy waits for the stream's queued work, stalling the host behind the last launch)."""
    t = x if torch.is_tensor(x) else torch.as_tensor(np.asarray(x), dtype=dtype)
    t = t.to(dtype)
    if t.device == dev:
        return t
    if dev.type == "cuda":
        return t.pin_memory().to(dev, non_blocking=True)
    return t.to(dev)


def _need(t, name, dtype, dev):
    if t.device != dev:
        raise ValueError(f"{name} is on {t.device}, expected {dev}")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")


# ---------------------------------------------------------------- codec
def quantize_blocks(k, v):
    """(M, 256, 4, 128) bf16 K (pre-RoPE) and V -> (M, 51200) uint8, bit-identical to kv800.py:56-76 on CPU torch."""
    L = ops()
    dev = k.device
    _need(k, "k", torch.bfloat16, dev); _need(v, "v", torch.bfloat16, dev)
    if k.shape != v.shape or k.dim() != 4 or tuple(k.shape[1:]) != (BLK, 4, 128):
        raise ValueError(f"k, v must be (M, 256, 4, 128), got {tuple(k.shape)} / {tuple(v.shape)}")
    k, v = k.contiguous(), v.contiguous()
    out = torch.empty(k.shape[0], SUB, dtype=torch.uint8, device=dev)
    _check(L.kv800_hip_quantize_blocks(_ptr(k), _ptr(v), k.shape[0], _ptr(out), _stream(dev)))
    return out


def dequantize_blocks(sb):
    """(M, 51200) uint8 -> K (M, 256, 4, 128) bf16, V (M, 256, 4, 128) fp32 (kv800.py:79-92)."""
    L = ops()
    dev = sb.device
    _need(sb, "sb", torch.uint8, dev)
    if sb.dim() != 2 or sb.shape[1] != SUB:
        raise ValueError(f"sb must be (M, 51200), got {tuple(sb.shape)}")
    sb = sb.contiguous()
    M = sb.shape[0]
    k = torch.empty(M, BLK, 4, 128, dtype=torch.bfloat16, device=dev)
    v = torch.empty(M, BLK, 4, 128, dtype=torch.float32, device=dev)
    _check(L.kv800_hip_dequantize_blocks(_ptr(sb), M, _ptr(k), _ptr(v), _stream(dev)))
    return k, v


def flush(epool, eoff, ebs, e_hs, e_ts, e_v, qpool, qbt, bsq, qs0, nq_prev, nq_new, max_new, latency=False):
    """Quantize sub-blocks j in [nq_prev[r], nq_new[r]) of every row r from the exact pages into the quant pool
    (one launch; see kv800_hip_flush). epool bf16 (any shape, element offsets), eoff (R, pages) int64 element
    offsets, qpool uint8 (byte offsets), qbt (R, >= 1) int64 quant block table, nq_prev / nq_new (R,) int32.
    latency=True: kv800_hip_flush_latency (same bytes; for steps that flush few sub-blocks, e.g. decode)."""
    L = ops()
    dev = epool.device
    _need(epool, "epool", torch.bfloat16, dev); _need(qpool, "qpool", torch.uint8, dev)
    _need(eoff, "eoff", torch.int64, dev); _need(qbt, "qbt", torch.int64, dev)
    _need(nq_prev, "nq_prev", torch.int32, dev); _need(nq_new, "nq_new", torch.int32, dev)
    if eoff.stride(-1) != 1 or qbt.stride(-1) != 1:
        raise ValueError("eoff and qbt rows must be contiguous")
    R = nq_prev.shape[0]
    nq_prev, nq_new = nq_prev.contiguous(), nq_new.contiguous()
    fn = L.kv800_hip_flush_latency if latency else L.kv800_hip_flush
    _check(fn(_ptr(epool), _ptr(eoff), eoff.stride(0), int(ebs), int(e_hs), int(e_ts), int(e_v), _ptr(qpool), _ptr(qbt),
              qbt.stride(0), int(bsq), int(qs0), _ptr(nq_prev), _ptr(nq_new), R, int(max_new), _stream(dev)))


def write_exact(ev, slot, k, v, pos=None, sk=None, sv=None, skoff=None, svoff=None):
    """Write the step's rows k, v (R, 4, 128) bf16 (pre-RoPE K, unrotated V) into the exact cache ev ([pages, 4, ebs,
    256] bf16 view, K | V) at slot (R,) int64 (< 0: skipped); with sink buffers (window layers) rows at pos < 4 also go
    to sk + skoff[r] / sv + svoff[r] (bf16 element offsets). One launch (vllm_attn.py:263-291)."""
    L = ops()
    dev = ev.device
    _need(ev, "ev", torch.bfloat16, dev); _need(slot, "slot", torch.int64, dev)
    k, v = k.contiguous(), v.contiguous()
    _need(k, "k", torch.bfloat16, dev); _need(v, "v", torch.bfloat16, dev)
    R = slot.shape[0]
    if k.shape != (R, 4, 128) or v.shape != (R, 4, 128):
        raise ValueError(f"k, v must be ({R}, 4, 128), got {tuple(k.shape)}, {tuple(v.shape)}")
    sinks = sk is not None
    if sinks:
        _need(sk, "sk", torch.bfloat16, dev); _need(sv, "sv", torch.bfloat16, dev)
        _need(pos, "pos", torch.int64, dev); _need(skoff, "skoff", torch.int64, dev); _need(svoff, "svoff", torch.int64, dev)
    _check(L.kv800_hip_write_exact(_ptr(ev), ev.stride(0), ev.stride(1), ev.stride(2), 128, ev.shape[2], _ptr(slot),
                                   _ptr(k), _ptr(v), R, _ptr(pos) if sinks else None, _ptr(sk) if sinks else None,
                                   _ptr(sv) if sinks else None, _ptr(skoff) if sinks else None,
                                   _ptr(svoff) if sinks else None, _stream(dev)))


def decode_tables(qbt, bsq, qs0, N, nqmax):
    """Quantized layer decode tables (vllm_attn.py:332-340): NQ (R,) int32 and boff (R, max(nqmax, 1)) int64 byte
    offsets of each row's first nqmax sub-blocks through the (R, blocks) int32 quant block table qbt."""
    L = ops()
    dev = N.device
    _need(qbt, "qbt", torch.int32, dev); _need(N, "N", torch.int32, dev)
    if qbt.stride(-1) != 1:
        raise ValueError("qbt rows must be contiguous")
    R = N.shape[0]
    boff = torch.empty(R, max(int(nqmax), 1), dtype=torch.int64, device=dev)
    NQ = torch.empty(R, dtype=torch.int32, device=dev)
    _check(L.kv800_hip_decode_tables(_ptr(qbt), qbt.stride(0), int(bsq), int(qs0), _ptr(N.contiguous()), R, int(nqmax),
                                     _ptr(boff), _ptr(NQ), _stream(dev)))
    return boff, NQ


def step_tables(qbt, bsq, qs0, N, nqmax, nnew=1, aux_scale=None, aux_add=0):
    """All per-step tables of the quant KV group in one launch (kv800_hip_step_tables): (boff, NQ, NP, qbt64, aux) with
    NP = sub-blocks flushed before the step's new tokens (nnew: an int for every row, or an (R,) int32 device tensor of
    per-row counts, a mixed step's query lengths), qbt64 = qbt as int64 and, if aux_scale is given,
    aux = qbt[:, 0] * aux_scale + aux_add (else None)."""
    L = ops()
    dev = N.device
    _need(qbt, "qbt", torch.int32, dev); _need(N, "N", torch.int32, dev)
    rows = None
    if torch.is_tensor(nnew):
        _need(nnew, "nnew", torch.int32, dev)
        if nnew.shape != (N.shape[0],):
            raise ValueError("per-row nnew must be (R,)")
        rows, nnew = nnew.contiguous(), 0
    if qbt.stride(-1) != 1:
        raise ValueError("qbt rows must be contiguous")
    R = N.shape[0]
    boff = torch.empty(R, max(int(nqmax), 1), dtype=torch.int64, device=dev)
    NQ = torch.empty(R, dtype=torch.int32, device=dev)
    NP = torch.empty(R, dtype=torch.int32, device=dev)
    qbt64 = torch.empty(R, qbt.shape[1], dtype=torch.int64, device=dev)
    aux = torch.empty(R, dtype=torch.int64, device=dev) if aux_scale is not None else None
    _check(L.kv800_hip_step_tables(_ptr(qbt), qbt.stride(0), int(bsq), int(qs0), _ptr(N.contiguous()), R, int(nqmax),
                                   int(nnew), _ptr(rows) if rows is not None else None, _ptr(boff), _ptr(NQ),
                                   _ptr(NP), _ptr(qbt64), _ptr(aux),
                                   int(aux_scale or 0), int(aux_add), _stream(dev)))
    return boff, NQ, NP, qbt64, aux


def step_meta(bt, lens, ebs):
    """(slot int64, pos int64, lens int32) of a decode step from the (R, pages) int32 block table and the (R,) int64
    device lengths including the new token (kv800_hip_step_meta)."""
    L = ops()
    dev = bt.device
    _need(bt, "bt", torch.int32, dev)
    _need(lens, "lens", torch.int64, dev)
    if bt.dim() != 2 or bt.stride(-1) != 1 or lens.dim() != 1 or lens.shape[0] != bt.shape[0]:
        raise ValueError("bt must be (R, pages) with contiguous rows and lens (R,)")
    R = bt.shape[0]
    slot = torch.empty(R, dtype=torch.int64, device=dev)
    pos = torch.empty(R, dtype=torch.int64, device=dev)
    l32 = torch.empty(R, dtype=torch.int32, device=dev)
    _check(L.kv800_hip_step_meta(_ptr(bt), bt.stride(0), bt.shape[1], _ptr(lens.contiguous()), R, int(ebs), _ptr(slot),
                                 _ptr(pos), _ptr(l32), _stream(dev)))
    return slot, pos, l32


def page_offsets(bt, scale, add=0):
    """(R, pages) int64 bt * scale + add of an (R, pages) int32 block table (kv800_hip_page_offsets)."""
    L = ops()
    dev = bt.device
    _need(bt, "bt", torch.int32, dev)
    if bt.dim() != 2 or bt.stride(-1) != 1:
        raise ValueError("bt must be (R, pages) with contiguous rows")
    out = torch.empty(bt.shape[0], bt.shape[1], dtype=torch.int64, device=dev)
    _check(L.kv800_hip_page_offsets(_ptr(bt), bt.stride(0), bt.shape[0], bt.shape[1], int(scale), int(add), _ptr(out),
                                    _stream(dev)))
    return out


def history(P, lens, cos_t=None, sin_t=None, out=None, offs=None):
    """Prefill over compressed history (kv800_hip_history, vllm_attn.py:351-380): rows b < len(lens) of the paged cache
    P, positions [0, lens[b]), as contiguous bf16 K (rotated with the (P, 32) cos_t / sin_t tables, or unrotated when
    they are None) and V, (sum(lens), 4, 128) each, row b's positions starting at offs[b]. Positions below
    256 * P.NQ[b] are dequantized from their sub-blocks, the others read from the exact pages. With out = (K, V)
    ((S, 4, 128) bf16 each) and offs (R,) the rows are written there instead, row b's positions at rows offs[b] + p
    (ranges that must fit in S); the other rows of out are left as they are. Returns (K, V, offs)."""
    L = ops()
    dev = P.epool.device
    lens = [int(x) for x in (lens.tolist() if torch.is_tensor(lens) else lens)]
    R = len(lens)
    if any(x < 0 for x in lens):
        raise ValueError("lens must be >= 0")
    if out is None:
        S = sum(lens)
        K = torch.empty(S, 4, 128, dtype=torch.bfloat16, device=dev)
        V = torch.empty_like(K)
        offs = [0] * R
        for b in range(1, R):
            offs[b] = offs[b - 1] + lens[b - 1]
    else:
        if offs is None:
            raise ValueError("history: out needs offs, each row's first output row")
        K, V = out
        _need(K, "K", torch.bfloat16, dev); _need(V, "V", torch.bfloat16, dev)
        if K.shape != V.shape or K.dim() != 3 or K.shape[1:] != (4, 128) or not (K.is_contiguous() and
                                                                               V.is_contiguous()):
            raise ValueError("out must be two contiguous (S, 4, 128) bf16 tensors")
        offs = [int(x) for x in offs]
        if len(offs) != R or any(o < 0 or o + n > K.shape[0] for o, n in zip(offs, lens)):
            raise ValueError("offs must give each row's range inside out")
    if R == 0 or sum(lens) == 0:
        return K, V, offs
    rot = cos_t is not None
    if rot:
        _need(cos_t, "cos_t", torch.bfloat16, dev); _need(sin_t, "sin_t", torch.bfloat16, dev)
        if cos_t.shape != sin_t.shape or cos_t.dim() != 2 or cos_t.shape[1] != 32:
            raise ValueError("cos_t / sin_t must be (P, 32)")
        cos_t, sin_t = cos_t.contiguous(), sin_t.contiguous()
    _need(P.epool, "epool", torch.bfloat16, dev); _need(P.eoff, "eoff", torch.int64, dev)
    _need(P.NQ, "NQ", torch.int32, dev)
    if P.eoff.stride(-1) != 1 or P.eoff.shape[0] < R or P.NQ.shape[0] < R:
        raise ValueError("eoff / NQ must cover the rows with contiguous eoff rows")
    s = Paged()
    s.epool, s.eoff, s.eoff_stride = P.epool.data_ptr(), P.eoff.data_ptr(), P.eoff.stride(0)
    s.ebs, s.e_hs, s.e_ts, s.e_v = int(P.ebs), int(P.e_hs), int(P.e_ts), int(P.e_v)
    N = host_to_device(lens, torch.int32, dev)   # the output extents, from the host lengths
    s.N, s.NQ = N.data_ptr(), P.NQ.data_ptr()
    qbytes = 0
    if P.qpool is not None and P.boff is not None and P.boff.numel():
        _need(P.qpool, "qpool", torch.uint8, dev); _need(P.boff, "boff", torch.int64, dev)
        if P.boff.stride(-1) != 1 or P.boff.shape[0] < R:
            raise ValueError("boff must cover the rows with contiguous rows")
        s.qpool, s.boff, s.boff_stride = P.qpool.data_ptr(), P.boff.data_ptr(), P.boff.stride(0)
        qbytes = _extent(P.qpool)
    offt = host_to_device(offs, torch.int64, dev)
    _check(L.kv800_hip_history(ctypes.byref(s), R, max(lens), _ptr(cos_t) if rot else None,
                               _ptr(sin_t) if rot else None, cos_t.shape[0] if rot else 0, qbytes, _extent(P.epool),
                               _ptr(offt), _ptr(K), _ptr(V), _stream(dev)))
    return K, V, offs



def rope_rows(k, pos, cos_t, sin_t):
    """Keys k (S, 4, 128) bf16 rotated at positions pos (S,) int64 with the (P, 32) bf16 tables (kv800_hip_rope_rows,
    bit-identical to vllm_attn.py:160-163's _rope over its 128-wide tables). Returns a new (S, 4, 128) bf16 tensor."""
    L = ops()
    dev = k.device
    k = k.contiguous()
    _need(k, "k", torch.bfloat16, dev); _need(pos, "pos", torch.int64, dev)
    _need(cos_t, "cos_t", torch.bfloat16, dev); _need(sin_t, "sin_t", torch.bfloat16, dev)
    if k.dim() != 3 or k.shape[1:] != (4, 128) or pos.shape != (k.shape[0],):
        raise ValueError(f"k must be (S, 4, 128) with pos (S,), got {tuple(k.shape)}, {tuple(pos.shape)}")
    if cos_t.shape != sin_t.shape or cos_t.dim() != 2 or cos_t.shape[1] != 32:
        raise ValueError("cos_t / sin_t must be (P, 32)")
    out = torch.empty_like(k)
    _check(L.kv800_hip_rope_rows(_ptr(k), _ptr(pos.contiguous()), k.shape[0], _ptr(cos_t.contiguous()),
                                 _ptr(sin_t.contiguous()), cos_t.shape[0], _ptr(out), _stream(dev)))
    return out


PREFILL_SPLIT_BELOW = 256   # workgroups (query tiles x 4 KV heads) under which the key range is split
PREFILL_SPLIT_TARGET = 512  # workgroups a split grid aims at (two per CU)


def prefill_splits(tiles, max_key_tiles):
    """Key splits of one prefill launch: 1 when its tiles x 4 workgroups nearly fill the GPU, else enough for about
    PREFILL_SPLIT_TARGET workgroups, with at least two 64-key tiles per split and at most 64 splits."""
    w = 4 * tiles
    if w >= PREFILL_SPLIT_BELOW or max_key_tiles < 4:
        return 1
    return int(max(1, min(64, -(-PREFILL_SPLIT_TARGET // w), max_key_tiles // 2)))


def prefill(q, qsl, qpos0, K, V, kp, ksl, window=0, nsink=0, splits=None):
    """Prefill attention of ragged rows (kv800_hip_prefill_split): row r's queries q[qsl[r]:qsl[r+1]] ((T, 16, 128)
    bf16) at positions qpos0[r], qpos0[r] + 1, ... over keys / values K, V[ksl[r]:ksl[r+1]] ((S, 4, 128) bf16) at
    positions kp (S,) (ascending within a row; None: key j of a row at position j). qsl / ksl / qpos0: host sequences
    (R + 1, R + 1, R). Mask: kp <= query
    position, and with window > 0 also kp > position - window or kp < nsink. splits: key splits per (query tile, KV
    head) (default prefill_splits: few query tiles over long rows are split and merged). Returns (T, 16, 128) bf16."""
    L = ops()
    dev = q.device
    q, K, V = q.contiguous(), K.contiguous(), V.contiguous()
    _need(q, "q", torch.bfloat16, dev); _need(K, "K", torch.bfloat16, dev); _need(V, "V", torch.bfloat16, dev)
    qsl, ksl, qpos0 = [int(x) for x in qsl], [int(x) for x in ksl], [int(x) for x in qpos0]
    R = len(qpos0)
    if len(qsl) != R + 1 or len(ksl) != R + 1:
        raise ValueError("qsl and ksl need R + 1 entries")
    if q.dim() != 3 or q.shape[1:] != (16, 128) or qsl[0] != 0 or qsl[-1] != q.shape[0]:
        raise ValueError(f"q must be (qsl[-1], 16, 128), got {tuple(q.shape)}")
    if K.shape != V.shape or K.dim() != 3 or K.shape[1:] != (4, 128) or ksl[0] != 0 or ksl[-1] != K.shape[0]:
        raise ValueError(f"K / V must be (ksl[-1], 4, 128), got {tuple(K.shape)}, {tuple(V.shape)}")
    if any(b < a for a, b in zip(qsl, qsl[1:])) or any(b < a for a, b in zip(ksl, ksl[1:])):
        raise ValueError("qsl / ksl must be non-decreasing")
    if kp is not None:
        kp = host_to_device(kp, torch.int32, dev).contiguous()
        if kp.shape != (K.shape[0],):
            raise ValueError("kp must be (S,)")
    out = torch.empty(q.shape, dtype=torch.bfloat16, device=dev)
    tiles = [0]
    for a, b in zip(qsl, qsl[1:]):
        tiles.append(tiles[-1] + (b - a + 31) // 32)   # 32-query tiles, one workgroup per tile and KV head
    if R == 0 or tiles[-1] == 0:
        return out
    if splits is None:
        splits = prefill_splits(tiles[-1], max(-(-(b - a) // 64) for a, b in zip(ksl, ksl[1:])))
    splits = int(splits)
    T = qsl[-1]
    part = torch.empty(T * 16 * splits * 132 if splits > 1 else 0, dtype=torch.float32, device=dev)
    meta = host_to_device(qsl + ksl + qpos0 + tiles, torch.int64, dev)
    m_qsl, m_ksl = meta[:R + 1], meta[R + 1:2 * R + 2]
    m_pos, m_tiles = meta[2 * R + 2:3 * R + 2], meta[3 * R + 2:]
    _check(L.kv800_hip_prefill_split(_ptr(q), _ptr(m_qsl), _ptr(m_pos), _ptr(K), _ptr(V), _ptr(kp), _ptr(m_ksl),
                                     _ptr(m_tiles), R, tiles[-1], T, int(window), int(nsink), splits,
                                     _ptr(part) if splits > 1 else None, part.numel(), _ptr(out), _stream(dev)))
    return out


def read_probe(buf, out, groups):
    """Streaming read of the whole of buf (a contiguous device tensor, a multiple of 16 bytes) by kv800_hip_read_probe
    with `groups` workgroups; out: an int32 device tensor of at least `groups` entries (one xor word each)."""
    L = ops()
    if not (buf.is_cuda and out.is_cuda and buf.is_contiguous() and out.numel() >= groups):
        raise ValueError("read_probe: contiguous device tensors, out with at least `groups` entries")
    _check(L.kv800_hip_read_probe(_ptr(buf), buf.numel() * buf.element_size(), _ptr(out), int(groups),
                                  _stream(buf.device)))


def fake_quant_k(x):
    """x (..., 256, C) float32 on the GPU -> float32 dequantized 800h K per (256-token group, channel)
    (kv800_hip_fake_quant_k; train.py:82-89)."""
    L = ops()
    if x.device.type != "cuda":
        raise ValueError(f"x must be on a ROCm device, got {x.device}")
    _need(x, "x", torch.float32, x.device)
    if x.dim() < 2 or x.shape[-2] != 256:
        raise ValueError(f"x must be (..., 256, C), got {tuple(x.shape)}")
    x = x.contiguous()
    out = torch.empty_like(x)
    C = x.shape[-1]
    G = x.numel() // (256 * C) if C else 0
    for g0 in range(0, G, 65535):                       # grid y holds at most 65535 groups
        g1 = min(G, g0 + 65535)
        _check(L.kv800_hip_fake_quant_k(ctypes.c_void_p(x.data_ptr() + g0 * 256 * C * 4), g1 - g0, C,
                                        ctypes.c_void_p(out.data_ptr() + g0 * 256 * C * 4), _stream(x.device)))
    return out


def fake_quant_v(v):
    """v (..., 4, 128) float32 on the GPU -> float32: per token the V of a quantize -> dequantize round trip
    (kv800_hip_fake_quant_v; train.py:92-100)."""
    L = ops()
    if v.device.type != "cuda":
        raise ValueError(f"v must be on a ROCm device, got {v.device}")
    _need(v, "v", torch.float32, v.device)
    if v.dim() < 2 or tuple(v.shape[-2:]) != (4, 128):
        raise ValueError(f"v must be (..., 4, 128), got {tuple(v.shape)}")
    v = v.contiguous()
    out = torch.empty_like(v)
    _check(L.kv800_hip_fake_quant_v(_ptr(v), v.numel() // 512, _ptr(out), _stream(v.device)))
    return out


def combine(MO, LO, AO, ns):
    """LSE merge of (B, ns+1, 16[, 128]) partials -> (B, 16, 128) bf16 (kv800.py:231-236)."""
    L = ops()
    dev = MO.device
    for t, nm in ((MO, "MO"), (LO, "LO"), (AO, "AO")):
        _need(t, nm, torch.float32, dev)
    MO, LO, AO = MO.contiguous(), LO.contiguous(), AO.contiguous()
    out = torch.empty(MO.shape[0], 16, 128, dtype=torch.bfloat16, device=dev)
    _check(L.kv800_hip_decode_merge(_ptr(MO), _ptr(LO), _ptr(AO), MO.shape[0], int(ns), _ptr(out), _stream(dev)))
    return out


# ---------------------------------------------------------------- decode
_PAIRS = OrderedDict()     # (device, cos ptr, sin ptr, rows) -> (cos_t, sin_t, versions, pair table)


def rope_pairs(cos_t, sin_t):
    """Packed bf16 (cos, sin) pair table of every row of the bf16 tables (kv800_hip_rope_table), cached per table
    tensors. The entry holds the two tables themselves, so their storage cannot be freed and reused by other tensors
    while it is cached; it is rebuilt when either tensor is modified in place (version counter) or replaced."""
    key = (str(cos_t.device), cos_t.data_ptr(), sin_t.data_ptr(), cos_t.shape[0])
    ent = _PAIRS.get(key)
    ver = (cos_t._version, sin_t._version)
    if ent is not None and ent[0] is cos_t and ent[1] is sin_t and ent[2] == ver:
        _PAIRS.move_to_end(key)
        return ent[3]
    L = ops()
    P = cos_t.shape[0]
    t = torch.empty(P, 32, dtype=torch.int32, device=cos_t.device)
    _check(L.kv800_hip_rope_table(_ptr(cos_t), _ptr(sin_t), P, _ptr(t), _stream(cos_t.device)))
    _PAIRS[key] = (cos_t, sin_t, ver, t)
    _PAIRS.move_to_end(key)
    while len(_PAIRS) > 8:
        _PAIRS.popitem(last=False)
    return t


def plan(B, nqmax, spb=None, target=None):
    """(ns, spb) of a decode call: explicit spb; or the reference's target rule (kv800.py:366-367); or the library
    plan (about two workgroups per CU)."""
    if not nqmax:
        return 0, 1
    if spb is None and target:
        spb = max(1, math.ceil(nqmax * B * 4 / target))
    if spb is not None:
        spb = max(1, int(spb))
        return math.ceil(nqmax / spb), spb
    ns, sp = ctypes.c_int64(), ctypes.c_int64()
    _check(ops().kv800_hip_plan(B, nqmax, ctypes.byref(ns), ctypes.byref(sp)))
    return ns.value, sp.value


def paged_struct(P, B):
    """kv800_paged_t of a kv800.Paged, plus the extents of its pools."""
    dev = P.epool.device
    _need(P.epool, "epool", torch.bfloat16, dev); _need(P.eoff, "eoff", torch.int64, dev)
    _need(P.N, "N", torch.int32, dev); _need(P.NQ, "NQ", torch.int32, dev)
    if P.eoff.stride(-1) != 1:
        raise ValueError("eoff rows must be contiguous")
    s = Paged()
    nqmax = 0 if P.win else int(P.nqmax or 0)
    if nqmax:
        _need(P.qpool, "qpool", torch.uint8, dev); _need(P.boff, "boff", torch.int64, dev)
        if P.boff.stride(-1) != 1:
            raise ValueError("boff rows must be contiguous")
        s.qpool, s.boff, s.boff_stride = P.qpool.data_ptr(), P.boff.data_ptr(), P.boff.stride(0)
        qbytes = _extent(P.qpool)
    else:
        qbytes = 0
    s.epool, s.eoff, s.eoff_stride = P.epool.data_ptr(), P.eoff.data_ptr(), P.eoff.stride(0)
    s.ebs, s.e_hs, s.e_ts, s.e_v = int(P.ebs), int(P.e_hs), int(P.e_ts), int(P.e_v)
    sink_elems = 0
    if P.win and P.sk is not None:
        _need(P.sk, "sk", torch.bfloat16, dev); _need(P.sv, "sv", torch.bfloat16, dev)
        _need(P.skoff, "skoff", torch.int64, dev); _need(P.svoff, "svoff", torch.int64, dev)
        s.sk, s.sv, s.skoff, s.svoff = P.sk.data_ptr(), P.sv.data_ptr(), P.skoff.data_ptr(), P.svoff.data_ptr()
        sink_elems = min(_extent(P.sk), _extent(P.sv))
    s.N, s.NQ = P.N.data_ptr(), P.NQ.data_ptr()
    s.nqmax, s.win = nqmax, int(P.win or 0)
    if P.N.shape[0] < B or P.NQ.shape[0] < B:
        raise ValueError("N / NQ have fewer rows than q")
    return s, qbytes, _extent(P.epool), sink_elems


def plan_balanced(B, nqmax):
    """Workgroup count of the balanced schedule (kv800_hip_plan_balanced)."""
    g = ctypes.c_int64()
    _check(ops().kv800_hip_plan_balanced(B, nqmax, ctypes.byref(g)))
    return g.value


def decode(P, q, cos_t, sin_t, spb=None, target=None, groups=None):
    """q (B, 16, 128) bf16 post-RoPE -> (B, 16, 128) bf16: the fused HIP decode of one layer (kv800_hip_decode).
    spb / target (the reference's split overrides, kv800.py:366-367) select the fixed (row, split) grid; otherwise the
    balanced schedule runs, with `groups` workgroups (default: the library's plan)."""
    L = ops()
    dev = q.device
    _need(q, "q", torch.bfloat16, dev); _need(cos_t, "cos_t", torch.bfloat16, dev); _need(sin_t, "sin_t", torch.bfloat16, dev)
    B = q.shape[0]
    if q.dim() != 3 or tuple(q.shape[1:]) != (16, 128):
        raise ValueError(f"q must be (B, 16, 128), got {tuple(q.shape)}")
    if cos_t.shape != sin_t.shape or cos_t.dim() != 2 or cos_t.shape[1] != 32:
        raise ValueError("cos_t / sin_t must be (P, 32)")
    q, cos_t, sin_t = q.contiguous(), cos_t.contiguous(), sin_t.contiguous()
    s, qbytes, eelems, selems = paged_struct(P, B)
    out = torch.empty(B, 16, 128, dtype=torch.bfloat16, device=dev)
    if B == 0:
        return out
    cs2 = rope_pairs(cos_t, sin_t) if s.nqmax else None
    if not s.nqmax:
        arg, wsb = 0, int(L.kv800_hip_decode_workspace(B, 0, 0))
    elif spb is None and not target:
        g = int(groups) if groups else plan_balanced(B, s.nqmax)
        if g < 1:
            raise ValueError("groups must be >= 1")
        arg, wsb = -g, int(L.kv800_hip_decode_workspace_balanced(B, g, 0))
    else:
        ns, arg = plan(B, s.nqmax, spb, target)
        wsb = int(L.kv800_hip_decode_workspace(B, ns, 0))
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    _check(L.kv800_hip_decode_sized(ctypes.byref(s), _ptr(q), B, _ptr(cos_t), _ptr(sin_t), cos_t.shape[0], _ptr(cs2),
                                    qbytes, eelems, selems, _ptr(out), _ptr(ws), wsb, arg, _stream(dev)))
    return out


def decode_parts(P, q, cos_t, sin_t, spb=None, target=None):
    """The three stages separately (decode_quant, decode_exact, decode_merge) with the partials returned:
    (out, MO, LO, AO, ns). Same result as decode(); used by tests of each stage."""
    L = ops()
    dev = q.device
    q, cos_t, sin_t = q.contiguous(), cos_t.contiguous(), sin_t.contiguous()
    B = q.shape[0]
    s, qbytes, eelems, selems = paged_struct(P, B)
    ns, sp = plan(B, s.nqmax, spb, target)
    MO = torch.empty(B, ns + 1, 16, dtype=torch.float32, device=dev)
    LO = torch.empty_like(MO)
    AO = torch.empty(B, ns + 1, 16, 128, dtype=torch.float32, device=dev)
    scale = 128 ** -0.5 * LOG2E
    st = _stream(dev)
    if ns:
        cs2 = rope_pairs(cos_t, sin_t)
        _check(L.kv800_hip_decode_quant_sized(_ptr(q), s.qpool, qbytes, s.boff, s.boff_stride, _ptr(P.NQ), _ptr(cs2),
                                              cos_t.shape[0], _ptr(MO), _ptr(LO), _ptr(AO), B, ns, sp, scale, st))
    _check(L.kv800_hip_decode_exact_sized(ctypes.byref(s), _ptr(q), _ptr(cos_t), _ptr(sin_t), cos_t.shape[0], eelems,
                                          selems, _ptr(MO), _ptr(LO), _ptr(AO), B, ns, scale, st))
    out = torch.empty(B, 16, 128, dtype=torch.bfloat16, device=dev)
    _check(L.kv800_hip_decode_merge(_ptr(MO), _ptr(LO), _ptr(AO), B, ns, _ptr(out), st))
    return out, MO, LO, AO, ns
