"""Paged 800h KV cache API with the MI355X `hip` backend: the reference's lfm3_kv800/kv800.py interface (layout
constants, hadamard, flat, quantize_blocks, dequantize_blocks, combine, Paged, decode with set_backend / get_backend
and LFM3KV_BACKEND, PagedStore), running on the gfx950 kernels of libkv800_hip.so.

Layout (kv800.py:3-15): quantized layer state = 256-token sub-blocks of 51,200 bytes addressed by BOFF[b, j] (bytes
from the quant pool's base):
  [0, 32768)      kc   [256, 4, 32]  planar 2-bit K (byte j = dims j, j+32, j+64, j+96 at bits 0-1/2-3/4-5/6-7)
  [32768, 49152)  vb   [256, 4, 16]  planar 1-bit V after the per-head Hadamard (byte j = dims j + 16i at bit i)
  [49152, 49664)  vlo  [256, 2] fp8  per (token, 2-head group)
  [49664, 50176)  vsc  [256, 2] fp8
  [50176, 50688)  klo  [4, 128] fp8  per (head, channel) over the 256 tokens, pre-RoPE
  [50688, 51200)  ksc  [4, 128] fp8
Exact tokens (pre-RoPE K, unrotated V, bf16) live in pages of EBS tokens at EOFF[b, p // EBS] (elements); K of
(head h, slot t) at + h*e_hs + t*e_ts, V at + e_v. Sinks of window layers: [4, 4, 128] blocks at SKOFF / SVOFF.
Sub-block j of a full layer is quantized once n >= 256 j + 384; window layers = 4 sinks + the last 256 tokens.

Backends: this package provides one, "hip" (ROCm torch, device type "cuda", gfx950). The reference's names "sycl",
"triton" and "torch" are recognised by LFM3KV_BACKEND / set_backend but are not part of this build: forcing one
raises, as forcing an unavailable backend does in the reference (kv800.py:306-317). auto on a device the hip backend
cannot serve raises too -- the product path never falls back to a CPU implementation."""
import math
import os

import torch

from . import get_logger

BLK, LAG, NSINK, WIN = 256, 128, 4, 256
SUB = 51200
KC_O, VB_O, VLO_O, VSC_O, KLO_O, KSC_O = 0, 32768, 49152, 49664, 50176, 50688
F8 = torch.float8_e4m3fn
LOG2E = 1.4426950408889634
BACKENDS = ("hip",)
REFERENCE_BACKENDS = ("sycl", "triton", "torch")     # accepted names that this build does not provide
_log = get_logger()


def hadamard(n=128, device=None):
    """Normalized Sylvester Hadamard (n x n, fp32): entries +-fp32(1/sqrt(n)), as kv800.py:43-46. The HIP kernels
    apply this matrix implicitly (sequential fma chain in the quantizer, FWHT in the merge); H arguments of the API
    are accepted for interface compatibility and must be this matrix."""
    i = torch.arange(n)
    par = torch.zeros(n, n, dtype=torch.int64)
    x = i[:, None] & i[None, :]
    while bool(x.any()):
        par ^= x & 1
        x = x >> 1
    H = torch.where(par.bool(), -1.0, 1.0).to(torch.float32) / n ** 0.5
    return H.to(device)


def flat(t):
    """1-D view of t's storage starting at t's first element (kv800.py:49-52)."""
    n = t.untyped_storage().nbytes() // t.element_size() - t.storage_offset()
    return torch.as_strided(t, (n,), (1,), t.storage_offset())


def _hip():
    from . import kv800_hip
    kv800_hip.ops()                                   # ImportError when the backend cannot run here
    return kv800_hip


# ---------------------------------------------------------------- codec (HIP)
def quantize_blocks(k, v, H=None):
    """k, v: (M, 256, 4, 128) bf16 (pre-RoPE K, unrotated V) on the GPU -> (M, 51200) uint8 sub-blocks
    (kv800.py:56-76). Bit-identical to the reference quantizer on CPU torch."""
    return _hip().quantize_blocks(k.to(torch.bfloat16), v.to(torch.bfloat16))


def dequantize_blocks(sb, H=None):
    """(M, 51200) uint8 -> pre-RoPE K (M, 256, 4, 128) bf16 and unrotated V (M, 256, 4, 128) fp32 (kv800.py:79-92)."""
    return _hip().dequantize_blocks(sb)


def combine(MO, LO, AO, ns, H=None):
    """LSE merge of split partials (kv800.py:231-236): H applied to the quantized splits, bf16 out."""
    return _hip().combine(MO, LO, AO, ns)


class Paged:
    """Everything the decode kernels read for one layer and one batch of decode sequences (kv800.py:239-248).
    qpool: uint8 tensor whose data_ptr is the byte base of BOFF; epool: bf16 tensor, base of EOFF (elements);
    sk/sv: bf16 tensors, bases of SKOFF/SVOFF (elements). N: seq lengths incl. the current token (int32); NQ: flushed
    sub-blocks per sequence (int32); nqmax: host int >= max(NQ). win: 0 = quantized layer, 256 = window+sinks layer."""
    __slots__ = ("qpool", "boff", "epool", "eoff", "ebs", "e_hs", "e_ts", "e_v", "sk", "sv", "skoff", "svoff",
                 "N", "NQ", "nqmax", "win")

    def __init__(self, **kw):
        for k in self.__slots__:
            setattr(self, k, kw.get(k))


# ---------------------------------------------------------------- backend selection (kv800.py:251-359)
_FORCED = None
_CHOSEN = {}
_VERIFIED = set()
_LAST = [None]


def _requested():
    v = _FORCED if _FORCED is not None else os.environ.get("LFM3KV_BACKEND", "auto")
    v = (v or "auto").strip().lower()
    if v not in BACKENDS + REFERENCE_BACKENDS + ("auto",):
        raise ValueError(f"LFM3KV_BACKEND={v!r}: expected one of {', '.join(BACKENDS + REFERENCE_BACKENDS)}, auto")
    return v


def set_backend(name=None):
    """Force a decode backend ('hip'), or 'auto' / None to pick per device (env LFM3KV_BACKEND is read when None)."""
    global _FORCED
    _FORCED = None if name is None else str(name).strip().lower()
    _requested()
    _CHOSEN.clear(); _VERIFIED.clear()


def get_backend(device_type=None):
    """Backend used by the last decode() (or the one in use on `device_type`)."""
    return _CHOSEN.get(device_type) if device_type else _LAST[0]


def _available(name, dt):
    """(ok, detail) for backend `name` on device type `dt`."""
    if name in REFERENCE_BACKENDS:
        return False, f"the {name} backend is not part of the MI355X build (use the reference package for it)"
    if name == "hip":
        if dt != "cuda":
            return False, f"the HIP backend runs on ROCm GPUs (torch device type 'cuda'), not {dt!r}"
        from . import kv800_hip
        try:
            kv800_hip.ops()
        except ImportError as e:
            return False, str(e)
        return True, kv800_hip.SOURCE
    raise ValueError(name)


def _chain(dt):
    return ("hip",) if dt == "cuda" else ()


def _resolve(dt):
    if dt in _CHOSEN:
        return _CHOSEN[dt]
    req = _requested()
    if req != "auto":
        ok, why = _available(req, dt)
        if not ok:
            raise RuntimeError(f"800h decode backend {req!r} was requested (LFM3KV_BACKEND / set_backend) but is not "
                               f"available on {dt}: {why}")
        _log.info("decode backend on %s: %s (forced; %s)", dt, req, why)
        _CHOSEN[dt] = req
        return req
    skipped = []
    for name in _chain(dt):
        ok, why = _available(name, dt)
        if ok:
            _log.info("decode backend on %s: %s (%s)", dt, name, why)
            _CHOSEN[dt] = name
            return name
        skipped.append(f"{name}: {why}")
    raise RuntimeError(f"no 800h decode backend for device type {dt!r}"
                       + (f" ({'; '.join(skipped)})" if skipped else " (the MI355X build serves ROCm GPUs only)"))


def decode(P, q, cos_t, sin_t, H=None, spb=None, target=None):
    """q: (B, 16, 128) bf16 post-RoPE -> (B, 16, 128) bf16 (kv800.py:330-349). cos_t / sin_t: (P, 32) bf16 tables of
    the 32 rotating frequencies (dims d and d + 64 share frequency d, d < 32). H: the normalized 128 Hadamard (implicit
    in the kernels). spb / target: split planning overrides (kv800.py:366-367)."""
    dt = q.device.type
    be = _resolve(dt)
    _LAST[0] = be
    out = _run(be, P, q, cos_t, sin_t, spb, target)
    _VERIFIED.add(dt)
    return out


def _run(be, P, q, cos_t, sin_t, spb, target):
    if be != "hip":
        raise RuntimeError(f"backend {be!r} is not part of this build")
    from . import kv800_hip
    return kv800_hip.decode(P, q, cos_t, sin_t, spb, target)


# ---------------------------------------------------------------- harness store with the paged layout
class PagedStore:
    """Test/bench store with the vLLM-style paged layout for `batch` equal-length sequences (kv800.py:387-441). Exact
    pages form a ring of `nring` pages of `ebs` tokens per sequence; sub-blocks are flushed by the HIP paged flush
    (one launch per append) with the same rule as the vLLM cache."""

    def __init__(self, batch, max_len, device, window=0, ebs=64, nring=10):
        self.B, self.win, self.dev, self.ebs, self.nring = batch, window, device, ebs, nring
        self.H = hadamard(128, device)
        nsub = 0 if window else max_len // BLK + 1
        self.qpool = torch.zeros(max(1, batch * nsub), SUB, dtype=torch.uint8, device=device)
        self.boff = (torch.arange(batch * max(nsub, 1), device=device, dtype=torch.int64) * SUB).view(batch, max(nsub, 1))
        self.epool = torch.zeros(batch * nring, 4, ebs, 256, dtype=torch.bfloat16, device=device)
        npg = max_len // ebs + 2
        pg = torch.arange(npg, device=device) % nring
        self.eoff = ((torch.arange(batch, device=device)[:, None] * nring + pg[None]) * (4 * ebs * 256)).to(torch.int64)
        self.e_hs, self.e_ts, self.e_v = ebs * 256, 256, 128
        self.sk = torch.zeros(batch, NSINK, 4, 128, dtype=torch.bfloat16, device=device)
        self.sv = torch.zeros_like(self.sk)
        self.skoff = torch.arange(batch, device=device, dtype=torch.int64) * NSINK * 512
        self.N = torch.zeros(batch, dtype=torch.int32, device=device)
        self.NQ = torch.zeros_like(self.N)
        self.n, self.nq = 0, 0
        if nring * ebs < 512 + ebs:
            raise ValueError("the exact ring must hold at least 512 + ebs tokens")

    def paged(self):
        return Paged(qpool=self.qpool, boff=self.boff, epool=self.epool, eoff=self.eoff, ebs=self.ebs,
                     e_hs=self.e_hs, e_ts=self.e_ts, e_v=self.e_v, sk=self.sk if self.win else None,
                     sv=self.sv if self.win else None, skoff=self.skoff, svoff=self.skoff, N=self.N, NQ=self.NQ,
                     nqmax=self.nq, win=self.win)

    def _exact_index(self, pos):
        """element offsets (B, len(pos), 4) of the K rows of positions `pos` for each head."""
        pg = self.eoff[:, pos // self.ebs]
        return pg[..., None] + torch.arange(4, device=self.dev) * self.e_hs + (pos % self.ebs)[None, :, None] * self.e_ts

    def append(self, k, v):
        """k: pre-RoPE keys, v: values, (B, T, 4, 128)."""
        T = k.shape[1]
        ef = flat(self.epool)
        for s in range(0, T, 128):
            kk, vv = k[:, s:s + 128].to(self.dev, torch.bfloat16), v[:, s:s + 128].to(self.dev, torch.bfloat16)
            t = kk.shape[1]
            pos = torch.arange(self.n, self.n + t, device=self.dev)
            idx = self._exact_index(pos)[..., None] + torch.arange(128, device=self.dev)
            ef[idx] = kk
            ef[idx + self.e_v] = vv
            if self.win and self.n < NSINK:
                m = pos < NSINK
                self.sk[:, pos[m]], self.sv[:, pos[m]] = kk[:, m], vv[:, m]
            self.n += t
            nq_new = 0 if self.win else max(0, (self.n - LAG) // BLK)
            if nq_new > self.nq:                     # one launch flushes every newly eligible sub-block of every row
                prev = torch.full((self.B,), self.nq, dtype=torch.int32, device=self.dev)
                new = torch.full((self.B,), nq_new, dtype=torch.int32, device=self.dev)
                _hip().flush(self.epool, self.eoff, self.ebs, self.e_hs, self.e_ts, self.e_v, self.qpool, self.boff,
                             BLK, 1, prev, new, nq_new - self.nq)
                self.nq = nq_new
        self.N.fill_(self.n)
        self.NQ.fill_(self.nq)
