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
class _Selection:
    """Decode-backend choice with the reference's controls: the LFM3KV_BACKEND environment variable (read at every
    resolution) and set_backend() name a backend or 'auto'; the choice is made once per device type and remembered
    until set_backend() is called again. This build serves one backend, 'hip', on ROCm devices (torch device type
    'cuda'). The reference's own names are valid values but cannot be served, so forcing one raises RuntimeError, and
    'auto' raises too on a device the HIP library cannot serve: there is no CPU path to fall back to."""

    def __init__(self):
        self.override = None          # set by set_backend(); None: the environment decides
        self.chosen = {}              # device type -> backend name resolved for it
        self.last = None              # backend of the most recent decode()

    @staticmethod
    def normalise(name):
        key = "auto" if name is None else (str(name).strip().lower() or "auto")
        known = BACKENDS + REFERENCE_BACKENDS + ("auto",)
        if key not in known:
            raise ValueError(f"LFM3KV_BACKEND={key!r}: expected one of {', '.join(known)}")
        return key

    def wanted(self):
        return self.normalise(self.override if self.override is not None else os.environ.get("LFM3KV_BACKEND"))

    @staticmethod
    def refusal(name, device_type):
        """None when backend `name` can run on `device_type`, else why it cannot."""
        if name in REFERENCE_BACKENDS:
            return f"the {name} backend is not part of the MI355X build (use the reference package for it)"
        if device_type != "cuda":
            return f"the HIP backend runs on ROCm GPUs (torch device type 'cuda'), not {device_type!r}"
        from . import kv800_hip
        try:
            kv800_hip.ops()
        except ImportError as e:
            return str(e)
        return None

    def backend_for(self, device_type):
        if device_type in self.chosen:
            return self.chosen[device_type]
        wanted = self.wanted()
        name = "hip" if wanted == "auto" else wanted
        why = self.refusal(name, device_type)
        if why is not None and wanted == "auto":
            raise RuntimeError(f"no 800h decode backend for device type {device_type!r} ({why})")
        if why is not None:
            raise RuntimeError(f"800h decode backend {wanted!r} was requested (LFM3KV_BACKEND / set_backend) but is "
                               f"not available on {device_type}: {why}")
        _log.info("decode backend on %s: %s (%s)", device_type, name, "forced" if wanted != "auto" else "auto")
        self.chosen[device_type] = name
        return name


_SEL = _Selection()


def set_backend(name=None):
    """Force a decode backend ('hip'), or 'auto' / None to pick per device (env LFM3KV_BACKEND is read when None).
    An unknown name raises ValueError and leaves the current setting as it was."""
    _SEL.override = None if name is None else _SEL.normalise(name)
    _SEL.chosen.clear()


def get_backend(device_type=None):
    """Backend used by the last decode() (or the one in use on `device_type`)."""
    return _SEL.chosen.get(device_type) if device_type else _SEL.last


def decode(P, q, cos_t, sin_t, H=None, spb=None, target=None):
    """q: (B, 16, 128) bf16 post-RoPE -> (B, 16, 128) bf16 (kv800.py:330-349). cos_t / sin_t: (P, 32) bf16 tables of
    the 32 rotating frequencies (dims d and d + 64 share frequency d, d < 32). H: the normalized 128 Hadamard (implicit
    in the kernels). spb / target: split planning overrides (kv800.py:366-367)."""
    _SEL.last = _SEL.backend_for(q.device.type)
    from . import kv800_hip
    return kv800_hip.decode(P, q, cos_t, sin_t, spb, target)


# ---------------------------------------------------------------- harness store with the paged layout
class PagedStore:
    """Cache of one layer for `batch` sequences of equal length, in the paged layout the decode reads (the reference's
    test/bench store, kv800.py:387-441, same constructor and methods).

    Exact pages: sequence b owns pages [b nring, (b + 1) nring) of `epool` and uses them as a ring, position p living
    in page b nring + (p // ebs) % nring, slot p % ebs. Quantized layers: sequence b's sub-block j lives at byte
    BOFF[b, j] = (b nsub + j) 51,200 of `qpool`. append() moves rows in with the HIP row-write kernel (one launch per
    step of at most 128 tokens, sinks included) and flushes the sub-blocks that became eligible (n >= 256 j + 384) with
    one HIP flush launch. A step of at most 128 tokens ends at most 511 positions after the first row of the oldest
    sub-block still to flush, so a ring of at least 512 + ebs tokens never overwrites a row before its flush."""

    STEP = 128

    def __init__(self, batch, max_len, device, window=0, ebs=64, nring=10):
        if nring * ebs < 512 + ebs:
            raise ValueError(f"the exact ring of {nring} x {ebs} tokens must hold at least 512 + ebs tokens")
        self.B, self.win, self.dev, self.ebs, self.nring = batch, window, device, ebs, nring
        self.H = hadamard(128, device)
        nsub = 1 if window else max_len // BLK + 1
        self.qpool = torch.zeros(batch * nsub, SUB, dtype=torch.uint8, device=device)
        self.boff = torch.arange(batch * nsub, dtype=torch.int64, device=device).view(batch, nsub) * SUB
        self.epool = torch.zeros(batch * nring, 4, ebs, 256, dtype=torch.bfloat16, device=device)
        self.e_hs, self.e_ts, self.e_v = self.epool.stride(1), self.epool.stride(2), 128
        self._ring0 = torch.arange(batch, dtype=torch.int64, device=device) * nring   # first ring page of each row
        logical = torch.arange(max_len // ebs + 2, dtype=torch.int64, device=device)
        self.eoff = (self._ring0[:, None] + logical % nring) * self.epool.stride(0)
        self.sk = torch.zeros(batch, NSINK, 4, 128, dtype=torch.bfloat16, device=device)
        self.sv = torch.zeros_like(self.sk)
        self.skoff = self._ring0 // nring * self.sk.stride(0)
        self.N = torch.zeros(batch, dtype=torch.int32, device=device)
        self.NQ = torch.zeros(batch, dtype=torch.int32, device=device)
        self.n = self.nq = 0

    def paged(self):
        return Paged(qpool=self.qpool, boff=self.boff, epool=self.epool, eoff=self.eoff, ebs=self.ebs,
                     e_hs=self.e_hs, e_ts=self.e_ts, e_v=self.e_v, sk=self.sk if self.win else None,
                     sv=self.sv if self.win else None, skoff=self.skoff, svoff=self.skoff, N=self.N, NQ=self.NQ,
                     nqmax=self.nq, win=self.win)

    def append(self, k, v):
        """k: pre-RoPE keys, v: values, (B, T, 4, 128), any float dtype (cast to bf16)."""
        kh = _hip()
        T = k.shape[1]
        for t0 in range(0, T, self.STEP):
            t1 = min(T, t0 + self.STEP)
            pos = torch.arange(self.n, self.n + t1 - t0, dtype=torch.int64, device=self.dev)
            slot = (self._ring0[:, None] + (pos // self.ebs) % self.nring) * self.ebs + pos % self.ebs      # (B, t)
            rows_k = k[:, t0:t1].to(self.dev, torch.bfloat16).reshape(-1, 4, 128)
            rows_v = v[:, t0:t1].to(self.dev, torch.bfloat16).reshape(-1, 4, 128)
            sinks = {}
            if self.win and self.n < NSINK:
                sinks = dict(pos=pos.expand(self.B, -1).reshape(-1), sk=self.sk, sv=self.sv,
                             skoff=self.skoff[:, None].expand(-1, t1 - t0).reshape(-1))
                sinks["svoff"] = sinks["skoff"]
            kh.write_exact(self.epool, slot.reshape(-1), rows_k, rows_v, **sinks)
            self.n += t1 - t0
            eligible = 0 if self.win else max(0, self.n - LAG) // BLK
            if eligible > self.nq:
                nq0 = torch.full((self.B,), self.nq, dtype=torch.int32, device=self.dev)
                nq1 = torch.full((self.B,), eligible, dtype=torch.int32, device=self.dev)
                kh.flush(self.epool, self.eoff, self.ebs, self.e_hs, self.e_ts, self.e_v, self.qpool, self.boff,
                         BLK, 1, nq0, nq1, eligible - self.nq)
                self.nq = eligible
        self.N.fill_(self.n)
        self.NQ.fill_(self.nq)
