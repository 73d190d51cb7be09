"""CPU oracle for the 800h path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this module. The product package
(lfm3-kv800_amd/) never imports it; its decode and quantizer run on the HIP library or raise.

Python side of oracle/kv800_oracle.c (ctypes) plus numpy helpers:
  * bf16 <-> float32 bit conversion (round to nearest even, as torch .to(bfloat16));
  * quantize_blocks / dequantize_blocks / decode / combine / fake_quant_k / fake_quant_v: the C restatements of
    kv800.py:56-92, 231-236, torch_decode.py:16-80 and train.py:82-100 (see the C file's header for what pins each
    one);
  * build_paged(): a numpy restatement of the paged store of kv800.py:387-441 (exact pages of `ebs` tokens as
    [4 heads, ebs, K 128 | V 128] bf16, 51,200-byte quantized sub-blocks, sinks [4, 4, 128]) with the reference flush
    rule NQ = (n - 128) // 256 (kv800.py:433) and optionally shuffled physical page tables;
  * reference_f64(): a float64 restatement of the reference's independent check tests/test_parity.py:36-64
    (fake-quant with fp8 lo / scale, fp32 RoPE rounded to bf16, one softmax).
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "libkv800_oracle.so")

BLK, LAG, NSINK, WIN, SUB = 256, 128, 4, 256, 51200
KC_O, VB_O, VLO_O, VSC_O, KLO_O, KSC_O = 0, 32768, 49152, 49664, 50176, 50688

_LIB = None


class Paged(ctypes.Structure):
    _fields_ = [("qpool", ctypes.c_void_p), ("boff", ctypes.c_void_p), ("boff_stride", ctypes.c_int64),
                ("epool", ctypes.c_void_p), ("eoff", ctypes.c_void_p), ("eoff_stride", ctypes.c_int64),
                ("ebs", ctypes.c_int64), ("e_hs", ctypes.c_int64), ("e_ts", ctypes.c_int64), ("e_v", ctypes.c_int64),
                ("sk", ctypes.c_void_p), ("sv", ctypes.c_void_p), ("skoff", ctypes.c_void_p), ("svoff", ctypes.c_void_p),
                ("N", ctypes.c_void_p), ("NQ", ctypes.c_void_p), ("nqmax", ctypes.c_int64), ("win", ctypes.c_int64)]


def build_lib():
    """Compile the C oracle (make -C oracle)."""
    import subprocess
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _LIB
    if _LIB is None:
        if not os.path.isfile(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built: run `make -C oracle` (or __graft_entry__.build())")
        L = ctypes.CDLL(LIB_PATH)
        vp, i64 = ctypes.c_void_p, ctypes.c_int64
        L.oracle_quantize_blocks.argtypes = [vp, vp, i64, vp]
        L.oracle_dequantize_blocks.argtypes = [vp, i64, vp, vp]
        L.oracle_decode.argtypes = [ctypes.POINTER(Paged), i64, vp, vp, vp, vp]
        L.oracle_decode.restype = ctypes.c_int
        L.oracle_decode_f32.argtypes = [ctypes.POINTER(Paged), i64, vp, vp, vp, vp, vp]
        L.oracle_decode_f32.restype = ctypes.c_int
        L.oracle_combine.argtypes = [vp, vp, vp, i64, i64, vp]
        L.oracle_fake_quant_k.argtypes = [vp, i64, i64, vp]
        L.oracle_fake_quant_v.argtypes = [vp, i64, vp]
        L.oracle_f8_encode_n.argtypes = [vp, i64, vp]
        L.oracle_f8_decode_n.argtypes = [vp, i64, vp]
        L.oracle_hadamard.argtypes = [vp]
        L.oracle_num_threads.restype = ctypes.c_int
        _LIB = L
    return _LIB


def _p(a):
    return ctypes.c_void_p(a.ctypes.data) if a is not None else None


# ---------------------------------------------------------------- bf16 / fp8 helpers
def f32_to_bf16(x):
    """float32 array -> uint16 bf16 bits, round to nearest even (finite inputs)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    r = (u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)
    return r.astype(np.uint16)


def bf16_to_f32(b):
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def f8_encode(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint8)
    lib().oracle_f8_encode_n(_p(x), x.size, _p(out))
    return out


def f8_decode(b):
    b = np.ascontiguousarray(b, dtype=np.uint8)
    out = np.empty(b.shape, np.float32)
    lib().oracle_f8_decode_n(_p(b), b.size, _p(out))
    return out


def hadamard():
    H = np.empty((128, 128), np.float32)
    lib().oracle_hadamard(_p(H))
    return H


# ---------------------------------------------------------------- codec
def quantize_blocks(k_bits, v_bits):
    """k, v: (M, 256, 4, 128) uint16 bf16 bits -> (M, 51200) uint8 (kv800.py:56-76)."""
    k = np.ascontiguousarray(k_bits, np.uint16); v = np.ascontiguousarray(v_bits, np.uint16)
    assert k.shape == v.shape and k.shape[1:] == (BLK, 4, 128), k.shape
    M = k.shape[0]
    out = np.empty((M, SUB), np.uint8)
    lib().oracle_quantize_blocks(_p(k), _p(v), M, _p(out))
    return out


def dequantize_blocks(sb):
    """(M, 51200) uint8 -> K (M,256,4,128) uint16 bf16 bits, V (M,256,4,128) float32 (kv800.py:79-92)."""
    sb = np.ascontiguousarray(sb, np.uint8)
    M = sb.shape[0]
    k = np.empty((M, BLK, 4, 128), np.uint16); v = np.empty((M, BLK, 4, 128), np.float32)
    lib().oracle_dequantize_blocks(_p(sb), M, _p(k), _p(v))
    return k, v


def fake_quant_k(x):
    """x (..., 256, C) float32 -> float32 dequantized 800h K per (group, channel) (train.py:82-89)."""
    x = np.ascontiguousarray(x, np.float32)
    assert x.ndim >= 2 and x.shape[-2] == BLK, x.shape
    out = np.empty_like(x)
    lib().oracle_fake_quant_k(_p(x), x.size // (BLK * x.shape[-1]), x.shape[-1], _p(out))
    return out


def fake_quant_v(v):
    """v (..., 4, 128) float32 -> float32: the V of a quantize -> dequantize round trip per token (train.py:92-100)."""
    v = np.ascontiguousarray(v, np.float32)
    assert v.shape[-2:] == (4, 128), v.shape
    out = np.empty_like(v)
    lib().oracle_fake_quant_v(_p(v), v.size // 512, _p(out))
    return out


def combine(MO, LO, AO, ns):
    """kv800.py:231-236 -> (B, 16, 128) uint16 bf16 bits."""
    MO = np.ascontiguousarray(MO, np.float32); LO = np.ascontiguousarray(LO, np.float32)
    AO = np.ascontiguousarray(AO, np.float32)
    B = MO.shape[0]
    out = np.empty((B, 16, 128), np.uint16)
    lib().oracle_combine(_p(MO), _p(LO), _p(AO), B, ns, _p(out))
    return out


# ---------------------------------------------------------------- paged case (kv800.py:387-441 layout)
class PagedCase:
    """numpy arrays of one layer's paged cache + per-row lengths, in the layout of kv800.Paged."""

    def __init__(self, **kw):
        self.__dict__.update(kw)

    def c_struct(self):
        s = Paged()
        s.qpool, s.boff, s.boff_stride = _p(self.qpool), _p(self.boff), self.boff.shape[1]
        s.epool, s.eoff, s.eoff_stride = _p(self.epool), _p(self.eoff), self.eoff.shape[1]
        s.ebs, s.e_hs, s.e_ts, s.e_v = self.ebs, self.e_hs, self.e_ts, self.e_v
        s.sk = _p(self.sk) if self.sinks else None
        s.sv = _p(self.sv) if self.sinks else None
        s.skoff, s.svoff = _p(self.skoff), _p(self.svoff)
        s.N, s.NQ, s.nqmax, s.win = _p(self.N), _p(self.NQ), self.nqmax, self.win
        return s


def nq_of(n):
    """Flushed sub-blocks at length n (kv800.py:433, vllm_attn.py:303-305)."""
    return max(0, (int(n) - LAG) // BLK)


def build_paged(gen_kv, lens, win=0, ebs=64, shuffle_seed=None, sinks=True):
    """Paged layer for rows with lengths `lens`.

    gen_kv(b, p0, p1) -> (K, V) uint16 bf16 bits of shape (p1 - p0, 4, 128) for row b, positions [p0, p1).
    Quantized layers (win == 0): sub-blocks j < NQ_b are quantized by the oracle into the quant pool at BOFF[b, j];
    exact pages hold positions >= 256 NQ_b. Window layers (win > 0): exact pages hold [max(0, n - win), n), and the
    sinks (positions < 4) are stored at SKOFF / SVOFF when `sinks`. shuffle_seed permutes the physical page order of
    both pools (vLLM block tables); None keeps them in row-major order."""
    lens = [int(n) for n in lens]
    B = len(lens)
    rng = np.random.RandomState(shuffle_seed) if shuffle_seed is not None else None
    NQ = np.array([0 if win else nq_of(n) for n in lens], np.int32)
    nqmax = int(NQ.max()) if B else 0
    nsub = max(1, nqmax)
    qslots = B * nsub
    qperm = rng.permutation(qslots) if rng is not None else np.arange(qslots)
    boff = (qperm.reshape(B, nsub).astype(np.int64) * SUB)
    qpool = np.zeros((max(1, qslots), SUB), np.uint8)
    # exact pages: only the pages covering [lo_b, n_b) are materialised
    lo = [max(NQ[b] * BLK, n - win) if win else NQ[b] * BLK for b, n in enumerate(lens)]
    lo = [max(0, x) for x in lo]
    npg = max(1, max(((n + ebs - 1) // ebs for n in lens), default=1))
    first = [l // ebs for l in lo]
    need = [max(0, (n + ebs - 1) // ebs - f) for n, f in zip(lens, first)]
    total = max(1, sum(need))
    eperm = rng.permutation(total) if rng is not None else np.arange(total)
    page_elems = 4 * ebs * 256
    epool = np.zeros((total, 4, ebs, 256), np.uint16)
    eoff = np.zeros((B, npg), np.int64)
    c = 0
    for b in range(B):
        for i in range(need[b]):
            eoff[b, first[b] + i] = int(eperm[c]) * page_elems
            c += 1
    sk = np.zeros((B, NSINK, 4, 128), np.uint16); sv = np.zeros_like(sk)
    for b, n in enumerate(lens):
        nq = int(NQ[b])
        if nq:
            K, V = gen_kv(b, 0, nq * BLK)
            sb = quantize_blocks(K.reshape(nq, BLK, 4, 128), V.reshape(nq, BLK, 4, 128))
            for j in range(nq):
                qpool[boff[b, j] // SUB] = sb[j]
        if n > lo[b]:
            K, V = gen_kv(b, lo[b], n)
            for i, p in enumerate(range(lo[b], n)):
                pg = eoff[b, p // ebs] // page_elems
                epool[pg, :, p % ebs, :128] = K[i]
                epool[pg, :, p % ebs, 128:] = V[i]
        if win and sinks and n > 0:
            m = min(NSINK, n)
            K, V = gen_kv(b, 0, m)
            sk[b, :m] = K; sv[b, :m] = V
    return PagedCase(qpool=qpool, boff=boff, epool=epool, eoff=eoff, ebs=ebs, e_hs=ebs * 256, e_ts=256, e_v=128,
                     sk=sk, sv=sv, skoff=(np.arange(B, dtype=np.int64) * NSINK * 512),
                     svoff=(np.arange(B, dtype=np.int64) * NSINK * 512), sinks=bool(win and sinks),
                     N=np.array(lens, np.int32), NQ=NQ, nqmax=nqmax, win=int(win), B=B)


def decode(case, q_bits, cos_bits, sin_bits):
    """torch_decode.decode (torch_decode.py:27-80) on a PagedCase. q (B,16,128) bf16 bits; cos/sin (P,32) bf16
    bits -> (B,16,128) bf16 bits."""
    q = np.ascontiguousarray(q_bits, np.uint16)
    cs = np.ascontiguousarray(cos_bits, np.uint16); sn = np.ascontiguousarray(sin_bits, np.uint16)
    out = np.empty((q.shape[0], 16, 128), np.uint16)
    st = case.c_struct()
    rc = lib().oracle_decode(ctypes.byref(st), q.shape[0], _p(q), _p(cs), _p(sn), _p(out))
    if rc != 0:
        raise MemoryError("oracle decode scratch allocation failed")
    return out


def decode_f32(case, q_bits, cos_bits, sin_bits):
    """decode() and, beside its bf16 bits, the same outputs before their final bf16 rounding (float32)."""
    q = np.ascontiguousarray(q_bits, np.uint16)
    cs = np.ascontiguousarray(cos_bits, np.uint16); sn = np.ascontiguousarray(sin_bits, np.uint16)
    out = np.empty((q.shape[0], 16, 128), np.uint16)
    outf = np.empty((q.shape[0], 16, 128), np.float32)
    st = case.c_struct()
    rc = lib().oracle_decode_f32(ctypes.byref(st), q.shape[0], _p(q), _p(cs), _p(sn), _p(out), _p(outf))
    if rc != 0:
        raise MemoryError("oracle decode scratch allocation failed")
    return out, outf


def num_threads():
    return int(lib().oracle_num_threads())


# ---------------------------------------------------------------- seeded inputs
def randn_bf16(rng, shape, scale=1.0, offset=None):
    x = rng.standard_normal(size=shape).astype(np.float32) * np.float32(scale)
    if offset is not None:
        x = x + offset.astype(np.float32)
    return f32_to_bf16(x)


def rope_tables(max_pos, theta=1e6):
    """cos / sin (max_pos, 32) bf16 bits of the 32 rotating frequencies, float32 product then bf16 rounding, as
    vllm_attn.py:147-154 and tests/test_parity.py:30-33. float32 cos / sin come from numpy here; the tests that
    compare against the GPU feed the same arrays to both sides."""
    inv = (np.float32(1.0) / np.power(np.float32(theta), np.arange(0, 64, 2, dtype=np.float32) / np.float32(128))).astype(np.float32)
    fr = np.arange(max_pos, dtype=np.float32)[:, None] * inv[None]
    return f32_to_bf16(np.cos(fr).astype(np.float32)), f32_to_bf16(np.sin(fr).astype(np.float32))


# ---------------------------------------------------------------- independent float64 check (test_parity.py:36-64)
def _f8_round(x):
    return f8_decode(f8_encode(np.asarray(x, np.float32))).astype(np.float64)


def _aq(x, bits, axis):
    """test_parity.py:36-42: asymmetric min/max fake quant along `axis`, lo and scale through fp8 e4m3."""
    lo = x.min(axis=axis, keepdims=True); hi = x.max(axis=axis, keepdims=True)
    sc = np.maximum((hi - lo) / (2 ** bits - 1), 1e-8)
    lo8, sc8 = _f8_round(lo), np.maximum(_f8_round(sc), 1e-8)
    return np.clip(np.round((x - lo8) / sc8), 0, 2 ** bits - 1) * sc8 + lo8


def reference_f64(q_bits, K_bits, V_bits, cos_bits, sin_bits, window=0, round_k=True):
    """q (B,16,128), K/V (B,n,4,128) bf16 bits (pre-RoPE K), cos/sin (P,32) bf16 bits -> (B,16,128) float64.
    The reference's independent check, in float64 (the fake quant itself works on float32 values as the reference
    does; everything after it is float64). round_k=False skips the two bf16 roundings of K (dequantized, then
    rotated) that the reference and torch_decode.py apply: the exact attention over the quantized cache."""
    q = bf16_to_f32(q_bits).astype(np.float64)
    Kh = bf16_to_f32(K_bits).astype(np.float64); Vh = bf16_to_f32(V_bits).astype(np.float64)
    B, n = Kh.shape[:2]
    H = hadamard().astype(np.float64)
    nq = 0 if window else nq_of(n)
    K, V = Kh.copy(), Vh.copy()
    if nq:
        x = Kh[:, :nq * BLK].reshape(B, nq, BLK, 512).astype(np.float32)
        kq = _aq(x.astype(np.float64), 2, 2).reshape(B, nq * BLK, 4, 128)
        K[:, :nq * BLK] = bf16_to_f32(f32_to_bf16(kq.astype(np.float32))).astype(np.float64) if round_k else kq
        y = (Vh[:, :nq * BLK] @ H).reshape(B, nq * BLK, 2, 256)
        V[:, :nq * BLK] = _aq(y, 1, -1).reshape(B, nq * BLK, 4, 128) @ H
    cs = bf16_to_f32(cos_bits[:n]).astype(np.float64)[None, :, None, :]
    sn = bf16_to_f32(sin_bits[:n]).astype(np.float64)[None, :, None, :]
    K0, K2 = K[..., :32], K[..., 64:96]
    Kr = K.copy()
    Kr[..., :32] = K0 * cs - K2 * sn
    Kr[..., 64:96] = K2 * cs + K0 * sn
    if round_k:
        Kr = bf16_to_f32(f32_to_bf16(Kr.astype(np.float32))).astype(np.float64)
    Kr, V = np.repeat(Kr, 4, axis=2), np.repeat(V, 4, axis=2)            # (B, n, 16, 128)
    sc = np.einsum("bhd,bnhd->bhn", q, Kr) * 128 ** -0.5
    if window:
        p = np.arange(n)
        keep = (p >= n - window) | (p < NSINK)
        sc = np.where(keep[None, None], sc, -np.inf)
    sc = sc - sc.max(-1, keepdims=True)
    w = np.exp(sc); w = w / w.sum(-1, keepdims=True)
    return np.einsum("bhn,bnhd->bhd", w, V)
