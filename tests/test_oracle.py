"""Pins the CPU oracle (oracle/) against the reference's semantics, on the CPU:
  * fp8 e4m3fn encode against torch's .to(float8_e4m3fn) on every rounding-relevant bit pattern, decode exhaustively;
  * quantize_blocks byte-for-byte against the committed golden fixtures and the torch statement of kv800.py:56-76;
  * the Hadamard chain against torch-CPU's float32 matmul (the order MKL uses for this shape);
  * dequantize_blocks against the torch statement of kv800.py:79-92 and as the inverse of the packing;
  * decode against an independent float64 restatement of tests/test_parity.py:45-64 on the reference's 12 cases
    (rel < 1e-2 as the reference requires, plus the 2e-2 max-abs / 1e-3 mean-abs bar);
  * combine against a float64 LSE merge.
Planted mistakes (a negated sin table, swapped V planes, an off-by-one flush) must fail the same checks."""
import hashlib
import math

import numpy as np
import pytest
import torch

import make_golden
import torch_statement as ts

F8 = torch.float8_e4m3fn


def t_bf16(bits):
    return torch.from_numpy(np.ascontiguousarray(bits).astype(np.int16)).view(torch.bfloat16)


# ---------------------------------------------------------------- fp8
def test_f8_encode_matches_torch(oracle):
    rng = np.random.RandomState(0)
    # every (sign, exponent, top-4 mantissa bits) with rounding-relevant low patterns, plus random floats
    top = np.arange(1 << 13, dtype=np.uint32) << np.uint32(19)                    # bits 19..31
    low = np.array([0, 1, 0x3FFFF, 0x40000, 0x40001, 0x7FFFF], dtype=np.uint32)
    pats = (top[:, None] | low[None, :]).ravel()
    pats = np.concatenate([pats, rng.randint(0, 2 ** 32, size=2_000_000, dtype=np.uint64).astype(np.uint32)])
    x = pats.view(np.float32)
    want = torch.from_numpy(x.copy()).to(F8).view(torch.uint8).numpy()
    got = oracle.f8_encode(x)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], want[~nan])
    assert np.all((got[nan] & 0x7F) == 0x7F)


def test_f8_decode_exhaustive(oracle):
    b = np.arange(256, dtype=np.uint8)
    want = torch.from_numpy(b.copy()).view(F8).float().numpy()
    got = oracle.f8_decode(b)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan) and np.array_equal(got[~nan], want[~nan])


# ---------------------------------------------------------------- Hadamard chain = torch-CPU matmul order
def test_hadamard_constant_and_chain(oracle):
    H = oracle.hadamard()
    Ht = ts.sylvester().numpy()
    assert np.array_equal(H.view(np.uint32), Ht.view(np.uint32))
    assert set(np.abs(H).view(np.uint32).ravel().tolist()) == {0x3DB504F3}
    # dequantize uses the same chain: (bits*vsc+vlo) @ H must equal torch's matmul bit for bit
    kb, vb = make_golden.case_inputs("outlier")
    sb = ts.quantize(t_bf16(kb), t_bf16(vb)).numpy()
    _, v = oracle.dequantize_blocks(sb)
    _, vt = ts.dequantize(torch.from_numpy(sb))
    assert np.array_equal(v.view(np.uint32), vt.numpy().view(np.uint32))


# ---------------------------------------------------------------- quantizer
@pytest.mark.parametrize("case", ["parity", "outlier", "edge", "scaled"])
def test_quantize_matches_golden(oracle, case):
    g = np.load(make_golden.os.path.join(make_golden.HERE, "quantize_golden.npz"))
    kb, vb = make_golden.case_inputs(case)
    assert make_golden.input_digest(kb, vb) == str(g[f"{case}_input_sha256"]), "seeded inputs drifted"
    out = oracle.quantize_blocks(kb, vb)
    if case == "scaled":
        got = [hashlib.sha256(out[m].tobytes()).hexdigest() for m in range(out.shape[0])]
        assert got == list(g["scaled_sha256"])
    else:
        want = g[f"{case}_out"]
        assert np.array_equal(out, want), f"{int((out != want).sum())} bytes differ"


def test_quantize_matches_torch_statement_random(oracle):
    rng = np.random.RandomState(7)
    k = make_golden.bf16_bits(rng.standard_normal((3, 256, 4, 128)).astype(np.float32) * rng.rand(1, 1, 4, 128).astype(np.float32) * 4 + 0.3)
    v = make_golden.bf16_bits(rng.standard_normal((3, 256, 4, 128)).astype(np.float32) * 2)
    assert np.array_equal(oracle.quantize_blocks(k, v), ts.quantize(t_bf16(k), t_bf16(v)).numpy())


def test_dequantize_is_inverse_of_packing(oracle):
    kb, vb = make_golden.case_inputs("parity")
    sb = oracle.quantize_blocks(kb, vb)
    k, v = oracle.dequantize_blocks(sb)
    kt, vt = ts.dequantize(torch.from_numpy(sb))
    assert np.array_equal(k, kt.view(torch.int16).numpy().view(np.uint16))
    assert np.array_equal(v.view(np.uint32), vt.numpy().view(np.uint32))
    # closed form: codes rebuilt from the dequantized K reproduce the kc bytes
    klo = oracle.f8_decode(sb[:, 50176:50688]).reshape(-1, 1, 4, 128)
    ksc = oracle.f8_decode(sb[:, 50688:]).reshape(-1, 1, 4, 128)
    kf = oracle.bf16_to_f32(k)
    codes = np.rint((kf - klo) / np.where(ksc > 0, ksc, 1)).astype(np.int64)
    codes = np.where(ksc > 0, codes, 0).clip(0, 3).reshape(-1, 256, 4, 4, 32)
    kc = codes[..., 0, :] | (codes[..., 1, :] << 2) | (codes[..., 2, :] << 4) | (codes[..., 3, :] << 6)
    assert np.array_equal(kc.reshape(sb.shape[0], -1).astype(np.uint8), sb[:, :32768])


def test_quantizer_equals_fake_quant(oracle):
    """tests/test_train_hook.py:92-106: dequantize(quantize(k)) equals the per-channel fake quant of K exactly."""
    kb, vb = make_golden.case_inputs("parity")
    k, _ = oracle.dequantize_blocks(oracle.quantize_blocks(kb, vb))
    x = oracle.bf16_to_f32(kb).reshape(2, 256, 512)
    lo, hi = x.min(1, keepdims=True), x.max(1, keepdims=True)
    lo8 = oracle.f8_decode(oracle.f8_encode(lo))
    sc8 = oracle.f8_decode(oracle.f8_encode(np.maximum((hi - lo) / np.float32(3), np.float32(1e-8))))
    c = np.clip(np.rint((x - lo8) / np.maximum(sc8, np.float32(1e-8))), 0, 3).astype(np.float32)
    fq = oracle.f32_to_bf16((c * sc8 + lo8).astype(np.float32)).reshape(k.shape)
    assert np.array_equal(fq, k)


# ---------------------------------------------------------------- decode (the reference's 12 parity cases)
QUANT_NS = (50, 383, 384, 700, 1500, 5000)
WINDOW_NS = (3, 10, 200, 259, 260, 1500)


def parity_inputs(oracle, n, win, seed=0):
    """B = 2 rows: K = N(0,1) + 3 N(0,1) per channel, V = N(0,1), q = 2 N(0,1) (tests/test_parity.py:83-87)."""
    rng = np.random.RandomState(seed * 100003 + n * 7 + win)
    K = oracle.randn_bf16(rng, (2, n, 4, 128), offset=3 * rng.standard_normal((1, 1, 4, 128)))
    V = oracle.randn_bf16(rng, (2, n, 4, 128))
    q = oracle.randn_bf16(rng, (2, 16, 128), scale=2.0)
    return q, K, V


def run_parity(oracle, n, win, mutate=None):
    q, K, V = parity_inputs(oracle, n, win)
    cos, sin = oracle.rope_tables(8192)
    case = oracle.build_paged(lambda b, p0, p1: (K[b, p0:p1], V[b, p0:p1]), [n, n], win=win, shuffle_seed=n)
    sin_used = oracle.f32_to_bf16(-oracle.bf16_to_f32(sin)) if mutate == "sin" else sin
    if mutate == "vplanes":
        vb = case.qpool[:, 32768:49152].copy()
        case.qpool[:, 32768:49152] = ((vb << 1) | (vb >> 7)).astype(np.uint8)
    if mutate == "flush":
        case.NQ = np.maximum(case.NQ - 1, 0).astype(np.int32)   # one sub-block too few read as quantized
    out = oracle.bf16_to_f32(oracle.decode(case, q, cos, sin_used)).astype(np.float64)
    ref = oracle.reference_f64(q, K, V, cos, sin, window=win)
    rel = np.linalg.norm(out - ref) / np.linalg.norm(ref)
    return out, ref, rel


@pytest.mark.parametrize("win,n", [(0, n) for n in QUANT_NS] + [(256, n) for n in WINDOW_NS])
def test_oracle_decode_parity(oracle, win, n):
    """The reference's bar (rel < 1e-2, test_parity.py:104), and sharper: the oracle's bf16 output is the bf16
    rounding of the independent float64 result to within one bf16 ulp (what remains is rounding noise)."""
    out, ref, rel = run_parity(oracle, n, win)
    assert math.isfinite(rel) and rel < 1e-2, rel
    refb = oracle.bf16_to_f32(oracle.f32_to_bf16(ref.astype(np.float32))).astype(np.float64)
    d = np.abs(out - refb)
    assert np.all(d <= np.abs(ref) * 2 ** -7 + 1e-6), d.max()
    assert d.mean() < 1e-4, d.mean()


@pytest.mark.parametrize("mutate", ["sin", "vplanes", "flush"])
def test_oracle_decode_planted_mistakes_fail(oracle, mutate):
    _, _, rel = run_parity(oracle, 1500, 0, mutate=mutate)
    assert rel > 3e-2, (mutate, rel)


def _torch_case(case):
    """An oracle PagedCase as CPU torch tensors with the kv800.Paged field names."""
    from types import SimpleNamespace
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a))
    bf = lambda a: T(a.view(np.int16)).view(torch.bfloat16)
    return SimpleNamespace(qpool=T(case.qpool), boff=T(case.boff), epool=bf(case.epool), eoff=T(case.eoff),
                           ebs=case.ebs, e_hs=case.e_hs, e_ts=case.e_ts, e_v=case.e_v,
                           sk=bf(case.sk) if case.sinks else None, sv=bf(case.sv) if case.sinks else None,
                           skoff=T(case.skoff), svoff=T(case.svoff), N=T(case.N), NQ=T(case.NQ), nqmax=case.nqmax,
                           win=case.win)


@pytest.mark.parametrize("win,n", [(0, 1024), (0, 5000), (256, 1500), (256, 3)])
def test_torch_port_matches_c_oracle(oracle, win, n):
    """oracle/torch_port.py (the pure-torch CPU baseline) and the C oracle restate the same decode: on the
    reference's parity inputs they agree to the bf16 rounding of their different summation orders."""
    import torch_port
    q, K, V = parity_inputs(oracle, n, win, seed=5)
    cos, sin = oracle.rope_tables(n + 8)
    case = oracle.build_paged(lambda b, p0, p1: (K[b, p0:p1], V[b, p0:p1]), [n, n], win=win, shuffle_seed=n)
    want = oracle.bf16_to_f32(oracle.decode(case, q, cos, sin))
    got = torch_port.decode(_torch_case(case), t_bf16(q), t_bf16(cos), t_bf16(sin)).float().numpy()
    d = np.abs(got - want)
    assert d.max() <= np.abs(want).max() * 2 ** -7 and d.mean() < 1e-4, (d.max(), d.mean())


def test_torch_port_dequantize_matches_statement():
    """torch_port.dequantize against the golden generator's dequantizer (tests/golden/torch_statement.py)."""
    import torch_port
    g = torch.Generator().manual_seed(2)
    k = torch.randn(3, 256, 4, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(3, 256, 4, 128, generator=g).to(torch.bfloat16)
    sb = ts.quantize(k, v)
    k1, v1 = torch_port.dequantize(sb, torch_port.hadamard128())
    k2, v2 = ts.dequantize(sb)
    assert torch.equal(k1, k2.float()) and torch.equal(v1, v2)
    assert torch.equal(torch_port.hadamard128(), ts.sylvester())


def test_oracle_combine():
    import oracle as o
    rng = np.random.RandomState(3)
    B, ns = 3, 4
    MO = (rng.standard_normal((B, ns + 1, 16)) * 4).astype(np.float32)
    LO = (rng.rand(B, ns + 1, 16) * 10 + 0.1).astype(np.float32)
    AO = rng.standard_normal((B, ns + 1, 16, 128)).astype(np.float32)
    out = o.bf16_to_f32(o.combine(MO, LO, AO, ns)).astype(np.float64)
    H = o.hadamard().astype(np.float64)
    w = np.exp2(MO - MO.max(1, keepdims=True)).astype(np.float64)
    L = (w * LO).sum(1)
    ref = (w[:, :ns, :, None] * AO[:, :ns]).sum(1) @ H + w[:, ns, :, None] * AO[:, ns]
    ref = ref / L[..., None]
    assert np.abs(out - ref).max() <= np.abs(ref).max() * 2 ** -7


# ---------------------------------------------------------------- training fake quant (train.py:82-100)
def _fq_k_numpy(oracle, x):
    """train.py:82-89 restated with numpy float32 ops (independent of the C oracle)."""
    x = np.asarray(x, np.float32)
    lo = x.min(axis=-2, keepdims=True); hi = x.max(axis=-2, keepdims=True)
    lo8 = oracle.f8_decode(oracle.f8_encode(lo))
    sc8 = oracle.f8_decode(oracle.f8_encode(np.maximum((hi - lo) / np.float32(3), np.float32(1e-8))))
    c = np.clip(np.rint((x - lo8) / np.maximum(sc8, np.float32(1e-8))), 0, 3).astype(np.float32)
    return (c * sc8 + lo8).astype(np.float32)


def _train_inputs(oracle, seed):
    """tests/test_train_hook.py:93-96 shapes: K with per-channel scale and offset, V x 2 (bf16 bits)."""
    rng = np.random.RandomState(seed)
    k = rng.standard_normal((3, 256, 4, 128)) * rng.rand(1, 1, 4, 128) * 4 + 0.3
    v = rng.standard_normal((3, 256, 4, 128)) * 2
    return oracle.f32_to_bf16(k.astype(np.float32)), oracle.f32_to_bf16(v.astype(np.float32))


def test_fake_quant_k_numpy_statement(oracle):
    """C oracle vs the numpy statement on float32 inputs that are not bf16 values, with constant and outlier channels."""
    rng = np.random.RandomState(3)
    x = (rng.standard_normal((2, 256, 300)) * rng.rand(1, 1, 300) * 5).astype(np.float32)
    x[0, :, 7] = 1.25                                 # constant channel: scale clamps to 1e-8
    x[1, ::17, 11] *= 40                              # outliers
    assert np.array_equal(oracle.fake_quant_k(x), _fq_k_numpy(oracle, x))


def test_fake_quant_k_equals_round_trip(oracle):
    """tests/test_train_hook.py:97-99 analogue: fake_quant_k on bf16 keys, cast to bf16, equals the K of
    dequantize(quantize(k, v)) bit for bit."""
    kb, vb = _train_inputs(oracle, 0)
    kr, _ = oracle.dequantize_blocks(oracle.quantize_blocks(kb, vb))
    kq = oracle.fake_quant_k(oracle.bf16_to_f32(kb).reshape(3, 256, 512)).reshape(3, 256, 4, 128)
    assert np.array_equal(oracle.f32_to_bf16(kq), kr)
    # a planted mistake (scale (hi - lo) / 4) must not pass
    x = oracle.bf16_to_f32(kb).reshape(3, 256, 512)
    lo = x.min(1, keepdims=True); hi = x.max(1, keepdims=True)
    sc8 = oracle.f8_decode(oracle.f8_encode(np.maximum((hi - lo) / np.float32(4), np.float32(1e-8))))
    lo8 = oracle.f8_decode(oracle.f8_encode(lo))
    bad = (np.clip(np.rint((x - lo8) / sc8), 0, 3) * sc8 + lo8).astype(np.float32).reshape(3, 256, 4, 128)
    assert not np.array_equal(oracle.f32_to_bf16(bad), kr)


def test_fake_quant_v_equals_round_trip(oracle):
    """tests/test_train_hook.py:100-101 analogue: fake_quant_v equals the V of dequantize(quantize(k, v)) (same fp32
    chains, so bit for bit here; the reference's bar is atol 1e-5)."""
    kb, vb = _train_inputs(oracle, 1)
    _, vr = oracle.dequantize_blocks(oracle.quantize_blocks(kb, vb))
    vq = oracle.fake_quant_v(oracle.bf16_to_f32(vb))
    assert np.array_equal(vq, vr)


def test_fake_quant_v_float64(oracle):
    """Against a float64 statement of train.py:92-100: tokens whose bits agree match within the fp32 rounding of the
    two 128-term chains (1e-5 relative to the token's largest output); a token whose bits differ (an error of about
    sc8 / sqrt(128), far above that) must hold a rounding tie (|(y - lo8) / sc8 - 1/2| tiny in float64)."""
    rng = np.random.RandomState(2)
    v = (rng.standard_normal((512, 4, 128)) * 2).astype(np.float32)
    got = oracle.fake_quant_v(v).astype(np.float64)
    H = oracle.hadamard().astype(np.float64)
    y = (v.astype(np.float64) @ H).reshape(512, 2, 256)
    lo = y.min(-1, keepdims=True); hi = y.max(-1, keepdims=True)
    lo8 = oracle.f8_decode(oracle.f8_encode(lo.astype(np.float32))).astype(np.float64)
    sc8 = oracle.f8_decode(oracle.f8_encode(np.maximum(hi - lo, 1e-8).astype(np.float32))).astype(np.float64)
    r = (y - lo8) / np.maximum(sc8, 1e-8)
    want = (np.clip(np.round(r), 0, 1) * sc8 + lo8).reshape(512, 4, 128) @ H
    diff = np.abs(got - want).max(axis=(1, 2))
    bad = np.nonzero(diff > 1e-5 * (1 + np.abs(want).max(axis=(1, 2))))[0]
    for t in bad:
        assert np.abs(np.abs(r[t] - np.floor(r[t])) - 0.5).min() < 1e-5, t
    assert len(bad) <= 2
