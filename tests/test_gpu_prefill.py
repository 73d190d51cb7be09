"""Prefill over compressed history on an MI355X: kv800_hip_history (the dequantize -> bf16 producer of
vllm_attn.py:351-380) bit-exact against the oracle, and the quantized-layer prefill rows (vllm_cache.prefill_quant_rows)
against a float64 restatement."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"
MAX_ABS, MEAN_ABS = 2e-2, 1e-3


def say(*a):
    print("[gpu-prefill]", *a, flush=True)


def to_dev_bf16(bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).to(DEV)


def bits_of(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def upload(case):
    import lfm3_kv800_amd.kv800 as kv
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    return kv.Paged(qpool=T(case.qpool), boff=T(case.boff), epool=to_dev_bf16(case.epool), eoff=T(case.eoff),
                    ebs=case.ebs, e_hs=case.e_hs, e_ts=case.e_ts, e_v=case.e_v, sk=None, sv=None, skoff=None,
                    svoff=None, N=T(case.N), NQ=T(case.NQ), nqmax=case.nqmax, win=0)


def rope_np(oracle, kbits, pos, cos, sin):
    """vllm_attn.py:160-163 in numpy float32 (each product and the sum rounded once), then bf16 bits."""
    k = oracle.bf16_to_f32(kbits)
    c32, s32 = oracle.bf16_to_f32(cos[pos]), oracle.bf16_to_f32(sin[pos])
    one, zero = np.ones_like(c32), np.zeros_like(s32)
    c = np.concatenate([c32, one, c32, one], 1)[:, None, :]
    s = np.concatenate([s32, zero, s32, zero], 1)[:, None, :]
    rot = np.concatenate([-k[..., 64:], k[..., :64]], -1)
    return oracle.f32_to_bf16((k * c + rot * s).astype(np.float32))


def history_np(oracle, K, V, n):
    """Positions [0, n) of one row as the reference assembles them: dequantized sub-blocks (K bf16, V fp32 -> bf16),
    then the exact rows; returns unrotated K bits and V bits."""
    nq = oracle.nq_of(n)
    kb, vb = K[:n].copy(), V[:n].copy()
    if nq:
        kq, vq = oracle.dequantize_blocks(oracle.quantize_blocks(K[:256 * nq].reshape(nq, 256, 4, 128),
                                                                 V[:256 * nq].reshape(nq, 256, 4, 128)))
        kb[:256 * nq] = kq.reshape(-1, 4, 128)
        vb[:256 * nq] = oracle.f32_to_bf16(vq.reshape(-1, 4, 128))
    return kb, vb


# the launch takes 64 positions per workgroup, or 16 / 4 when that leaves fewer than 1,024 workgroups: the first set
# runs at 4 (578 tiles x 5 rows), the single 16K row at 16 (1,025 tiles), the four rows at 64 (257 tiles x 4)
@pytest.mark.parametrize("lens", [[50, 384, 640, 1000, 2311], [16400], [16400, 300, 9000, 16390]],
                         ids=["tiles4", "tiles16", "tiles64"])
def test_history_bitexact(hip, oracle, lens):
    rng = np.random.RandomState(5)
    K = [oracle.randn_bf16(rng, (n, 4, 128), offset=rng.standard_normal((1, 4, 128))) for n in lens]
    V = [oracle.randn_bf16(rng, (n, 4, 128)) for n in lens]
    cos, sin = oracle.rope_tables(max(lens) + 16)
    case = oracle.build_paged(lambda b, p0, p1: (K[b][p0:p1], V[b][p0:p1]), lens, ebs=64, shuffle_seed=3)
    P = upload(case)
    say("history", lens)
    Kh, Vh, offs = hip.history(P, lens, to_dev_bf16(cos), to_dev_bf16(sin))
    Ku, Vu, _ = hip.history(P, lens)                          # unrotated (sliding layers)
    kh, vh, ku, vu = bits_of(Kh), bits_of(Vh), bits_of(Ku), bits_of(Vu)
    for b, n in enumerate(lens):
        kb, vb = history_np(oracle, K[b], V[b], n)
        sl = slice(offs[b], offs[b] + n)
        assert np.array_equal(vh[sl], vb), b
        assert np.array_equal(vu[sl], vb), b
        assert np.array_equal(ku[sl], kb), b
        assert np.array_equal(kh[sl], rope_np(oracle, kb, np.arange(n), cos, sin)), b


def check_quant_rows(oracle, prev, new, seed):
    """prefill_quant_rows over rows with histories prev and new-query counts new, against a float64 attention over
    the reference's assembled keys / values (dequantized history + exact rows, RoPE at every position)."""
    from lfm3_kv800_amd import vllm_cache as vc
    rng = np.random.RandomState(seed)
    R = len(prev)
    lens = [p + t for p, t in zip(prev, new)]
    K = [oracle.randn_bf16(rng, (n, 4, 128)) for n in lens]
    V = [oracle.randn_bf16(rng, (n, 4, 128)) for n in lens]
    cos, sin = oracle.rope_tables(max(lens) + 8)
    case = oracle.build_paged(lambda b, p0, p1: (K[b][p0:p1], V[b][p0:p1]), prev, ebs=64, shuffle_seed=seed)
    P = upload(case)
    q = oracle.randn_bf16(rng, (sum(new), 16, 128))
    qsl = np.concatenate([[0], np.cumsum(new)]).astype(np.int64)
    kn = np.concatenate([K[b][prev[b]:] for b in range(R)])
    vn = np.concatenate([V[b][prev[b]:] for b in range(R)])
    say("prefill rows", R, "rows: prev", prev[:8], "new", new[:8], "query tiles", sum((t + 31) // 32 for t in new))
    out = vc.prefill_quant_rows(P, to_dev_bf16(q), to_dev_bf16(kn), to_dev_bf16(vn), qsl, prev, to_dev_bf16(cos),
                                to_dev_bf16(sin))
    assert tuple(out.shape) == (sum(new), 16, 128)
    o = torch.from_numpy(bits_of(out).view(np.int16)).view(torch.bfloat16).float().numpy()
    assert np.isfinite(o).all()
    worst = 0.0
    for b in range(R):
        n0, n = prev[b], lens[b]
        if n == n0:
            continue
        kb, vb = history_np(oracle, K[b], V[b], n0)
        kb = np.concatenate([kb, K[b][n0:n]]); vb = np.concatenate([vb, V[b][n0:n]])
        Kr = oracle.bf16_to_f32(rope_np(oracle, kb, np.arange(n), cos, sin)).astype(np.float64)
        Vf = oracle.bf16_to_f32(vb).astype(np.float64)
        qf = oracle.bf16_to_f32(q[qsl[b]:qsl[b + 1]]).astype(np.float64)
        Kr, Vf = np.repeat(Kr, 4, axis=1), np.repeat(Vf, 4, axis=1)                   # (n, 16, 128)
        sc = np.einsum("thd,shd->hts", qf, Kr) * 128 ** -0.5
        qp = np.arange(n0, n)
        sc = np.where(np.arange(n)[None, None, :] <= qp[None, :, None], sc, -np.inf)
        w = np.exp(sc - sc.max(-1, keepdims=True)); w /= w.sum(-1, keepdims=True)
        want = np.einsum("hts,shd->thd", w, Vf)
        d = np.abs(o[qsl[b]:qsl[b + 1]] - want)
        worst = max(worst, float(d.max()))
        if R <= 4:
            say(f"row {b}: max-abs {d.max():.3e} mean-abs {d.mean():.3e}")
        assert d.max() < MAX_ABS and d.mean() < MEAN_ABS, (b, d.max(), d.mean())
    say(f"{R} rows: worst max-abs {worst:.3e}")


def test_prefill_key_splits(hip, oracle):
    """kv800_hip_prefill_split: the same rows with the key range of every (query tile, KV head) split 1, 2, 5, 24 and
    64 ways (partials merged by log-sum-exp): each against float64 at the bar, and each within 4e-3 of the unsplit
    kernel (a split rescales its probabilities by its own running max before their bf16 rounding, so single outputs
    move by a few bf16 steps of the row's magnitude, not of their own)."""
    from lfm3_kv800_amd import vllm_cache as vc
    import lfm3_kv800_amd.kv800_hip as kh
    rng = np.random.RandomState(19)
    prev, new = [3000, 700, 0], [5, 40, 3]
    lens = [p + t for p, t in zip(prev, new)]
    K = [oracle.randn_bf16(rng, (n, 4, 128)) for n in lens]
    V = [oracle.randn_bf16(rng, (n, 4, 128)) for n in lens]
    cos, sin = oracle.rope_tables(max(lens) + 8)
    case = oracle.build_paged(lambda b, p0, p1: (K[b][p0:p1], V[b][p0:p1]), prev, ebs=64, shuffle_seed=19)
    P = upload(case)
    q = oracle.randn_bf16(rng, (sum(new), 16, 128))
    qsl = np.concatenate([[0], np.cumsum(new)]).astype(np.int64)
    kn = np.concatenate([K[b][prev[b]:] for b in range(3)])
    vn = np.concatenate([V[b][prev[b]:] for b in range(3)])
    args = vc.prefill_quant_inputs(P, to_dev_bf16(q), to_dev_bf16(kn), to_dev_bf16(vn), qsl, prev, to_dev_bf16(cos),
                                   to_dev_bf16(sin))
    want = []
    for b in range(3):
        n0, n = prev[b], lens[b]
        kb, vb = history_np(oracle, K[b], V[b], n0)
        kb = np.concatenate([kb, K[b][n0:n]]); vb = np.concatenate([vb, V[b][n0:n]])
        Kr = np.repeat(oracle.bf16_to_f32(rope_np(oracle, kb, np.arange(n), cos, sin)).astype(np.float64), 4, axis=1)
        Vf = np.repeat(oracle.bf16_to_f32(vb).astype(np.float64), 4, axis=1)
        qf = oracle.bf16_to_f32(q[qsl[b]:qsl[b + 1]]).astype(np.float64)
        sc = np.einsum("thd,shd->hts", qf, Kr) * 128 ** -0.5
        sc = np.where(np.arange(n)[None, None, :] <= np.arange(n0, n)[None, :, None], sc, -np.inf)
        w = np.exp(sc - sc.max(-1, keepdims=True)); w /= w.sum(-1, keepdims=True)
        want.append(np.einsum("hts,shd->thd", w, Vf))
    want = np.concatenate(want)
    # the assembled rows carry no position array (key j of a row is at position j): the same output, bit for bit, as
    # the explicit positions
    kp = torch.from_numpy(np.concatenate([np.arange(n) for n in lens]).astype(np.int32))
    assert args[5] is None
    explicit = kh.prefill(*args[:5], kp, args[6], window=0, splits=1)
    assert torch.equal(explicit.view(torch.int16), kh.prefill(*args, window=0, splits=1).view(torch.int16))
    base = None
    for splits in (1, 2, 5, 24, 64):
        say("prefill key splits", splits)
        out = kh.prefill(*args, window=0, splits=splits)
        o = torch.from_numpy(bits_of(out).view(np.int16)).view(torch.bfloat16).float().numpy()
        d = np.abs(o - want)
        say(f"splits {splits}: max-abs {d.max():.3e} mean-abs {d.mean():.3e}")
        assert np.isfinite(o).all() and d.max() < MAX_ABS and d.mean() < MEAN_ABS, (splits, d.max(), d.mean())
        if base is None:
            base = o
        dd = float(np.abs(o - base).max())
        say(f"splits {splits}: max |split - unsplit| {dd:.3e}")
        assert dd <= 4e-3, (splits, dd)
    assert kh.prefill_splits(3, 48) > 1                                   # the default for these rows splits


def test_prefill_quant_rows(hip, oracle):
    """Extend rows of a quantized layer: queries at positions n0 .. n-1 over the compressed history + new rows, against
    a float64 attention over the reference's assembled keys / values."""
    check_quant_rows(oracle, [700, 383, 1500], [37, 5, 64], 8)


def test_prefill_many_ragged_rows(hip, oracle):
    """41 rows: empty histories, rows with no new queries, 1..90 queries (a query-tile count whose grid is no multiple
    of the 8 XCDs), histories across and inside flush boundaries; and a call whose rows bring no queries at all."""
    rng = np.random.RandomState(77)
    prev = [int(x) for x in rng.randint(0, 1200, 41)]
    new = [int(x) for x in rng.randint(1, 91, 41)]
    prev[0], prev[5], prev[9] = 0, 0, 383
    new[3], new[17], new[30] = 0, 0, 0
    new[11], new[12] = 32, 33
    if sum((t + 31) // 32 for t in new) % 2 == 0:
        new[40] += 32                                 # an odd tile count: 4 x tiles workgroups, 4 left over per 8
    tiles = sum((t + 31) // 32 for t in new)
    assert (4 * tiles) % 8 != 0
    check_quant_rows(oracle, prev, new, 77)
    check_quant_rows(oracle, [0, 500], [0, 0], 78)


def upload_window(case):
    import lfm3_kv800_amd.kv800 as kv
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    return kv.Paged(qpool=to_dev_bf16(case.epool), boff=T(case.eoff), epool=to_dev_bf16(case.epool), eoff=T(case.eoff),
                    ebs=case.ebs, e_hs=case.e_hs, e_ts=case.e_ts, e_v=case.e_v, sk=to_dev_bf16(case.sk),
                    sv=to_dev_bf16(case.sv), skoff=T(case.skoff), svoff=T(case.svoff), N=T(case.N), NQ=T(case.NQ),
                    nqmax=0, win=case.win)


def test_prefill_window_rows(hip, oracle):
    """Extend rows of a window layer: queries at positions n0 .. n-1 over the sinks, the last 255 exact positions
    and the new rows, with the window + sinks mask (vllm_attn.py:351-402, 168-184), against a float64 attention over
    the same keys / values taken from the inputs (not from the pages)."""
    from lfm3_kv800_amd import vllm_cache as vc
    rng = np.random.RandomState(13)
    prev = [0, 3, 200, 256, 700, 1300]
    new = [6, 9, 70, 1, 300, 40]
    lens = [p + t for p, t in zip(prev, new)]
    K = [oracle.randn_bf16(rng, (n, 4, 128)) for n in lens]
    V = [oracle.randn_bf16(rng, (n, 4, 128)) for n in lens]
    cos, sin = oracle.rope_tables(1400)
    case = oracle.build_paged(lambda b, p0, p1: (K[b][p0:p1], V[b][p0:p1]), prev, win=256, ebs=64, shuffle_seed=6)
    P = upload_window(case)
    q = oracle.randn_bf16(rng, (sum(new), 16, 128))
    qsl = np.concatenate([[0], np.cumsum(new)])
    kn = np.concatenate([K[b][prev[b]:] for b in range(len(prev))])
    vn = np.concatenate([V[b][prev[b]:] for b in range(len(prev))])
    say("window prefill rows", prev, new)
    out = vc.prefill_window_rows(P, to_dev_bf16(q), to_dev_bf16(kn), to_dev_bf16(vn), qsl, prev, to_dev_bf16(cos),
                                 to_dev_bf16(sin))
    o = torch.from_numpy(bits_of(out).view(np.int16)).view(torch.bfloat16).float().numpy()
    W, NS = 256, 4
    for b in range(len(prev)):
        n0, n = prev[b], lens[b]
        lo = max(0, n0 - (W - 1))
        kp = np.concatenate([np.arange(min(NS, lo)), np.arange(lo, n)])
        Kr = oracle.bf16_to_f32(rope_np(oracle, K[b][kp], kp, cos, sin)).astype(np.float64)
        Vf = oracle.bf16_to_f32(V[b][kp]).astype(np.float64)
        qf = oracle.bf16_to_f32(q[qsl[b]:qsl[b + 1]]).astype(np.float64)
        Kr, Vf = np.repeat(Kr, 4, axis=1), np.repeat(Vf, 4, axis=1)
        sc = np.einsum("thd,shd->hts", qf, Kr) * 128 ** -0.5
        qp = np.arange(n0, n)[None, :, None]
        keep = (kp[None, None, :] <= qp) & ((kp[None, None, :] > qp - W) | (kp[None, None, :] < NS))
        sc = np.where(keep, sc, -np.inf)
        w = np.exp(sc - sc.max(-1, keepdims=True)); w /= w.sum(-1, keepdims=True)
        want = np.einsum("hts,shd->thd", w, Vf)
        d = np.abs(o[qsl[b]:qsl[b + 1]] - want)
        say(f"window row {b} (n0={n0}, {n - n0} new): max-abs {d.max():.3e} mean-abs {d.mean():.3e}")
        assert np.isfinite(o).all() and d.max() < MAX_ABS and d.mean() < MEAN_ABS, (b, d.max(), d.mean())


def test_rope_rows_bitexact(hip, oracle):
    """kv800_hip_rope_rows against vllm_attn.py:160-163 restated in numpy float32, bit for bit, on offset keys at
    random positions (signed zeros included)."""
    rng = np.random.RandomState(21)
    S = 3000
    k = oracle.randn_bf16(rng, (S, 4, 128), offset=3 * rng.standard_normal((1, 4, 128)))
    k[::97, 1, 40] = 0x8000                                   # -0.0 on a dim without a frequency
    k[::89, 2, 5] = 0x8000                                    # -0.0 on a rotating dim
    cos, sin = oracle.rope_tables(40000)
    pos = rng.randint(0, 40000, size=S).astype(np.int64)
    got = bits_of(hip.rope_rows(to_dev_bf16(k), torch.from_numpy(pos).to(DEV), to_dev_bf16(cos), to_dev_bf16(sin)))
    want = rope_np(oracle, k, pos, cos, sin)
    say("rope_rows", S, "rows, mismatches", int((got != want).sum()))
    assert np.array_equal(got, want)


def test_prefill_slide_rows(hip, oracle):
    """Extend rows of a native sliding layer: window 256 without sinks, keys stored after RoPE and used as stored
    (cos_t None), against a float64 attention over the same keys / values taken from the inputs."""
    from lfm3_kv800_amd import vllm_cache as vc
    import lfm3_kv800_amd.kv800 as kv
    rng = np.random.RandomState(17)
    prev = [0, 2, 255, 256, 900]
    new = [3, 40, 1, 77, 130]
    lens = [p + t for p, t in zip(prev, new)]
    K = [oracle.randn_bf16(rng, (n, 4, 128)) for n in lens]
    V = [oracle.randn_bf16(rng, (n, 4, 128)) for n in lens]
    case = oracle.build_paged(lambda b, p0, p1: (K[b][p0:p1], V[b][p0:p1]), prev, win=256, ebs=64, shuffle_seed=2,
                              sinks=False)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    P = kv.Paged(qpool=None, boff=None, epool=to_dev_bf16(case.epool), eoff=T(case.eoff), ebs=case.ebs, e_hs=case.e_hs,
                 e_ts=case.e_ts, e_v=case.e_v, sk=None, sv=None, skoff=None, svoff=None, N=T(case.N), NQ=T(case.NQ),
                 nqmax=0, win=256)
    q = oracle.randn_bf16(rng, (sum(new), 16, 128))
    qsl = np.concatenate([[0], np.cumsum(new)])
    kn = np.concatenate([K[b][prev[b]:] for b in range(len(prev))])
    vn = np.concatenate([V[b][prev[b]:] for b in range(len(prev))])
    say("slide prefill rows", prev, new)
    out = vc.prefill_window_rows(P, to_dev_bf16(q), to_dev_bf16(kn), to_dev_bf16(vn), qsl, prev, None, None)
    o = torch.from_numpy(bits_of(out).view(np.int16)).view(torch.bfloat16).float().numpy()
    W = 256
    for b in range(len(prev)):
        n0, n = prev[b], lens[b]
        kp = np.arange(max(0, n0 - (W - 1)), n)
        Kf = np.repeat(oracle.bf16_to_f32(K[b][kp]).astype(np.float64), 4, axis=1)
        Vf = np.repeat(oracle.bf16_to_f32(V[b][kp]).astype(np.float64), 4, axis=1)
        qf = oracle.bf16_to_f32(q[qsl[b]:qsl[b + 1]]).astype(np.float64)
        sc = np.einsum("thd,shd->hts", qf, Kf) * 128 ** -0.5
        qp = np.arange(n0, n)[None, :, None]
        sc = np.where((kp[None, None, :] <= qp) & (kp[None, None, :] > qp - W), sc, -np.inf)
        w = np.exp(sc - sc.max(-1, keepdims=True)); w /= w.sum(-1, keepdims=True)
        want = np.einsum("hts,shd->thd", w, Vf)
        d = np.abs(o[qsl[b]:qsl[b + 1]] - want)
        say(f"slide row {b} (n0={n0}, {n - n0} new): max-abs {d.max():.3e} mean-abs {d.mean():.3e}")
        assert np.isfinite(o).all() and d.max() < MAX_ABS and d.mean() < MEAN_ABS, (b, d.max(), d.mean())


def test_prefill_long_chunk(hip, oracle):
    """One 2048-query chunk over a 6,000-token quantized history (the reference's 2048-query prefill chunk): property
    checks at full size (finite, |out| <= max |V|), and 64 sampled queries against float64."""
    from lfm3_kv800_amd import vllm_cache as vc
    rng = np.random.RandomState(31)
    n0, t = 6000, 2048
    n = n0 + t
    K = oracle.randn_bf16(rng, (n, 4, 128))
    V = oracle.randn_bf16(rng, (n, 4, 128))
    cos, sin = oracle.rope_tables(n + 8)
    case = oracle.build_paged(lambda b, p0, p1: (K[p0:p1], V[p0:p1]), [n0], ebs=64, shuffle_seed=9)
    P = upload(case)
    q = oracle.randn_bf16(rng, (t, 16, 128))
    say("long prefill chunk", n0, t)
    out = vc.prefill_quant_rows(P, to_dev_bf16(q), to_dev_bf16(K[n0:]), to_dev_bf16(V[n0:]), [0, t], [n0],
                                to_dev_bf16(cos), to_dev_bf16(sin))
    o = torch.from_numpy(bits_of(out).view(np.int16)).view(torch.bfloat16).float().numpy()
    assert np.isfinite(o).all()
    kb, vb = history_np(oracle, K, V, n0)
    kb = np.concatenate([kb, K[n0:]]); vb = np.concatenate([vb, V[n0:]])
    Vf = oracle.bf16_to_f32(vb).astype(np.float64)
    assert np.abs(o).max() <= np.abs(Vf).max() + 1e-2
    Kr = np.repeat(oracle.bf16_to_f32(rope_np(oracle, kb, np.arange(n), cos, sin)).astype(np.float64), 4, axis=1)
    Vr = np.repeat(Vf, 4, axis=1)
    pick = np.sort(rng.choice(t, 64, replace=False))
    qf = oracle.bf16_to_f32(q[pick]).astype(np.float64)
    sc = np.einsum("thd,shd->hts", qf, Kr) * 128 ** -0.5
    sc = np.where(np.arange(n)[None, None, :] <= (n0 + pick)[None, :, None], sc, -np.inf)
    w = np.exp(sc - sc.max(-1, keepdims=True)); w /= w.sum(-1, keepdims=True)
    want = np.einsum("hts,shd->thd", w, Vr)
    d = np.abs(o[pick] - want)
    say(f"long chunk: max-abs {d.max():.3e} mean-abs {d.mean():.3e}")
    assert d.max() < MAX_ABS and d.mean() < MEAN_ABS
