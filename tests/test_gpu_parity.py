"""Parity of the HIP backend (through the C ABI) with the CPU oracle and the golden fixtures, on an MI355X.

Bars:
  * quantizer / flush / dequantizer: bit-exact with the oracle and the golden fixtures;
  * decode, every input (the benchmark configurations' N(0, 1) q / K / V, the reference's own 12 parity cases with K offset
    per channel by 3 N(0, 1) and q x 2, ragged batches, fp8 range edges): within 2e-2 max-abs and 1e-3 mean-abs of the
    oracle's restatement of torch_decode.py (both bf16 outputs, same cache bytes), a one-step rounding of a near-tie
    excepted (decode_bar.py states the rule and its margin), and for the 12 parity cases also the reference's own bar,
    rel < 1e-2 against its independent check (tests/test_parity.py:104)."""
import hashlib
import os

import numpy as np
import pytest
import torch

import decode_bar
import make_golden

pytestmark = pytest.mark.gpu

MAX_ABS, MEAN_ABS = 2e-2, 1e-3
DEV = "cuda"


def say(*a):
    print("[gpu-parity]", *a, flush=True)


def to_dev_bf16(bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).to(DEV)


def bits_of(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def upload(case):
    """oracle PagedCase (numpy) -> kv800.Paged on the GPU."""
    import lfm3_kv800_amd.kv800 as kv
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    return kv.Paged(qpool=T(case.qpool), boff=T(case.boff), epool=to_dev_bf16(case.epool), eoff=T(case.eoff),
                    ebs=case.ebs, e_hs=case.e_hs, e_ts=case.e_ts, e_v=case.e_v,
                    sk=to_dev_bf16(case.sk) if case.sinks else None, sv=to_dev_bf16(case.sv) if case.sinks else None,
                    skoff=T(case.skoff), svoff=T(case.svoff), N=T(case.N), NQ=T(case.NQ), nqmax=case.nqmax, win=case.win)


def download(P, oracle):
    """kv800.Paged on the GPU -> oracle PagedCase over the same bytes."""
    C = lambda t: t.detach().cpu().contiguous().numpy()
    sinks = P.sk is not None
    B = P.N.shape[0]
    zoff = np.zeros(B, np.int64)
    return oracle.PagedCase(qpool=C(P.qpool), boff=C(P.boff), epool=bits_of(P.epool), eoff=C(P.eoff), ebs=P.ebs,
                            e_hs=P.e_hs, e_ts=P.e_ts, e_v=P.e_v, sk=bits_of(P.sk) if sinks else np.zeros(1, np.uint16),
                            sv=bits_of(P.sv) if sinks else np.zeros(1, np.uint16),
                            skoff=C(P.skoff) if P.skoff is not None else zoff,
                            svoff=C(P.svoff) if P.svoff is not None else zoff, sinks=sinks, N=C(P.N), NQ=C(P.NQ),
                            nqmax=int(P.nqmax or 0), win=int(P.win or 0), B=B)


def close(out_bits, ref_bits, what):
    """Decode outputs against oracle.decode_f32's (bits, unrounded) pair: the shared decode bar (decode_bar.py);
    anything else against bf16 bits: 2e-2 max-abs, 1e-3 mean-abs."""
    if isinstance(ref_bits, tuple):
        decode_bar.check(out_bits, ref_bits, what, say)
        return
    o = torch.from_numpy(out_bits.view(np.int16)).view(torch.bfloat16).float().numpy()
    r = torch.from_numpy(ref_bits.view(np.int16)).view(torch.bfloat16).float().numpy()
    d = np.abs(o - r)
    say(f"{what}: max-abs {d.max():.3e} mean-abs {d.mean():.3e}")
    assert np.isfinite(o).all(), what
    assert d.max() < MAX_ABS and d.mean() < MEAN_ABS, (what, d.max(), d.mean())


# ---------------------------------------------------------------- quantizer / flush / dequantizer: bit-exact
@pytest.mark.parametrize("case", ["parity", "outlier", "edge", "scaled"])
def test_quantize_golden(hip, case):
    g = np.load(os.path.join(make_golden.HERE, "quantize_golden.npz"))
    kb, vb = make_golden.case_inputs(case)
    say("quantize golden", case, kb.shape)
    out = hip.quantize_blocks(to_dev_bf16(kb), to_dev_bf16(vb)).cpu().numpy()
    if case == "scaled":
        assert [hashlib.sha256(out[m].tobytes()).hexdigest() for m in range(out.shape[0])] == list(g["scaled_sha256"])
    else:
        want = g[f"{case}_out"]
        assert np.array_equal(out, want), f"{int((out != want).sum())} of {out.size} bytes differ"


@pytest.mark.parametrize("dist", ["normal", "offset", "outlier", "wide"])
def test_quantize_random_vs_oracle(hip, oracle, dist):
    rng = np.random.RandomState({"normal": 11, "offset": 12, "outlier": 13, "wide": 14}[dist])
    M = 24
    k = rng.standard_normal((M, 256, 4, 128)).astype(np.float32)
    v = rng.standard_normal((M, 256, 4, 128)).astype(np.float32)
    if dist == "offset":
        k += 3 * rng.standard_normal((1, 1, 4, 128)).astype(np.float32)
    if dist == "outlier":
        k[rng.random_sample(k.shape) < 0.01] *= 8
        v[rng.random_sample(v.shape) < 0.01] *= 8
    if dist == "wide":
        k *= np.exp2(rng.randint(-12, 6, size=(M, 1, 4, 128))).astype(np.float32)
        v *= np.exp2(rng.randint(-12, 6, size=(M, 256, 4, 1))).astype(np.float32)
    kb, vb = oracle.f32_to_bf16(k), oracle.f32_to_bf16(v)
    say("quantize random", dist, M)
    got = hip.quantize_blocks(to_dev_bf16(kb), to_dev_bf16(vb)).cpu().numpy()
    want = oracle.quantize_blocks(kb, vb)
    assert np.array_equal(got, want), f"{int((got != want).sum())} bytes differ"


@pytest.mark.parametrize("latency", [False, True])
def test_flush_two_kv_groups(hip, oracle, latency):
    """vLLM geometry: two exact KV groups (different shuffled block tables, ebs 128, [pages, 4, 128, 256] bf16) and one
    quant layer per group with 1280-token quant pages of 262,144 bytes. Each layer must gather from its own group's
    pages (the 0.1.1 fix, vllm_attn.py:301); reading the other group's table must give different bytes. Both flush
    kernels: the throughput one and the latency one of decode steps."""
    rng = np.random.RandomState(5)
    R, n_tok, ebs = 6, 2048 + 384, 128
    pages_per_row = (n_tok + ebs - 1) // ebs
    nq_new = np.array([(n_tok - 128) // 256 - r % 3 for r in range(R)], np.int32)     # ragged: 9, 8, 7 sub-blocks
    nq_prev = np.array([r % 2 for r in range(R)], np.int32)                             # some already flushed
    K = [oracle.randn_bf16(rng, (R, n_tok, 4, 128)) for _ in range(2)]
    V = [oracle.randn_bf16(rng, (R, n_tok, 4, 128)) for _ in range(2)]
    npages = R * pages_per_row + 3
    elems = 4 * ebs * 256
    tables, pools = [], []
    for gidx in range(2):
        perm = rng.permutation(npages)[:R * pages_per_row].reshape(R, pages_per_row)
        pool = np.zeros((npages, 4, ebs, 256), np.uint16)
        for r in range(R):
            for p in range(n_tok):
                pg = perm[r, p // ebs]
                pool[pg, :, p % ebs, :128] = K[gidx][r, p]
                pool[pg, :, p % ebs, 128:] = V[gidx][r, p]
        tables.append(perm.astype(np.int64))
        pools.append(pool)
    qpages = R * 2 + 2
    qperm = rng.permutation(qpages)[:R * 2].reshape(R, 2).astype(np.int64)
    outs = []
    for gidx in range(2):
        epool = to_dev_bf16(pools[gidx])
        eoff = torch.from_numpy(tables[gidx] * elems).to(DEV)
        qpool = torch.zeros(qpages * 262144, dtype=torch.uint8, device=DEV)
        say("flush group", gidx, "latency" if latency else "throughput")
        hip.flush(epool, eoff, ebs, ebs * 256, 256, 128, qpool, torch.from_numpy(qperm).to(DEV), 1280, 262144,
                  torch.from_numpy(nq_prev).to(DEV), torch.from_numpy(nq_new).to(DEV), int((nq_new - nq_prev).max()),
                  latency=latency)
        outs.append(qpool.cpu().numpy())
    for gidx in range(2):
        q = outs[gidx]
        for r in range(R):
            js = list(range(nq_prev[r], nq_new[r]))
            want = oracle.quantize_blocks(np.stack([K[gidx][r, 256 * j:256 * j + 256] for j in js]),
                                          np.stack([V[gidx][r, 256 * j:256 * j + 256] for j in js]))
            for i, j in enumerate(js):
                off = qperm[r, (256 * j) // 1280] * 262144 + ((256 * j) % 1280) // 256 * 51200
                assert np.array_equal(q[off:off + 51200], want[i]), (gidx, r, j)
                other = oracle.quantize_blocks(K[1 - gidx][r, 256 * j:256 * j + 256][None],
                                               V[1 - gidx][r, 256 * j:256 * j + 256][None])[0]
                assert not np.array_equal(q[off:off + 51200], other)
            for j in range(nq_prev[r]):                   # already-flushed sub-blocks are left untouched
                off = qperm[r, (256 * j) // 1280] * 262144 + ((256 * j) % 1280) // 256 * 51200
                assert not q[off:off + 51200].any()


def test_flush_c2_full_size(hip, oracle):
    """config C2 at full size: 64 sequences x a 2048-token chunk in vLLM-geometry exact pages (shuffled), K / V
    ~ N(0,1) with 1 % of the elements x 8, one flush launch into shuffled 1280-token quant pages: all 448 sub-blocks
    (the flush rule gives 7 per sequence) must equal the oracle quantizer's bytes."""
    B, n, ebs = 64, 2048, 128
    nq = (n - 128) // 256
    pages = n // ebs
    g = torch.Generator(device=DEV).manual_seed(21)
    x = torch.randn(B * pages, 4, ebs, 256, generator=g, device=DEV)
    x[torch.rand(x.shape, generator=g, device=DEV) < 0.01] *= 8
    epool = x.to(torch.bfloat16)
    del x
    perm = torch.randperm(B * pages, generator=g, device=DEV).view(B, pages)
    eoff = (perm * (4 * ebs * 256)).to(torch.int64)
    qpp = (nq * 256 + 1279) // 1280
    qbt = torch.randperm(B * qpp, generator=g, device=DEV).view(B, qpp).to(torch.int64)
    qpool = torch.zeros(B * qpp * 262144, dtype=torch.uint8, device=DEV)
    say("flush C2", B, "x", nq, "sub-blocks")
    hip.flush(epool, eoff, ebs, ebs * 256, 256, 128, qpool, qbt, 1280, 262144,
              torch.zeros(B, dtype=torch.int32, device=DEV), torch.full((B,), nq, dtype=torch.int32, device=DEV), nq)
    q = qpool.cpu().numpy()
    ep = bits_of(epool).reshape(B * pages, 4, ebs, 256)
    pm, qb = perm.cpu().numpy(), qbt.cpu().numpy()
    rows = ep[pm].transpose(0, 1, 3, 2, 4).reshape(B, pages * ebs, 4, 256)   # (row, token, head, K | V)
    want = oracle.quantize_blocks(np.ascontiguousarray(rows[:, :nq * 256, :, :128].reshape(B * nq, 256, 4, 128)),
                                  np.ascontiguousarray(rows[:, :nq * 256, :, 128:].reshape(B * nq, 256, 4, 128)))
    bad = 0
    for r in range(B):
        for j in range(nq):
            off = qb[r, (256 * j) // 1280] * 262144 + ((256 * j) % 1280) // 256 * 51200
            bad += not np.array_equal(q[off:off + 51200], want[r * nq + j])
    assert bad == 0, f"{bad} of {B * nq} sub-blocks differ"


def test_dequantize_vs_oracle(hip, oracle):
    kb, vb = make_golden.case_inputs("outlier")
    sb = oracle.quantize_blocks(kb, vb)
    say("dequantize", sb.shape)
    k, v = hip.dequantize_blocks(torch.from_numpy(sb).to(DEV))
    kw, vw = oracle.dequantize_blocks(sb)
    assert np.array_equal(bits_of(k), kw)
    assert np.array_equal(v.cpu().numpy().view(np.uint32), vw.view(np.uint32))


# ---------------------------------------------------------------- decode
QUANT_NS = (50, 383, 384, 700, 1500, 5000)
WINDOW_NS = (3, 10, 200, 259, 260, 1500)


@pytest.mark.parametrize("seed", [0, 1, 2])
@pytest.mark.parametrize("win,n", [(0, n) for n in QUANT_NS] + [(256, n) for n in WINDOW_NS])
def test_decode_reference_cases(hip, oracle, win, n, seed):
    """tests/test_parity.py's 12 cases (its run_case takes a seed, test_parity.py:80) at seeds 0, 1 and 2, through the
    product PagedStore (HIP flush) and kv800.decode."""
    import lfm3_kv800_amd.kv800 as kv
    import test_oracle as T
    q, K, V = T.parity_inputs(oracle, n, win, seed=seed)
    cos, sin = oracle.rope_tables(8192)
    say("decode case", win, n, "seed", seed)
    st = kv.PagedStore(2, n + 8, DEV, window=win)
    pre = max(1, n - 5)
    st.append(to_dev_bf16(K[:, :pre]), to_dev_bf16(V[:, :pre]))
    for i in range(pre, n):
        st.append(to_dev_bf16(K[:, i:i + 1]), to_dev_bf16(V[:, i:i + 1]))
    kv.set_backend("hip")
    try:
        out = kv.decode(st.paged(), to_dev_bf16(q), to_dev_bf16(cos), to_dev_bf16(sin), st.H)
        assert kv.get_backend() == "hip"
    finally:
        kv.set_backend(None)
    ob = bits_of(out)
    want = oracle.decode_f32(download(st.paged(), oracle), q, cos, sin)
    ref = oracle.reference_f64(q, K, V, cos, sin, window=win)
    o = oracle.bf16_to_f32(ob).astype(np.float64)
    rel = np.linalg.norm(o - ref) / np.linalg.norm(ref)
    say(f"win={win} n={n} seed={seed}: rel {rel:.2e} vs the independent check")
    assert rel < 1e-2
    close(ob, want, f"win={win} n={n} seed={seed} vs oracle")


@pytest.mark.parametrize("B,n", [(4, 1024), (2, 384), (3, 5000), (1, 9000)])
def test_decode_baseline_inputs(hip, oracle, B, n):
    """config C1 (B = 4, n = 1024, q / K / V ~ N(0, 1)) and other lengths, shuffled pages: the strict bar."""
    rng = np.random.RandomState(B * 1000 + n)
    K = oracle.randn_bf16(rng, (B, n, 4, 128)); V = oracle.randn_bf16(rng, (B, n, 4, 128))
    q = oracle.randn_bf16(rng, (B, 16, 128))
    cos, sin = oracle.rope_tables(n + 1)
    case = oracle.build_paged(lambda b, p0, p1: (K[b, p0:p1], V[b, p0:p1]), [n] * B, ebs=128, shuffle_seed=n)
    say("decode baseline inputs", B, n)
    out = hip.decode(upload(case), to_dev_bf16(q), to_dev_bf16(cos), to_dev_bf16(sin))
    close(bits_of(out), oracle.decode_f32(case, q, cos, sin), f"N(0,1) B={B} n={n}")


@pytest.mark.parametrize("win", [0, 256])
def test_decode_shuffled_ragged(hip, oracle, win):
    rng = np.random.RandomState(21 + win)
    lens = [1, 127, 128, 383, 384, 385, 700, 1024, 2311, 4096]
    K = [oracle.randn_bf16(rng, (n, 4, 128), offset=rng.standard_normal((1, 4, 128))) for n in lens]
    V = [oracle.randn_bf16(rng, (n, 4, 128)) for n in lens]
    q = oracle.randn_bf16(rng, (len(lens), 16, 128), scale=1.5)
    cos, sin = oracle.rope_tables(4200)
    case = oracle.build_paged(lambda b, p0, p1: (K[b][p0:p1], V[b][p0:p1]), lens, win=win, ebs=128, shuffle_seed=9)
    say("decode ragged", win, lens)
    P = upload(case)
    want = oracle.decode_f32(case, q, cos, sin)
    # fixed grids (spb) and balanced schedules: one workgroup over every row, 5 groups (ranges that start and end
    # inside rows), and more groups than sub-blocks (most workgroups empty)
    for spb, groups in ((None, None), (1, None), (3, None), (None, 1), (None, 5), (None, 2000)):
        out = hip.decode(P, to_dev_bf16(q), to_dev_bf16(cos), to_dev_bf16(sin), spb=spb, groups=groups)
        close(bits_of(out), want, f"ragged win={win} spb={spb} groups={groups}")


@pytest.mark.parametrize("B", [128, 129])
def test_decode_window_either_side_of_one_wave_switch(hip, oracle, B):
    """Window + sinks layer at the two batch sizes either side of the exact kernel's switch from 4-wave workgroups per
    (row, KV head) to one-wave workgroups (4 B workgroups against one resident round, 512 on MI355X): ragged rows
    (empty-window, sink-only and just-full rows among them), shuffled pages, every row against the oracle."""
    rng = np.random.RandomState(400 + B)
    lens = rng.randint(1, 700, size=B)
    lens[:5] = [1, 4, 5, 260, 261]
    K = [oracle.randn_bf16(rng, (int(n), 4, 128), offset=rng.standard_normal((1, 4, 128))) for n in lens]
    V = [oracle.randn_bf16(rng, (int(n), 4, 128)) for n in lens]
    q = oracle.randn_bf16(rng, (B, 16, 128), scale=1.5)
    cos, sin = oracle.rope_tables(704)
    case = oracle.build_paged(lambda b, p0, p1: (K[b][p0:p1], V[b][p0:p1]), lens, win=256, ebs=128,
                              shuffle_seed=B)
    say("decode window", B, "rows")
    P = upload(case)
    want = oracle.decode_f32(case, q, cos, sin)
    out = hip.decode(P, to_dev_bf16(q), to_dev_bf16(cos), to_dev_bf16(sin))
    close(bits_of(out), want, f"window B={B}")


def test_decode_many_rows_few_groups(hip, oracle):
    """Balanced schedule with few workgroups over 150 ragged rows: a single workgroup (one slice per row), slices that
    start and end inside rows, rows without quantized sub-blocks between them."""
    rng = np.random.RandomState(57)
    lens = [int(x) for x in rng.randint(1, 1400, size=150)]
    lens[10:20] = [1, 2, 127, 128, 129, 383, 384, 385, 639, 640]
    K = [oracle.randn_bf16(rng, (n, 4, 128)) for n in lens]
    V = [oracle.randn_bf16(rng, (n, 4, 128)) for n in lens]
    q = oracle.randn_bf16(rng, (len(lens), 16, 128))
    cos, sin = oracle.rope_tables(1500)
    case = oracle.build_paged(lambda b, p0, p1: (K[b][p0:p1], V[b][p0:p1]), lens, ebs=128, shuffle_seed=57)
    say("decode many rows", len(lens), "sub-blocks", int(case.NQ.sum()))
    P = upload(case)
    want = oracle.decode_f32(case, q, cos, sin)
    for groups in (1, 2, 7, None):
        out = hip.decode(P, to_dev_bf16(q), to_dev_bf16(cos), to_dev_bf16(sin), groups=groups)
        close(bits_of(out), want, f"150 rows groups={groups}")


def test_decode_list_wise_cut(hip, oracle):
    """The balanced schedule's list-wise cut: 700 rows of 0-3 sub-blocks with group counts whose row-wise cut needs
    two rounds of the 512 resident workgroups and the list-wise cut one, so the list-wise cut runs: workgroups whose
    sub-blocks span 2 (groups 400) or ~7 rows (groups 97), each row segment its own partial, rows entered from an
    earlier workgroup and rows without sub-blocks on the way."""
    rng = np.random.RandomState(83)
    lens = [int(x) for x in rng.randint(380, 1100, size=700)]
    lens[::37] = [int(x) for x in rng.randint(1, 384, size=len(lens[::37]))]
    K = [oracle.randn_bf16(rng, (n, 4, 128)) for n in lens]
    V = [oracle.randn_bf16(rng, (n, 4, 128)) for n in lens]
    q = oracle.randn_bf16(rng, (len(lens), 16, 128))
    cos, sin = oracle.rope_tables(1200)
    case = oracle.build_paged(lambda b, p0, p1: (K[b][p0:p1], V[b][p0:p1]), lens, ebs=128, shuffle_seed=83)
    say("decode 700 rows list-wise, sub-blocks", int(case.NQ.sum()))
    P = upload(case)
    want = oracle.decode_f32(case, q, cos, sin)
    for groups in (400, 97):
        out = hip.decode(P, to_dev_bf16(q), to_dev_bf16(cos), to_dev_bf16(sin), groups=groups)
        close(bits_of(out), want, f"700 rows groups={groups}")


def test_decode_batch_over_1024_rows(hip, oracle):
    """Balanced schedule with more than 1024 rows: each scan thread owns 5 rows, more than it keeps in registers, so
    the later rows' counts are read again; rows with no quantized sub-block among them."""
    rng = np.random.RandomState(71)
    lens = [int(x) for x in rng.randint(1, 520, size=1100)]
    K = [oracle.randn_bf16(rng, (n, 4, 128)) for n in lens]
    V = [oracle.randn_bf16(rng, (n, 4, 128)) for n in lens]
    q = oracle.randn_bf16(rng, (len(lens), 16, 128))
    cos, sin = oracle.rope_tables(1000)
    case = oracle.build_paged(lambda b, p0, p1: (K[b][p0:p1], V[b][p0:p1]), lens, ebs=64, shuffle_seed=71)
    say("decode 1100 rows, sub-blocks", int(case.NQ.sum()))
    P = upload(case)
    want = oracle.decode_f32(case, q, cos, sin)
    for groups in (None, 5):
        out = hip.decode(P, to_dev_bf16(q), to_dev_bf16(cos), to_dev_bf16(sin), groups=groups)
        close(bits_of(out), want, f"1100 rows groups={groups}")


def test_decode_stages_and_merge(hip, oracle):
    rng = np.random.RandomState(31)
    lens = [900, 3000, 1500]
    K = [oracle.randn_bf16(rng, (n, 4, 128)) for n in lens]
    V = [oracle.randn_bf16(rng, (n, 4, 128)) for n in lens]
    q = oracle.randn_bf16(rng, (3, 16, 128))
    cos, sin = oracle.rope_tables(3100)
    case = oracle.build_paged(lambda b, p0, p1: (K[b][p0:p1], V[b][p0:p1]), lens, shuffle_seed=4)
    say("decode stages")
    P = upload(case)
    out, MO, LO, AO, ns = hip.decode_parts(P, to_dev_bf16(q), to_dev_bf16(cos), to_dev_bf16(sin), spb=2)
    assert ns == 6
    merged = oracle.combine(MO.cpu().numpy(), LO.cpu().numpy(), AO.cpu().numpy(), ns)
    close(bits_of(out), merged, "HIP merge vs oracle combine of the same partials")
    close(bits_of(out), oracle.decode_f32(case, q, cos, sin), "staged decode vs oracle")
    fused = hip.decode(P, to_dev_bf16(q), to_dev_bf16(cos), to_dev_bf16(sin), spb=2)
    assert torch.equal(fused, out)


def test_decode_merge_many_partials(hip, oracle):
    """The merge with more partials per row than its 16 lane groups take in one memory round trip (the fixed grid at
    one sub-block per split: 77 and 33 quantized partials), against the oracle's combine of the same partials; then
    single long rows through the balanced plan, which cuts a batch that fills under half a resident round into one
    sub-block per workgroup (a 32K row: 127 slices)."""
    rng = np.random.RandomState(43)
    lens = [20000, 8600]
    K = [oracle.randn_bf16(rng, (n, 4, 128)) for n in lens]
    V = [oracle.randn_bf16(rng, (n, 4, 128)) for n in lens]
    q = oracle.randn_bf16(rng, (2, 16, 128))
    cos, sin = oracle.rope_tables(max(lens) + 1)
    case = oracle.build_paged(lambda b, p0, p1: (K[b][p0:p1], V[b][p0:p1]), lens, shuffle_seed=43)
    say("decode merge of many partials", lens)
    P = upload(case)
    out, MO, LO, AO, ns = hip.decode_parts(P, to_dev_bf16(q), to_dev_bf16(cos), to_dev_bf16(sin), spb=1)
    assert ns == 77
    merged = oracle.combine(MO.cpu().numpy(), LO.cpu().numpy(), AO.cpu().numpy(), ns)
    close(bits_of(out), merged, "HIP merge of 77 partials vs oracle combine")
    close(bits_of(out), oracle.decode_f32(case, q, cos, sin), "77 splits vs oracle")
    res = hip.plan_balanced(64, 127)                     # one round of resident workgroups
    assert hip.plan_balanced(1, 127) == 127 and hip.plan_balanced(2, 127) == 254
    assert hip.plan_balanced(4, 127) == (508 + 1) // 2 and hip.plan_balanced(16, 127) == min(res, 508)
    n = 32768
    K1 = oracle.randn_bf16(rng, (1, n, 4, 128)); V1 = oracle.randn_bf16(rng, (1, n, 4, 128))
    q1 = oracle.randn_bf16(rng, (1, 16, 128))
    cos, sin = oracle.rope_tables(n + 1)
    case1 = oracle.build_paged(lambda b, p0, p1: (K1[b, p0:p1], V1[b, p0:p1]), [n], ebs=128, shuffle_seed=44)
    say("decode one 32K row, plan", hip.plan_balanced(1, int(case1.nqmax)))
    out1 = hip.decode(upload(case1), to_dev_bf16(q1), to_dev_bf16(cos), to_dev_bf16(sin))
    close(bits_of(out1), oracle.decode_f32(case1, q1, cos, sin), "one 32K row, one sub-block per workgroup")


def test_decode_full_size_all_rows(hip, oracle):
    """config C3 at full size (64 x 32,768, permuted tables): cache built on the GPU by the HIP quantizer,
    decoded by the HIP kernels; every row is decoded again by the oracle from the downloaded pages (the strict bar), and
    every output is finite and within the range of its row's dequantized values."""
    import lfm3_kv800_amd.kv800 as kv
    B, n, ebs = 64, 32768, 128
    nq = (n - 128) // 256
    g = torch.Generator(device=DEV).manual_seed(3)
    say("full size: building", B, n)
    qperm = torch.randperm(B * nq, generator=g, device=DEV)
    boff = (qperm.view(B, nq) * 51200).to(torch.int64)
    qpool = torch.empty(B * nq * 51200, dtype=torch.uint8, device=DEV)
    for b0 in range(0, B, 8):
        k = torch.randn(8 * nq, 256, 4, 128, generator=g, device=DEV).to(torch.bfloat16)
        v = torch.randn(8 * nq, 256, 4, 128, generator=g, device=DEV).to(torch.bfloat16)
        sb = hip.quantize_blocks(k, v)
        dst = boff[b0:b0 + 8].reshape(-1)[:, None] + torch.arange(51200, device=DEV)
        qpool[dst.reshape(-1)] = sb.reshape(-1)
    pages = (n + ebs - 1) // ebs
    ex0 = nq * 256 // ebs
    npg = B * (pages - ex0)
    eperm = torch.randperm(npg, generator=g, device=DEV).view(B, pages - ex0)
    eoff = torch.zeros(B, pages, dtype=torch.int64, device=DEV)
    eoff[:, ex0:] = eperm * (4 * ebs * 256)
    epool = torch.randn(npg, 4, ebs, 256, generator=g, device=DEV).to(torch.bfloat16)
    N = torch.full((B,), n, dtype=torch.int32, device=DEV)
    NQ = torch.full((B,), nq, dtype=torch.int32, device=DEV)
    P = kv.Paged(qpool=qpool, boff=boff, epool=epool, eoff=eoff, ebs=ebs, e_hs=ebs * 256, e_ts=256, e_v=128,
                 sk=None, sv=None, skoff=None, svoff=None, N=N, NQ=NQ, nqmax=nq, win=0)
    q = torch.randn(B, 16, 128, generator=g, device=DEV).to(torch.bfloat16)
    cos, sin = oracle.rope_tables(n)
    say("full size: decode")
    out = hip.decode(P, q, to_dev_bf16(cos), to_dev_bf16(sin))
    torch.cuda.synchronize()
    o = out.float()
    assert bool(torch.isfinite(o).all())
    # |out| <= max |V| over the row's tokens, per KV head: V of the quantized sub-blocks through the dequantizer, and
    # the exact tail from its pages
    for b in range(B):
        sbs = qpool[(boff[b][:, None] + torch.arange(51200, device=DEV)).reshape(-1)].view(nq, 51200)
        _, vq = hip.dequantize_blocks(sbs)
        vmax = vq.abs().amax(dim=(0, 1, 3))                                           # (4,)
        tail = epool.view(-1)[(eoff[b, ex0:][:, None] + torch.arange(4 * ebs * 256, device=DEV)).reshape(-1)]
        vmax = torch.maximum(vmax, tail.view(-1, 4, ebs, 256)[..., 128:].float().abs().amax(dim=(0, 2, 3)))
        omax = o[b].abs().view(4, 4, 128).amax(dim=(1, 2))
        assert bool((omax <= vmax * (1 + 2 ** -7)).all()), (b, omax.tolist(), vmax.tolist())
    case = download(P, oracle)
    say("full size: oracle, all", B, "rows")
    want = oracle.decode_f32(case, bits_of(q), cos, sin)
    close(bits_of(out), want, "64x32768 all rows")


def test_rope_pairs_cache_follows_tables(hip, oracle):
    """The packed RoPE pair table is cached per (cos, sin) tensor pair: a different table of the same shape built after
    the first one is dropped, and a table rewritten in place, are each decoded with their own values."""
    rng = np.random.RandomState(44)
    lens = [1500, 900]
    K = [oracle.randn_bf16(rng, (n, 4, 128)) for n in lens]
    V = [oracle.randn_bf16(rng, (n, 4, 128)) for n in lens]
    q = oracle.randn_bf16(rng, (2, 16, 128))
    case = oracle.build_paged(lambda b, p0, p1: (K[b][p0:p1], V[b][p0:p1]), lens, ebs=128, shuffle_seed=44)
    P = upload(case)
    ca, sa = oracle.rope_tables(1600, theta=1e6)
    cb, sb = oracle.rope_tables(1600, theta=1e4)
    say("rope pair cache: table A, then B, then B rewritten as A")
    cos, sin = to_dev_bf16(ca), to_dev_bf16(sa)
    close(bits_of(hip.decode(P, to_dev_bf16(q), cos, sin)), oracle.decode_f32(case, q, ca, sa), "table A")
    del cos, sin
    torch.cuda.synchronize()
    cos, sin = to_dev_bf16(cb), to_dev_bf16(sb)
    close(bits_of(hip.decode(P, to_dev_bf16(q), cos, sin)), oracle.decode_f32(case, q, cb, sb), "table B after A")
    cos.copy_(to_dev_bf16(ca)); sin.copy_(to_dev_bf16(sa))
    close(bits_of(hip.decode(P, to_dev_bf16(q), cos, sin)), oracle.decode_f32(case, q, ca, sa), "B rewritten in place")
