"""Mixed prefill + decode steps of the vLLM-geometry cache path (vllm_cache.KV800DecodeLayer / KV800SlideLayer with
mixed_step_meta, the counterpart of KV800Attention.forward, vllm_attn.py:244-402) on an MI355X.

Three steps over 9 rows, every row's K / V history known on the host:
  A  prefill: all rows are extend rows starting at position 0 (1 .. 2300 tokens);
  B  mixed: rows 0-5 decode one token (rows 0 and 3 cross a flush boundary, row 2 writes a sink), rows 6-8 extend by
     37, 1100 (from position 3: it writes the last sink) and 2300 tokens (nine sub-blocks become eligible);
  C  decode: every row one token.
Layers: window + sinks 2 (exact group A, sinks in the aux of 6 (K) and 10 (V)), quantized 6 (exact group A) and 10
(exact group B: the 0.1.1 multi-group flush), native sliding 4 (its own group, post-RoPE keys). After each step:
  * every exact page and every quant page (sub-blocks and aux) equals the pools built on the host from the histories,
    byte for byte: sub-block j of a row is the oracle quantizer's bytes of positions [256 j, 256 j + 256) for every
    j < nq(seq_len), nothing else was written;
  * decode rows are within 2e-2 max-abs / 1e-3 mean-abs of the oracle's torch_decode over a cache built
    independently from the same history (near-tie roundings excepted: decode_bar.py);
  * extend rows are within the same bar of a float64 attention over the keys the reference assembles for them
    (vllm_attn.py:351-402): quantized layers their nq(prev) dequantized sub-blocks, the exact rows from 256 nq(prev)
    on and the new rows; window layers the sinks, the last 255 positions and the new rows; sampled queries on long
    rows."""
import numpy as np
import pytest
import torch

import decode_bar

from test_gpu_prefill import history_np, rope_np

pytestmark = pytest.mark.gpu

DEV = "cuda"
EBS, QBLOCK, QPAGE, AUX = 128, 1280, 262144, 256000
MAX_ABS, MEAN_ABS = 2e-2, 1e-3
LAYERS = (2, 6, 10, 4)
GROUP = {2: "A", 6: "A", 10: "B", 4: "C"}


def say(*a):
    print("[gpu-mixed]", *a, flush=True)


def bf16_dev(bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).to(DEV)


def bits_of(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def as_f32(bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).float().numpy()


def nq_of(n):
    return max(0, int(n) - 128) // 256


def attention64(qf, Kf, Vf, kp, qp, keep):
    """float64 softmax attention of queries (t, 16, 128) at positions qp over keys (s, 4, 128) at kp; keep(kp, qp)
    -> bool (t, s) mask."""
    Kr, Vr = np.repeat(Kf, 4, axis=1), np.repeat(Vf, 4, axis=1)
    sc = np.einsum("thd,shd->hts", qf, Kr) * 128 ** -0.5
    sc = np.where(keep(kp[None, :], qp[:, None])[None], sc, -np.inf)
    w = np.exp(sc - sc.max(-1, keepdims=True))
    w /= w.sum(-1, keepdims=True)
    return np.einsum("hts,shd->thd", w, Vr)


def test_mixed_prefill_decode_steps(hip, oracle):
    from lfm3_kv800_amd import vllm_cache as vc
    rng = np.random.RandomState(2024)
    A = np.array([1407, 999, 2, 383, 2300, 1663, 700, 3, 1500], np.int64)      # step A: prompt chunks from 0
    B_new = np.array([1, 1, 1, 1, 1, 1, 37, 1100, 2300], np.int64)              # step B: 6 decode + 3 extend rows
    steps = [(np.zeros(9, np.int64), A, 0), (A, B_new, 6), (A + B_new, np.ones(9, np.int64), 9)]
    R = 9
    nmax = int((A + B_new + 1).max())
    hist = {l: (oracle.randn_bf16(rng, (R, nmax, 4, 128), offset=rng.standard_normal((1, 1, 4, 128))),
                oracle.randn_bf16(rng, (R, nmax, 4, 128))) for l in LAYERS}
    cos, sin = oracle.rope_tables(nmax + 8)
    cos_d, sin_d = bf16_dev(cos), bf16_dev(sin)

    # block tables: every logical page of a row its own shuffled physical page, exact groups A / B / C, quant group Q
    epr, qpr = nmax // EBS + 1, nmax // QBLOCK + 1
    bt = {g: rng.permutation(R * epr + 7)[:R * epr].reshape(R, epr).astype(np.int32) for g in "ABC"}
    qbt = rng.permutation(R * qpr + 3)[:R * qpr].reshape(R, qpr).astype(np.int32)
    ev = {l: torch.zeros(R * epr + 7, 4, EBS, 256, dtype=torch.bfloat16, device=DEV) for l in LAYERS}
    qv = {l: torch.zeros(R * qpr + 3, QPAGE, dtype=torch.uint8, device=DEV) for l in (6, 10)}
    lay = {l: (vc.KV800SlideLayer(l, ev[l]) if l == 4 else vc.KV800DecodeLayer(l, ev[l], qv.get(l))) for l in LAYERS}

    for si, (prev, new, nd) in enumerate(steps):
        n = prev + new
        say(f"step {'ABC'[si]}: prev {prev.tolist()} new {new.tolist()} decode rows {nd}")
        me = {g: vc.mixed_step_meta(torch.from_numpy(bt[g]), torch.from_numpy(n), torch.from_numpy(new), EBS, DEV,
                                    num_decodes=nd) for g in "ABC"}
        mq = vc.mixed_step_meta(torch.from_numpy(qbt), torch.from_numpy(n), torch.from_numpy(new), QBLOCK, DEV,
                                num_decodes=nd)
        qsl = np.concatenate([[0], np.cumsum(new)])
        T = int(qsl[-1])
        rows_tok = np.repeat(np.arange(R), new)
        pos_tok = np.concatenate([np.arange(p, p + c) for p, c in zip(prev, new)])
        q = {l: oracle.randn_bf16(rng, (T, 16, 128)) for l in LAYERS}
        outs = {}
        for l in LAYERS:
            K, V = hist[l]
            kn, vn = bf16_dev(K[rows_tok, pos_tok]), bf16_dev(V[rows_tok, pos_tok])
            if l == 4:
                o = lay[l].forward(bf16_dev(q[l]), kn, vn, me[GROUP[l]])
            else:
                o = lay[l].forward(bf16_dev(q[l]), kn, vn, me[GROUP[l]], mq, hosts=lay, cos_t=cos_d, sin_t=sin_d)
            outs[l] = as_f32(bits_of(o))
        torch.cuda.synchronize()

        # ---- pools, byte for byte
        for l in LAYERS:
            K, V = hist[l]
            want = np.zeros((R * epr + 7, 4, EBS, 256), np.uint16)
            for r in range(R):
                for p0 in range(0, int(n[r]), EBS):
                    p1 = min(int(n[r]), p0 + EBS)
                    pg = bt[GROUP[l]][r, p0 // EBS]
                    want[pg, :, :p1 - p0, :128] = K[r, p0:p1].transpose(1, 0, 2)
                    want[pg, :, :p1 - p0, 128:] = V[r, p0:p1].transpose(1, 0, 2)
            assert np.array_equal(bits_of(ev[l]).reshape(want.shape), want), ("exact pages", l)
        for l in (6, 10):
            K, V = hist[l]
            want = np.zeros((R * qpr + 3, QPAGE), np.uint8)
            for r in range(R):
                m = nq_of(n[r])
                if m:
                    sb = oracle.quantize_blocks(K[r, :256 * m].reshape(m, 256, 4, 128),
                                                V[r, :256 * m].reshape(m, 256, 4, 128))
                    for j in range(m):
                        off = (256 * j) % QBLOCK // 256 * 51200
                        want[qbt[r, 256 * j // QBLOCK], off:off + 51200] = sb[j]
                sinks = hist[2][0] if l == 6 else hist[2][1]            # layer 2's sink K in 6's aux, V in 10's
                for p in range(min(4, int(n[r]))):
                    want[qbt[r, 0]].view(np.uint16)[AUX // 2 + p * 512:AUX // 2 + (p + 1) * 512] = sinks[r, p].reshape(-1)
            got = qv[l].cpu().numpy()
            bad = np.argwhere((got != want).any(axis=1)).ravel()
            assert bad.size == 0, ("quant pages", l, bad[:8])
        say(f"step {'ABC'[si]}: exact and quant pools equal the host-built pools")

        # ---- decode rows against the oracle's torch_decode
        for l in LAYERS:
            if nd == 0:
                break
            K, V = hist[l]
            win = 256 if l in (2, 4) else 0
            case = oracle.build_paged(lambda b, p0, p1: (K[b, p0:p1], V[b, p0:p1]), list(n[:nd]), win=win, ebs=EBS,
                                      shuffle_seed=l, sinks=l != 4)
            if l == 4:
                cs = oracle.f32_to_bf16(np.ones_like(oracle.bf16_to_f32(cos)))
                sn = np.zeros_like(sin)
            else:
                cs, sn = cos, sin
            decode_bar.check(outs[l][:nd], oracle.decode_f32(case, q[l][:nd], cs, sn),
                             f"step {'ABC'[si]} layer {l} decode rows", say)

        # ---- extend rows against float64 attention over the keys the reference assembles
        for l in LAYERS:
            K, V = hist[l]
            for r in range(nd, R):
                n0, n1 = int(prev[r]), int(n[r])
                t0 = int(qsl[r])
                pick = np.arange(n1 - n0)
                if pick.size > 96:
                    pick = np.unique(np.concatenate([[0, pick.size - 1], rng.choice(pick.size, 94, replace=False)]))
                qp = n0 + pick
                qf = as_f32(q[l][t0 + pick]).astype(np.float64)
                if l in (6, 10):
                    kb, vb = history_np(oracle, K[r], V[r], n0)
                    kb = np.concatenate([kb, K[r, n0:n1]])
                    vb = np.concatenate([vb, V[r, n0:n1]])
                    kp = np.arange(n1)
                    Kf = as_f32(rope_np(oracle, kb, kp, cos, sin)).astype(np.float64)
                    keep = lambda a, b: a <= b
                else:
                    lo = max(0, n0 - 255)
                    ns = min(4, lo) if l == 2 else 0
                    kp = np.concatenate([np.arange(ns), np.arange(lo, n1)])
                    kb, vb = K[r, kp], V[r, kp]
                    Kf = as_f32(rope_np(oracle, kb, kp, cos, sin) if l == 2 else kb).astype(np.float64)
                    keep = ((lambda a, b: (a <= b) & ((a > b - 256) | (a < 4))) if l == 2
                            else (lambda a, b: (a <= b) & (a > b - 256)))
                want = attention64(qf, Kf, as_f32(vb).astype(np.float64), kp, qp, keep)
                got = outs[l][t0 + pick]
                d = np.abs(got - want)
                say(f"step {'ABC'[si]} layer {l} extend row {r} ({n0} + {n1 - n0}, {pick.size} queries): "
                    f"max-abs {d.max():.3e} mean-abs {d.mean():.3e}")
                assert np.isfinite(got).all() and d.max() < MAX_ABS and d.mean() < MEAN_ABS, (l, r, d.max(), d.mean())


def test_mixed_step_meta_and_tables(hip):
    """mixed_step_meta's slots / positions / token rows against their definitions, and kv800_hip_step_tables with
    per-row new-token counts: NP = nq(seq_len - query_len)."""
    from lfm3_kv800_amd import vllm_cache as vc
    g = torch.Generator().manual_seed(9)
    R, pages, ebs = 6, 40, 128
    bt = torch.randperm(R * pages + 3, generator=g)[:R * pages].view(R, pages).to(torch.int32)
    sl = torch.tensor([1, 385, 1408, 700, 3800, 2], dtype=torch.int64)
    ql = torch.tensor([1, 1, 1, 300, 2300, 2], dtype=torch.int64)
    m = vc.mixed_step_meta(bt, sl, ql, ebs, DEV)
    assert m.num_decodes == 3 and m.mixed
    pos = torch.cat([torch.arange(a - b, a) for a, b in zip(sl.tolist(), ql.tolist())])
    req = torch.repeat_interleave(torch.arange(R), ql)
    assert torch.equal(m.positions.cpu(), pos) and torch.equal(m.req_of_tok.cpu(), req)
    assert torch.equal(m.slot_mapping.cpu(), bt[req, pos // ebs].long() * ebs + pos % ebs)
    assert torch.equal(m.query_start_loc_cpu, torch.cat([torch.zeros(1, dtype=torch.int64), ql.cumsum(0)]))
    qbt = torch.randperm(R * 4 + 1, generator=g)[:R * 4].view(R, 4).to(torch.int32)
    nqmax = int(((sl - 128).clamp(min=0) // 256).max())
    boff, NQ, NP, qbt64, aux = hip.step_tables(qbt.to(DEV), 1280, 262144, sl.to(torch.int32).to(DEV), nqmax,
                                                nnew=ql.to(torch.int32).to(DEV))
    nq = lambda x: (x - 128).clamp(min=0) // 256
    assert torch.equal(NQ.cpu(), nq(sl).to(torch.int32)) and torch.equal(NP.cpu(), nq(sl - ql).to(torch.int32))
    assert vc._max_flush(m) == int((nq(sl) - nq(sl - ql)).max())
    with pytest.raises(ValueError):
        vc.mixed_step_meta(bt, sl, ql, ebs, DEV, num_decodes=4)          # row 3 has 300 tokens
    with pytest.raises(ValueError):
        vc.mixed_step_meta(bt, torch.tensor([5]), torch.tensor([6]), ebs, DEV)
