"""One decode step of the vLLM-geometry cache path (lfm3-kv800_amd/vllm_cache.py, the counterpart of
vllm_attn.py:214-350) on an MI355X, checked against the CPU oracle.

Setup: ragged rows whose step crosses flush boundaries (n = 256 j + 384) on some rows and writes a sink (position < 4)
on another; exact caches of 128-token pages in two exact KV groups (layers 2, 6 share one block table, layer 10 has
its own: the 0.1.1 multi-group case), one quant KV group of 1280-token pages for layers 6 and 10, all page tables
shuffled; window layer 2 keeps its sinks in the aux area of layers 6 (K) and 10 (V). After the step:
  * the step's K / V rows sit at their slots, and the sink rows in the hosts' aux (bit-exact);
  * every sub-block that became eligible was flushed from the layer's own exact group, bit-exact with the oracle
    quantizer, and no other quant sub-block changed;
  * each layer's decode output is within 2e-2 max-abs / 1e-3 mean-abs of the oracle's torch_decode over a cache built
    independently from the rows' full K / V history (near-tie roundings excepted: decode_bar.py)."""
import numpy as np
import pytest
import torch

import decode_bar

pytestmark = pytest.mark.gpu

DEV = "cuda"
EBS, QBLOCK, QPAGE, AUX = 128, 1280, 262144, 256000
MAX_ABS, MEAN_ABS = 2e-2, 1e-3


def say(*a):
    print("[gpu-vllm]", *a, flush=True)


def bf16_dev(bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).to(DEV)


def bits_of(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("early_flush", [False, True])
def test_vllm_decode_step(hip, oracle, early_flush):
    from lfm3_kv800_amd import vllm_cache as vc
    rng = np.random.RandomState(77)
    L0 = np.array([1407, 999, 2, 383, 3000, 1663], np.int64)   # lengths before the step
    n = L0 + 1
    R, nmax = len(L0), int(n.max())
    layers = (2, 6, 10)
    hist = {l: (oracle.randn_bf16(rng, (R, nmax, 4, 128)), oracle.randn_bf16(rng, (R, nmax, 4, 128))) for l in layers}
    q = {l: oracle.randn_bf16(rng, (R, 16, 128)) for l in layers}
    cos, sin = oracle.rope_tables(4096)

    # ---- block tables: exact groups A (layers 2, 6) and B (layer 10), quant group Q (layers 6, 10)
    epr = nmax // EBS + 1
    qpr = nmax // QBLOCK + 1
    bt = {g: rng.permutation(R * epr + 5)[:R * epr].reshape(R, epr).astype(np.int32) for g in "AB"}
    qbt = rng.permutation(R * qpr + 3)[:R * qpr].reshape(R, qpr).astype(np.int32)
    group = {2: "A", 6: "A", 10: "B"}
    nq_prev = np.maximum(L0 - 128, 0) // 256
    nq_new = np.maximum(n - 128, 0) // 256
    say("rows", list(n), "flushes", int((nq_new - nq_prev).sum()))

    # ---- caches before the step: history positions [0, L0) in exact pages, sub-blocks j < nq_prev in quant pages
    exact, quant = {}, {}
    for l in layers:
        K, V = hist[l]
        ep = np.zeros((R * epr + 5, 4, EBS, 256), np.uint16)
        for r in range(R):
            for p in range(L0[r]):
                pg = bt[group[l]][r, p // EBS]
                ep[pg, :, p % EBS, :128] = K[r, p]
                ep[pg, :, p % EBS, 128:] = V[r, p]
        exact[l] = ep
        if l != 2:
            qp = np.zeros((R * qpr + 3, QPAGE), np.uint8)
            for r in range(R):
                if nq_prev[r]:
                    sb = oracle.quantize_blocks(K[r, :256 * nq_prev[r]].reshape(-1, 256, 4, 128),
                                                V[r, :256 * nq_prev[r]].reshape(-1, 256, 4, 128))
                    for j in range(nq_prev[r]):
                        off = (256 * j) % QBLOCK // 256 * 51200
                        qp[qbt[r, 256 * j // QBLOCK], off:off + 51200] = sb[j]
            quant[l] = qp
    for r in range(R):                                   # sinks of window layer 2: K in layer 6's aux, V in 10's
        for p in range(min(4, L0[r])):
            for host, arr in ((6, hist[2][0]), (10, hist[2][1])):
                page = quant[host][qbt[r, 0]].view(np.uint16)
                page[AUX // 2 + p * 512: AUX // 2 + (p + 1) * 512] = arr[r, p].reshape(-1)
    before = {l: quant[l].copy() for l in quant}

    # ---- the step on the GPU
    ev = {l: bf16_dev(exact[l]) for l in layers}
    qv = {l: torch.from_numpy(quant[l]).to(DEV) for l in quant}
    lay = {l: vc.KV800DecodeLayer(l, ev[l], qv.get(l)) for l in layers}
    metas = {g: vc.step_meta(torch.from_numpy(bt[g]), torch.from_numpy(n), EBS, DEV) for g in "AB"}
    mq = vc.step_meta(torch.from_numpy(qbt), torch.from_numpy(n), QBLOCK, DEV)
    cos_d, sin_d = bf16_dev(cos), bf16_dev(sin)
    if early_flush:                                      # all quant layers' flushes ahead, on the side stream
        say("launch_flushes")
        vc.launch_flushes(list(lay.values()), {l: metas[group[l]] for l in layers}, mq)
    outs = {}
    for l in layers:
        K, V = hist[l]
        kn = bf16_dev(np.stack([K[r, L0[r]] for r in range(R)]))
        vn = bf16_dev(np.stack([V[r, L0[r]] for r in range(R)]))
        say("layer", l)
        outs[l] = bits_of(lay[l].forward(bf16_dev(q[l]), kn, vn, metas[group[l]], mq, hosts=lay, cos_t=cos_d,
                                         sin_t=sin_d))
    torch.cuda.synchronize()

    # ---- writes, sinks and flushes
    for l in layers:
        K, V = hist[l]
        ep = bits_of(ev[l]).reshape(exact[l].shape)
        for r in range(R):
            p = L0[r]
            pg = bt[group[l]][r, p // EBS]
            assert np.array_equal(ep[pg, :, p % EBS, :128], K[r, p]) and np.array_equal(ep[pg, :, p % EBS, 128:], V[r, p])
    for host, arr in ((6, hist[2][0]), (10, hist[2][1])):
        qb = qv[host].cpu().numpy()
        for r in range(R):
            if L0[r] < 4:
                page = qb[qbt[r, 0]].view(np.uint16)
                assert np.array_equal(page[AUX // 2 + L0[r] * 512: AUX // 2 + (L0[r] + 1) * 512], arr[r, L0[r]].reshape(-1))
    for l in (6, 10):
        K, V = hist[l]
        qb = qv[l].cpu().numpy()
        changed = set()
        for r in range(R):
            for j in range(nq_prev[r], nq_new[r]):
                want = oracle.quantize_blocks(K[r, 256 * j:256 * j + 256][None], V[r, 256 * j:256 * j + 256][None])[0]
                off = (256 * j) % QBLOCK // 256 * 51200
                assert np.array_equal(qb[qbt[r, 256 * j // QBLOCK], off:off + 51200], want), (l, r, j)
                changed.add((int(qbt[r, 256 * j // QBLOCK]), off))
        qb2 = qb.copy()
        for pg, off in changed:
            qb2[pg, off:off + 51200] = before[l][pg, off:off + 51200]
        qb2[:, AUX:] = before[l][:, AUX:]                  # the aux may hold this step's sinks
        assert np.array_equal(qb2, before[l]), l

    # ---- decode against the oracle on an independently built cache of the full history
    for l in layers:
        K, V = hist[l]
        case = oracle.build_paged(lambda b, p0, p1: (K[b, p0:p1], V[b, p0:p1]), list(n), win=256 if l == 2 else 0,
                                  ebs=EBS, shuffle_seed=l)
        decode_bar.check(outs[l], oracle.decode_f32(case, q[l], cos, sin), f"layer {l}", say)


def test_step_tables(hip):
    """kv800_hip_step_tables / kv800_hip_page_offsets against the torch formulas the reference uses per step
    (vllm_attn.py:276-291, 297-317, 320-340), including rows with no flushed sub-block and a step of 3 new tokens."""
    g = torch.Generator().manual_seed(5)
    R, blocks, bsq, qs0 = 7, 9, 1280, 262144
    qbt = torch.randperm(R * blocks + 4, generator=g)[:R * blocks].view(R, blocks).to(torch.int32)
    N = torch.tensor([1, 128, 384, 385, 1663, 5000, 11520], dtype=torch.int32)
    nqmax = int(((N.long() - 128).clamp(min=0) // 256).max())
    boff, NQ, NP, qbt64, aux = hip.step_tables(qbt.to(DEV), bsq, qs0, N.to(DEV), nqmax, nnew=3, aux_scale=qs0 // 2,
                                                aux_add=AUX // 2)
    assert torch.equal(NQ.cpu(), ((N.long() - 128).clamp(min=0) // 256).to(torch.int32))
    assert torch.equal(NP.cpu(), ((N.long() - 3 - 128).clamp(min=0) // 256).to(torch.int32))
    sub = torch.arange(nqmax) * 256
    assert torch.equal(boff.cpu(), qbt[:, sub // bsq].long() * qs0 + ((sub % bsq) // 256) * 51200)
    assert torch.equal(qbt64.cpu(), qbt.long())
    assert torch.equal(aux.cpu(), qbt[:, 0].long() * (qs0 // 2) + AUX // 2)
    eoff = hip.page_offsets(qbt.to(DEV), 131072, 5)
    assert torch.equal(eoff.cpu(), qbt.long() * 131072 + 5)


def test_step_meta_matches_torch(hip):
    """The per-step metadata launch (kv800_hip_step_meta) against the torch statement it replaces (slot = page of
    pos // ebs times ebs plus pos % ebs, pos = len - 1): random block tables with a padded row stride, lengths on page
    boundaries, 1, and a full table; a row of length 0 and one past its table get slot -1."""
    from lfm3_kv800_amd import kv800_hip
    g = torch.Generator(device=DEV).manual_seed(5)
    R, pages, stride, ebs = 37, 9, 12, 16
    bt_full = torch.randint(0, 1000, (R, stride), generator=g, device=DEV, dtype=torch.int32)
    bt = bt_full[:, :pages]
    lens = torch.randint(1, pages * ebs + 1, (R,), generator=g, device=DEV, dtype=torch.int64)
    lens[0], lens[1], lens[2], lens[3] = 1, ebs, ebs + 1, pages * ebs
    slot, pos, l32 = kv800_hip.step_meta(bt, lens, ebs)
    p = lens - 1
    want = bt.gather(1, (p // ebs)[:, None].long())[:, 0].long() * ebs + p % ebs
    assert torch.equal(slot, want) and torch.equal(pos, p) and torch.equal(l32, lens.to(torch.int32))
    lens[4], lens[5] = 0, pages * ebs + 1
    slot, pos, _ = kv800_hip.step_meta(bt, lens, ebs)
    assert int(slot[4]) == -1 and int(pos[4]) == -1 and int(slot[5]) == -1 and int(pos[5]) == pages * ebs


def test_vllm_decode_step_full_size(hip, oracle):
    """the shape of config C4 through the vLLM cache path, all six attention layers: 398 rows with
    lengths U[1K, 32K] (rows 0-7 placed so the step flushes a sub-block), window + sinks layers 2 and 18 (sinks in the
    aux areas of 6 / 10 and 14 / 22) and quantized layers 6, 10, 14, 22, in two exact KV groups (A: 6, 14, 22; B: 2,
    10, 18). Each row's history is a slice of a per-layer N(0,1) pool; its last 640 positions sit in a ring of 8
    shuffled exact pages, its sub-blocks j < nq(n - 1) are quantized from the slice by the HIP quantizer. One step
    (flushes ahead on the side stream, then each layer's write + decode): every output finite, the flushed sub-blocks
    of rows 0-7 equal the oracle quantizer's bytes, and sampled rows (shortest, longest, a flushing row, three more)
    are within the decode bar of the oracle on their full histories."""
    from lfm3_kv800_amd import vllm_cache as vc
    dev = torch.device(DEV)
    R, lo_n, hi_n = 398, 1024, 32768
    rng = np.random.RandomState(41)
    L0 = rng.randint(lo_n, hi_n + 1, size=R).astype(np.int64)
    L0[:8] = 256 * rng.randint(5, 120, size=8) + 127          # n - 128 = 256 k: sub-block k - 1 flushes this step
    n = L0 + 1
    nq_prev = np.maximum(L0 - 128, 0) // 256
    assert ((np.maximum(n - 128, 0) // 256) > nq_prev).sum() >= 8
    layers = (2, 6, 10, 14, 18, 22)
    group = {6: "A", 14: "A", 22: "A", 2: "B", 10: "B", 18: "B"}
    g = torch.Generator(device=dev).manual_seed(41)
    POOL, RING = 1 << 16, 8
    pools = {l: tuple(torch.randn(POOL, 4, 128, generator=g, device=dev).to(torch.bfloat16) for _ in range(2))
             for l in layers}
    base = torch.from_numpy((np.arange(R) * 7919) % (POOL - hi_n - 2)).to(dev)

    def hist(l, rows, p0, p1):
        """(len(rows), p1 - p0, 4, 128) K and V of positions [p0, p1) of the rows (p0, p1 scalars)."""
        idx = base[torch.as_tensor(rows, device=dev)][:, None] + torch.arange(p0, p1, device=dev)
        return pools[l][0][idx], pools[l][1][idx]

    # exact pages: row r's logical page p is page perm[r, p % RING] of its group
    lp = (hi_n + 1) // EBS + 2
    bt = {grp: np.ascontiguousarray(rng.permutation(R * RING).reshape(R, RING)[:, np.arange(lp) % RING], np.int32)
          for grp in "AB"}
    qneed = (n + QBLOCK - 1) // QBLOCK
    qpr = int(qneed.max())
    qbt = np.zeros((R, qpr), np.int32)
    qbt[np.arange(qpr)[None, :] < qneed[:, None]] = rng.permutation(int(qneed.sum()))
    say("full size: rows", R, "tokens", int(n.sum()), "layers", layers)
    ev, qv = {}, {}
    W = 640
    pos = torch.from_numpy(L0[:, None] - W + np.arange(W)[None, :]).to(dev)         # (R, W) last positions
    rr = torch.arange(R, device=dev)[:, None].expand(R, W)
    btd = {grp: torch.from_numpy(bt[grp]).to(dev).long() for grp in "AB"}
    for l in layers:
        e = torch.zeros(R * RING, 4, EBS, 256, dtype=torch.bfloat16, device=dev)
        idx = base[:, None] + pos
        pg = btd[group[l]][rr, pos // EBS]
        e[pg, :, pos % EBS, :128] = pools[l][0][idx]
        e[pg, :, pos % EBS, 128:] = pools[l][1][idx]
        ev[l] = e
    # quant pages: every sub-block j < nq_prev[r] from the HIP quantizer
    pairs = np.array([(r, j) for r in range(R) for j in range(int(nq_prev[r]))], np.int64)
    for l in (6, 10, 14, 22):
        q_l = torch.zeros(int(qneed.sum()), QPAGE, dtype=torch.uint8, device=dev)
        slots = q_l[:, :AUX].view(-1, 5, 51200)
        for i in range(0, len(pairs), 2048):
            part = torch.from_numpy(pairs[i:i + 2048]).to(dev)
            idx = base[part[:, 0]][:, None] + 256 * part[:, 1:2] + torch.arange(256, device=dev)
            sb = hip.quantize_blocks(pools[l][0][idx], pools[l][1][idx])
            qpage = torch.from_numpy(qbt).to(dev).long()[part[:, 0], 256 * part[:, 1] // QBLOCK]
            slots[qpage, (256 * part[:, 1]) % QBLOCK // 256] = sb
        qv[l] = q_l
    # sinks (positions 0-3) of the window layers: K in the first host's aux, V in the second's
    qbt0 = torch.from_numpy(qbt[:, 0]).to(dev).long()
    for wl in (2, 18):
        ks, vs = hist(wl, list(range(R)), 0, 4)
        for host, arr in zip(vc.SINK_HOST[wl], (ks, vs)):
            aux = qv[host].view(torch.bfloat16).view(-1, QPAGE // 2)[:, AUX // 2:AUX // 2 + 2048]
            aux[qbt0] = arr.reshape(R, 2048)
    torch.cuda.synchronize()

    lay = {l: vc.KV800DecodeLayer(l, ev[l], qv.get(l)) for l in layers}
    metas = {grp: vc.step_meta(torch.from_numpy(bt[grp]), torch.from_numpy(n), EBS, DEV) for grp in "AB"}
    mq = vc.step_meta(torch.from_numpy(qbt), torch.from_numpy(n), QBLOCK, DEV)
    cos, sin = oracle.rope_tables(hi_n + 64)
    cos_d, sin_d = bf16_dev(cos), bf16_dev(sin)
    qs = {l: torch.randn(R, 16, 128, generator=g, device=dev).to(torch.bfloat16) for l in layers}
    kn = {l: torch.randn(R, 4, 128, generator=g, device=dev).to(torch.bfloat16) for l in layers}
    vn = {l: torch.randn(R, 4, 128, generator=g, device=dev).to(torch.bfloat16) for l in layers}
    say("full size: step")
    vc.launch_flushes(list(lay.values()), {l: metas[group[l]] for l in layers}, mq)
    outs = {l: lay[l].forward(qs[l], kn[l], vn[l], metas[group[l]], mq, hosts=lay, cos_t=cos_d, sin_t=sin_d)
            for l in layers}
    torch.cuda.synchronize()
    for l in layers:
        assert bool(torch.isfinite(outs[l].float()).all()), l

    # the sub-block each of rows 0-7 flushed in this step, against the oracle quantizer
    for l in (6, 10, 14, 22):
        qb = qv[l]
        for r in range(8):
            j = int(nq_prev[r])
            K, V = hist(l, [r], 256 * j, 256 * j + 256)
            want = oracle.quantize_blocks(bits_of(K), bits_of(V))[0]
            pg, off = int(qbt[r, 256 * j // QBLOCK]), (256 * j) % QBLOCK // 256 * 51200
            assert np.array_equal(qb[pg, off:off + 51200].cpu().numpy(), want), (l, r, j)

    sample = sorted({int(np.argmin(n)), int(np.argmax(n)), 3, *rng.choice(np.arange(8, R), 3, replace=False).tolist()})
    for l in layers:
        Ks, Vs = [], []
        for r in sample:
            pg = int(bt[group[l]][r, L0[r] // EBS])                        # the step's row in the exact pages
            assert torch.equal(ev[l][pg, :, L0[r] % EBS, :128], kn[l][r]), (l, r)
            assert torch.equal(ev[l][pg, :, L0[r] % EBS, 128:], vn[l][r]), (l, r)
            K, V = hist(l, [r], 0, int(L0[r]))
            Ks.append(np.concatenate([bits_of(K[0]), bits_of(kn[l][r:r + 1])]))
            Vs.append(np.concatenate([bits_of(V[0]), bits_of(vn[l][r:r + 1])]))
        if l in vc.WINDOW_LAYERS:                         # the window layer's sinks come from the host layers' aux
            for b, r in enumerate(sample):
                for hl, arr in zip(vc.SINK_HOST[l], (Ks, Vs)):
                    aux = qv[hl].view(torch.bfloat16).view(-1, QPAGE // 2)[int(qbt[r, 0]), AUX // 2:AUX // 2 + 2048]
                    assert np.array_equal(bits_of(aux).reshape(4, 4, 128), arr[b][:4]), (l, r)
        case = oracle.build_paged(lambda b, p0, p1: (Ks[b][p0:p1], Vs[b][p0:p1]), [int(n[r]) for r in sample],
                                  win=256 if l in vc.WINDOW_LAYERS else 0, ebs=EBS, shuffle_seed=l)
        decode_bar.check(outs[l][sample].float().cpu().numpy(), oracle.decode_f32(case, bits_of(qs[l][sample]), cos, sin),
                         f"full size layer {l}: rows {sample}", say)
    del ev, qv, lay, outs, pools
    torch.cuda.empty_cache()
