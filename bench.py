"""Benchmark of the 800h decode path on one MI355X: one layer of paged split-K decode attention
over 64 sequences x 32,768 tokens (127 quantized 256-token sub-blocks + 256 exact tokens per sequence, permuted page
tables), 16 query heads over 4 KV heads x 128 (the reference format's head shape; same bytes and flops per token as
32 / 8 / 64).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--c3-only] [--calib]
                    [--c2-only | --c4-only | --prefill-only | --window-only | --e2e-only [--e2e-which both|256|398]
                     [--e2e-steps S]]

A step = one kv800.decode call over one layer (the quantized-split grid with the exact tail, then the split merge).
Warm-up: the GPU reaches its sustained-load clocks only after tens of milliseconds of work (the first 50 C3 kernel
launches after setup average 178 us, the following ones 152 us), so every timed section follows its own untimed work
whatever --warmup says: the C3 layer steps and the C3 kernel launches each at least max(W, 300) calls and 250 ms of
GPU time (warm_up; the JSON records what ran), 200 flushes for C2, 20 steps for C4.
Inputs are resident in HBM; two cache copies (2 x 450 MB, above the 256 MB MALL) alternate between steps. Prints one
JSON line. roofline: the quantized-split kernel's algorithmic bytes (NQ * 51,200 per sequence) over its average
launch duration, K launches back to back between one HIP event pair on their own stream; traffic from the
committed rocprofv3 counter summary;
cpu_baseline: a pure-torch CPU restatement of the reference's torch_decode.py on a sample of the same rows (the C
oracle's time beside it). Extra
fields: flush_c2 (config C2, the flush kernel alone), c4 (config 4, one decode step of all 6 attention
layers over 398 ragged sequences), e2e (config 5, greedy decode tok/s of an LFM3-shaped model over 256
sequences), e2e_398x32k (the same loop at the reference's published point, 398 sequences of 32K tokens), prefill
(prefill over compressed history: 8 rows x a 2048-token chunk over 16K-token histories, the attention kernel against
the MFMA peak), fake_quant (training fake quantization of one layer's K and V), window_398 (one window + sinks layer
of 398 rows at 32K context against the HBM peak), hbm_copy (a plain 1 GiB device
copy: the bandwidth the box sustains) and hbm_read (a 4 GiB streaming read by kv800_hip_read_probe: the read
bandwidth the part sustains for plain loads, and the decode kernel's achieved bandwidth as a fraction of it) and
decode_small_batch (one decode layer's latency for 1, 8 and 16 rows of 32K tokens). Every
timed loop runs with the interpreter's garbage collector frozen (frozen_heap). --calib runs a plain copy of known size
instead (rocprof FETCH/WRITE calibration)."""
import argparse
import gc
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

B, N_CTX, EBS = 64, 32768, 128
NQ = (N_CTX - 128) // 256                           # 127 flushed sub-blocks per sequence
QBYTES = B * NQ * 51200                             # compressed bytes read by the quantized-split kernel
XBYTES = B * (N_CTX - NQ * 256) * 2048              # exact tail bytes (256 tokens x 4 heads x (K + V) bf16)
ALG_BYTES = QBYTES + XBYTES                         # the reference's accounting (nvidia/check_nvidia.py:563)
HBM_PEAK_GBS = 8000.0


def measured_traffic():
    """HBM bytes per decode_quant launch from the committed rocprofv3 counter summary: FETCH_SIZE + WRITE_SIZE, each
    scaled by what the counter reads for a plain 1 GiB copy (rocprofv3 cannot run inside this process). None if absent."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "decode_quant_c3_pmc.txt")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1])
    except (OSError, ValueError):
        pass
    return None


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


class frozen_heap:
    """Runs a timed loop with the interpreter's collector off: collects once, moves every live object to the permanent
    generation (gc.freeze) and disables collection until the block ends. A full collection of this process's heap takes
    ~40 ms (torch's import alone leaves ~10^6 objects); one landing inside a timed loop stalls the launches that long
    (measured: one 40 ms idle gap on the GPU in an otherwise unchanged C4 loop, 2.2 -> 3.5 ms per step). A serving
    engine freezes its heap after start-up for the same reason."""

    def __enter__(self):
        gc.collect()
        gc.freeze()
        gc.disable()
        return self

    def __exit__(self, *exc):
        gc.enable()
        gc.unfreeze()
        return False


C3_WARM_CALLS, C3_WARM_MS = 300, 250.0


def warm_up(torch, fn, calls, min_ms):
    """Untimed calls of fn(i) until at least `calls` calls and `min_ms` of wall time (GPU-bound: synchronized every 50
    calls) have run. Returns (calls, ms) actually run."""
    t0 = time.perf_counter()
    i = 0
    while True:
        fn(i)
        i += 1
        if i % 50 == 0 or i >= calls:
            torch.cuda.synchronize()
            ms = (time.perf_counter() - t0) * 1e3
            if i >= calls and ms >= min_ms:
                return i, round(ms, 1)


def build_layer(torch, kh, seed, dev):
    """One layer's cache for the 64 x 32K workload: sub-blocks quantized on the GPU by the HIP quantizer from seeded
    bf16 N(0,1) K / V, written through a random permutation of the quant pool; exact pages permuted likewise."""
    import lfm3_kv800_amd.kv800 as kv
    g = torch.Generator(device=dev).manual_seed(seed)
    boff = (torch.randperm(B * NQ, generator=g, device=dev).view(B, NQ) * 51200).to(torch.int64)
    qpool = torch.empty(B * NQ * 51200, dtype=torch.uint8, device=dev)
    for b0 in range(0, B, 8):
        k = torch.randn(8 * NQ, 256, 4, 128, generator=g, device=dev).to(torch.bfloat16)
        v = torch.randn(8 * NQ, 256, 4, 128, generator=g, device=dev).to(torch.bfloat16)
        sb = kh.quantize_blocks(k, v)
        idx = boff[b0:b0 + 8].reshape(-1)[:, None] + torch.arange(51200, device=dev)
        qpool[idx.reshape(-1)] = sb.reshape(-1)
        del k, v, sb, idx
    pages = N_CTX // EBS
    ex0 = NQ * 256 // EBS
    npg = B * (pages - ex0)
    eoff = torch.zeros(B, pages, dtype=torch.int64, device=dev)
    eoff[:, ex0:] = torch.randperm(npg, generator=g, device=dev).view(B, pages - ex0) * (4 * EBS * 256)
    epool = torch.randn(npg, 4, EBS, 256, generator=g, device=dev).to(torch.bfloat16)
    N = torch.full((B,), N_CTX, dtype=torch.int32, device=dev)
    NQt = torch.full((B,), NQ, dtype=torch.int32, device=dev)
    return kv.Paged(qpool=qpool, boff=boff, epool=epool, eoff=eoff, ebs=EBS, e_hs=EBS * 256, e_ts=256, e_v=128,
                    sk=None, sv=None, skoff=None, svoff=None, N=N, NQ=NQt, nqmax=NQ, win=0)


C2_B, C2_N, C2_EBS = 64, 2048, 128
C2_NQ = (C2_N - 128) // 256                         # 7 flushed sub-blocks per sequence (kv800.py:433 flush rule)
C2_READ = C2_B * C2_NQ * 256 * 4 * 128 * 2 * 2      # bf16 K + V gathered from the exact pages
C2_WRITE = C2_B * C2_NQ * 51200
C2_FMA = C2_B * C2_NQ * 256 * 4 * 16 * 688          # fp32 fma of the bit-exact V Hadamard chains: 688 per lane's 8
                                                    # outputs (16 lanes per head row), 86 per output
FMA_PEAK = 256 * 64 * 2.4e9                         # non-packed fp32 fma/s: 256 CUs x 64 lanes x 2.4 GHz


def bench_flush_c2(torch, kh, dev, steps, warmup):
    """config C2, the flush kernel alone: 64 sequences x a 2048-token prefill chunk in vLLM-geometry exact
    pages (128 tokens x 4 heads x [K128 | V128] bf16 per page, shuffled physical pages), K / V ~ N(0,1) with 1 % of
    the elements x 8, flushed by one launch into shuffled 1280-token quant pages (5 x 51,200 B per 262,144-B page):
    448 sub-blocks. Per-launch HIP events on the current stream."""
    g = torch.Generator(device=dev).manual_seed(11)
    pages = C2_N // C2_EBS
    npg = C2_B * pages
    x = torch.randn(npg, 4, C2_EBS, 256, generator=g, device=dev)
    x[torch.rand(x.shape, generator=g, device=dev) < 0.01] *= 8
    epool = x.to(torch.bfloat16)
    del x
    eoff = (torch.randperm(npg, generator=g, device=dev).view(C2_B, pages) * (4 * C2_EBS * 256)).to(torch.int64)
    qpp = (C2_NQ * 256 + 1279) // 1280
    qpool = torch.zeros(C2_B * qpp * 262144, dtype=torch.uint8, device=dev)
    qbt = torch.randperm(C2_B * qpp, generator=g, device=dev).view(C2_B, qpp).to(torch.int64)
    nq0 = torch.zeros(C2_B, dtype=torch.int32, device=dev)
    nq1 = torch.full((C2_B,), C2_NQ, dtype=torch.int32, device=dev)

    def flush():
        kh.flush(epool, eoff, C2_EBS, C2_EBS * 256, 256, 128, qpool, qbt, 1280, 262144, nq0, nq1, C2_NQ)

    s = torch.cuda.current_stream(dev)
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    with frozen_heap():
        for _ in range(warmup):
            flush()
        torch.cuda.synchronize()
        for e0, e1 in ev:
            e0.record(s)
            flush()
            e1.record(s)
        ev[-1][1].synchronize()
    ms = sum(e0.elapsed_time(e1) for e0, e1 in ev) / steps
    gbps = (C2_READ + C2_WRITE) / (ms * 1e-3) / 1e9
    return {"workload": "C2: flush of 64 seqs x 2048-token chunk = 448 sub-blocks, vLLM page geometry, shuffled "
                        "exact and quant page tables, N(0,1) K/V with 1% outliers x8",
            "ms": round(ms, 5), "bytes": C2_READ + C2_WRITE, "gbps": round(gbps, 1),
            "hbm_frac": round(gbps / HBM_PEAK_GBS, 4), "bound": "valu",
            "fma_per_launch": C2_FMA, "fma_frac": round(C2_FMA / (ms * 1e-3) / FMA_PEAK, 4)}


C4_R, C4_MIN, C4_MAX = 398, 1024, 32768
C4_GROUP = {6: "A", 14: "A", 22: "A", 2: "B", 10: "B", 18: "B"}   # two exact KV groups of three layers


def bench_c4(torch, kh, dev, steps, warmup, cos, sin):
    """config C4: the 6 attention layers of an LFM3-1.7B-shaped stack (quantized 6, 10, 14, 22; window + sinks
    2, 18) over 398 sequences with lengths U[1K, 32K] (seeded), vLLM page geometry (exact: 128-token pages in two exact
    KV groups; quant: 1280-token pages in one group, sinks in the hosts' aux), one decode step per layer per step:
    the new token's rows, the flush of the sub-blocks that became eligible, decode tables and decode
    (lfm3-kv800_amd/vllm_cache.py). Quant pages are filled from a pool of sub-blocks quantized from N(0,1) bf16 K / V;
    exact pages, sinks and q / k / v are N(0,1)."""
    import numpy as np
    from lfm3_kv800_amd import vllm_cache as vc
    g = torch.Generator(device=dev).manual_seed(41)
    L0 = np.random.RandomState(41).randint(C4_MIN, C4_MAX + 1, size=C4_R).astype(np.int64)
    nmax = int(L0.max()) + steps + warmup + 1
    ebs, qb = 128, vc.QBLOCK
    epr, qpr = nmax // ebs + 1, nmax // qb + 1
    gc = torch.Generator().manual_seed(41)
    bt = {grp: torch.randperm(C4_R * epr, generator=gc).view(C4_R, epr).to(torch.int32) for grp in "AB"}
    n_ep = C4_R * epr
    qperm = torch.randperm(C4_R * qpr, generator=gc).view(C4_R, qpr).to(torch.int32)
    # a pool of real sub-blocks, copied into every quant page slot
    pool = kh.quantize_blocks(torch.randn(256, 256, 4, 128, generator=g, device=dev).to(torch.bfloat16),
                              torch.randn(256, 256, 4, 128, generator=g, device=dev).to(torch.bfloat16))
    layers = {}
    for l in (2, 6, 10, 14, 18, 22):
        ev = torch.randn(n_ep, 4, ebs, 256, generator=g, device=dev).to(torch.bfloat16)
        qv = None
        if l not in vc.WINDOW_LAYERS:
            qv = torch.empty(C4_R * qpr, vc.QPAGE, dtype=torch.uint8, device=dev)
            pick = torch.randint(0, pool.shape[0], (C4_R * qpr * 5,), generator=g, device=dev)
            qv[:, :vc.AUX_BYTES].view(-1, 5, 51200).copy_(pool[pick].view(-1, 5, 51200))
            qv[:, vc.AUX_BYTES:].view(torch.bfloat16).copy_(
                torch.randn(C4_R * qpr, (vc.QPAGE - vc.AUX_BYTES) // 2, generator=g, device=dev))
        layers[l] = vc.KV800DecodeLayer(l, ev, qv)
    qkv = {l: (torch.randn(C4_R, 16, 128, generator=g, device=dev).to(torch.bfloat16),
               torch.randn(C4_R, 4, 128, generator=g, device=dev).to(torch.bfloat16),
               torch.randn(C4_R, 4, 128, generator=g, device=dev).to(torch.bfloat16)) for l in layers}
    torch.cuda.synchronize()
    # per-step metadata (slot mapping, lengths, device block tables) is the scheduler's input; it is built before the
    # timed steps, as vLLM builds it on the host while the previous step runs on the GPU
    metas = []
    for i in range(warmup + steps):
        lens = torch.from_numpy(L0 + 1 + i)
        metas.append(({grp: vc.step_meta(bt[grp], lens, ebs, dev) for grp in "AB"}, vc.step_meta(qperm, lens, qb, dev)))
    torch.cuda.synchronize()

    def step(i):
        me, mq = metas[i]
        # the step's flushes start at once on a side stream, under the decode of the layers before them
        vc.launch_flushes(list(layers.values()), {l: me[C4_GROUP[l]] for l in layers}, mq)
        for l in (2, 6, 10, 14, 18, 22):
            q, k, v = qkv[l]
            layers[l].forward(q, k, v, me[C4_GROUP[l]], mq, hosts=layers, cos_t=cos, sin_t=sin)

    with frozen_heap():
        for i in range(warmup):
            step(i)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(warmup, warmup + steps):
            step(i)
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1e3 / steps
    # one more step (past the timed ones) whose layer outputs are checked
    me, mq = metas[-1]
    outs = [layers[l].forward(*qkv[l], me[C4_GROUP[l]], mq, hosts=layers, cos_t=cos, sin_t=sin)
            for l in (2, 6, 10, 14, 18, 22)]
    finite = all(bool(torch.isfinite(o.float()).all()) for o in outs)
    # algorithmic bytes of one step (the reference's accounting), at the mean step length
    nmid = L0 + 1 + warmup + steps // 2
    nq = np.maximum(nmid - 128, 0) // 256
    qbytes = int((nq * 51200 + (nmid - 256 * nq) * 2048).sum()) * 4
    wbytes = int(((np.minimum(4, np.maximum(nmid - 256, 0)) + np.minimum(256, nmid)) * 2048).sum()) * 2
    gbps = (qbytes + wbytes) / (ms * 1e-3) / 1e9
    return {"workload": "C4: 6 attention layers (4 quantized + 2 window+sinks), 398 seqs, lengths U[1K, 32K], vLLM "
                        "page geometry, two exact KV groups, new-token write + flush + decode per layer",
            "ms_per_step": round(ms, 4), "tok_s": round(C4_R / (ms * 1e-3), 1), "bytes_per_step": qbytes + wbytes,
            "gbps": round(gbps, 1), "hbm_frac": round(gbps / HBM_PEAK_GBS, 4), "outputs_finite": finite}


E2E_R, E2E_MIN, E2E_MAX = 256, 1024, 32768


def bench_e2e(torch, dev, steps, lens=None, seed=51, graph=False):
    """config C5: greedy decode of a random-init LFM3-1.7B-shaped model (lfm3-kv800_amd/model.py: 24 layers,
    13 short-conv, 6 full-attention on the 800h caches, 5 sliding-window; weights N(0, 0.02) bf16) over 256 sequences
    with prompt lengths U[1K, 32K] (seeded), `steps` greedy steps; `lens` replaces the prompt lengths (the reference's
    published throughput point is 398 sequences of 32,768 tokens, RESULTS_RELEASE.md:90-96). tok/s = c (steps - 1) /
    time, time from the end of the first step to the end of the last (the reference's decode tok/s,
    RESULTS_RELEASE.md:83-85). The prompts' K / V histories are synthetic N(0, 1), written into the caches before the
    first step by the attention layers' own step path in 2048-token prefill chunks (exact pages, sinks, flushes:
    model.PagedAttention800.fill); prompt processing is not part of the measurement. Each step is launched
    kernel by kernel from the host (the loop is GPU-bound at these batch sizes: replaying one recorded HIP graph of the
    step, graph=True / model.DecodeGraph, measured the same step time)."""
    import numpy as np
    from lfm3_kv800_amd import model as M
    cfg = M.Lfm3Config()
    L0 = (np.random.RandomState(seed).randint(E2E_MIN, E2E_MAX + 1, size=E2E_R) if lens is None
          else np.asarray(lens)).astype(np.int64)
    R = len(L0)
    g = torch.Generator(device=dev).manual_seed(seed)

    # prompt K / V: slices of per-layer N(0, 1) pools at row- and position-dependent offsets (the fill asks for each
    # row's history in prefill chunks, ~R x 16 x 11 slices at 32K prompts)
    POOL = 1 << 16
    pools = {}

    def history(l, r, p0, p1):
        if l not in pools:
            pools[l] = tuple(torch.randn(POOL, 4, 128, generator=g, device=dev).to(torch.bfloat16) for _ in range(2))
        o = (r * 7919 + p0 * 13) % (POOL - (p1 - p0) + 1)
        return pools[l][0][o:o + p1 - p0], pools[l][1][o:o + p1 - p0]

    t = time.perf_counter()
    attn = M.PagedAttention800(L0.tolist(), steps + 1, dev, seed=seed)
    attn.fill(history)
    model = M.Lfm3Decoder(cfg, attn, R, dev, seed=seed)
    model.randomize_conv_states(seed)
    tokens = torch.randint(0, cfg.vocab, (R,), generator=g, device=dev)
    torch.cuda.synchronize()
    log(f"e2e: caches of {R} prompts ({int(L0.sum())} tokens) and weights ready in {time.perf_counter() - t:.1f} s")
    # first step (and the recording of the graph): outside the measured window
    if graph:
        dg = M.DecodeGraph(model, attn, tokens, steps - 1)
        advance = dg.step
    else:
        tokens = model.greedy(tokens, attn.begin_step())
        advance = lambda: model.greedy(tokens, attn.begin_step())
    torch.cuda.synchronize()
    with frozen_heap():
        t0 = time.perf_counter()
        for _ in range(steps - 1):
            tokens = advance()
        torch.cuda.synchronize()
        dt = time.perf_counter() - t0
    assert bool(((tokens >= 0) & (tokens < cfg.vocab)).all())
    ctx = L0 + steps
    prompts = "U[1K, 32K]" if lens is None else f"{int(L0.min())}..{int(L0.max())} tokens"
    out = {"workload": f"greedy decode, random-init LFM3-1.7B-shaped model (hidden 2048, 24 layers: 13 conv, "
                       f"6 full attention on 800h caches, 5 sliding 256; vocab {cfg.vocab}, ffn {cfg.ffn}), "
                       f"{R} seqs, prompts {prompts}, {steps} steps",
           "data": "synthetic N(0,1) K/V prompt histories written through the mixed-step cache path, random token ids",
           "tok_s": round(R * (steps - 1) / dt, 1), "ms_per_step": round(dt * 1e3 / (steps - 1), 3),
           "steps": steps, "seqs": R, "context_tokens_end": int(ctx.sum()),
           "launch": "one HIP graph per step" if graph else "eager"}
    del attn, model, pools
    torch.cuda.empty_cache()
    return out


PF_R, PF_HIST, PF_NEW = 8, 16384, 2048                # prefill rows, history tokens per row, new tokens per row
MFMA_BF16_PEAK = 2500.0                               # TFLOP/s, MI355X dense bf16 / fp16


def median_us(torch, fn, n, warmup=10):
    """Median duration (us) of fn() over n calls, one HIP event pair per call on the current stream."""
    for _ in range(warmup):
        fn()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
    for e0, e1 in ev:
        e0.record()
        fn()
        e1.record()
    ev[-1][1].synchronize()
    t = sorted(e0.elapsed_time(e1) * 1e3 for e0, e1 in ev)
    return round(t[len(t) // 2], 1)


def events_ms(torch, fn, n, warmup):
    """Average duration of fn() over n calls, one HIP event pair per call on the current stream, after warmup calls."""
    for _ in range(warmup):
        fn()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
    for e0, e1 in ev:
        e0.record()
        fn()
        e1.record()
    ev[-1][1].synchronize()
    return sum(e0.elapsed_time(e1) for e0, e1 in ev) / n


def bench_prefill(torch, kh, dev, steps, warmup):
    """Prefill over compressed history (vllm_attn.py:351-402 for quantized layers): PF_R rows, each
    extending a PF_HIST-token history by one PF_NEW-query chunk (the reference's prefill chunk, vllm_attn.py:190-200),
    through vllm_cache.prefill_quant_rows: the history producer (flushed sub-blocks dequantized and rotated to bf16,
    exact rows rotated), the new rows' key RoPE, one flash-attention launch over all rows. The cache is a PagedStore
    filled with seeded N(0,1) K / V by the HIP row writes and flushes. Whole calls host-timed (the row bookkeeping is
    host work, as in the reference); the attention kernel alone by HIP events, against the MFMA bf16 peak: 4 x 128
    flops per (query, visible key, query head)."""
    import lfm3_kv800_amd.kv800 as kv
    from lfm3_kv800_amd import vllm_cache as vc
    g = torch.Generator(device=dev).manual_seed(61)
    st = kv.PagedStore(PF_R, PF_HIST + 8, dev)
    for c0 in range(0, PF_HIST, 2048):
        n = min(PF_HIST, c0 + 2048) - c0
        st.append(torch.randn(PF_R, n, 4, 128, generator=g, device=dev).to(torch.bfloat16),
                  torch.randn(PF_R, n, 4, 128, generator=g, device=dev).to(torch.bfloat16))
    P = st.paged()
    T = PF_R * PF_NEW
    q = torch.randn(T, 16, 128, generator=g, device=dev).to(torch.bfloat16)
    k = torch.randn(T, 4, 128, generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn(T, 4, 128, generator=g, device=dev).to(torch.bfloat16)
    cos, sin = rope_tables(torch, PF_HIST + PF_NEW + 8, dev)
    qsl = [i * PF_NEW for i in range(PF_R + 1)]
    prev = [PF_HIST] * PF_R
    run = lambda: vc.prefill_quant_rows(P, q, k, v, qsl, prev, cos, sin)
    for _ in range(warmup):
        run()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        out = run()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    assert bool(torch.isfinite(out.float()).all())
    args = vc.prefill_quant_inputs(P, q, k, v, qsl, prev, cos, sin)
    ms_k = events_ms(torch, lambda: kh.prefill(*args, window=0), steps, warmup)
    pairs = PF_R * (PF_NEW * PF_HIST + PF_NEW * (PF_NEW + 1) // 2)      # (query, visible key) pairs, causal
    flop = pairs * 16 * 4 * 128
    tflops = flop / (ms_k * 1e-3) / 1e12
    # a short extend chunk: row 0 alone with 16 new queries over its 16K history (the key-split path), HIP events
    # around the attention call (its host preparation included), median of 50
    import lfm3_kv800_amd.kv800 as kv
    P1 = kv.Paged(qpool=P.qpool, boff=P.boff[:1].contiguous(), epool=P.epool, eoff=P.eoff[:1].contiguous(), ebs=P.ebs,
                  e_hs=P.e_hs, e_ts=P.e_ts, e_v=P.e_v, sk=None, sv=None, skoff=None, svoff=None,
                  N=P.N[:1].contiguous(), NQ=P.NQ[:1].contiguous(), nqmax=P.nqmax, win=0)
    args1 = vc.prefill_quant_inputs(P1, q[:16], k[:16], v[:16], [0, 16], [PF_HIST], cos, sin)
    short = median_us(torch, lambda: kh.prefill(*args1, window=0), 50)
    return {"workload": f"f3: prefill over compressed history, {PF_R} rows x {PF_NEW}-token chunk over "
                        f"{PF_HIST}-token histories ({(PF_HIST - 128) // 256} flushed sub-blocks each), "
                        "PagedStore geometry, N(0,1) q/K/V",
            "ms": round(ms, 4), "tok_s": round(T / (ms * 1e-3), 1), "attention_kernel_ms": round(ms_k, 4),
            "attention_flop": flop, "tflops": round(tflops, 1), "mfma_frac": round(tflops / MFMA_BF16_PEAK, 4),
            "bound": "mfma",
            "short_chunk_us": {"workload": f"1 row x 16 queries over a {PF_HIST}-token history (key-split path)",
                               "attention_call_us": short}}


FQ_B, FQ_T = 8, 4096                                  # training batch of the fake-quant measurement


WIN_R, WIN_W, WIN_SINKS = 398, 256, 4      # a window + sinks layer (LFM3 layers 2 / 18) at 398 rows of 32K context


def bench_window(torch, kh, dev, steps, warmup):
    """One window + sinks layer (vllm_attn.py:34: the last 256 positions and the 4 sinks) of 398 rows at 32,768 tokens
    through the fused HIP decode (NQ = 0): 128-token exact pages in vLLM geometry, shuffled, N(0,1) K / V / sinks /
    q. kv800_hip_decode_sized is called directly with its buffers allocated once, the K launches back to back between
    one HIP event pair; 2,048 algorithmic bytes per (visible token, layer)."""
    import ctypes
    import lfm3_kv800_amd.kv800 as kv
    g = torch.Generator(device=dev).manual_seed(61)
    ebs, pages = 128, N_CTX // 128
    lo = (N_CTX - WIN_W) // ebs
    npg = WIN_R * (pages - lo)
    eoff = torch.zeros(WIN_R, pages, dtype=torch.int64, device=dev)
    eoff[:, lo:] = torch.randperm(npg, generator=g, device=dev).view(WIN_R, pages - lo) * (4 * ebs * 256)
    epool = torch.randn(npg, 4, ebs, 256, generator=g, device=dev).to(torch.bfloat16)
    sk = torch.randn(WIN_R, WIN_SINKS, 4, 128, generator=g, device=dev).to(torch.bfloat16)
    sv = torch.randn(WIN_R, WIN_SINKS, 4, 128, generator=g, device=dev).to(torch.bfloat16)
    so = torch.arange(WIN_R, device=dev, dtype=torch.int64) * (WIN_SINKS * 4 * 128)
    P = kv.Paged(qpool=None, boff=None, epool=epool, eoff=eoff, ebs=ebs, e_hs=ebs * 256, e_ts=256, e_v=128, sk=sk,
                 sv=sv, skoff=so, svoff=so.clone(), N=torch.full((WIN_R,), N_CTX, dtype=torch.int32, device=dev),
                 NQ=torch.zeros(WIN_R, dtype=torch.int32, device=dev), nqmax=0, win=WIN_W)
    q = torch.randn(WIN_R, 16, 128, generator=g, device=dev).to(torch.bfloat16)
    cos, sin = rope_tables(torch, N_CTX + 64, dev)
    assert torch.isfinite(kh.decode(P, q, cos, sin).float()).all()
    L = kh.ops()
    st, qbytes, eelems, selems = kh.paged_struct(P, WIN_R)
    wsb = int(L.kv800_hip_decode_workspace(WIN_R, 0, 0))
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    out = torch.empty(WIN_R, 16, 128, dtype=torch.bfloat16, device=dev)
    ptr = lambda t: ctypes.c_void_p(t.data_ptr())
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)

    def call():
        rc = L.kv800_hip_decode_sized(ctypes.byref(st), ptr(q), WIN_R, ptr(cos), ptr(sin), cos.shape[0], None, qbytes,
                                      eelems, selems, ptr(out), ptr(ws), wsb, 0, stream)
        assert rc == 0, L.kv800_hip_last_error()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with frozen_heap():
        for _ in range(warmup):
            call()
        e0.record()
        for _ in range(steps):
            call()
        e1.record()
        e1.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / steps
    byt = WIN_R * (WIN_W + WIN_SINKS) * 2048
    return {"workload": f"window + sinks layer ({WIN_W} + {WIN_SINKS} tokens) of {WIN_R} rows at {N_CTX} tokens, one "
                        "workgroup of one wave per (row, KV head)", "us": round(us, 2), "bytes": byt,
            "gbps": round(byt / (us * 1e-6) / 1e9, 1), "hbm_frac": round(byt / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}


def bench_fake_quant(torch, kh, dev, steps, warmup):
    """Training fake quantization (train.py:82-100): one quantized layer's keys and values of a training
    batch of FQ_B sequences x FQ_T tokens, float32, 4 KV heads x 128: kv800_hip_fake_quant_k over (B, T / 256, 256,
    512) and kv800_hip_fake_quant_v over (B T, 4, 128), HIP events per launch. Each reads and writes its tensor once;
    V also runs the quantizer's and the dequantizer's fp32 Hadamard chains per token."""
    g = torch.Generator(device=dev).manual_seed(71)
    x = torch.randn(FQ_B, FQ_T // 256, 256, 512, generator=g, device=dev)
    vv = torch.randn(FQ_B * FQ_T, 4, 128, generator=g, device=dev)
    ms_k = events_ms(torch, lambda: kh.fake_quant_k(x), steps, warmup)
    ms_v = events_ms(torch, lambda: kh.fake_quant_v(vv), steps, warmup)
    nb = x.numel() * 4 * 2                                            # float32 read + written
    return {"workload": f"f4: fake quantization of one layer's K and V, {FQ_B} x {FQ_T} tokens x 4 heads x 128, "
                        "float32, N(0,1)",
            "k_ms": round(ms_k, 4), "v_ms": round(ms_v, 4), "bytes_each": nb,
            "k_gbps": round(nb / (ms_k * 1e-3) / 1e9, 1), "v_gbps": round(nb / (ms_v * 1e-3) / 1e9, 1),
            "tok_s": round(FQ_B * FQ_T / ((ms_k + ms_v) * 1e-3), 1)}


def bench_copy(torch, dev, steps):
    """A plain 1 GiB device copy (read + write), HIP events: the HBM bandwidth this box sustains, beside the 8 TB/s
    peak the roofline fractions use."""
    x = torch.empty(1 << 28, dtype=torch.int32, device=dev)
    y = torch.empty_like(x)
    ms = events_ms(torch, lambda: y.copy_(x), steps, 3)
    gbps = 2 * x.numel() * 4 / (ms * 1e-3) / 1e9
    del x, y
    return {"bytes": 2 * (1 << 30), "ms": round(ms, 4), "gbps": round(gbps, 1), "frac_of_peak": round(gbps / HBM_PEAK_GBS, 4)}


def bench_read(torch, kh, dev, steps):
    """A 4 GiB streaming read by kv800_hip_read_probe (plain 16-byte loads, 8 in flight per lane, 512 workgroups),
    HIP events: the read bandwidth the part sustains for the decode kernels' kind of load, beside the 8 TB/s peak."""
    x = torch.empty(1 << 32, dtype=torch.uint8, device=dev)
    out = torch.empty(512, dtype=torch.int32, device=dev)
    ms = events_ms(torch, lambda: kh.read_probe(x, out, 512), steps, 3)
    gbps = x.numel() / (ms * 1e-3) / 1e9
    del x, out
    return {"bytes": 1 << 32, "ms": round(ms, 4), "gbps": round(gbps, 1), "frac_of_peak": round(gbps / HBM_PEAK_GBS, 4)}


def decode_small_batches(torch, kh, P, q, cos, sin, sizes=(1, 8, 16)):
    """Latency of one decode layer for the first B rows of the C3 layer (32,768 tokens each): kv800.decode's default
    plan, HIP events, median of 200 launches after 100; the small-batch regime of a serving engine, where each
    workgroup's sub-block chain and not HBM sets the time."""
    import lfm3_kv800_amd.kv800 as kv
    s = torch.cuda.current_stream(q.device)
    res = {}
    for b in sizes:
        Pb = kv.Paged(qpool=P.qpool, boff=P.boff[:b].contiguous(), epool=P.epool, eoff=P.eoff[:b].contiguous(),
                      ebs=P.ebs, e_hs=P.e_hs, e_ts=P.e_ts, e_v=P.e_v, sk=None, sv=None, skoff=None, svoff=None,
                      N=P.N[:b].contiguous(), NQ=P.NQ[:b].contiguous(), nqmax=P.nqmax, win=0)
        qb = q[:b].contiguous()
        for _ in range(100):
            kh.decode(Pb, qb, cos, sin)
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(200)]
        for e0, e1 in ev:
            e0.record(s)
            kh.decode(Pb, qb, cos, sin)
            e1.record(s)
        ev[-1][1].synchronize()
        t = sorted(e0.elapsed_time(e1) * 1e3 for e0, e1 in ev)
        res[str(b)] = round(t[len(t) // 2], 1)
    return {"workload": "first B rows of the C3 layer (32,768 tokens each), whole kv800.decode, HIP events, median",
            "unit": "us", "us": res}


def rope_tables(torch, n, dev):
    """(cos, sin) (n, 32) bf16 of LFM3's full-attention layers (theta 1e6, fp32 product, bf16 cast)."""
    inv = 1.0 / (1e6 ** (torch.arange(0, 64, 2, dtype=torch.float32) / 128))
    fr = torch.arange(n, dtype=torch.float32)[:, None] * inv[None]
    return fr.cos().to(torch.bfloat16).to(dev), fr.sin().to(torch.bfloat16).to(dev)


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(torch, P, q, cos, sin, rows):
    """The reference's pure-torch decode restated on CPU torch (oracle/torch_port.py, torch_decode.py:27-80) over
    rows 0 .. rows-1 of the layer, on this host's cores (at most 16, the box's CPU share); and the C oracle
    (oracle/kv800_oracle.c, OpenMP) over the same rows. Returns ((port s, threads), (C oracle s, threads))."""
    import numpy as np
    from types import SimpleNamespace
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    import torch_port
    threads = max(1, min(16, len(os.sched_getaffinity(0))))
    torch.set_num_threads(threads)
    C = lambda t: t.detach().cpu()
    cp = SimpleNamespace(qpool=C(P.qpool), boff=C(P.boff), epool=C(P.epool), eoff=C(P.eoff), ebs=P.ebs, e_hs=P.e_hs,
                         e_ts=P.e_ts, e_v=P.e_v, sk=None, sv=None, skoff=None, svoff=None, N=C(P.N), NQ=C(P.NQ),
                         nqmax=P.nqmax, win=P.win)
    qc, cc, sc = C(q), C(cos), C(sin)
    torch_port.decode(cp, qc, cc, sc, rows=[0])                      # page in, warm the allocator
    t0 = time.perf_counter()
    torch_port.decode(cp, qc, cc, sc, rows=range(rows))
    t_port = time.perf_counter() - t0
    # the C oracle over the same rows (its sub-blocks re-addressed into a compact pool)
    N2 = lambda t: t.detach().cpu().contiguous().numpy()
    B16 = lambda t: N2(t).view(np.uint16)
    sel = list(range(rows))
    blocks = torch.from_numpy((N2(P.boff)[sel] // 51200).reshape(-1)).to(P.qpool.device)
    qpool = N2(P.qpool.view(-1, 51200).index_select(0, blocks))
    case = oracle.PagedCase(qpool=qpool, boff=(np.arange(rows * NQ, dtype=np.int64) * 51200).reshape(rows, NQ),
                            epool=B16(P.epool.view(torch.int16)), eoff=N2(P.eoff)[sel], ebs=P.ebs, e_hs=P.e_hs,
                            e_ts=P.e_ts, e_v=P.e_v, sk=np.zeros(1, np.uint16), sv=np.zeros(1, np.uint16),
                            skoff=np.zeros(rows, np.int64), svoff=np.zeros(rows, np.int64), sinks=False,
                            N=N2(P.N)[sel], NQ=N2(P.NQ)[sel], nqmax=NQ, win=0, B=rows)
    qb, cb, sb = B16(q.view(torch.int16))[sel], B16(cos.view(torch.int16)), B16(sin.view(torch.int16))
    t0 = time.perf_counter()
    oracle.decode(case, qb, cb, sb)
    t_c = time.perf_counter() - t0
    return (t_port, threads), (t_c, oracle.num_threads())


C1_B, C1_N, C1_ITERS = 4, 1024, 10


def build_c1(torch, dev):
    """config C1: one quantized layer of 4 sequences x 1024 tokens in PagedStore's default geometry
    (ebs 64, ring of 10 pages), q / K / V ~ N(0, 1) bf16 from seed 1, written and flushed by this build's HIP path
    (3 sub-blocks + 256 exact tokens per row). Returns (Paged, q, cos, sin) on the device."""
    import lfm3_kv800_amd.kv800 as kv
    g = torch.Generator(device=dev).manual_seed(1)
    st = kv.PagedStore(C1_B, C1_N + 8, dev)
    st.append(torch.randn(C1_B, C1_N, 4, 128, generator=g, device=dev).to(torch.bfloat16),
              torch.randn(C1_B, C1_N, 4, 128, generator=g, device=dev).to(torch.bfloat16))
    q = torch.randn(C1_B, 16, 128, generator=g, device=dev).to(torch.bfloat16)
    cos, sin = rope_tables(torch, C1_N + 8, dev)
    return st.paged(), q, cos, sin


def cpu_baseline_c1(torch, host, threads):
    """C1 on this host's cores: the pure-torch restatement of torch_decode.decode (oracle/torch_port.py), one warm-up
    call then C1_ITERS timed calls. Returns ms per call."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import torch_port
    torch.set_num_threads(threads)
    P, q, cos, sin = host
    torch_port.decode(P, q, cos, sin)
    t0 = time.perf_counter()
    for _ in range(C1_ITERS):
        torch_port.decode(P, q, cos, sin)
    return (time.perf_counter() - t0) * 1e3 / C1_ITERS


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=500)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-rows", type=int, default=64)
    ap.add_argument("--calib", action="store_true", help="plain copy of known size (rocprof FETCH/WRITE calibration)")
    ap.add_argument("--c3-only", action="store_true", help="skip the C2 / C4 / C5 workloads (counter passes of the C3 kernel)")
    ap.add_argument("--e2e-only", action="store_true", help="only the C5 decode loop; prints its record")
    ap.add_argument("--c2-only", action="store_true", help="only the C2 flush (counter passes of the flush kernel)")
    ap.add_argument("--c4-only", action="store_true", help="only the C4 step; prints its record")
    ap.add_argument("--prefill-only", action="store_true", help="only the prefill workload; prints its record")
    ap.add_argument("--window-only", action="store_true", help="only the 398-row window layer; prints its record")
    ap.add_argument("--e2e-steps", type=int, default=128)
    ap.add_argument("--e2e-which", choices=("both", "256", "398"), default="both",
                    help="with --e2e-only: the 256-sequence loop, the 398 x 32K one, or both")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py: this build measures one GPU only (--gpus {a.gpus} requested); the 800h path shards by "
              "sequence with no exchange, so N GPUs would run N independent copies of this workload", file=sys.stderr)
        sys.exit(2)
    import torch
    import lfm3_kv800_amd.kv800_hip as kh
    kh.ops()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)

    if a.e2e_only:
        rec = {}
        if a.e2e_which in ("both", "256"):
            rec["e2e"] = bench_e2e(torch, dev, a.e2e_steps)
            torch.cuda.empty_cache()
        if a.e2e_which in ("both", "398"):
            rec["e2e_398x32k"] = bench_e2e(torch, dev, 32, lens=[C4_MAX] * C4_R)
        print(json.dumps(rec), flush=True)
        return

    if a.c2_only:
        print(json.dumps({"flush_c2": bench_flush_c2(torch, kh, dev, a.steps, a.warmup)}), flush=True)
        return

    if a.window_only:
        print(json.dumps({"window_398": bench_window(torch, kh, dev, max(a.steps, 20), max(a.warmup, 200))}),
              flush=True)
        return

    if a.prefill_only:
        print(json.dumps({"prefill": bench_prefill(torch, kh, dev, max(3, a.steps), 2)}), flush=True)
        return

    if a.c4_only:
        cos4, sin4 = rope_tables(torch, C4_MAX + 64, dev)
        print(json.dumps({"c4": bench_c4(torch, kh, dev, max(5, min(a.steps, 20)), 20, cos4, sin4)}), flush=True)
        return

    if a.calib:
        x = torch.empty(1 << 28, dtype=torch.int32, device=dev)      # 1 GiB
        y = torch.empty_like(x)
        for _ in range(3):
            y.copy_(x)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(a.steps):
            y.copy_(x)
        e1.record(); e1.synchronize()
        ms = e0.elapsed_time(e1) / a.steps
        print(json.dumps({"calib": "copy", "bytes_read": x.numel() * 4, "bytes_written": x.numel() * 4,
                          "ms": ms, "gbps": 2 * x.numel() * 4 / ms / 1e6}))
        return

    t_build = time.perf_counter()
    layers = [build_layer(torch, kh, seed, dev) for seed in (1, 2)]
    g = torch.Generator(device=dev).manual_seed(7)
    q = torch.randn(B, 16, 128, generator=g, device=dev).to(torch.bfloat16)
    cos, sin = rope_tables(torch, N_CTX, dev)
    kh.rope_pairs(cos, sin)                                          # model-constant table, built once
    torch.cuda.synchronize()
    log(f"built 2 cache copies in {time.perf_counter() - t_build:.1f} s")

    # ---- whole-layer timing: W warmup + K timed steps, synchronized on both sides
    with frozen_heap():
        warm_layer = warm_up(torch, lambda i: kh.decode(layers[i & 1], q, cos, sin), max(a.warmup, C3_WARM_CALLS),
                             C3_WARM_MS)
        t0 = time.perf_counter()
        for i in range(a.steps):
            kh.decode(layers[i & 1], q, cos, sin)
        torch.cuda.synchronize()
        ms_step = (time.perf_counter() - t0) * 1e3 / a.steps

    # ---- dominant kernel alone (decode_quant), HIP events on the stream it runs on
    import ctypes
    L = kh.ops()
    s = torch.cuda.Stream(device=dev)
    ns, spb = kh.plan(B, NQ)
    MO = torch.empty(B, ns + 1, 16, dtype=torch.float32, device=dev)
    LO = torch.empty_like(MO)
    AO = torch.empty(B, ns + 1, 16, 128, dtype=torch.float32, device=dev)
    cs2 = kh.rope_pairs(cos, sin)
    scale = 128 ** -0.5 * 1.4426950408889634
    structs = [kh.paged_struct(P, B) for P in layers]

    def quant(i):
        P, (st, qbytes, _, _) = layers[i & 1], structs[i & 1]
        rc = L.kv800_hip_decode_quant_sized(ctypes.c_void_p(q.data_ptr()), st.qpool, qbytes, st.boff, st.boff_stride,
                                            ctypes.c_void_p(P.NQ.data_ptr()), ctypes.c_void_p(cs2.data_ptr()),
                                            cos.shape[0], ctypes.c_void_p(MO.data_ptr()), ctypes.c_void_p(LO.data_ptr()),
                                            ctypes.c_void_p(AO.data_ptr()), B, ns, spb, scale,
                                            ctypes.c_void_p(s.cuda_stream))
        assert rc == 0, L.kv800_hip_last_error()

    # the K launches back to back between one event pair on their stream: the average launch duration, including the
    # short dispatch gap between consecutive kernels; then one event pair around each launch, whose average also
    # carries the event packets' own time (reported beside it)
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(a.steps)]
    e_all = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
    with torch.cuda.stream(s), frozen_heap():
        warm_kernel = warm_up(torch, quant, max(a.warmup, C3_WARM_CALLS), C3_WARM_MS)
        e_all[0].record(s)
        for i in range(a.steps):
            quant(i)
        e_all[1].record(s)
        for i in range(a.steps):
            ev[i][0].record(s)
            quant(i)
            ev[i][1].record(s)
        ev[-1][1].synchronize()
    ms_quant = e_all[0].elapsed_time(e_all[1]) / a.steps
    ms_quant_each = sum(e0.elapsed_time(e1) for e0, e1 in ev) / a.steps
    torch.cuda.synchronize()

    out = kh.decode(layers[0], q, cos, sin)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    small = decode_small_batches(torch, kh, layers[0], q, cos, sin) if not a.c3_only else None

    achieved = QBYTES / (ms_quant * 1e-3) / 1e9
    layer_gbps = ALG_BYTES / (ms_step * 1e-3) / 1e9
    # the CPU baseline runs last, on a host copy of the layer: its 16 busy threads would otherwise share the host with
    # the launches of the GPU sections below (a C4 step issues ~60 launches)
    from types import SimpleNamespace
    P0 = layers[0]
    C = lambda t: t.detach().cpu() if t is not None else None
    host_layer = SimpleNamespace(qpool=C(P0.qpool), boff=C(P0.boff), epool=C(P0.epool), eoff=C(P0.eoff), ebs=P0.ebs,
                                 e_hs=P0.e_hs, e_ts=P0.e_ts, e_v=P0.e_v, sk=None, sv=None, skoff=None, svoff=None,
                                 N=C(P0.N), NQ=C(P0.NQ), nqmax=P0.nqmax, win=P0.win) if not a.no_cpu else None
    host_q, host_cos, host_sin = C(q), C(cos), C(sin)
    # C1: built and timed on the GPU here (whole kv800.decode call), its host copy timed on the CPU at the end
    c1_gpu_ms = host_c1 = None
    if not a.no_cpu:
        P1, q1, cos1, sin1 = build_c1(torch, dev)
        for _ in range(20):
            kh.decode(P1, q1, cos1, sin1)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(200):
            kh.decode(P1, q1, cos1, sin1)
        torch.cuda.synchronize()
        c1_gpu_ms = (time.perf_counter() - t0) * 1e3 / 200
        host_c1 = (SimpleNamespace(qpool=C(P1.qpool), boff=C(P1.boff), epool=C(P1.epool), eoff=C(P1.eoff),
                                   ebs=P1.ebs, e_hs=P1.e_hs, e_ts=P1.e_ts, e_v=P1.e_v, sk=None, sv=None, skoff=None,
                                   svoff=None, N=C(P1.N), NQ=C(P1.NQ), nqmax=P1.nqmax, win=P1.win),
                   C(q1), C(cos1), C(sin1))
        del P1, q1, cos1, sin1

    # ---- the other BASELINE.json configs with a GPU workload: C2 (flush alone), C4 (6-layer decode step), C5 (engine loop)
    del layers, structs
    torch.cuda.empty_cache()
    extra_steps = max(5, min(a.steps, 20))
    flush_c2 = c4 = e2e = e2e_398 = prefill = fake_quant = copy = read = window = None
    if not a.c3_only:
        copy = bench_copy(torch, dev, 10)
        read = bench_read(torch, kh, dev, 10)
        read["decode_quant_frac_of_read"] = round(achieved / read["gbps"], 4)
        prefill = bench_prefill(torch, kh, dev, max(3, min(a.steps, 10)), 2)
        torch.cuda.empty_cache()
        fake_quant = bench_fake_quant(torch, kh, dev, extra_steps, 5)
        torch.cuda.empty_cache()
        window = bench_window(torch, kh, dev, max(a.steps, 20), 200)
        torch.cuda.empty_cache()
        flush_c2 = bench_flush_c2(torch, kh, dev, extra_steps, 200)
        torch.cuda.empty_cache()
        cos4, sin4 = rope_tables(torch, C4_MAX + 64, dev)
        c4 = bench_c4(torch, kh, dev, extra_steps, 20, cos4, sin4)
        del cos4, sin4
        torch.cuda.empty_cache()
        e2e = bench_e2e(torch, dev, a.e2e_steps)
        e2e["workload"] = "C5: " + e2e["workload"]
        e2e_398 = bench_e2e(torch, dev, 32, lens=[C4_MAX] * C4_R)
    cpu = None
    if not a.no_cpu:
        rows = max(1, min(B, a.cpu_rows))
        (dt, cores), (dt_c, cores_c) = cpu_baseline(torch, host_layer, host_q, host_cos, host_sin, rows)
        cpu = {"value": round(dt * 1e3 * B / rows, 1), "unit": "ms/layer (64x32K, scaled from the sample)",
               "cores": cores, "cpu_model": cpu_model(), "kind": "port",
               "sample": f"pure-torch restatement of torch_decode.decode (oracle/torch_port.py) on rows 0..{rows - 1} "
                         f"of the 64 x 32768 layer, {cores} torch threads: {dt:.2f} s, scaled by 64/{rows}",
               "c_oracle_ms_per_layer": round(dt_c * 1e3 * B / rows, 1), "c_oracle_threads": cores_c}
        c1_ms = cpu_baseline_c1(torch, host_c1, cores)
        cpu["c1"] = {"workload": "C1: one quantized layer, 4 seqs x 1024 tokens (3 sub-blocks + 256 exact tokens per "
                                 "seq), PagedStore default geometry, N(0,1) q/K/V",
                     "cpu_ms_per_call": round(c1_ms, 3), "iters": C1_ITERS, "cores": cores,
                     "gpu_ms_per_call": round(c1_gpu_ms, 4),
                     "sample": f"oracle/torch_port.py decode of all 4 rows, {C1_ITERS} timed calls after one warm-up"}
    res = {
        "metric": "800h decode ms/layer @64x32K",
        "value": round(ms_step, 5), "unit": "ms", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": round(ms_step, 5), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "u8 codes / bf16 QK + fp16 PV MFMA / fp32 accumulate", "data": "synthetic",
        "c3_warmup": {"layer_steps": warm_layer[0], "layer_ms": warm_layer[1], "kernel_launches": warm_kernel[0],
                      "kernel_ms": warm_kernel[1], "rule": f"max(--warmup, {C3_WARM_CALLS}) calls and >= "
                                                          f"{C3_WARM_MS:.0f} ms per timed C3 section"},
        "config": {"workload": "C3: one layer paged decode, 64 seqs x 32768 tokens, 16 q / 4 kv heads x 128, "
                               "NQ=127 sub-blocks + 256 exact tokens per seq, permuted page tables, 2 rotating copies",
                   "global_batch": B, "seq_len": N_CTX, "parallelism": "none (1 GPU)"},
        "layer": {"algorithmic_bytes": ALG_BYTES, "gbps": round(layer_gbps, 1),
                  "hbm_frac": round(layer_gbps / HBM_PEAK_GBS, 4), "decode_tok_s": round(B / (ms_step * 1e-3), 1)},
        "roofline": {"bound": "hbm", "kernel": "decode_quant_kernel", "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(), "kernel_ms": round(ms_quant, 5),
                     "kernel_ms_event_pair_each": round(ms_quant_each, 5), "bytes_per_launch": QBYTES},
        "cpu_baseline": cpu,
        "flush_c2": flush_c2,
        "c4": c4,
        "e2e": e2e,
        "e2e_398x32k": e2e_398,
        "prefill": prefill,
        "fake_quant": fake_quant,
        "window_398": window,
        "hbm_copy": copy,
        "hbm_read": read,
        "decode_small_batch": small,
    }
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
