"""One step of the 800h attention layers on caches with vLLM's page geometry, without vLLM.

Counterpart of the reference's vLLM integration (vllm_attn.py:214-402, KV800Attention.forward), with the same cache
layout so that pages written here are the pages vLLM would hold:

  quantized layers (6, 10, 14, 22): a quant cache of 1280-token pages, 5 x 51,200-byte sub-blocks padded to 262,144 B
      (vllm_attn.py:36-37, 126-131), block table shared by the four layers (one FullAttention KV group), plus an exact
      cache of [4 heads, ebs, K128 | V128] bf16 pages (sliding window 640) in the layer's exact KV group;
  window layers (2, 18): the exact cache only; their 4 sink tokens live in the 6,144-byte aux area at byte 256,000 of
      the first quant page of the host layers (6, 10) / (14, 22) (vllm_attn.py:3-9, 276-291).

One step of one layer takes a vLLM-shaped batch: decode rows (one token each) first, then extend / prefill rows of
any chunk length (query_start_loc, seq_lens). It writes the K / V rows of every scheduled token into the exact pages
(and positions < 4 into the sink aux), flushes the sub-blocks that became eligible (n >= 256 j + 384) in
[nq(seq_len - query_len), nq(seq_len)) per row from this layer's own exact group (the 0.1.1 fix, vllm_attn.py:301),
decodes the decode rows with the fused decode and attends the extend rows over their compressed history
(vllm_attn.py:351-402). Every piece is a launch of libkv800_hip.so on the current stream; the only host values are
the ones the reference also reads on the host (the rows' sequence and query lengths)."""
from dataclasses import dataclass, field

import numpy as np
import torch

from . import kv800, kv800_hip

QUANT_LAYERS, WINDOW_LAYERS = (6, 10, 14, 22), (2, 18)
SLIDE_LAYERS = (4, 8, 12, 16, 20)              # LFM3's native sliding-window layers (vllm_attn.py:217-222)
SINK_HOST = {2: (6, 10), 18: (14, 22)}     # window layer -> (layer whose aux holds the sink K, ... the sink V)
EXACT_WINDOW = 640
QBLOCK, QPAGE = 1280, 262144
AUX_BYTES = (QBLOCK // kv800.BLK) * kv800.SUB  # 256,000: start of the aux area in a quant page


@dataclass
class StepMeta:
    """Per-step metadata of one KV-cache group (the KV800Meta fields the attention reads, vllm_attn.py:64-75).
    block_table (R, blocks) int32; slot_mapping (T,) int64 slot of each scheduled token (-1: none); seq_lens (R,)
    int32 including the step's tokens; seq_lens_cpu the same on the host; positions (T,) int64. `cache` holds values
    shared by the layers of the group within the step.
    Mixed steps (mixed_step_meta) also carry query_start_loc_cpu (R + 1,) host int64, num_decodes (rows
    [0, num_decodes) have one token each, the rest are extend rows), query_lens (R,) int32 and req_of_tok (T,) int64
    (each token's row) on the device; a decode step (step_meta) leaves them None: one token per row, T = R."""
    block_table: torch.Tensor
    slot_mapping: torch.Tensor
    seq_lens: torch.Tensor
    seq_lens_cpu: torch.Tensor
    positions: torch.Tensor
    cache: dict = field(default_factory=dict)
    query_start_loc_cpu: torch.Tensor = None
    num_decodes: int = None
    query_lens: torch.Tensor = None
    req_of_tok: torch.Tensor = None

    @property
    def mixed(self):
        return self.query_start_loc_cpu is not None


def step_lens(seq_lens_cpu, device):
    """The rows' lengths on the device (int64). On a GPU the copy goes through freshly pinned host memory and does not
    block the host, so the next step can be prepared while the GPU still runs this one."""
    sl = seq_lens_cpu.to(torch.int64)
    device = torch.device(device)
    return sl.pin_memory().to(device, non_blocking=True) if device.type == "cuda" else sl.to(device)


def step_meta(block_table, seq_lens_cpu, ebs, device, seq_lens_dev=None):
    """StepMeta of a decode step in which every row appends one token at position seq_len - 1. seq_lens_dev: the same
    lengths already on the device (step_lens), shared by the KV groups of a step."""
    sl = seq_lens_cpu.to(torch.int64)
    dsl = step_lens(sl, device) if seq_lens_dev is None else seq_lens_dev
    bt = block_table.to(device=device, dtype=torch.int32)
    if bt.device.type == "cuda":   # one launch (kv800_hip_step_meta)
        slot, pos, dsl32 = kv800_hip.step_meta(bt.contiguous(), dsl, ebs)
        return StepMeta(bt, slot, dsl32, sl, pos)
    pos = dsl - 1
    page = bt.gather(1, (pos // ebs)[:, None].long())[:, 0].long()
    slot = page * ebs + pos % ebs
    return StepMeta(bt, slot, dsl.to(torch.int32), sl, pos)


def mixed_step_meta(block_table, seq_lens_cpu, query_lens_cpu, ebs, device, num_decodes=None):
    """StepMeta of a vLLM-shaped step of one KV group: row r schedules query_lens[r] >= 1 tokens at positions
    seq_lens[r] - query_lens[r] .. seq_lens[r] - 1 (decode rows first, then extend rows, as vLLM orders a batch,
    vllm_attn.py:244-277). block_table (R, blocks) on the host; num_decodes defaults to the leading rows with one
    token. Slots and positions are formed on the host, as vLLM's scheduler forms slot_mapping."""
    bt = torch.as_tensor(block_table).to(torch.int32).cpu()
    sl = torch.as_tensor(seq_lens_cpu).to(torch.int64).cpu()
    ql = torch.as_tensor(query_lens_cpu).to(torch.int64).cpu()
    R = sl.shape[0]
    if bt.dim() != 2 or bt.shape[0] != R or ql.shape != (R,):
        raise ValueError("block_table (R, blocks), seq_lens (R,) and query_lens (R,) must agree")
    if bool((ql < 1).any()) or bool((ql > sl).any()):
        raise ValueError("every row needs 1 <= query_len <= seq_len")
    qsl = torch.zeros(R + 1, dtype=torch.int64)
    qsl[1:] = torch.cumsum(ql, 0)
    T = int(qsl[-1])
    req = torch.repeat_interleave(torch.arange(R), ql)
    pos = torch.arange(T) - qsl[:-1][req] + (sl - ql)[req]
    if bool((pos // ebs >= bt.shape[1]).any()):
        raise ValueError("the block table does not cover the step's positions")
    slot = bt[req, pos // ebs].to(torch.int64) * ebs + pos % ebs
    if num_decodes is None:
        nd = 0
        while nd < R and int(ql[nd]) == 1:
            nd += 1
    else:
        nd = int(num_decodes)
        if not 0 <= nd <= R or bool((ql[:nd] != 1).any()):
            raise ValueError("decode rows must come first, one token each")
    dev = torch.device(device)
    up = (lambda t: t.pin_memory().to(dev, non_blocking=True)) if dev.type == "cuda" else (lambda t: t.to(dev))
    return StepMeta(up(bt), up(slot), up(sl.to(torch.int32)), sl, up(pos), query_start_loc_cpu=qsl, num_decodes=nd,
                    query_lens=up(ql.to(torch.int32)), req_of_tok=up(req))


def _max_flush(m):
    """Most sub-blocks any row of the step becomes eligible for (host values): nq(seq_len) - nq(seq_len - query_len)."""
    sl = m.seq_lens_cpu.to(torch.int64)
    ql = (m.query_start_loc_cpu[1:] - m.query_start_loc_cpu[:-1]) if m.mixed else torch.ones_like(sl)
    nq = lambda n: torch.clamp(n - kv800.LAG, min=0) // kv800.BLK
    return int((nq(sl) - nq(sl - ql)).max()) if sl.numel() else 0


class KV800DecodeLayer:
    """One LFM3 full-attention layer's decode step over its 800h caches. exact: (pages, 4, ebs, 256) bf16 [K | V];
    quant: (qpages, 262144) uint8 for quantized layers, None for window layers."""

    def __init__(self, layer_idx, exact, quant=None):
        self.l = layer_idx
        self.win = layer_idx in WINDOW_LAYERS
        if self.win == (quant is not None):
            raise ValueError(f"layer {layer_idx}: window layers take no quant cache, quantized layers need one")
        if exact.dtype != torch.bfloat16 or exact.dim() != 4 or exact.shape[1] != 4 or exact.shape[3] != 256:
            raise ValueError("exact cache must be (pages, 4, ebs, 256) bf16")
        if quant is not None and (quant.dtype != torch.uint8 or quant.dim() != 2 or quant.shape[1] != QPAGE
                                  or quant.stride(0) != QPAGE or quant.stride(1) != 1):
            raise ValueError(f"quant cache must be a contiguous (pages, {QPAGE}) uint8 tensor")
        self.ev, self.qv = exact, quant
        self.ebs = exact.shape[2]
        self._zeros = None   # NQ = 0 rows of the window decode

    def forward(self, q, k, v, mx: StepMeta, mq: StepMeta = None, hosts=None, cos_t=None, sin_t=None, max_new=1):
        """q (T, 16, 128) post-RoPE, k (T, 4, 128) pre-RoPE, v (T, 4, 128), all bf16, one row per scheduled token.
        mx: this layer's exact-group metadata; mq: the quant group's (quantized layers, and the sink hosts of window
        layers); hosts: {layer: KV800DecodeLayer} holding the sink hosts' quant caches (window layers); cos_t / sin_t
        (P, 32) bf16 RoPE tables; max_new: most sub-blocks any row can become eligible for in a decode step (1).
        A mixed step (mx.mixed) runs the decode rows and the extend rows of the batch (vllm_attn.py:244-402)."""
        if mx.mixed:
            return self._forward_mixed(q, k, v, mx, mq, hosts, cos_t, sin_t)
        ev, ebs = self.ev, self.ebs
        s0, s1, s2 = ev.stride(0), ev.stride(1), ev.stride(2)
        R = q.shape[0]
        # ---- per-step tables, built once per KV group and shared by its layers: the exact group's page offsets, and
        # the quant group's decode / flush / sink tables (one launch each)
        eoff = self._eoff(mx)
        boff, NQ, NP, qbt64, aux, nqmax = _step_tables(mq)
        N = mx.seq_lens
        if self.win:
            # ---- step rows into the exact window pages, sink rows into the hosts' aux, then the window decode
            kh, vh = (hosts[h] for h in SINK_HOST[self.l])
            skb, svb = kh.qv.view(torch.bfloat16), vh.qv.view(torch.bfloat16)
            kv800_hip.write_exact(ev, mx.slot_mapping, k, v, pos=mx.positions, sk=skb, sv=svb, skoff=aux, svoff=aux)
            if self._zeros is None or self._zeros.shape[0] < R:
                self._zeros = torch.zeros(max(R, 64), dtype=torch.int32, device=ev.device)
            P = kv800.Paged(qpool=ev, boff=eoff, epool=ev, eoff=eoff, ebs=ebs, e_hs=s1, e_ts=s2, e_v=128, sk=skb, sv=svb,
                            skoff=aux, svoff=aux, N=N, NQ=self._zeros[:R], nqmax=0, win=kv800.WIN)
            return kv800_hip.decode(P, q, cos_t, sin_t)
        kv800_hip.write_exact(ev, mx.slot_mapping, k, v)
        # ---- flush the sub-blocks that became eligible this step ([NP, NQ) per row), from this layer's own exact group;
        # if launch_flushes ran it ahead on the side stream, wait for it instead
        done = mq.cache.get(("flushed", self.l))
        if done is not None:
            torch.cuda.current_stream(ev.device).wait_event(done)
        else:
            self._flush(mx, mq, max_new)
        # ---- the fused decode
        P = kv800.Paged(qpool=self.qv, boff=boff, epool=ev, eoff=eoff, ebs=ebs, e_hs=s1, e_ts=s2, e_v=128, sk=None,
                        sv=None, skoff=None, svoff=None, N=N, NQ=NQ, nqmax=nqmax, win=0)
        return kv800_hip.decode(P, q, cos_t, sin_t)

    def _sinks(self, hosts):
        """The sink buffers of a window layer: the quant caches of its two host layers as bf16."""
        kh, vh = (hosts[h] for h in SINK_HOST[self.l])
        return kh.qv.view(torch.bfloat16), vh.qv.view(torch.bfloat16)

    def write_step(self, k, v, mx: StepMeta, mq: StepMeta, hosts=None):
        """The cache half of a step (vllm_attn.py:255-317): the K / V rows of every scheduled token (k, v (T, 4, 128)
        bf16, pre-RoPE K) into this layer's exact pages; window layers also put positions < 4 into the sink aux of
        their hosts; quantized layers then flush, from their own exact group, the sub-blocks [NP, NQ) of every row
        (NP = nq(seq_len - query_len)), after this step's rows are in the pages (an extend row's new sub-blocks are
        made of them)."""
        ev = self.ev
        boff, NQ, NP, qbt64, aux, nqmax = _step_tables(mq)
        if self.win:
            skb, svb = self._sinks(hosts)
            at = aux.index_select(0, mx.req_of_tok) if mx.mixed else aux
            kv800_hip.write_exact(ev, mx.slot_mapping, k, v, pos=mx.positions, sk=skb, sv=svb, skoff=at, svoff=at)
            return
        kv800_hip.write_exact(ev, mx.slot_mapping, k, v)
        mnew = _max_flush(mq)
        if mnew > 0:
            kv800_hip.flush(ev, self._eoff(mx), self.ebs, ev.stride(1), ev.stride(2), 128, self.qv, qbt64, QBLOCK, QPAGE,
                            NP, NQ, mnew, latency=mnew <= 2)

    def _forward_mixed(self, q, k, v, mx, mq, hosts, cos_t, sin_t):
        """A mixed step: write_step, then the decode rows through the fused decode and the extend rows through the
        prefill over compressed history (quantized layers: the row's nq(prev) sub-blocks dequantized, the exact rows
        from 256 nq(prev) on, then its new rows; window layers: sinks, the last 255 exact rows, the new rows)."""
        ev, ebs = self.ev, self.ebs
        s1, s2 = ev.stride(1), ev.stride(2)
        qsl = mx.query_start_loc_cpu
        R, T, nd = qsl.shape[0] - 1, int(qsl[-1]), mx.num_decodes
        self.write_step(k, v, mx, mq, hosts)
        eoff = self._eoff(mx)
        boff, NQ, NP, qbt64, aux, nqmax = _step_tables(mq)
        out = torch.empty(T, 16, 128, dtype=torch.bfloat16, device=q.device)
        prev = (mx.seq_lens_cpu - (qsl[1:] - qsl[:-1])).tolist()
        t0 = int(qsl[nd])
        eq = (qsl[nd:] - t0).tolist()
        if self.win:
            skb, svb = self._sinks(hosts)
            if self._zeros is None or self._zeros.shape[0] < R:
                self._zeros = torch.zeros(max(R, 64), dtype=torch.int32, device=ev.device)
            if nd:
                P = kv800.Paged(qpool=ev, boff=eoff[:nd], epool=ev, eoff=eoff[:nd], ebs=ebs, e_hs=s1, e_ts=s2, e_v=128,
                                sk=skb, sv=svb, skoff=aux[:nd], svoff=aux[:nd], N=mx.seq_lens[:nd],
                                NQ=self._zeros[:nd], nqmax=0, win=kv800.WIN)
                out[:nd] = kv800_hip.decode(P, q[:nd], cos_t, sin_t)
            if R > nd:
                P = kv800.Paged(qpool=None, boff=None, epool=ev, eoff=eoff[nd:], ebs=ebs, e_hs=s1, e_ts=s2, e_v=128,
                                sk=skb, sv=svb, skoff=aux[nd:], svoff=aux[nd:], N=mx.seq_lens[nd:],
                                NQ=self._zeros[:R - nd], nqmax=0, win=kv800.WIN)
                out[t0:] = prefill_window_rows(P, q[t0:T], k[t0:T], v[t0:T], eq, prev[nd:], cos_t, sin_t)
            return out
        if nd:
            P = kv800.Paged(qpool=self.qv, boff=boff[:nd], epool=ev, eoff=eoff[:nd], ebs=ebs, e_hs=s1, e_ts=s2, e_v=128,
                            sk=None, sv=None, skoff=None, svoff=None, N=mx.seq_lens[:nd], NQ=NQ[:nd], nqmax=nqmax,
                            win=0)
            out[:nd] = kv800_hip.decode(P, q[:nd], cos_t, sin_t)
        if R > nd:
            P = kv800.Paged(qpool=self.qv, boff=boff[nd:], epool=ev, eoff=eoff[nd:], ebs=ebs, e_hs=s1, e_ts=s2, e_v=128,
                            sk=None, sv=None, skoff=None, svoff=None, N=mx.seq_lens[nd:], NQ=NP[nd:], nqmax=nqmax,
                            win=0)
            out[t0:] = prefill_quant_rows(P, q[t0:T], k[t0:T], v[t0:T], eq, prev[nd:], cos_t, sin_t)
        return out

    def _eoff(self, mx):
        """The exact group's page offsets for this cache's page stride (one launch per group and step)."""
        key = ("eoff", self.ev.stride(0))
        if key not in mx.cache:
            mx.cache[key] = kv800_hip.page_offsets(mx.block_table, self.ev.stride(0))
        return mx.cache[key]

    def _flush(self, mx, mq, max_new=1):
        """This step's flush of a quantized layer on the current stream: rows r quantize sub-blocks [NP[r], NQ[r])
        of this layer's own exact group into its quant pages."""
        ev = self.ev
        _, NQ, NP, qbt64, _, _ = _step_tables(mq)
        kv800_hip.flush(ev, self._eoff(mx), self.ebs, ev.stride(1), ev.stride(2), 128, self.qv, qbt64, QBLOCK, QPAGE, NP,
                        NQ, max_new, latency=True)


class KV800SlideLayer:
    """One LFM3 native sliding-window layer's decode step (vllm_attn.py:217-222, 253-254, 325-326 with slide=True):
    window 256 without sinks, K stored after the layer's own RoPE (theta 1e4, all 64 frequencies) and read with the
    identity tables, so the exact-window kernel only attends. exact: (pages, 4, ebs, 256) bf16 [K | V] of the layer's
    own sliding KV group."""

    def __init__(self, layer_idx, exact):
        if exact.dtype != torch.bfloat16 or exact.dim() != 4 or exact.shape[1] != 4 or exact.shape[3] != 256:
            raise ValueError("exact cache must be (pages, 4, ebs, 256) bf16")
        self.l, self.ev, self.ebs = layer_idx, exact, exact.shape[2]
        self.win = True
        self._zeros = None
        self._ident = None

    def identity_tables(self, rows):
        """(cos, sin) (rows, 32) bf16 of ones / zeros: the kernel's RoPE then leaves the stored keys as they are."""
        if self._ident is None or self._ident[0].shape[0] < rows:
            n = max(2 * rows, 4096)   # grown ahead: a decode step asks for one more row each time
            self._ident = (torch.ones(n, 32, dtype=torch.bfloat16, device=self.ev.device),
                           torch.zeros(n, 32, dtype=torch.bfloat16, device=self.ev.device))
        return self._ident

    def write_step(self, k, v, mx: StepMeta):
        """The K / V rows (post-RoPE K) of every scheduled token into the sliding pages."""
        kv800_hip.write_exact(self.ev, mx.slot_mapping, k, v)

    def forward(self, q, k, v, mx: StepMeta):
        """q (T, 16, 128) post-RoPE, k (T, 4, 128) POST-RoPE, v (T, 4, 128), bf16, one row per scheduled token;
        mx: the layer's sliding-group metadata. A mixed step's extend rows attend their last 255 positions and their
        new rows (vllm_attn.py:351-402 with slide=True)."""
        ev, ebs = self.ev, self.ebs
        R = mx.seq_lens.shape[0]
        key = ("eoff", ev.stride(0))
        if key not in mx.cache:
            mx.cache[key] = kv800_hip.page_offsets(mx.block_table, ev.stride(0))
        eoff = mx.cache[key]
        self.write_step(k, v, mx)
        if self._zeros is None or self._zeros.shape[0] < R:
            self._zeros = torch.zeros(max(R, 64), dtype=torch.int32, device=ev.device)
        nd = mx.num_decodes if mx.mixed else R
        cos1, sin0 = self.identity_tables(int(mx.seq_lens_cpu.max()) + 1)
        out = torch.empty(q.shape[0], 16, 128, dtype=torch.bfloat16, device=q.device) if mx.mixed else None
        if nd:
            P = kv800.Paged(qpool=ev, boff=eoff[:nd], epool=ev, eoff=eoff[:nd], ebs=ebs, e_hs=ev.stride(1),
                            e_ts=ev.stride(2), e_v=128, sk=None, sv=None, skoff=None, svoff=None, N=mx.seq_lens[:nd],
                            NQ=self._zeros[:nd], nqmax=0, win=kv800.WIN)
            o = kv800_hip.decode(P, q[:nd], cos1, sin0)
            if not mx.mixed:
                return o
            out[:nd] = o
        if R > nd:
            qsl = mx.query_start_loc_cpu
            t0, T = int(qsl[nd]), int(qsl[-1])
            prev = (mx.seq_lens_cpu - (qsl[1:] - qsl[:-1])).tolist()
            P = kv800.Paged(qpool=None, boff=None, epool=ev, eoff=eoff[nd:], ebs=ebs, e_hs=ev.stride(1),
                            e_ts=ev.stride(2), e_v=128, sk=None, sv=None, skoff=None, svoff=None, N=mx.seq_lens[nd:],
                            NQ=self._zeros[:R - nd], nqmax=0, win=kv800.WIN)
            out[t0:] = prefill_window_rows(P, q[t0:T], k[t0:T], v[t0:T], (qsl[nd:] - t0).tolist(), prev[nd:], None,
                                           None)
        return out


def _step_tables(mq):
    """(boff, NQ, NP, qbt64, aux, nqmax) of the quant group for this step, built once (kv800_hip_step_tables); NP
    counts each row's sub-blocks before its query_len new tokens (one for a decode step)."""
    if ("step",) not in mq.cache:
        nqmax = int(torch.clamp(mq.seq_lens_cpu.to(torch.int64) - kv800.LAG, min=0).max()) // kv800.BLK
        nnew = mq.query_lens if mq.mixed else 1
        mq.cache[("step",)] = kv800_hip.step_tables(mq.block_table, QBLOCK, QPAGE, mq.seq_lens, nqmax, nnew=nnew,
                                                    aux_scale=QPAGE // 2, aux_add=AUX_BYTES // 2) + (nqmax,)
    return mq.cache[("step",)]


_SIDE = {}


def launch_flushes(layers, metas, mq, max_new=1):
    """Start this step's flushes of the quantized layers at once, on a side stream (default priority), so that they
    run under the layers queued before the first quantized one (a window layer, the new-token writes); each quantized
    layer's forward waits for all of them. A flush running beside a quantized layer's decode grid slows that grid far
    more than the flush takes alone (C4: one decode 400 -> 650 us beside the next layer's flush; the step 2.06 -> 1.97
    ms with every flush done before the first quantized decode). A step's flush reads tokens written in earlier steps
    only (sub-block j flushes at n >= 256 j + 384, so it ends 128 tokens before the step's token), and the side stream
    first waits for everything queued so far on the current stream.
    layers: the KV800DecodeLayer objects of the step; metas: {layer index: its exact group's StepMeta}; mq: the quant
    group's StepMeta. Call once per step, before the step's first attention layer. A mixed step starts none (its
    extend rows flush sub-blocks made of this step's own tokens): each layer's forward flushes after its writes."""
    quant = [l for l in layers if not l.win]
    if not quant or mq.mixed:
        return
    dev = quant[0].ev.device
    main = torch.cuda.current_stream(dev)
    tabs = _step_tables(mq)                        # tables built on the current stream, before the fork
    eoffs = {l.l: l._eoff(metas[l.l]) for l in quant}
    side = _SIDE.get(dev)
    if side is None:
        side = _SIDE[dev] = torch.cuda.Stream(device=dev)
    fork = torch.cuda.Event()
    fork.record(main)
    side.wait_event(fork)
    with torch.cuda.stream(side):
        for t in tabs[:5]:
            if t is not None:
                t.record_stream(side)
        for l in quant:
            eoffs[l.l].record_stream(side)
            l._flush(metas[l.l], mq, max_new)
        done = torch.cuda.Event()
        done.record(side)
    for l in quant:
        mq.cache[("flushed", l.l)] = done


# ---------------------------------------------------------------- prefill / extend rows over compressed history
def _ranges(starts, counts):
    """Concatenation of range(s, s + c) over the pairs, as an int64 numpy array."""
    starts, counts = np.asarray(starts, np.int64), np.asarray(counts, np.int64)
    if counts.sum() == 0:
        return np.zeros(0, np.int64)
    base = np.repeat(starts - np.concatenate(([0], np.cumsum(counts)[:-1])), counts)
    return base + np.arange(int(counts.sum()), dtype=np.int64)


def prefill_quant_rows(P, q, k, v, qsl, prev, cos_t, sin_t):
    """Prefill / extend rows of a quantized layer (vllm_attn.py:351-402 for quant layers): row i has queries
    q[qsl[i]:qsl[i+1]] (post-RoPE) at positions prev[i] .. prev[i] + (qsl[i+1] - qsl[i]) - 1, new pre-RoPE keys and
    values k / v at the same rows, and a history of prev[i] positions in the cache P (its first (prev - 128) // 256
    sub-blocks flushed, P.NQ, the rest in the exact pages). The history comes out of one kv800_hip_history launch
    (dequantized, rotated, bf16), the new keys out of one kv800_hip_rope_rows launch; each row's keys are its history
    followed by its new rows, and one kv800_hip_prefill launch attends all rows. qsl / prev are host sequences.
    Returns (T, 16, 128) bf16."""
    return kv800_hip.prefill(*prefill_quant_inputs(P, q, k, v, qsl, prev, cos_t, sin_t), window=0)


def prefill_quant_inputs(P, q, k, v, qsl, prev, cos_t, sin_t):
    """The arguments of prefill_quant_rows' attention launch, (q, qsl, prev, K, V, key positions, key row starts):
    the rows' keys (history, then new rows) and values assembled as prefill_quant_rows describes. The key positions
    are None: key j of a row is at position j."""
    dev = q.device
    prev, qsl = [int(x) for x in prev], [int(x) for x in qsl]
    new = [b - a for a, b in zip(qsl, qsl[1:])]
    T = qsl[-1]
    # key order: row 0's history, row 0's new rows, row 1's history, ...; the history launch writes each row's history
    # in place, the new rows (rotated) follow by one index_copy_ each for K and V
    ksl = np.concatenate(([0], np.cumsum(np.asarray(prev) + np.asarray(new)))).astype(np.int64)
    Kc = torch.empty(int(ksl[-1]), 4, 128, dtype=torch.bfloat16, device=dev)
    Vc = torch.empty_like(Kc)
    kv800_hip.history(P, prev, cos_t, sin_t, out=(Kc, Vc), offs=ksl[:-1])
    # the new rows' positions and their key indices, in one copy
    pi = kv800_hip.host_to_device(np.concatenate((_ranges(prev, new), _ranges(ksl[:-1] + np.asarray(prev, np.int64),
                                                                              new))), torch.int64, dev)
    pos_new, idx = pi[:T], pi[T:]
    Kn = kv800_hip.rope_rows(k[:T].to(torch.bfloat16), pos_new, cos_t, sin_t)
    Kc.index_copy_(0, idx, Kn)
    Vc.index_copy_(0, idx, v[:T].to(torch.bfloat16))
    return q, qsl, prev, Kc, Vc, None, ksl   # key positions: the index within the row (kp = None)


def prefill_window_rows(P, q, k, v, qsl, prev, cos_t, sin_t):
    """Prefill / extend rows of a window layer (vllm_attn.py:351-402 with win set): row i has queries
    q[qsl[i]:qsl[i+1]] (post-RoPE) at positions prev[i] .. prev[i] + (qsl[i+1] - qsl[i]) - 1 and new keys and values
    k / v at the same rows. Its history is what the layer keeps: the sinks (positions < min(NSINK, lo), when P.sk is
    set) at P.skoff / P.svoff in P.sk / P.sv, and the exact rows [lo, prev[i]) with lo = max(0, prev[i] - (WIN - 1)) in
    the exact pages of P (P.eoff element offsets per ebs positions, e_hs / e_ts / e_v strides). With cos_t / sin_t all
    keys are rotated at their positions (window + sinks layers keep pre-RoPE keys); None leaves them as stored (sliding
    layers keep post-RoPE keys). One gather of the history, then one kv800_hip_prefill launch with the window mask
    (and the sinks). qsl / prev are host sequences. Returns (T, 16, 128) bf16."""
    dev = q.device
    prev, qsl = [int(x) for x in prev], [int(x) for x in qsl]
    R = len(prev)
    new = np.asarray([b - a for a, b in zip(qsl, qsl[1:])], np.int64)
    p0 = np.asarray(prev, np.int64)
    lo = np.maximum(0, p0 - (kv800.WIN - 1))
    sinks = P.sk is not None
    ns = np.minimum(kv800.NSINK, lo) if sinks else np.zeros(R, np.int64)
    nx = p0 - lo
    rows = np.arange(R)
    # ---- exact rows [lo, prev): element offset of each (position, head) K row through the page table
    xr = np.repeat(rows, nx)
    xp = _ranges(lo, nx)
    h2d = lambda a: kv800_hip.host_to_device(a, torch.int64, dev)
    page = P.eoff[h2d(xr), h2d(xp // P.ebs)]                                      # (Sx,) element offsets
    ko = (page + h2d((xp % P.ebs) * P.e_ts))[:, None] + torch.arange(4, device=dev) * P.e_hs
    d128 = torch.arange(128, device=dev)
    ef = kv800.flat(P.epool)
    Kx, Vx = ef[ko[..., None] + d128], ef[ko[..., None] + P.e_v + d128]                          # (Sx, 4, 128)
    # ---- sink rows
    if sinks:
        sr = np.repeat(rows, ns)
        st = _ranges(np.zeros(R, np.int64), ns)
        so = h2d(st * 512)[:, None] + torch.arange(4, device=dev) * 128
        srd = h2d(sr)
        Ks = kv800.flat(P.sk)[(P.skoff[srd][:, None] + so)[..., None] + d128]
        Vs = kv800.flat(P.sv)[(P.svoff[srd][:, None] + so)[..., None] + d128]
    else:
        Ks = Vs = torch.empty(0, 4, 128, dtype=torch.bfloat16, device=dev)
    # ---- per row: sinks, exact rows, new rows, as rows of cat(sinks, exact, new)
    cnt = ns + nx + new
    ksl = np.concatenate(([0], np.cumsum(cnt))).astype(np.int64)
    order = np.concatenate([np.concatenate((_ranges([s0], [a]), len(Ks) + _ranges([x0], [b]),
                                            len(Ks) + len(Kx) + _ranges([q0], [c])))
                            for s0, x0, q0, a, b, c in zip(np.cumsum(ns) - ns, np.cumsum(nx) - nx, qsl[:-1], ns, nx,
                                                           new)]) if R else np.zeros(0, np.int64)
    kpos = np.concatenate([np.concatenate((np.arange(a), np.arange(l0, n0), np.arange(n0, n0 + c)))
                           for a, l0, n0, c in zip(ns, lo, p0, new)]) if R else np.zeros(0, np.int64)
    idx = h2d(order.astype(np.int64))
    Kc = torch.cat((Ks, Kx, k[:qsl[-1]].to(torch.bfloat16))).index_select(0, idx)
    Vc = torch.cat((Vs, Vx, v[:qsl[-1]].to(torch.bfloat16))).index_select(0, idx)
    if cos_t is not None:
        Kc = kv800_hip.rope_rows(Kc, h2d(kpos), cos_t, sin_t)
    return kv800_hip.prefill(q, qsl, prev, Kc, Vc, torch.from_numpy(kpos.astype(np.int32)), ksl, window=kv800.WIN,
                             nsink=kv800.NSINK if sinks else 0)
