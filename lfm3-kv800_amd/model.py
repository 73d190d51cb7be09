"""Decode loop of an LFM3-1.7B-shaped model whose attention layers run on the 800h path (config C5), without
vLLM.

The layer stack follows the reference's vLLM model (vllm_model.py:542-653) and its attention routing with
LFM3_KV800=1 (vllm_model.py:268-304): 24 layers of width 2048, each `h += post_norm(op(norm(h)))` then
`h += post_ffn_norm(ffn(ffn_norm(h)))` (sandwich norms, vllm_model.py:446-471), then a final norm and the tied LM head.
  * 13 gated short-conv layers (width 7, vllm_model.py:327-431): in_proj -> B, C, x; y = C * conv(B * x); out_proj.
  * 6 full-attention layers, 16 query / 4 KV heads of 128, QK RMSNorm per head, RoPE theta 1e6 on 32 of the 64
    frequencies (zero tail), per-head sigmoid output gate (vllm_model.py:195-304): quantized 6, 10, 14, 22 and window +
    sinks 2, 18 on the 800h caches (vllm_cache.KV800DecodeLayer), keys handed over before RoPE.
  * 5 native sliding layers 4, 8, 12, 16, 20 (RoPE theta 1e4 on all frequencies, window 256) on exact window caches
    (vllm_cache.KV800SlideLayer), keys handed over after RoPE.
The vocabulary and feed-forward sizes are not in the reference (its weights are not available offline): 65,536 and
8,192 here, about 1.67 B parameters. Weights are random N(0, 0.02) in bf16, norm weights 1.

Attention goes through an object with begin_step() -> the new tokens' positions and attend(layer, q, k_pre, k_post, v)
-> (R, 16, 128): PagedAttention800 (below) keeps vLLM's page geometry and runs every layer on libkv800_hip.so; tests
substitute an oracle implementation to check the logits. Between the GEMMs, the model's elementwise work runs on the
fused kernels of model_ops (include/lfm3_model.h). DecodeGraph captures one whole decode step (metadata, 24 layers,
greedy token) as a HIP graph and replays it per step."""
from dataclasses import dataclass

import torch
import torch.nn.functional as F

from . import kv800, kv800_hip
from . import model_ops as mo
from . import vllm_cache as vc

CONV, FULL, SLIDE = "conv", "full", "slide"
EXACT_GROUPS = {"A": (2, 10, 18), "B": (6, 14, 22)}       # exact KV groups of the full layers (sliding window 640)
SLIDE_GROUPS = {"C": (4, 12, 20), "D": (8, 16)}           # KV groups of the native sliding layers (window 256)


@dataclass
class Lfm3Config:
    hidden: int = 2048
    heads: int = 16
    kv_heads: int = 4
    head_dim: int = 128
    ffn: int = 8192
    vocab: int = 65536
    layers: int = 24
    conv_len: int = 7
    window: int = 256
    eps: float = 1e-5

    def layer_type(self, l):
        if l in vc.QUANT_LAYERS or l in vc.WINDOW_LAYERS:
            return FULL
        if l in vc.SLIDE_LAYERS:
            return SLIDE
        return CONV


def model_rope_tables(theta, angles, n, device):
    """(cos, sin) (n, 64) bf16 of the model's neox RoPE (vllm_model.py:106-151): frequency f < angles is
    theta^(-2f/128), the rest 0 (cos 1, sin 0); angles in fp32, then bf16, as the reference's cos / sin caches."""
    inv = 1.0 / (theta ** (torch.arange(0, 2 * angles, 2, dtype=torch.float32) / 128))
    inv = torch.cat((inv, torch.zeros(64 - angles)))
    fr = torch.arange(n, dtype=torch.float32)[:, None] * inv[None]
    return fr.cos().to(torch.bfloat16).to(device), fr.sin().to(torch.bfloat16).to(device)


def kernel_tables(n, device):
    """(cos, sin) (n, 32) bf16 of the full layers' 32 rotating frequencies, the tables the decode kernels read
    (vllm_attn.py:147-159)."""
    inv = 1.0 / (1e6 ** (torch.arange(0, 64, 2, dtype=torch.float32) / 128))
    fr = torch.arange(n, dtype=torch.float32)[:, None] * inv[None]
    return fr.cos().to(torch.bfloat16).to(device), fr.sin().to(torch.bfloat16).to(device)


def glu_rows(rows):
    """Whether the fused up-projection + gated activation (128-row tiles) is used for a batch of `rows`: measured
    on MI355X against hipBLASLt + silu_mul at hidden 2048, ffn 8192 (device time per layer): 192 rows 28.7 vs 29.8 us,
    256 rows 25.7 vs 33.2, 320 rows 38.6 vs 35.2 (a third row tile a quarter full), 398 rows 41.1 vs 41.7, 128 rows
    23.1 vs 22.1."""
    return 128 < rows <= 256 or rows > 384


class Lfm3Decoder:
    """Random-init LFM3-shaped model for batched decode: step(tokens) appends one token to every row and returns the
    logits. The dense products are torch GEMMs; everything between them is one fused HIP kernel (model_ops): the
    sandwich norms with the residual add, the q / k norms with RoPE, the short-conv step, the gated activation and
    the attention output gate. The FFN's up-projection and gated activation run as one HIP GEMM (model_ops.linear on
    a [g | u] weight) at the batch sizes where it beats the library product plus the activation kernel (glu_rows).
    conv_state: per conv layer (R, hidden, conv_len - 1) bf16. max_pos bounds the positions of the model's RoPE
    tables."""

    def __init__(self, cfg: Lfm3Config, attention, rows, device, seed=0, max_pos=65536):
        self.cfg, self.attn, self.R, self.dev = cfg, attention, rows, device
        g = torch.Generator(device=device).manual_seed(seed)
        H, D, G = cfg.hidden, cfg.head_dim, cfg.heads

        def w(*shape):
            return (torch.randn(*shape, generator=g, device=device) * 0.02).to(torch.bfloat16)

        ones = lambda n: torch.ones(n, dtype=torch.bfloat16, device=device)
        self.embed = w(cfg.vocab, H)
        self.final_norm = ones(H)
        self.tables = {FULL: model_rope_tables(1e6, 32, max_pos, device),
                       SLIDE: model_rope_tables(1e4, 64, max_pos, device)}
        self.fused_ffn = glu_rows(rows)
        self.layers = []
        for l in range(cfg.layers):
            t = cfg.layer_type(l)
            L = {"type": t, "norm": ones(H), "post_norm": ones(H), "ffn_norm": ones(H), "post_ffn_norm": ones(H),
                 "w13": w(2 * cfg.ffn, H), "w2": w(H, cfg.ffn)}
            if self.fused_ffn:
                L["w13p"] = mo.PackedWeight(L["w13"], glu=True)
            if t == CONV:
                L.update(in_proj=w(3 * H, H), conv=w(H, cfg.conv_len), out_proj=w(H, H),
                         state=torch.zeros(rows, H, cfg.conv_len - 1, dtype=torch.bfloat16, device=device))
            else:
                # q, k, v and the 16 output-gate logits from one product: rows [q | k | v | gate]
                L.update(qkvg=torch.cat((w((G + 2 * cfg.kv_heads) * D, H), w(G, H))), q_norm=ones(D), k_norm=ones(D),
                         o_proj=w(H, G * D))
            self.layers.append(L)

    def randomize_conv_states(self, seed):
        g = torch.Generator(device=self.dev).manual_seed(seed)
        for L in self.layers:
            if L["type"] == CONV:
                L["state"].copy_(torch.randn(L["state"].shape, generator=g, device=self.dev) * 0.1)

    def _conv(self, L, n):
        return F.linear(mo.conv_step(F.linear(n, L["in_proj"]), L["conv"], L["state"]), L["out_proj"])

    def _attention(self, l, L, n, pos):
        cfg = self.cfg
        qkvg = F.linear(n, L["qkvg"])                                                   # (R, 3088)
        cos, sin = self.tables[L["type"]]
        q, k_pre, k_rot, v = mo.qkv_post(qkvg, L["q_norm"], L["k_norm"], cos, sin, pos, cfg.eps)
        o = self.attn.attend(l, q, k_pre, k_rot, v)
        o = mo.gate_mul(o, qkvg[:, (cfg.heads + 2 * cfg.kv_heads) * cfg.head_dim:])
        return F.linear(o.reshape(o.shape[0], -1), L["o_proj"])

    def step(self, tokens, pos, fp32=True):
        """tokens (R,) int64, pos (R,) int64 the new tokens' positions (device); the attention object's begin_step
        has been called with the rows' lengths including this token. Returns (R, vocab) logits, fp32 (the bf16 LM-head
        output widened) or, with fp32=False, bf16."""
        cfg = self.cfg
        x = self.embed[tokens]
        _, n = mo.add_rmsnorm(None, x, None, self.layers[0]["norm"], cfg.eps)
        for l, L in enumerate(self.layers):
            h = self._conv(L, n) if L["type"] == CONV else self._attention(l, L, n, pos)
            x, n = mo.add_rmsnorm(h, x, L["post_norm"], L["ffn_norm"], cfg.eps)
            a = mo.linear(n, L["w13p"]) if self.fused_ffn else mo.silu_mul(F.linear(n, L["w13"]))
            h = F.linear(a, L["w2"])
            nxt = self.layers[l + 1]["norm"] if l + 1 < len(self.layers) else self.final_norm
            x, n = mo.add_rmsnorm(h, x, L["post_ffn_norm"], nxt, cfg.eps)
        logits = F.linear(n, self.embed)
        return logits.float() if fp32 else logits

    def greedy(self, tokens, pos):
        """One step's greedy tokens (R,) int64: the first index of each row's largest logit (one HIP launch on the
        bf16 logits, the same choice as argmax over their fp32 widening)."""
        return mo.argmax(self.step(tokens, pos, fp32=False))


class PagedAttention800:
    """The model's 11 attention layers on libkv800_hip.so with vLLM's page geometry: one quant KV group (1280-token
    pages of 262,144 B) for layers 6, 10, 14, 22; exact KV groups A (2, 10, 18) and B (6, 14, 22) of ebs-token pages
    holding each row's last positions; sliding KV groups C (4, 12, 20) and D (8, 16) (window 256). Each row of an exact
    or sliding group owns a ring of `ring` shuffled physical pages and logical page p maps to its (p % ring)-th one
    (the pages a sliding-window KV group recycles): the ring holds a prompt chunk of FILL tokens plus the 384 exact
    positions before it, and the decode steps' windows.

    lens0: the rows' history lengths; steps: decode steps to provide for."""

    FILL = 2048   # prompt tokens per row per fill step (the reference's prefill chunk, vllm_attn.py:196)

    def __init__(self, lens0, steps, device, ebs=128, seed=0):
        self.dev, self.ebs = device, ebs
        self.lens = torch.tensor([int(x) for x in lens0], dtype=torch.int64)
        R = self.R = len(lens0)
        nmax = int(self.lens.max()) + steps + 1
        self.cos, self.sin = kernel_tables(nmax + 64, device)
        rng = torch.Generator().manual_seed(seed)
        lp = nmax // ebs + 1                                                   # logical exact pages per row

        # a fill step writes FILL positions and flushes sub-blocks starting up to 383 positions before them; a decode
        # step reads the 384 positions before its token: the ring spans both with a page to spare
        self.ring = ring = max(self.FILL, 384 + steps + 1) // ebs + 5

        def table():
            """block table (R, lp) int32: row r's logical page p -> the (p % ring)-th of its ring of shuffled pages."""
            perm = torch.randperm(R * ring, generator=rng).view(R, ring).to(torch.int32)
            return perm[:, torch.arange(lp) % ring].contiguous(), R * ring

        self.bt, npages = {}, {}
        for grp in (*EXACT_GROUPS, *SLIDE_GROUPS):
            bt, npages[grp] = table()
            self.bt[grp] = bt.to(device)
        self.bt_cpu = {g: t.cpu() for g, t in self.bt.items()}
        qlp = nmax // vc.QBLOCK + 1
        self.qbt_cpu = torch.randperm(R * qlp, generator=rng).view(R, qlp).to(torch.int32)
        self.qbt = self.qbt_cpu.to(device)
        self.group_of = {l: g for g, ls in {**EXACT_GROUPS, **SLIDE_GROUPS}.items() for l in ls}
        self.layers = {}
        for l in (2, 6, 10, 14, 18, 22):
            ev = torch.zeros(npages[self.group_of[l]], 4, ebs, 256, dtype=torch.bfloat16, device=device)
            qv = None if l in vc.WINDOW_LAYERS else torch.zeros(R * qlp, vc.QPAGE, dtype=torch.uint8, device=device)
            self.layers[l] = vc.KV800DecodeLayer(l, ev, qv)
        for l in vc.SLIDE_LAYERS:
            ev = torch.zeros(npages[self.group_of[l]], 4, ebs, 256, dtype=torch.bfloat16, device=device)
            self.layers[l] = vc.KV800SlideLayer(l, ev)
        self.metas = None
        self.lens_dev = self.lens_bound = None   # set by freeze()

    # ---- prompt history
    def fill(self, history):
        """Write every row's history into the caches through the layers' step path (vllm_cache write_step: exact rows,
        sinks of window layers in the hosts' aux areas, flush of every sub-block that becomes eligible, from the
        layer's own exact group), in prefill steps of up to FILL positions per row, as vLLM schedules prompt chunks:
        step c carries positions [c FILL, min(n, (c + 1) FILL)) of every row still short of its length n. Prompt
        attention is not computed (no queries exist for a synthetic history). history(l, r, p0, p1) -> (K, V)
        (p1 - p0, 4, 128) bf16 on the device: pre-RoPE K for full layers, post-RoPE K for sliding layers."""
        lens = self.lens
        for c0 in range(0, int(lens.max()) if self.R else 0, self.FILL):
            rows = torch.nonzero(lens > c0).flatten()
            sl = torch.clamp(lens[rows], max=c0 + self.FILL)
            ql = sl - c0
            me = {g: vc.mixed_step_meta(self.bt_cpu[g][rows], sl, ql, self.ebs, self.dev, num_decodes=0)
                  for g in self.bt}
            mq = vc.mixed_step_meta(self.qbt_cpu[rows], sl, ql, vc.QBLOCK, self.dev, num_decodes=0)
            for l, layer in self.layers.items():
                parts = [history(l, int(r), c0, int(n)) for r, n in zip(rows.tolist(), sl.tolist())]
                K = torch.cat([p[0] for p in parts])
                V = torch.cat([p[1] for p in parts])
                if isinstance(layer, vc.KV800SlideLayer):
                    layer.write_step(K, V, me[self.group_of[l]])
                else:
                    layer.write_step(K, V, me[self.group_of[l]], mq, hosts=self.layers)
                del K, V, parts

    # ---- decode steps
    def freeze(self, steps):
        """Make the next `steps` decode steps replayable from one recorded step: the rows' lengths then advance on the
        device (an add inside the step instead of a copy from the host), and the host values of the step metadata are
        taken at the lengths after the last of those steps. Those values are bounds that hold for every step in
        between: the largest flushed sub-block count (the width of the decode tables and the clamp of each row's own
        count, which the kernels read on the device) and the rows of the sliding layers' identity tables."""
        self.lens_dev = self.lens.to(self.dev)
        self.lens_bound = self.lens + steps

    def begin_step(self):
        """Metadata of the next decode step (every row appends one token) and the start of its flushes."""
        self.lens += 1
        if self.lens_dev is None:
            host, dl = self.lens, vc.step_lens(self.lens, self.dev)
        else:
            self.lens_dev += 1
            host, dl = self.lens_bound, self.lens_dev
        me = {g: vc.step_meta(self.bt[g], host, self.ebs, self.dev, dl) for g in self.bt}
        mq = vc.step_meta(self.qbt, host, vc.QBLOCK, self.dev, dl)
        self.metas = (me, mq)
        full = [self.layers[l] for l in (2, 6, 10, 14, 18, 22)]
        vc.launch_flushes(full, {l.l: me[self.group_of[l.l]] for l in full}, mq)
        return mq.positions

    def attend(self, l, q, k_pre, k_post, v):
        me, mq = self.metas
        layer = self.layers[l]
        if isinstance(layer, vc.KV800SlideLayer):
            return layer.forward(q, k_post, v, me[self.group_of[l]])
        return layer.forward(q, k_pre, v, me[self.group_of[l]], mq, hosts=self.layers, cos_t=self.cos, sin_t=self.sin)


class DecodeGraph:
    """Greedy decode with one HIP graph per step. Construction runs the first step eagerly on the graph's own stream
    (it builds the cached tables, library handles and the flush stream that the recorded step reuses; its tokens are
    `tokens` afterwards, its bf16 logits `first_logits`), then freezes the attention for `steps` further steps and records
    one step, whose input is the token buffer and whose greedy tokens are copied back into it. Each step() replays it:
    one graph launch instead of ~250 kernel launches from the host. `tokens` and `logits` (the last replay's bf16
    logits) are buffers that the next step overwrites. The attention must be a PagedAttention800."""

    def __init__(self, model, attention, tokens, steps):
        self.attn, self.left = attention, int(steps)
        self.stream = torch.cuda.Stream(device=tokens.device)
        self.stream.wait_stream(torch.cuda.current_stream(tokens.device))
        with torch.cuda.stream(self.stream):
            self.first_logits = model.step(tokens, attention.begin_step(), fp32=False)
            self.tokens = mo.argmax(self.first_logits)
        self.stream.synchronize()
        attention.freeze(self.left)
        lens = attention.lens.clone()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=self.stream):
            logits = model.step(self.tokens, attention.begin_step(), fp32=False)
            self.tokens.copy_(mo.argmax(logits))
        attention.lens = lens          # recording ran no step
        self.logits = logits
        torch.cuda.current_stream(tokens.device).wait_stream(self.stream)

    def step(self):
        """One decode step: returns the (R,) greedy tokens."""
        if self.left <= 0:
            raise RuntimeError("DecodeGraph: the steps it was recorded for are used up")
        self.left -= 1
        self.attn.lens += 1
        self.graph.replay()
        return self.tokens


def decode_loop(model, attention, tokens, steps, graph=False):
    """Greedy decode: `steps` steps from `tokens` (R,) int64; returns the (steps, R) generated tokens. graph=True runs
    the steps after the first as replays of one recorded step (DecodeGraph; PagedAttention800 only)."""
    if graph and steps > 0:
        dg = DecodeGraph(model, attention, tokens, steps - 1)
        out = [dg.tokens.clone()]
        for _ in range(steps - 1):
            out.append(dg.step().clone())
        return torch.stack(out)
    out = []
    for _ in range(steps):
        tokens = model.greedy(tokens, attention.begin_step())
        out.append(tokens)
    return torch.stack(out)
