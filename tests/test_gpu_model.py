"""The LFM3-shaped decode model (lfm3-kv800_amd/model.py, config C5) on an MI355X: its attention layers on the
HIP path (vLLM page geometry: quantized, window + sinks and native sliding layers) against the same model, same
weights and conv states, whose attention is the CPU oracle's torch_decode restatement over each layer's full K / V
history (quantized by the oracle quantizer, sinks and windows as torch_decode.py:27-80 selects them). Teacher forcing:
both models read the oracle model's greedy tokens. The models differ only in attention, whose outputs agree within
bf16 rounding; the bar on the logits is rel-L2 2e-2 per step with the same greedy token (or one whose logit is tied
with the top within the two models' largest logit difference).

Also the native sliding layer alone (vllm_cache.KV800SlideLayer: window 256, no sinks, post-RoPE keys, identity RoPE
tables) against the oracle, at the north-star bar; the decode steps replayed from one recorded HIP graph
(model.DecodeGraph) against the same steps launched from the host; and the fused kernels against torch."""
import numpy as np
import pytest
import torch

import decode_bar

pytestmark = pytest.mark.gpu
DEV = "cuda"


def say(*a):
    print("[gpu-model]", *a, flush=True)


def dev_bf16(bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).to(DEV)


def bits_of(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


class OracleAttention:
    """Attention of the 11 layers by the CPU oracle over full histories (numpy bf16 bits, (R, nmax, 4, 128) per layer;
    pre-RoPE keys for full layers, post-RoPE keys for sliding layers)."""

    def __init__(self, oracle, hist, lens0, cos_bits, sin_bits):
        from lfm3_kv800_amd import vllm_cache as vc
        self.o, self.vc, self.hist = oracle, vc, hist
        self.lens = np.array(lens0, np.int64)
        self.cos, self.sin = cos_bits, sin_bits
        self.one = oracle.f32_to_bf16(np.ones_like(oracle.bf16_to_f32(cos_bits)))
        self.zero = np.zeros_like(sin_bits)

    def begin_step(self):
        self.lens += 1
        return torch.from_numpy(self.lens - 1).to(DEV)

    def attend(self, l, q, k_pre, k_post, v):
        vc, o = self.vc, self.o
        K, V = self.hist[l]
        slide = l in vc.SLIDE_LAYERS
        p = self.lens - 1
        for r in range(len(p)):
            K[r, p[r]] = bits_of((k_post if slide else k_pre)[r])
            V[r, p[r]] = bits_of(v[r])
        win = 256 if (slide or l in vc.WINDOW_LAYERS) else 0
        case = o.build_paged(lambda b, p0, p1: (K[b, p0:p1], V[b, p0:p1]), list(self.lens), win=win, ebs=128,
                             shuffle_seed=l, sinks=not slide)
        cs, sn = (self.one, self.zero) if slide else (self.cos, self.sin)
        self.last = o.decode_f32(case, bits_of(q), cs, sn)            # (bf16 bits, f32 before rounding)
        return dev_bf16(self.last[0])


class TeeAttention:
    """The HIP attention, with every layer's output also computed by the oracle on the same inputs and compared at the
    north-star bar (max-abs 2e-2, mean-abs 1e-3, near-tie roundings excepted: decode_bar.py)."""

    def __init__(self, hip_attn, ref_attn):
        self.h, self.r, self.worst = hip_attn, ref_attn, {}

    def begin_step(self):
        p, pr = self.h.begin_step(), self.r.begin_step()
        assert torch.equal(p, pr)
        return p

    def attend(self, l, q, k_pre, k_post, v):
        o = self.h.attend(l, q, k_pre, k_post, v)
        self.r.attend(l, q, k_pre, k_post, v)
        mx, mean, _ = decode_bar.check(bits_of(o), self.r.last, f"layer {l}", say=lambda *a: None)
        w = self.worst.get(l, (0.0, 0.0))
        self.worst[l] = (max(w[0], mx), max(w[1], mean))
        return o


def test_model_decode_matches_oracle_attention(hip, oracle):
    from lfm3_kv800_amd import model as M
    cfg = M.Lfm3Config()
    lens0, steps = [1405, 700], 4          # row 0 crosses the flush boundary n = 1408 during the steps
    R, nmax = len(lens0), max(lens0) + steps + 1
    rng = np.random.RandomState(8)
    layers = [l for l in range(cfg.layers) if cfg.layer_type(l) != M.CONV]
    hist = {l: (oracle.randn_bf16(rng, (R, nmax, 4, 128)), oracle.randn_bf16(rng, (R, nmax, 4, 128))) for l in layers}
    copy = lambda: {l: (hist[l][0].copy(), hist[l][1].copy()) for l in layers}
    say("filling caches", lens0)
    hip_attn = M.PagedAttention800(lens0, steps, DEV, seed=3)
    hip_attn.fill(lambda l, r, p0, p1: (dev_bf16(hist[l][0][r, p0:p1]), dev_bf16(hist[l][1][r, p0:p1])))
    cs, sn = bits_of(hip_attn.cos), bits_of(hip_attn.sin)
    tee = TeeAttention(hip_attn, OracleAttention(oracle, copy(), lens0, cs, sn))
    ref_attn = OracleAttention(oracle, copy(), lens0, cs, sn)
    say("building two models")
    hip_model = M.Lfm3Decoder(cfg, tee, R, DEV, seed=5)
    ref_model = M.Lfm3Decoder(cfg, ref_attn, R, DEV, seed=5)
    for m in (hip_model, ref_model):
        m.randomize_conv_states(6)
    tokens = torch.tensor([11, 22], dtype=torch.int64, device=DEV)
    for s in range(steps):
        pos_h, pos_r = tee.begin_step(), ref_attn.begin_step()
        assert torch.equal(pos_h, pos_r)
        lh, lr = hip_model.step(tokens, pos_h), ref_model.step(tokens, pos_r)
        torch.cuda.synchronize()
        assert torch.isfinite(lh).all()
        rel = float((lh - lr).norm() / lr.norm())
        ah, ar = lh.argmax(-1), lr.argmax(-1)
        # the same greedy token, unless the two are tied within the logits' own difference
        gap = lr.max(-1).values - lr.gather(1, ah[:, None])[:, 0]
        tol = 2 * float((lh - lr).abs().max())
        say(f"step {s}: logits rel-L2 {rel:.3e}, greedy tokens {ah.tolist()} vs {ar.tolist()}, gap {gap.tolist()}")
        assert rel < 1e-1 and bool((gap <= tol).all())
        tokens = ar
    say("per-layer worst (max-abs, mean-abs) vs oracle:", {l: (f"{a:.2e}", f"{b:.2e}") for l, (a, b) in tee.worst.items()})


def test_slide_layer_decode(hip, oracle):
    from lfm3_kv800_amd import vllm_cache as vc
    rng = np.random.RandomState(4)
    L0 = np.array([1000, 3, 255, 256, 600], np.int64)
    n = L0 + 1
    R, ebs = len(L0), 128
    nmax = int(n.max())
    K = oracle.randn_bf16(rng, (R, nmax, 4, 128)); V = oracle.randn_bf16(rng, (R, nmax, 4, 128))
    q = oracle.randn_bf16(rng, (R, 16, 128))
    epr = nmax // ebs + 1
    bt = rng.permutation(R * epr).reshape(R, epr).astype(np.int32)
    ev = np.zeros((R * epr, 4, ebs, 256), np.uint16)
    for r in range(R):
        for p in range(L0[r]):
            ev[bt[r, p // ebs], :, p % ebs, :128] = K[r, p]
            ev[bt[r, p // ebs], :, p % ebs, 128:] = V[r, p]
    layer = vc.KV800SlideLayer(4, dev_bf16(ev))
    mx = vc.step_meta(torch.from_numpy(bt), torch.from_numpy(n), ebs, DEV)
    say("slide layer rows", list(n))
    out = layer.forward(dev_bf16(q), dev_bf16(K[np.arange(R), L0]), dev_bf16(V[np.arange(R), L0]), mx)
    torch.cuda.synchronize()
    case = oracle.build_paged(lambda b, p0, p1: (K[b, p0:p1], V[b, p0:p1]), list(n), win=256, ebs=ebs, shuffle_seed=4,
                              sinks=False)
    one = oracle.f32_to_bf16(np.ones((nmax + 1, 32), np.float32))
    decode_bar.check(out.float().cpu().numpy(), oracle.decode_f32(case, q, one, np.zeros_like(one)), "slide layer", say)


def test_fused_model_ops_match_torch(hip):
    """The engine loop's fused kernels (model_ops) against the torch statements of the same ops on bf16 tensors, within
    2 bf16 ulps per element (the kernels sum means and the 7-tap conv in their own fp32 order and use the hardware
    exp)."""
    import torch.nn.functional as F
    from lfm3_kv800_amd import model as M
    from lfm3_kv800_amd import model_ops as mo
    g = torch.Generator(device=DEV).manual_seed(12)
    R, H, FF, eps = 37, 2048, 8192, 1e-5
    bf = lambda *s, scale=1.0: (torch.randn(*s, generator=g, device=DEV) * scale).to(torch.bfloat16)

    def rms(x, w):
        xf = x.float()
        return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * w.float()).to(torch.bfloat16)

    def close(a, b, what):
        a, b = a.float(), b.float()
        d = (a - b).abs()
        bad = d > b.abs() * 2 ** -7 + 1e-30
        say(f"{what}: max-abs {float(d.max()):.3e}, equal {float((d == 0).float().mean()):.4f}, over 2 ulp {int(bad.sum())}")
        assert not bool(bad.any()), what

    x, h, wp, wn = bf(R, H), bf(R, H), bf(H, scale=0.5) + 1, bf(H, scale=0.5) + 1
    xo, no = mo.add_rmsnorm(h, x, wp, wn, eps)
    x_ref = x + rms(h, wp)
    close(xo, x_ref, "add_rmsnorm x"); close(no, rms(x_ref, wn), "add_rmsnorm n")
    _, n0 = mo.add_rmsnorm(None, x, None, wn, eps)
    close(n0, rms(x, wn), "rmsnorm")
    gu = bf(R, 2 * FF, scale=3.0)
    close(mo.silu_mul(gu), F.silu(gu[:, :FF]) * gu[:, FF:], "silu_mul")
    qkvg = bf(R, 3088, scale=2.0)
    qw, kw = bf(128, scale=0.3) + 1, bf(128, scale=0.3) + 1
    pos = torch.randint(0, 40000, (R,), generator=g, device=DEV)
    for theta, angles in ((1e6, 32), (1e4, 64)):
        cos, sin = M.model_rope_tables(theta, angles, 40000, DEV)
        q, kp, kr, v = mo.qkv_post(qkvg, qw, kw, cos, sin, pos, eps)
        qn = rms(qkvg[:, :2048].reshape(R, 16, 128), qw)
        kn = rms(qkvg[:, 2048:2560].reshape(R, 4, 128), kw)
        c, s = cos[pos].float()[:, None], sin[pos].float()[:, None]
        rot = lambda t: (t.float() * torch.cat((c, c), -1) +
                         torch.cat((-t.float()[..., 64:], t.float()[..., :64]), -1) * torch.cat((s, s), -1)).to(torch.bfloat16)
        close(q, rot(qn), f"qkv_post q theta {theta:g}"); close(kp, kn, "qkv_post k_pre")
        close(kr, rot(kn), f"qkv_post k_rot theta {theta:g}")
        assert torch.equal(v, qkvg[:, 2560:3072].reshape(R, 4, 128))
    bcx, cw = bf(R, 3 * H), bf(H, 7, scale=0.3)
    st = bf(R, H, 6)
    st_ref = st.clone()
    out = mo.conv_step(bcx, cw, st)
    Bx = bcx[:, :H] * bcx[:, 2 * H:]
    win = torch.cat((st_ref, Bx.unsqueeze(-1)), -1)
    close(out, bcx[:, H:2 * H] * (win * cw).sum(-1), "conv_step out")
    assert torch.equal(st, win[..., 1:])
    o = bf(R, 16, 128)
    close(mo.gate_mul(o, qkvg[:, 3072:]), o * torch.sigmoid(qkvg[:, 3072:].float()).to(torch.bfloat16).unsqueeze(-1),
          "gate_mul")
    # inputs of the wrong type or shape are rejected on the host, before any launch
    with pytest.raises(TypeError):
        mo.qkv_post(qkvg, qw, kw, cos, sin, pos.to(torch.int32), eps)
    with pytest.raises(TypeError):
        mo.conv_step(bcx, cw, st.float())
    with pytest.raises(ValueError):
        mo.conv_step(bcx[:, :3 * H - 8], cw, st)
    with pytest.raises(ValueError):
        mo.gate_mul(o, qkvg[:, 3072:3080])
    with pytest.raises(ValueError):
        mo.add_rmsnorm(h, x, wp[:1024], wn, eps)


def _decode_setup(lens0, steps):
    """A model and its paged attention with seeded weights, conv states and K / V histories (the same every call)."""
    from lfm3_kv800_amd import model as M
    cfg = M.Lfm3Config()
    g = torch.Generator(device=DEV).manual_seed(21)

    def history(l, r, p0, p1):
        return (torch.randn((p1 - p0, 4, 128), generator=g, device=DEV).to(torch.bfloat16),
                torch.randn((p1 - p0, 4, 128), generator=g, device=DEV).to(torch.bfloat16))

    attn = M.PagedAttention800(lens0, steps, DEV, seed=3)
    attn.fill(history)
    model = M.Lfm3Decoder(cfg, attn, len(lens0), DEV, seed=5)
    model.randomize_conv_states(6)
    return model, attn


def test_model_full_size_c5(hip, oracle):
    """config C5 at full size: 256 rows with prompt lengths U[1K, 32K] (the bench's seed), the
    prompt caches written through the attention layers' step path in 2048-token prefill chunks
    (PagedAttention800.fill -> vllm_cache write_step: exact pages, sinks, flushes), then 3 greedy steps of the
    LFM3-shaped model: every step's logits finite and tokens in range; sub-blocks the fill flushed (first, middle and
    last of two rows, quantized layers 6 and 22) equal the oracle quantizer's bytes of the rows' history."""
    from lfm3_kv800_amd import model as M
    from lfm3_kv800_amd import model_ops as mo
    cfg = M.Lfm3Config()
    R, steps = 256, 3
    lens0 = np.random.RandomState(51).randint(1024, 32768 + 1, size=R).astype(np.int64)
    g = torch.Generator(device=DEV).manual_seed(51)
    POOL = 1 << 16
    pools = {}

    def history(l, r, p0, p1):
        if l not in pools:
            pools[l] = tuple(torch.randn(POOL, 4, 128, generator=g, device=DEV).to(torch.bfloat16) for _ in range(2))
        o = (r * 7919 + p0 * 13) % (POOL - (p1 - p0) + 1)
        return pools[l][0][o:o + p1 - p0], pools[l][1][o:o + p1 - p0]

    say("full-size C5: fill", R, "rows,", int(lens0.sum()), "prompt tokens")
    attn = M.PagedAttention800(lens0.tolist(), steps + 1, DEV, seed=51)
    attn.fill(history)
    torch.cuda.synchronize()
    F = attn.FILL
    for l in (6, 22):
        qv = attn.layers[l].qv
        for r in (int(np.argmin(lens0)), int(np.argmax(lens0))):
            n = int(lens0[r])
            m = max(0, n - 128) // 256
            for j in sorted({0, m // 2, m - 1}):
                c0 = (256 * j) // F * F
                K, V = history(l, r, c0, min(n, c0 + F))
                i0 = 256 * j - c0
                want = oracle.quantize_blocks(bits_of(K[i0:i0 + 256])[None], bits_of(V[i0:i0 + 256])[None])[0]
                pg, off = int(attn.qbt_cpu[r, 256 * j // 1280]), (256 * j) % 1280 // 256 * 51200
                assert np.array_equal(qv[pg, off:off + 51200].cpu().numpy(), want), (l, r, j)
    say("full-size C5: model and", steps, "greedy steps")
    model = M.Lfm3Decoder(cfg, attn, R, DEV, seed=51)
    model.randomize_conv_states(51)
    tok = torch.randint(0, cfg.vocab, (R,), generator=g, device=DEV)
    for s in range(steps):
        logits = model.step(tok, attn.begin_step(), fp32=False)
        tok = mo.argmax(logits)
        torch.cuda.synchronize()
        say(f"step {s}: logits finite {bool(torch.isfinite(logits.float()).all())}")
        assert bool(torch.isfinite(logits.float()).all()) and bool(((tok >= 0) & (tok < cfg.vocab)).all()), s
    del model, attn, pools
    torch.cuda.empty_cache()


def test_decode_graph_replays_match_eager(hip):
    """DecodeGraph (the first step eager, the others replays of one recorded step, lengths advanced on the device and
    the step metadata's host values taken at the last step's lengths) against the same steps launched one kernel at a
    time from the host, on identical models and caches: every step's greedy tokens and bf16 logits equal bit for bit.
    Eager GPU work and synchronisations run between the replays. Row 0 flushes a sub-block at the third step
    (n = 1408 = 256 * 4 + 384) and row 3 crosses an exact page boundary."""
    from lfm3_kv800_amd import model as M
    from lfm3_kv800_amd import model_ops as mo
    lens0, steps = [1405, 700, 2000, 127], 6
    tok0 = torch.tensor([11, 22, 33, 44], dtype=torch.int64, device=DEV)
    say("eager run", lens0, steps)
    model, attn = _decode_setup(lens0, steps)
    want, tok = [], tok0
    for s in range(steps):
        logits = model.step(tok, attn.begin_step(), fp32=False)
        tok = mo.argmax(logits)
        assert torch.equal(tok, logits.float().argmax(-1))
        want.append((tok.clone(), logits.clone()))
    torch.cuda.synchronize()
    del model, attn
    say("graph run")
    model, attn = _decode_setup(lens0, steps)
    dg = M.DecodeGraph(model, attn, tok0, steps - 1)
    got = [(dg.tokens.clone(), dg.first_logits.clone())]
    junk = torch.randn(512, 512, device=DEV)
    for s in range(1, steps):
        dg.step()
        got.append((dg.tokens.clone(), dg.logits.clone()))
        junk = (junk @ junk.t()).tanh()     # eager work between the replays
        torch.cuda.synchronize()
    assert int(attn.lens.sum()) == sum(lens0) + len(lens0) * steps
    for s, ((tw, lw), (tg, lg)) in enumerate(zip(want, got)):
        d = float((lw.float() - lg.float()).abs().max())
        say(f"step {s}: tokens {tg.tolist()} (eager {tw.tolist()}), logits max-abs difference {d:.3e}")
        assert torch.equal(tw, tg) and torch.equal(lw, lg), s
    with pytest.raises(RuntimeError):
        dg.step()


def test_argmax_matches_torch(hip):
    """The greedy-token kernel against torch.argmax over the same bf16 values: random rows, rows whose maximum is
    repeated (the first index wins), rows with NaN (the first NaN wins), -inf / +inf rows and a strided view; a batch of
    600 rows takes the 512-thread form."""
    from lfm3_kv800_amd import model_ops as mo
    g = torch.Generator(device=DEV).manual_seed(3)
    R, V = 9, 65536
    x = torch.randn(R, V, generator=g, device=DEV).to(torch.bfloat16)
    x[1, 100] = x[1, 40000] = x[1, 65535] = 50.0          # ties: first index
    x[2].fill_(1.0)                                       # all equal: index 0
    x[3, 7] = x[3, 9000] = float("nan")                   # NaN ranks first
    x[4].fill_(float("-inf"))
    x[5, 60000] = float("inf")
    x[6, 65535] = 100.0                                   # the last element
    for t in (x, torch.cat((x, x), 1)[:, 8:V + 8]):
        got, want = mo.argmax(t), t.float().argmax(-1)
        say("argmax", got.tolist(), want.tolist())
        assert torch.equal(got, want)
    # more rows than CUs: the 512-thread workgroups (two rows per CU), same special rows repeated down the batch
    big = torch.randn(600, V, generator=g, device=DEV).to(torch.bfloat16)
    big[::60] = x[:1].expand(10, V)
    big[1::60] = x[1:2].expand(10, V)
    big[3::60] = x[3:4].expand(10, V)
    big[4::60] = x[4:5].expand(10, V)
    got, want = mo.argmax(big), big.float().argmax(-1)
    say("argmax 600 rows: mismatches", int((got != want).sum()))
    assert torch.equal(got, want)


@pytest.mark.parametrize("R,N,K,split", [(256, 2048, 2048, 1), (256, 16384, 2048, 1), (398, 3088, 2048, 1),
                                         (37, 640, 8192, 4), (398, 2048, 8192, 8), (1, 128, 64, 1), (130, 256, 320, 1),
                                         (256, 2048, 2048, 8)])
def test_linear_matches_fp32(hip, R, N, K, split):
    """The engine loop's GEMM (lfm3_hip_linear over a shuffled weight) against an fp32 product of the same bf16
    operands, rounded to bf16: within one bf16 rounding of the fp32 result plus fp32 summation-order noise
    (|d| <= 2^-8 |ref| + 1e-3 max |ref|); the padded columns are zero; split-K sums its parts in a fixed order, so
    two runs give identical bits. Shapes cover partial 128-row tiles (398, 130, 37 rows), a padded width (3088),
    K = 8192 with 4- and 8-way splits, slab counts below and off the weight ring's depth (1, 5, 4 per part)."""
    from lfm3_kv800_amd import model_ops as mo
    g = torch.Generator(device=DEV).manual_seed(R + N + K)
    x = torch.randn(R, K, generator=g, device=DEV).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g, device=DEV) * 0.02).to(torch.bfloat16)
    pw = mo.PackedWeight(w)
    y = mo.linear(x, pw, split=split)
    torch.cuda.synchronize()
    ref = x.float() @ w.float().t()
    d = (y[:, :N].float() - ref).abs()
    bar = ref.abs() * 2.0 ** -8 + 1e-3 * ref.abs().max()
    say("linear", R, N, K, split, "max |d|", float(d.max()), "max |ref|", float(ref.abs().max()))
    assert bool((d <= bar).all())
    assert not bool(y[:, N:].any())
    y2 = mo.linear(x, pw, split=split)
    assert torch.equal(y, y2)


@pytest.mark.parametrize("R,F,K", [(256, 8192, 2048), (398, 256, 2048), (5, 64, 64)])
def test_linear_glu_matches_unfused(hip, R, F, K):
    """The gated-activation epilogue (a [g | u] weight regrouped in 64-row pairs) against the plain product of the same
    kernel followed by the silu_mul kernel: the same k order per output, so identical bits."""
    from lfm3_kv800_amd import model_ops as mo
    g = torch.Generator(device=DEV).manual_seed(R + F)
    x = torch.randn(R, K, generator=g, device=DEV).to(torch.bfloat16)
    w = (torch.randn(2 * F, K, generator=g, device=DEV) * 0.05).to(torch.bfloat16)
    fused = mo.linear(x, mo.PackedWeight(w, glu=True))
    plain = mo.silu_mul(mo.linear(x, mo.PackedWeight(w))[:, :2 * F].contiguous())
    torch.cuda.synchronize()
    say("glu", R, F, K, "equal", bool(torch.equal(fused, plain)))
    assert fused.shape == (R, F) and torch.equal(fused, plain)
