"""Range robustness of the quantized decode on an MI355X: hand-built sub-blocks whose scale bytes and score / weight
ranges are chosen to hit the kernel's conversions at their edges, decoded by the HIP kernels and by the oracle over
the same bytes.

  * every finite fp8 e4m3fn byte (zeros, subnormals, the smallest normals, +-448) as klo, ksc, vlo and vsc: the HIP
    path converts scale bytes with the hardware fp8 conversion, the oracle with integer arithmetic
    (kv800.py:83-91 decodes them through torch's float8_e4m3fn);
  * the fp16 P.V weights p * vsc at their largest: vsc = 448 on every token and a score that climbs by just under, and
    by just over, 7 log2 units from one sub-block to the next (the kernel's running max rescales on every new maximum,
    so p <= 1 and the weights stay <= 448; the climb also exercises the rescale of a state built from probabilities
    2^-7 below the new maximum).

Bar: finite outputs and rel-L2 < 1e-2 per row against the oracle (the reference's own decode bar,
tests/test_parity.py:104); the outputs reach magnitudes of hundreds here, where an absolute 2e-2 is below one bf16
step."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"
FINITE = np.array([b for b in range(256) if (b & 0x7F) != 0x7F], np.uint8)       # 254 finite e4m3fn bytes
SMALL = np.array([b for b in range(256) if (b & 0x78) <= 0x08], np.uint8)        # zeros, subnormals, min normals


def say(*a):
    print("[gpu-range]", *a, flush=True)


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


def block(rng, klo, ksc, vlo, vsc, kc=None):
    """One 51,200-byte sub-block: random K codes (or kc) and V bits, the given scale bytes."""
    sb = rng.randint(0, 256, size=51200).astype(np.uint8)
    if kc is not None:
        sb[0:32768] = kc
    sb[49152:49664], sb[49664:50176] = vlo, vsc
    sb[50176:50688], sb[50688:51200] = klo, ksc
    return sb


def run(hip, oracle, blocks, q, tail_seed, tail_scale=None):
    """Rows b with len(blocks[b]) hand-built sub-blocks and a 37-token exact tail, K ~ N(0, tail_scale[b]^2) and
    V ~ N(0, 1); returns (HIP, oracle) fp32."""
    rng = np.random.RandomState(tail_seed)
    lens = [128 + 256 * len(bl) + 37 for bl in blocks]
    nmax = max(lens)
    ts = np.ones(len(blocks), np.float32) if tail_scale is None else np.asarray(tail_scale, np.float32)
    K = oracle.f32_to_bf16(rng.standard_normal((len(blocks), nmax, 4, 128)).astype(np.float32) * ts[:, None, None, None])
    V = oracle.randn_bf16(rng, (len(blocks), nmax, 4, 128))
    case = oracle.build_paged(lambda b, p0, p1: (K[b, p0:p1], V[b, p0:p1]), lens, ebs=128, shuffle_seed=tail_seed)
    for b, bl in enumerate(blocks):
        assert case.NQ[b] == len(bl)
        for j, sb in enumerate(bl):
            case.qpool[case.boff[b, j] // 51200] = sb
    cos, sin = oracle.rope_tables(nmax + 1)
    want = oracle.decode(case, q, cos, sin)
    got = hip.decode(upload(case), to_dev_bf16(q), to_dev_bf16(cos), to_dev_bf16(sin))
    f = lambda bits: torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).float().numpy()
    return f(bits_of(got)), f(want)


def check(got, want, what):
    for b in range(got.shape[0]):
        rel = np.linalg.norm(got[b] - want[b]) / max(np.linalg.norm(want[b]), 1e-30)
        say(f"{what} row {b}: rel-L2 {rel:.3e}, max |out| {np.abs(want[b]).max():.3e}")
        assert np.isfinite(got[b]).all(), (what, b)
        assert rel < 1e-2, (what, b, rel)


def test_decode_every_fp8_scale_byte(hip, oracle):
    rng = np.random.RandomState(3)
    i = np.arange(512)
    rows = []
    # row 0: all 254 finite bytes in each of klo / ksc / vlo / vsc (multipliers coprime to 254: bijections)
    rows.append([block(rng, FINITE[(i + 128 * j) % 254], FINITE[(3 * i + 7 * j) % 254],
                       FINITE[(5 * i + 11 * j) % 254], FINITE[(7 * i + 13 * j) % 254]) for j in range(4)])
    # row 1: only zeros, subnormals and the smallest normals (its exact tail's keys as small, so that the sub-blocks
    # carry the softmax)
    S = len(SMALL)
    rows.append([block(rng, SMALL[(i + 5 * j) % S], SMALL[(3 * i + j) % S], SMALL[(5 * i + 3 * j) % S],
                       SMALL[(7 * i + 2 * j) % S]) for j in range(4)])
    q = np.stack([oracle.randn_bf16(rng, (16, 128), scale=0.02), oracle.randn_bf16(rng, (16, 128), scale=64.0)])
    say("every finite fp8 scale byte: 2 rows x 4 sub-blocks")
    got, want = run(hip, oracle, rows, q, tail_seed=3, tail_scale=[1.0, 0.01])
    check(got, want, "fp8 bytes")


@pytest.mark.parametrize("step", [6.98, 7.49])
def test_decode_fp16_weight_range(hip, oracle, step):
    """vsc = 448 (0x7E), vlo = -224 (0xF6) on every token; K is klo_j on dim 40 (a dim without a RoPE frequency, ksc 0)
    and 0 elsewhere, klo_j = -24, -16, ..., 32 over 8 sub-blocks; q is alpha on dim 40, with alpha chosen so that the
    score climbs by `step` log2 units per sub-block."""
    rng = np.random.RandomState(int(step * 100))
    klo_ramp = [0xDC, 0xD8, 0xD0, 0x00, 0x50, 0x58, 0x5C, 0x60]       # -24, -16, -8, 0, 8, 16, 24, 32 in e4m3fn
    f8 = oracle.f8_decode(np.array(klo_ramp, np.uint8))
    assert np.allclose(f8, [-24, -16, -8, 0, 8, 16, 24, 32]), f8
    blocks = []
    for j in range(8):
        klo = np.zeros(512, np.uint8)
        klo[np.arange(4) * 128 + 40] = klo_ramp[j]
        blocks.append(block(rng, klo, np.zeros(512, np.uint8), np.full(512, 0xF6, np.uint8),
                            np.full(512, 0x7E, np.uint8)))
    alpha = step / (8 * 128 ** -0.5 * 1.4426950408889634)
    qf = np.zeros((1, 16, 128), np.float32)
    qf[0, :, 40] = alpha
    q = oracle.f32_to_bf16(qf)
    say(f"fp16 weight range: step {step} log2 units per sub-block, alpha {alpha:.4f}")
    got, want = run(hip, oracle, [blocks], q, tail_seed=11)
    check(got, want, f"fp16 weights step {step}")


def test_read_probe_reads_every_unit(hip):
    """kv800_hip_read_probe (bench.py's read-bandwidth measurement): the xor of its per-workgroup words equals the xor
    of every dword of the buffer, for a buffer that is not a multiple of the grid's stride and for more workgroups
    than the buffer has strides."""
    import lfm3_kv800_amd.kv800_hip as kh
    g = torch.Generator(device="cuda").manual_seed(5)
    for n16, groups in ((1_000_003, 512), (4097, 64), (1, 8)):
        x = torch.randint(-2 ** 31, 2 ** 31 - 1, (4 * n16,), generator=g, device="cuda", dtype=torch.int64)
        x = x.to(torch.int32)
        out = torch.full((groups,), 0x5A5A5A5A, dtype=torch.int32, device="cuda")
        kh.read_probe(x, out, groups)
        torch.cuda.synchronize()
        xs = x.cpu().numpy().view(np.uint32)
        want = int(np.bitwise_xor.reduce(xs)) if xs.size else 0
        got = int(np.bitwise_xor.reduce(out.cpu().numpy().view(np.uint32)))
        print(f"[gpu-range] read_probe n16={n16} groups={groups}: xor {got:#010x} vs {want:#010x}", flush=True)
        assert got == want
