"""Pure-torch CPU restatement of the reference's torch decode path -- TEST INFRASTRUCTURE, not product code.

bench.py times it on the GPU box's host cores as the CPU baseline (`cpu_baseline.kind = "port"`): the reference's own
pure-torch backend (lfm3_kv800/torch_decode.py:27-80, with the dequantizer of kv800.py:79-92) cannot travel to the
box, so this file states the same algorithm on CPU torch -- per row, the flushed sub-blocks dequantized (2-bit K codes
times the fp8 scale plus the fp8 offset, rounded to bf16; 1-bit V planes times the scale plus the offset, times the
normalised Hadamard), the exact rows gathered from their pages, the sinks of window layers, every key rotated on the
dim pairs (d, d + 64), d < 32, in fp32 and rounded to bf16, then one fp32 softmax over all positions (scale 128^-0.5)
with 4 query heads per KV head. tests/test_oracle.py pins it against the C oracle (oracle/kv800_oracle.c) on the
config C1 inputs. Only tests/ and bench.py's cpu_baseline leg import it."""
import torch

BLK, SUB, NSINK = 256, 51200, 4
KC, VB, VLO, VSC, KLO, KSC = 0, 32768, 49152, 49664, 50176, 50688


def hadamard128():
    """Normalised Sylvester Hadamard of order 128 (kv800.py:43-46): +-1/sqrt(128) by the parity of popcount(i & j)."""
    i = torch.arange(128)
    x = i[:, None] & i[None, :]
    parity = torch.zeros(128, 128, dtype=torch.int64)
    for s in range(7):
        parity ^= (x >> s) & 1
    return (1.0 - 2.0 * parity.to(torch.float32)) / 128 ** 0.5


def _fp8(b):
    return b.contiguous().view(torch.float8_e4m3fn).float()


def dequantize(sb, H):
    """(M, 51200) uint8 sub-blocks -> K (M, 256, 4, 128) fp32 holding bf16 values, V (M, 256, 4, 128) fp32."""
    M = sb.shape[0]
    kc = sb[:, KC:VB].view(M, BLK, 4, 32).to(torch.int32)
    codes = torch.cat([(kc >> (2 * plane)) & 3 for plane in range(4)], dim=-1).float()      # dim = 32 plane + j
    k = codes * _fp8(sb[:, KSC:SUB]).view(M, 1, 4, 128) + _fp8(sb[:, KLO:KSC]).view(M, 1, 4, 128)
    vb = sb[:, VB:VLO].view(M, BLK, 4, 16).to(torch.int32)
    bits = torch.cat([(vb >> plane) & 1 for plane in range(8)], dim=-1).float()            # dim = 16 plane + j
    scale = _fp8(sb[:, VSC:KLO]).view(M, BLK, 2, 1).repeat_interleave(2, dim=2)             # per 2-head group
    offset = _fp8(sb[:, VLO:VSC]).view(M, BLK, 2, 1).repeat_interleave(2, dim=2)
    return k.to(torch.bfloat16).float(), (bits * scale + offset) @ H


def _rope(K, pos, cos_t, sin_t):
    c = cos_t[pos].float().unsqueeze(1)
    s = sin_t[pos].float().unsqueeze(1)
    lo, hi = K[..., 0:32], K[..., 64:96]
    out = K.clone()
    out[..., 0:32], out[..., 64:96] = lo * c - hi * s, hi * c + lo * s
    return out.to(torch.bfloat16).float()


def _row_keys(P, b, n, lo, nq, H):
    """(K, V, positions) of row b before RoPE: its nq sub-blocks, its sinks (window layers), its exact rows [lo, n)."""
    parts = []
    if nq:
        sb = P.qpool.view(-1)[P.boff[b, :nq, None] + torch.arange(SUB)]
        k, v = dequantize(sb, H)
        parts.append((k.reshape(-1, 4, 128), v.reshape(-1, 4, 128), torch.arange(nq * BLK)))
    if P.win and P.sk is not None:
        m = min(NSINK, lo, n)
        if m > 0:
            rows = (torch.arange(m)[:, None] * 4 + torch.arange(4)) * 128
            ks = P.sk.view(-1)[P.skoff[b] + rows[..., None] + torch.arange(128)].float()
            vs = P.sv.view(-1)[P.svoff[b] + rows[..., None] + torch.arange(128)].float()
            parts.append((ks, vs, torch.arange(m)))
    if n > lo:
        p = torch.arange(lo, n)
        row0 = P.eoff[b, p // P.ebs] + (p % P.ebs) * P.e_ts                                  # (S,) element offsets
        kidx = (row0[:, None] + torch.arange(4) * P.e_hs)[..., None] + torch.arange(128)    # (S, 4, 128)
        e = P.epool.view(-1)
        parts.append((e[kidx].float(), e[kidx + P.e_v].float(), p))
    if not parts:
        return None
    return tuple(torch.cat(x) for x in zip(*parts))


def decode(P, q, cos_t, sin_t, rows=None):
    """P: an object with the kv800.Paged fields as CPU tensors; q (B, 16, 128) bf16 -> (B, 16, 128) bf16. rows: the
    subset of rows to decode (others stay zero)."""
    H = hadamard128()
    B = q.shape[0]
    out = torch.zeros(B, 16, 128, dtype=torch.bfloat16)
    N, NQ = P.N.tolist(), P.NQ.tolist()
    for b in (range(B) if rows is None else rows):
        n = int(N[b])
        nq = 0 if P.win else min(int(NQ[b]), int(P.nqmax or 0))
        lo = int(NQ[b]) * BLK
        if P.win:
            lo = max(lo, n - P.win)
        got = _row_keys(P, b, n, lo, nq, H)
        if got is None:
            continue
        K, V, pos = got
        K = _rope(K, pos, cos_t, sin_t)                                                       # (S, 4, 128)
        qg = q[b].float().view(4, 4, 128)                                                     # (kv head, row, dim)
        scores = torch.matmul(qg, K.permute(1, 2, 0)) * 128 ** -0.5                          # (4, 4, S)
        o = torch.matmul(scores.softmax(-1), V.permute(1, 0, 2))                              # (4, 4, 128)
        out[b] = o.reshape(16, 128).to(torch.bfloat16)
    return out
