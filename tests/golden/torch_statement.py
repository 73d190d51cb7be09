"""CPU-torch statement of the reference quantizer / dequantizer (kv800.py:56-92), written for this build.

It evaluates the reference's arithmetic with the same torch library routines the reference uses -- float32 min / max,
true division, .round() (half to even), .to(float8_e4m3fn) and the float32 `@ H` matmul (MKL on CPU) -- so its output
bytes are what lfm3_kv800.kv800.quantize_blocks produces on CPU torch for the same input. It is the generator of the
golden fixtures (make_golden.py) and the torch-side check of the C oracle (tests/test_oracle.py); it is never
imported by the product package."""
import torch

BLK, SUB = 256, 51200
F8 = torch.float8_e4m3fn


def sylvester(n=128):
    h = torch.ones(1, 1)
    while h.shape[0] < n:
        h = torch.cat((torch.cat((h, h), 1), torch.cat((h, -h), 1)), 0)
    return h / n ** 0.5


def _fp8_pair(lo, span):
    """fp8 bytes of lo and of max(span, 1e-8), and the float32 values the reference divides by."""
    lo8 = lo.to(F8)
    sc8 = span.clamp_min(1e-8).to(F8)
    return lo8, sc8, lo8.float(), sc8.float().clamp_min(1e-8)


def quantize(k, v):
    """k, v (M, 256, 4, 128) bf16 -> (M, 51200) uint8."""
    M = k.shape[0]
    H = sylvester()
    xk = k.float()                                                   # (M, 256, 4, 128)
    klo8, ksc8, klo, kden = _fp8_pair(xk.amin(1), (xk.amax(1) - xk.amin(1)) / 3)
    codes = ((xk - klo[:, None]) / kden[:, None]).round().clamp(0, 3).to(torch.uint8)   # (M, 256, 4, 128)
    planes = codes.view(M, BLK, 4, 4, 32)                             # dim = 32 * plane + j
    kc = planes[..., 0, :] | (planes[..., 1, :] << 2) | (planes[..., 2, :] << 4) | (planes[..., 3, :] << 6)
    y = (v.float() @ H).view(M, BLK, 2, 256)                          # per (token, 2-head group)
    vlo8, vsc8, vlo, vden = _fp8_pair(y.amin(-1), y.amax(-1) - y.amin(-1))
    bits = ((y - vlo[..., None]) / vden[..., None]).round().clamp(0, 1).to(torch.uint8).view(M, BLK, 4, 8, 16)
    vb = torch.zeros(M, BLK, 4, 16, dtype=torch.uint8)
    for i in range(8):                                                # dim = 16 * i + j at bit i of byte j
        vb |= bits[..., i, :] << i
    out = torch.cat([kc.reshape(M, -1), vb.reshape(M, -1), vlo8.view(torch.uint8).reshape(M, -1),
                     vsc8.view(torch.uint8).reshape(M, -1), klo8.view(torch.uint8).reshape(M, -1),
                     ksc8.view(torch.uint8).reshape(M, -1)], 1)
    assert out.shape[1] == SUB
    return out


def dequantize(sb):
    """(M, 51200) uint8 -> K (M, 256, 4, 128) bf16, V (M, 256, 4, 128) float32."""
    M = sb.shape[0]
    H = sylvester()
    kc = sb[:, :32768].reshape(M, BLK, 4, 32)
    codes = torch.cat([(kc >> (2 * p)) & 3 for p in range(4)], -1).float()           # (M, 256, 4, 128)
    klo = sb[:, 50176:50688].contiguous().view(F8).float().view(M, 1, 4, 128)
    ksc = sb[:, 50688:].contiguous().view(F8).float().view(M, 1, 4, 128)
    k = (codes * ksc + klo).to(torch.bfloat16)
    vb = sb[:, 32768:49152].reshape(M, BLK, 4, 16)
    bits = torch.cat([(vb >> i) & 1 for i in range(8)], -1).float()                  # dim = 16 i + j
    vlo = sb[:, 49152:49664].contiguous().view(F8).float().view(M, BLK, 2, 1).repeat_interleave(2, 2)
    vsc = sb[:, 49664:50176].contiguous().view(F8).float().view(M, BLK, 2, 1).repeat_interleave(2, 2)
    return k, (bits * vsc + vlo) @ H
