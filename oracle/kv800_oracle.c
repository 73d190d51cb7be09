/* kv800_oracle.c -- CPU restatement of the lfm3-kv800 800h path. TEST INFRASTRUCTURE ONLY.
 *
 * This file is the parity checker for the HIP backend. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product library never links or calls it.
 *
 * It restates, in plain C with the same IEEE float32 operation sequence, the reference's
 *   - fp8 e4m3fn encode (torch .to(float8_e4m3fn): round-to-nearest-even, >464 -> 0x7F NaN, no saturation)
 *     and decode (kv800.py:98-104, kv800_sycl.sycl:41-45);
 *   - quantize_blocks (kv800.py:56-76), including `v.float() @ H` as a sequential fmaf chain over k = 0..127,
 *     which is bit-identical to torch-CPU's MKL sgemm for this shape (probed on 3.3 M outputs);
 *   - dequantize_blocks (kv800.py:79-92);
 *   - the pure-torch decode (torch_decode.py:16-80): per row dequantize, RoPE of all keys in fp32 rounded to bf16,
 *     one fp32 softmax (scale 1/sqrt(128)), 4 query rows per KV head, bf16 output;
 *   - the split merge `combine` (kv800.py:231-236);
 *   - the training fake quantization fake_quant_k / fake_quant_v (train.py:82-100).
 * Pinning (tests/test_oracle.py): fp8 encode exhaustively against torch; quantize_blocks byte-for-byte against a
 * torch statement of kv800.py:56-76 and against the committed golden fixtures; dequantize as the inverse of the
 * packing; decode against an independent float64 restatement of tests/test_parity.py:45-64 (the reference's own
 * independent check) on its 12 cases; fake_quant_k against a numpy float32 statement of train.py:82-89 and, on bf16
 * inputs, against the quantize -> dequantize round trip (tests/test_train_hook.py:92-106); fake_quant_v against the
 * round trip and against a float64 statement of train.py:92-100 away from rounding ties.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define BLK 256
#define SUB 51200
#define KC_O 0
#define VB_O 32768
#define VLO_O 49152
#define VSC_O 49664
#define KLO_O 50176
#define KSC_O 50688
#define NSINK 4

typedef union { float f; uint32_t u; } fu_t;

static inline float bf2f(uint16_t b) { fu_t x; x.u = (uint32_t)b << 16; return x.f; }

/* float -> bf16 bits, round to nearest even (torch .to(bfloat16); NaN stays NaN). */
static inline uint16_t f2bf(float f) {
  fu_t x; x.f = f;
  if ((x.u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((x.u >> 16) | 0x40u);
  uint32_t r = x.u + 0x7FFFu + ((x.u >> 16) & 1u);
  return (uint16_t)(r >> 16);
}
static inline float bfround(float f) { return bf2f(f2bf(f)); }

/* fp8 e4m3fn byte -> float (exact). 0x7F / 0xFF are NaN. kv800.py:98-104 */
float oracle_f8_decode(uint8_t b) {
  const uint32_t e = (b >> 3) & 15u, m = b & 7u;
  if (e == 15u && m == 7u) return NAN;
  float mag;
  if (e == 0) mag = (float)m * 0.001953125f;            /* subnormal: m * 2^-9 */
  else { fu_t x; x.u = ((e + 120u) << 23) | (m << 20); mag = x.f; }
  return (b & 0x80u) ? -mag : mag;
}

/* float -> fp8 e4m3fn byte with torch's semantics: RNE on the e4m3 grid, results past 448 (|x| > 464) -> NaN 0x7F
 * with the sign bit, inf/NaN -> 0x7F (NaN keeps its sign bit in torch: -nan -> 0xFF). */
uint8_t oracle_f8_encode(float f) {
  fu_t x; x.f = f;
  const uint8_t sign = (uint8_t)((x.u >> 24) & 0x80u);
  const uint32_t a = x.u & 0x7FFFFFFFu;
  if (a >= 0x7F800000u) return (uint8_t)(sign | 0x7Fu);   /* inf, NaN */
  fu_t y; y.u = a;
  const float v = y.f;
  if (v < 0.015625f) {                                      /* below 2^-6: subnormal grid, step 2^-9 */
    const float q = v * 512.0f;                              /* exact (power of two scaling) */
    float r = nearbyintf(q);                                 /* current rounding mode: nearest even */
    return (uint8_t)(sign | (uint8_t)r);                     /* r in 0..8; 8 == 0x08 == 2^-6 (min normal) */
  }
  /* normal: keep 3 mantissa bits, round to nearest even on the f32 bit pattern */
  const uint32_t exp = (a >> 23) & 0xFFu;                    /* >= 121 */
  uint32_t mant = a & 0x7FFFFFu;
  uint32_t keep = mant >> 20, rest = mant & 0xFFFFFu;
  uint32_t e8 = exp - 120u;                                  /* e4m3 exponent field (bias 7) */
  if (rest > 0x80000u || (rest == 0x80000u && (keep & 1u))) {
    keep += 1u;
    if (keep == 8u) { keep = 0u; e8 += 1u; }
  }
  if (e8 > 15u || (e8 == 15u && keep == 7u)) return (uint8_t)(sign | 0x7Fu);   /* past 448: NaN */
  return (uint8_t)(sign | (e8 << 3) | keep);
}

static inline float clamp_min_1e8(float a) { const float t = 1e-8f; return a < t ? t : a; }

/* torch .round(): half to even */
static inline float rne(float a) { return nearbyintf(a); }

/* y[0..127] = x[0..127] @ H, sequential fmaf over k (torch-CPU / MKL order for (M,128)@(128,128) fp32). */
static void had_seq(const float* x, const float* H, float* y) {
  for (int d = 0; d < 128; ++d) {
    float acc = 0.f;
    for (int k = 0; k < 128; ++k) acc = fmaf(x[k], H[k * 128 + d], acc);
    y[d] = acc;
  }
}

/* Sylvester Hadamard / sqrt(n) in fp32, as kv800.py:43-46 (entries are +-fp32(1/sqrt(128))). */
void oracle_hadamard(float* H) {
  const float c = (float)(1.0 / sqrt(128.0));
  for (int i = 0; i < 128; ++i)
    for (int j = 0; j < 128; ++j) H[i * 128 + j] = (__builtin_popcount((unsigned)(i & j)) & 1) ? -c : c;
}

/* kv800.py:56-76. k, v: (M, 256, 4, 128) bf16 bits -> out (M, 51200) bytes. */
void oracle_quantize_blocks(const uint16_t* k, const uint16_t* v, int64_t M, uint8_t* out) {
  float H[128 * 128];
  oracle_hadamard(H);
#pragma omp parallel for schedule(static)
  for (int64_t m = 0; m < M; ++m) {
    const uint16_t* km = k + m * (int64_t)BLK * 512;
    const uint16_t* vm = v + m * (int64_t)BLK * 512;
    uint8_t* o = out + m * (int64_t)SUB;
    uint8_t* codes = (uint8_t*)malloc(BLK * 512);
    /* ---- K: per (head, channel) over the 256 tokens */
    for (int hc = 0; hc < 512; ++hc) {
      float lo = INFINITY, hi = -INFINITY;
      for (int t = 0; t < BLK; ++t) { const float x = bf2f(km[t * 512 + hc]); lo = x < lo ? x : lo; hi = x > hi ? x : hi; }
      const uint8_t lo8 = oracle_f8_encode(lo);
      const uint8_t sc8 = oracle_f8_encode(clamp_min_1e8((hi - lo) / 3.0f));
      const float lof = oracle_f8_decode(lo8), den = clamp_min_1e8(oracle_f8_decode(sc8));
      for (int t = 0; t < BLK; ++t) {
        float c = rne((bf2f(km[t * 512 + hc]) - lof) / den);
        c = c < 0.f ? 0.f : (c > 3.f ? 3.f : c);
        codes[t * 512 + hc] = (c == c) ? (uint8_t)c : 0;
      }
      o[KLO_O + hc] = lo8;
      o[KSC_O + hc] = sc8;
    }
    for (int t = 0; t < BLK; ++t)
      for (int h = 0; h < 4; ++h)
        for (int j = 0; j < 32; ++j) {
          const uint8_t* c = codes + t * 512 + h * 128;
          o[KC_O + (t * 4 + h) * 32 + j] = (uint8_t)(c[j] | (c[j + 32] << 2) | (c[j + 64] << 4) | (c[j + 96] << 6));
        }
    /* ---- V: y = v @ H per (token, head); 1 bit per dim over groups of 2 heads (256 dims) per token */
    for (int t = 0; t < BLK; ++t) {
      float x[128], y[512];
      for (int h = 0; h < 4; ++h) {
        for (int d = 0; d < 128; ++d) x[d] = bf2f(vm[t * 512 + h * 128 + d]);
        had_seq(x, H, y + h * 128);
      }
      for (int g = 0; g < 2; ++g) {
        const float* yg = y + g * 256;
        float lo = INFINITY, hi = -INFINITY;
        for (int i = 0; i < 256; ++i) { lo = yg[i] < lo ? yg[i] : lo; hi = yg[i] > hi ? yg[i] : hi; }
        const uint8_t lo8 = oracle_f8_encode(lo);
        const uint8_t sc8 = oracle_f8_encode(clamp_min_1e8(hi - lo));
        const float lof = oracle_f8_decode(lo8), den = clamp_min_1e8(oracle_f8_decode(sc8));
        for (int hh = 0; hh < 2; ++hh) {
          const int h = 2 * g + hh;
          for (int j = 0; j < 16; ++j) {
            uint32_t byte = 0;
            for (int i = 0; i < 8; ++i) {
              float b = rne((yg[hh * 128 + j + 16 * i] - lof) / den);
              b = b < 0.f ? 0.f : (b > 1.f ? 1.f : b);
              byte |= (uint32_t)((b == b) ? (uint32_t)b : 0u) << i;
            }
            o[VB_O + (t * 4 + h) * 16 + j] = (uint8_t)byte;
          }
        }
        o[VLO_O + t * 2 + g] = lo8;
        o[VSC_O + t * 2 + g] = sc8;
      }
    }
    free(codes);
  }
}

/* kv800.py:79-92. sb (M, 51200) -> K (M,256,4,128) bf16 bits (bf16(code*ksc + klo)), V (M,256,4,128) f32
 * ((bit*vsc + vlo) @ H, sequential fmaf). */
void oracle_dequantize_blocks(const uint8_t* sb, int64_t M, uint16_t* kout, float* vout) {
  float H[128 * 128];
  oracle_hadamard(H);
#pragma omp parallel for schedule(static)
  for (int64_t m = 0; m < M; ++m) {
    const uint8_t* s = sb + m * (int64_t)SUB;
    uint16_t* ko = kout + m * (int64_t)BLK * 512;
    float* vo = vout + m * (int64_t)BLK * 512;
    for (int t = 0; t < BLK; ++t)
      for (int h = 0; h < 4; ++h) {
        const uint8_t* kc = s + KC_O + (t * 4 + h) * 32;
        for (int d = 0; d < 128; ++d) {
          const int code = (kc[d & 31] >> (2 * (d >> 5))) & 3;
          const float sc = oracle_f8_decode(s[KSC_O + h * 128 + d]), lo = oracle_f8_decode(s[KLO_O + h * 128 + d]);
          const float prod = (float)code * sc;
          ko[(t * 4 + h) * 128 + d] = f2bf(prod + lo);
        }
        const uint8_t* vb = s + VB_O + (t * 4 + h) * 16;
        const float vsc = oracle_f8_decode(s[VSC_O + t * 2 + (h >> 1)]), vlo = oracle_f8_decode(s[VLO_O + t * 2 + (h >> 1)]);
        float x[128];
        for (int d = 0; d < 128; ++d) {
          const float bit = (float)((vb[d & 15] >> (d >> 4)) & 1);
          const float prod = bit * vsc;
          x[d] = prod + vlo;
        }
        had_seq(x, H, vo + (t * 4 + h) * 128);
      }
  }
}

/* ---------------------------------------------------------------- training fake quant (train.py:82-100) */
/* x (G, 256, C) fp32 -> out: per (group, channel) code * sc8 + lo8 with the quantizer's K arithmetic (train.py:82-89:
 * float32 min / max, lo and (hi - lo) / 3 through fp8, IEEE subtract and divide, half-even round, clamp to [0, 3], then
 * the product and the sum rounded separately). */
void oracle_fake_quant_k(const float* x, int64_t G, int64_t C, float* out) {
#pragma omp parallel for schedule(static)
  for (int64_t g = 0; g < G; ++g)
    for (int64_t c = 0; c < C; ++c) {
      const float* xg = x + g * BLK * C + c;
      float lo = INFINITY, hi = -INFINITY;
      for (int t = 0; t < BLK; ++t) { const float v = xg[t * C]; lo = v < lo ? v : lo; hi = v > hi ? v : hi; }
      const float lof = oracle_f8_decode(oracle_f8_encode(lo));
      const float scf = oracle_f8_decode(oracle_f8_encode(clamp_min_1e8((hi - lo) / 3.0f)));
      const float den = clamp_min_1e8(scf);
      for (int t = 0; t < BLK; ++t) {
        float code = rne((xg[t * C] - lof) / den);
        code = code < 0.f ? 0.f : (code > 3.f ? 3.f : code);
        const float prod = code * scf;
        out[g * BLK * C + t * C + c] = prod + lof;
      }
    }
}

/* v (N, 4, 128) fp32 -> per token the V of a quantize -> dequantize round trip (train.py:92-100): y = v @ H by the
 * sequential chain, one bit per dim over each pair of heads with fp8 lo and scale = hi - lo, then
 * (bit * sc8 + lo8) @ H by the same chain. */
void oracle_fake_quant_v(const float* v, int64_t N, float* out) {
  float H[128 * 128];
  oracle_hadamard(H);
#pragma omp parallel for schedule(static)
  for (int64_t t = 0; t < N; ++t) {
    float y[512], z[512];
    for (int h = 0; h < 4; ++h) had_seq(v + t * 512 + h * 128, H, y + h * 128);
    for (int g = 0; g < 2; ++g) {
      const float* yg = y + g * 256;
      float* zg = z + g * 256;
      float lo = INFINITY, hi = -INFINITY;
      for (int i = 0; i < 256; ++i) { lo = yg[i] < lo ? yg[i] : lo; hi = yg[i] > hi ? yg[i] : hi; }
      const float lof = oracle_f8_decode(oracle_f8_encode(lo));
      const float scf = oracle_f8_decode(oracle_f8_encode(clamp_min_1e8(hi - lo)));
      const float den = clamp_min_1e8(scf);
      for (int i = 0; i < 256; ++i) {
        float b = rne((yg[i] - lof) / den);
        b = b < 0.f ? 0.f : (b > 1.f ? 1.f : b);
        const float prod = b * scf;
        zg[i] = prod + lof;
      }
    }
    for (int h = 0; h < 4; ++h) had_seq(z + h * 128, H, out + t * 512 + h * 128);
  }
}

/* ---------------------------------------------------------------- decode (torch_decode.py:27-80) */
/* Paged descriptor fields as in kv800.py:239-248. Offsets: boff bytes into qpool; eoff / skoff / svoff elements. */
typedef struct {
  const uint8_t* qpool; const int64_t* boff; int64_t boff_stride;
  const uint16_t* epool; const int64_t* eoff; int64_t eoff_stride;
  int64_t ebs, e_hs, e_ts, e_v;
  const uint16_t* sk; const uint16_t* sv; const int64_t* skoff; const int64_t* svoff;   /* sk == NULL: no sinks */
  const int32_t* N; const int32_t* NQ; int64_t nqmax; int64_t win;
} oracle_paged_t;

/* y = x @ H via a radix-2 FWHT (same value as the matmul to within float rounding; used inside decode only, where the
 * reference's own tolerance applies). */
static void had_fwht(const float* x, float* y) {
  float a[128];
  for (int d = 0; d < 128; ++d) a[d] = x[d];
  for (int len = 1; len < 128; len <<= 1)
    for (int i = 0; i < 128; i += 2 * len)
      for (int j = i; j < i + len; ++j) { const float u = a[j], w = a[j + len]; a[j] = u + w; a[j + len] = u - w; }
  const float c = (float)(1.0 / sqrt(128.0));
  for (int d = 0; d < 128; ++d) y[d] = a[d] * c;
}

/* Key row (4 heads x 128, f32, pre-RoPE) and value row of one position, gathered like torch_decode.py:52-70. */
static void rope_round(float* kr, const uint16_t* cos_t, const uint16_t* sin_t, int64_t p) {
  for (int j = 0; j < 32; ++j) {
    const float cs = bf2f(cos_t[p * 32 + j]), sn = bf2f(sin_t[p * 32 + j]);
    for (int h = 0; h < 4; ++h) {
      float* k = kr + h * 128;
      const float k0 = k[j], k2 = k[j + 64];
      const float a = k0 * cs, bb = k2 * sn, c = k2 * cs, dd = k0 * sn;
      k[j] = a - bb;
      k[j + 64] = c + dd;
    }
  }
  for (int i = 0; i < 512; ++i) kr[i] = bfround(kr[i]);
}

/* sc[r * smax + s] = q_r . k_(head r/4), float64 accumulation. */
static void score16(const float qf[16][128], const float* kr, float* sc, int64_t smax, int64_t s) {
  for (int r = 0; r < 16; ++r) {
    double acc = 0.0;
    const float* k = kr + (r >> 2) * 128;
    for (int d = 0; d < 128; ++d) acc += (double)qf[r][d] * (double)k[d];
    sc[(int64_t)r * smax + s] = (float)acc;
  }
}

/* One row b of torch_decode.decode. q (16,128) bf16 bits, cos/sin (P,32) bf16 bits; out (16,128) bf16 bits and, if
 * outf is not NULL, the same outputs before their bf16 rounding (f32).
 * Scratch: V (S, 512) f32 and sc (16, S) f32 with S >= nq*256 + 4 + (n - lo). */
static void decode_row(const oracle_paged_t* P, int64_t b, const uint16_t* q, const uint16_t* cos_t,
                       const uint16_t* sin_t, uint16_t* out, float* outf, float* V, float* sc, int64_t smax) {
  const int64_t n = P->N[b], nq_b = P->NQ[b];
  const int64_t nqmax = P->win ? 0 : P->nqmax;
  const int64_t nq = nq_b < nqmax ? nq_b : nqmax;
  int64_t lo = nq_b * BLK;
  if (P->win) lo = (n - P->win) > lo ? (n - P->win) : lo;
  float qf[16][128];
  for (int r = 0; r < 16; ++r) for (int d = 0; d < 128; ++d) qf[r][d] = bf2f(q[r * 128 + d]);
  int64_t S = 0;
  float kr[512];
  /* quantized sub-blocks j < nq: K = bf16(code*ksc + klo), V = (bit*vsc + vlo) @ H */
  for (int64_t j = 0; j < nq; ++j) {
    const uint8_t* s = P->qpool + P->boff[b * P->boff_stride + j];
    for (int t = 0; t < BLK; ++t) {
      for (int h = 0; h < 4; ++h) {
        const uint8_t* kc = s + KC_O + (t * 4 + h) * 32;
        for (int d = 0; d < 128; ++d) {
          const int code = (kc[d & 31] >> (2 * (d >> 5))) & 3;
          const float prod = (float)code * oracle_f8_decode(s[KSC_O + h * 128 + d]);
          kr[h * 128 + d] = bfround(prod + oracle_f8_decode(s[KLO_O + h * 128 + d]));
        }
        const uint8_t* vb = s + VB_O + (t * 4 + h) * 16;
        const float vsc = oracle_f8_decode(s[VSC_O + t * 2 + (h >> 1)]), vlo = oracle_f8_decode(s[VLO_O + t * 2 + (h >> 1)]);
        float x[128];
        for (int d = 0; d < 128; ++d) { const float prod = (float)((vb[d & 15] >> (d >> 4)) & 1) * vsc; x[d] = prod + vlo; }
        had_fwht(x, V + S * 512 + h * 128);
      }
      rope_round(kr, cos_t, sin_t, j * BLK + t);
      score16(qf, kr, sc, smax, S);
      ++S;
    }
  }
  if (P->win && P->sk) {
    int64_t cnt = NSINK; if (lo < cnt) cnt = lo; if (n < cnt) cnt = n;
    for (int64_t t = 0; t < cnt; ++t) {
      for (int i = 0; i < 512; ++i) {
        kr[i] = bf2f(P->sk[P->skoff[b] + t * 512 + i]);
        V[S * 512 + i] = bf2f(P->sv[P->svoff[b] + t * 512 + i]);
      }
      rope_round(kr, cos_t, sin_t, t);
      score16(qf, kr, sc, smax, S);
      ++S;
    }
  }
  for (int64_t p = lo; p < n; ++p) {
    const int64_t page = P->eoff[b * P->eoff_stride + p / P->ebs];
    for (int h = 0; h < 4; ++h) {
      const int64_t ko = page + (p % P->ebs) * P->e_ts + h * P->e_hs;
      for (int d = 0; d < 128; ++d) {
        kr[h * 128 + d] = bf2f(P->epool[ko + d]);
        V[S * 512 + h * 128 + d] = bf2f(P->epool[ko + P->e_v + d]);
      }
    }
    rope_round(kr, cos_t, sin_t, p);
    score16(qf, kr, sc, smax, S);
    ++S;
  }
  if (S == 0) {
    for (int i = 0; i < 16 * 128; ++i) { out[i] = 0; if (outf) outf[i] = 0.f; }
    return;
  }
  const float scale = (float)pow(128.0, -0.5);
  for (int r = 0; r < 16; ++r) {
    float* sr = sc + (int64_t)r * smax;
    float mx = -INFINITY;
    for (int64_t s = 0; s < S; ++s) { sr[s] *= scale; mx = sr[s] > mx ? sr[s] : mx; }
    double den = 0.0;
    for (int64_t s = 0; s < S; ++s) { sr[s] = expf(sr[s] - mx); den += sr[s]; }
    double acc[128];
    for (int d = 0; d < 128; ++d) acc[d] = 0.0;
    const int h = r >> 2;
    for (int64_t s = 0; s < S; ++s) {
      const double p = (double)(float)(sr[s] / den);
      const float* vr = V + s * 512 + h * 128;
      for (int d = 0; d < 128; ++d) acc[d] += p * (double)vr[d];
    }
    for (int d = 0; d < 128; ++d) {
      out[r * 128 + d] = f2bf((float)acc[d]);
      if (outf) outf[r * 128 + d] = (float)acc[d];
    }
  }
}

/* torch_decode.decode over all B rows (rows in parallel). q (B,16,128) bf16; out (B,16,128) bf16; outf (B,16,128)
 * f32 (or NULL): the outputs before their final bf16 rounding. */
int oracle_decode_f32(const oracle_paged_t* P, int64_t B, const uint16_t* q, const uint16_t* cos_t,
                      const uint16_t* sin_t, uint16_t* out, float* outf) {
  int64_t smax = 1;
  for (int64_t b = 0; b < B; ++b) {
    int64_t s = (int64_t)P->NQ[b] * BLK + NSINK + (P->N[b] > 0 ? P->N[b] : 0);
    if (s > smax) smax = s;
  }
  int bad = 0;
#pragma omp parallel
  {
    float* V = (float*)malloc(sizeof(float) * (size_t)smax * 512);
    float* sc = (float*)malloc(sizeof(float) * (size_t)smax * 16);
    if (!V || !sc) {
#pragma omp atomic write
      bad = 1;
    } else {
#pragma omp for schedule(dynamic, 1)
      for (int64_t b = 0; b < B; ++b)
        decode_row(P, b, q + b * 2048, cos_t, sin_t, out + b * 2048, outf ? outf + b * 2048 : NULL, V, sc, smax);
    }
    free(V); free(sc);
  }
  return bad ? -1 : 0;
}

int oracle_decode(const oracle_paged_t* P, int64_t B, const uint16_t* q, const uint16_t* cos_t, const uint16_t* sin_t,
                  uint16_t* out) {
  return oracle_decode_f32(P, B, q, cos_t, sin_t, out, NULL);
}

/* kv800.py:231-236: MO, LO (B, ns+1, 16) f32; AO (B, ns+1, 16, 128) f32 -> out (B, 16, 128) bf16 bits. */
void oracle_combine(const float* MO, const float* LO, const float* AO, int64_t B, int64_t ns, uint16_t* out) {
  float H[128 * 128];
  oracle_hadamard(H);
  const int64_t S = ns + 1;
  for (int64_t b = 0; b < B; ++b)
    for (int r = 0; r < 16; ++r) {
      float M = -INFINITY;
      for (int64_t s = 0; s < S; ++s) { const float m = MO[(b * S + s) * 16 + r]; M = m > M ? m : M; }
      float L = 0.f, xq[128], o[128];
      for (int d = 0; d < 128; ++d) xq[d] = 0.f;
      for (int64_t s = 0; s < S; ++s) {
        const float w = exp2f(MO[(b * S + s) * 16 + r] - M);
        L += w * LO[(b * S + s) * 16 + r];
        const float* a = AO + ((b * S + s) * 16 + r) * 128;
        if (s < ns) for (int d = 0; d < 128; ++d) xq[d] += w * a[d];
        else for (int d = 0; d < 128; ++d) o[d] = w * a[d];
      }
      if (ns) {
        float y[128];
        had_seq(xq, H, y);
        for (int d = 0; d < 128; ++d) o[d] += y[d];
      }
      for (int d = 0; d < 128; ++d) out[(b * 16 + r) * 128 + d] = f2bf(o[d] / L);
    }
}

int oracle_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* Batch forms for the Python wrapper. */
void oracle_f8_encode_n(const float* x, int64_t n, uint8_t* out) { for (int64_t i = 0; i < n; ++i) out[i] = oracle_f8_encode(x[i]); }
void oracle_f8_decode_n(const uint8_t* x, int64_t n, float* out) { for (int64_t i = 0; i < n; ++i) out[i] = oracle_f8_decode(x[i]); }
