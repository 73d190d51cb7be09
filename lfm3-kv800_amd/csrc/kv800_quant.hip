// kv800_quant.hip -- 800h quantize / paged flush / dequantize kernels for gfx950 and their C-ABI entry points.
//
// Reference semantics: kv800.py:56-76 (quantize_blocks), kv800.py:79-92 (dequantize_blocks), the flush plan of
// vllm_attn.py:297-317 and the PagedStore flush loop kv800.py:433-440. Output bytes are bit-identical to the
// reference quantizer on CPU torch:
//   * K: per (head, channel) min / max over the 256 tokens; lo8 = fp8(lo), sc8 = fp8(max((hi - lo) / 3, 1e-8));
//     code = clamp(rne((x - f32(lo8)) / max(f32(sc8), 1e-8)), 0, 3) with IEEE division;
//   * V: y = f32(v) @ H per (token, head) as the sequential fma chain over k = 0..127 that torch-CPU's sgemm
//     evaluates for this shape, then per (token, 2-head group) lo8 / sc8 and 1-bit codes the same way.
// Workgroups of 8 waves quantize one 256-token sub-block: its K per head, its V per token range; the input is
// gathered straight from the exact pages (paged flush) or from dense (M, 256, 4, 128) tensors, and the 51,200-byte
// result is written through the quant block table, so a flush is one launch with no host loop and no intermediate
// copies.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "kv800_common.h"
#include "../../include/kv800_hip.h"

namespace kv800 {

static thread_local char g_err[512];

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: %s", what, hipGetErrorString(e));
    return KV800_EHIP;
  }
  return KV800_OK;
}

namespace {

constexpr int QTHREADS = 512;    // 8 waves per sub-block, 32 tokens each
constexpr int QW = QTHREADS / 64, TPW = BLK / QW;

// ---------------------------------------------------------------- token-row sources
struct DenseSrc {   // (M, 256, 4, 128) contiguous K and V
  const uint16_t* k;
  const uint16_t* v;
  int64_t m;
  __device__ void prepare(int64_t*) {}
  __device__ const uint16_t* krow(int t, int h) const { return k + ((m * BLK + t) * 4 + h) * 128; }
  __device__ const uint16_t* vrow(int t, int h) const { return v + ((m * BLK + t) * 4 + h) * 128; }
};

struct PagedSrc {   // exact pages: K of (position p, head h) at eoff[r, p / ebs] + h e_hs + (p % ebs) e_ts; V at + e_v
  const uint16_t* ep;
  const int64_t* et;   // this row's page table
  int64_t ebs, e_hs, e_ts, e_v, p0;
  const int64_t* rowoff = nullptr;   // LDS: element offset of token t's head-0 K row, t < 256
  // One page-table lookup and division per token for the whole workgroup (every thread must call it).
  __device__ void prepare(int64_t* tab) {
    for (int t = threadIdx.x; t < BLK; t += blockDim.x) {
      const int64_t p = p0 + t;
      tab[t] = et[p / ebs] + (p % ebs) * e_ts;
    }
    __syncthreads();
    rowoff = tab;
  }
  __device__ const uint16_t* krow(int t, int h) const { return ep + rowoff[t] + h * e_hs; }
  __device__ const uint16_t* vrow(int t, int h) const { return krow(t, h) + e_v; }
};

// K code clamp(rne(fl(d / den)), 0, 3) without the division. fl(q) > 1/2 <=> d > den / 2 (a float above den / 2 is
// at least an ulp of den / 2 above it); fl(q) >= 3/2 <=> q >= 3/2 - 2^-24 and fl(q) > 5/2 <=> q > 5/2 + 2^-23 (the
// midpoints round to the even 3/2 and 5/2). Those two are decided on r = fl(d - t den) (one fma): near the threshold
// d - t den is a small multiple of 2^-24 times den's power of two, hence exact, and a second fma adds the margin
// den 2^-24 (den 2^-23) with the sign of the exact sum; far from it |r| dwarfs the margin. den >= 1e-8 is normal; a
// NaN d or den gives code 0, as the clamp of a NaN quotient does.
__device__ __forceinline__ uint32_t kcode(float d, float den) {
  const bool c1 = d > den * 0.5f;
  const bool c2 = __builtin_fmaf(den, 0x1p-24f, __builtin_fmaf(-den, 1.5f, d)) >= 0.f;
  const bool c3 = __builtin_fmaf(-den, 0x1p-23f, __builtin_fmaf(-den, 2.5f, d)) > 0.f;
  return (uint32_t)c1 + (uint32_t)c2 + (uint32_t)c3;
}

// x of the lane `n` places further round its 16-lane row (DPP row_ror)
__device__ __forceinline__ uint32_t row_ror(uint32_t x, int n) {
  return n == 4 ? (uint32_t)__builtin_amdgcn_update_dpp((int)x, (int)x, 0x124, 0xF, 0xF, false)
                : (uint32_t)__builtin_amdgcn_update_dpp((int)x, (int)x, 0x128, 0xF, 0xF, false);
}

struct QuantLds {                  // K path: per-wave min / max partials, then per-column lo and divisor
  float red_min[QW][512];
  float red_max[QW][512];
  float col_lo[512];
  float col_den[512];
};

// K codes and scales of one sub-block, all 4 heads in one workgroup: per (head, channel) min / max over its 256
// tokens (8 waves x 32 tokens). The latency flush uses it (one workgroup per sub-block's K); the throughput grids
// take the per-head form below, which reads each row once.
template <typename Src, int KG = 4>
__device__ void quantize_k(const Src& src, uint8_t* __restrict__ out, char* lds) {
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  QuantLds& S = *reinterpret_cast<QuantLds*>(lds);
  float* red_min = &S.red_min[0][0];
  float* red_max = &S.red_max[0][0];
  float* col_lo = S.col_lo;
  float* col_den = S.col_den;

  // ---------------- K: wave w = tokens 32w .. 32w + 31, lane = columns 8 lane .. 8 lane + 7 (head lane / 16). The
  // rows are read in groups of KG tokens, twice (min / max, then codes): the code pass walks the groups in reverse, so
  // it starts with the rows read last, the ones most likely still in L2 while the rest of the grid streams through it.
  // KG = 4 keeps the pass within the 64 VGPRs of the V pass it shares a grid with (8 waves per SIMD).
  const int h = lane >> 4, c0 = 8 * (lane & 15);
  float mn[8], mx[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) { mn[e] = INFINITY; mx[e] = -INFINITY; }
#pragma unroll 1
  for (int t0 = 0; t0 < TPW; t0 += KG) {
    uint4 kx[KG];
#pragma unroll
    for (int tt = 0; tt < KG; ++tt) kx[tt] = *reinterpret_cast<const uint4*>(src.krow(TPW * w + t0 + tt, h) + c0);
#pragma unroll
    for (int tt = 0; tt < KG; ++tt) {
      const uint32_t wd[4] = {kx[tt].x, kx[tt].y, kx[tt].z, kx[tt].w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = (e & 1) ? bf2f_hi(wd[e >> 1]) : bf2f_lo(wd[e >> 1]);
        mn[e] = fminf(mn[e], x);
        mx[e] = fmaxf(mx[e], x);
      }
    }
  }
  const int hc0 = h * 128 + c0;
#pragma unroll
  for (int e = 0; e < 8; ++e) { red_min[w * 512 + hc0 + e] = mn[e]; red_max[w * 512 + hc0 + e] = mx[e]; }
  __syncthreads();
  if (tid < 512) {
    float lo = red_min[tid], hi = red_max[tid];
#pragma unroll
    for (int ww = 1; ww < QW; ++ww) { lo = fminf(lo, red_min[ww * 512 + tid]); hi = fmaxf(hi, red_max[ww * 512 + tid]); }
    const uint32_t lo8 = f8e(lo);
    const uint32_t sc8 = f8e(clamp_min_1e8(__fdiv_rn(__fsub_rn(hi, lo), 3.0f)));
    out[KLO_O + tid] = (uint8_t)lo8;
    out[KSC_O + tid] = (uint8_t)sc8;
    col_lo[tid] = f8d(lo8);
    col_den[tid] = clamp_min_1e8(f8d(sc8));
  }
  __syncthreads();
  {
    float lof[8], den[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) { lof[e] = col_lo[hc0 + e]; den[e] = col_den[hc0 + e]; }
    const int p = (lane & 15) >> 2, q = lane & 3;   // plane of these 8 channels, byte quarter 8q .. 8q + 7
#pragma unroll 1
    for (int t0 = TPW - KG; t0 >= 0; t0 -= KG) {
      uint4 kx[KG];
#pragma unroll
      for (int tt = 0; tt < KG; ++tt) kx[tt] = *reinterpret_cast<const uint4*>(src.krow(TPW * w + t0 + tt, h) + c0);
#pragma unroll
      for (int tt = 0; tt < KG; ++tt) {
        __builtin_amdgcn_sched_barrier(0);   // one token row at a time
        const uint32_t wd[4] = {kx[tt].x, kx[tt].y, kx[tt].z, kx[tt].w};
        uint32_t d0 = 0, d1 = 0;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float x = (e & 1) ? bf2f_hi(wd[e >> 1]) : bf2f_lo(wd[e >> 1]);
          const uint32_t code = kcode(__fsub_rn(x, lof[e]), den[e]) << (2 * p);
          if (e < 4) d0 |= code << (8 * e); else d1 |= code << (8 * (e - 4));
        }
        // the 4 planes of these bytes sit in the lanes 4, 8, 12 apart within the 16-lane row
        d0 |= row_ror(d0, 4); d1 |= row_ror(d1, 4);
        d0 |= row_ror(d0, 8); d1 |= row_ror(d1, 8);
        if (p == 0) {
          const int t = TPW * w + t0 + tt;
          *reinterpret_cast<uint2*>(out + KC_O + (t * 4 + h) * 32 + 8 * q) = make_uint2(d0, d1);
        }
      }
    }
  }
}

// K codes and scales of one head hh of one sub-block, its 256 token rows read once: lane (g, c) of wave w holds the
// 8 channels 8 c .. 8 c + 7 of the tokens 32 i + 4 w + g (i = 0..7) in registers through both passes (min / max, then
// codes), so each row is fetched from memory once (the all-heads pass above reads its rows twice). Min / max across
// the 4 token rows of a wave by permlane swaps, across the 8 waves through LDS.
struct QuantLds1 {
  float red_min[QW][128];
  float red_max[QW][128];
  float col_lo[128];
  float col_den[128];
};
__device__ __forceinline__ float min4rows(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fminf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fminf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max4rows(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
template <typename Src>
__device__ void quantize_k1(const Src& src, uint8_t* __restrict__ out, char* lds, int hh) {
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, g = lane >> 4, c16 = lane & 15, c0 = 8 * c16;
  QuantLds1& S = *reinterpret_cast<QuantLds1*>(lds);
  constexpr int NT = BLK / 32;   // tokens per lane
  uint4 kx[NT];
#pragma unroll
  for (int i = 0; i < NT; ++i) kx[i] = *reinterpret_cast<const uint4*>(src.krow(32 * i + 4 * w + g, hh) + c0);
  {
    float mn[8], mx[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) { mn[e] = INFINITY; mx[e] = -INFINITY; }
#pragma unroll
    for (int i = 0; i < NT; ++i) {
      __builtin_amdgcn_sched_barrier(0);   // one token row at a time
      const uint32_t wd[4] = {kx[i].x, kx[i].y, kx[i].z, kx[i].w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = (e & 1) ? bf2f_hi(wd[e >> 1]) : bf2f_lo(wd[e >> 1]);
        mn[e] = fminf(mn[e], x);
        mx[e] = fmaxf(mx[e], x);
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      __builtin_amdgcn_sched_barrier(0);
      mn[e] = min4rows(mn[e]);
      mx[e] = max4rows(mx[e]);
    }
    if (g == 0) {
#pragma unroll
      for (int e = 0; e < 8; ++e) { S.red_min[w][c0 + e] = mn[e]; S.red_max[w][c0 + e] = mx[e]; }
    }
  }
  __syncthreads();
  if (tid < 128) {
    float lo = S.red_min[0][tid], hi = S.red_max[0][tid];
#pragma unroll
    for (int ww = 1; ww < QW; ++ww) { lo = fminf(lo, S.red_min[ww][tid]); hi = fmaxf(hi, S.red_max[ww][tid]); }
    const uint32_t lo8 = f8e(lo);
    const uint32_t sc8 = f8e(clamp_min_1e8(__fdiv_rn(__fsub_rn(hi, lo), 3.0f)));
    out[KLO_O + hh * 128 + tid] = (uint8_t)lo8;
    out[KSC_O + hh * 128 + tid] = (uint8_t)sc8;
    S.col_lo[tid] = f8d(lo8);
    S.col_den[tid] = clamp_min_1e8(f8d(sc8));
  }
  __syncthreads();
  // the rows stay packed across the passes: their unpacked floats are formed again here, not kept from the first
  // pass (64 registers instead of 32)
#pragma unroll
  for (int i = 0; i < NT; ++i) asm volatile("" : "+v"(kx[i].x), "+v"(kx[i].y), "+v"(kx[i].z), "+v"(kx[i].w));
  float lof[8], den[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) { lof[e] = S.col_lo[c0 + e]; den[e] = S.col_den[c0 + e]; }
  const int p = c16 >> 2, q = c16 & 3;   // plane of these 8 channels, byte quarter 8q .. 8q + 7
#pragma unroll
  for (int i = 0; i < NT; ++i) {
    __builtin_amdgcn_sched_barrier(0);   // one token row at a time
    const uint32_t wd[4] = {kx[i].x, kx[i].y, kx[i].z, kx[i].w};
    uint32_t d0 = 0, d1 = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float x = (e & 1) ? bf2f_hi(wd[e >> 1]) : bf2f_lo(wd[e >> 1]);
      const uint32_t code = kcode(__fsub_rn(x, lof[e]), den[e]) << (2 * p);
      if (e < 4) d0 |= code << (8 * e); else d1 |= code << (8 * (e - 4));
    }
    // the 4 planes of these bytes sit in the lanes 4, 8, 12 apart within the 16-lane row
    d0 |= row_ror(d0, 4); d1 |= row_ror(d1, 4);
    d0 |= row_ror(d0, 8); d1 |= row_ror(d1, 8);
    if (p == 0) {
      const int t = 32 * i + 4 * w + g;
      *reinterpret_cast<uint2*>(out + KC_O + (t * 4 + hh) * 32 + 8 * q) = make_uint2(d0, d1);
    }
  }
}

// ---------------------------------------------------------------- V path
// One lane owns 8 dims of one head row: lane = 16 hh + jj computes head hh's dims jj + 16 i (i = 0..7), which are
// exactly the 8 bits of the row's code byte jj. For k = 16 m + kl (m, i < 8, kl < 16),
// H[k][jj + 16 i] = H[kl][jj] (-1)^popcount(m & i), so the lane keeps the 16 values H[kl][jj] and every other sign is
// a compile-time negation.
__device__ __forceinline__ void hadamard_low(float (&hl)[16], int jj) {
  const float c = __uint_as_float(0x3DB504F3u);   // fp32(1 / sqrt(128))
#pragma unroll
  for (int kl = 0; kl < 16; ++kl) hl[kl] = (__builtin_popcount(kl & jj) & 1) ? -c : c;
}

__device__ __forceinline__ constexpr bool hneg(int m, int i) { return __builtin_popcount(m & i) & 1; }

// y[i] = sum_k x[k] H[k][jj + 16 i], each output by torch-CPU's sequential fma chain over k = 0..127. Outputs whose
// signs agree on a prefix of k share its partial sums: one chain for k < 16, two for k < 32 (by i & 1), four for
// k < 64 (by i & 3), eight after (688 fmas for the 8 outputs instead of 1024). x (the lane's staged row) is read one
// float4 at a time, two reads ahead of their use.
__device__ __forceinline__ void hadamard_row8(const float* x, const float (&hl)[16], float (&y)[8]) {
  float4 buf[3];
  buf[0] = *reinterpret_cast<const float4*>(x);
  buf[1] = *reinterpret_cast<const float4*>(x + 4);
  float ch[8];
  ch[0] = 0.f;
#pragma unroll
  for (int g = 0; g < 32; ++g) {   // k = 4 g .. 4 g + 3
    if (g + 2 < 32) buf[(g + 2) % 3] = *reinterpret_cast<const float4*>(x + 4 * (g + 2));
    const float4 v = buf[g % 3];
    const float xv[4] = {v.x, v.y, v.z, v.w};
    const int m = g >> 2;   // k >> 4
    if (g == 4) ch[1] = ch[0];
    if (g == 8) { ch[2] = ch[0]; ch[3] = ch[1]; }
    if (g == 16) { ch[4] = ch[0]; ch[5] = ch[1]; ch[6] = ch[2]; ch[7] = ch[3]; }
    const int nch = m == 0 ? 1 : m == 1 ? 2 : m < 4 ? 4 : 8;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float h = hl[(4 * g + e) & 15];
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (i < nch) ch[i] = __builtin_fmaf(xv[e], hneg(m, i) ? -h : h, ch[i]);
    }
    // the group's fmas stay before this point and the next group's reads after it: two reads ahead, no further (the
    // live chains only; the last group's results stay plain fma results)
    if (nch == 1) asm volatile("" : "+v"(ch[0])::"memory");
    else if (nch == 2) asm volatile("" : "+v"(ch[0]), "+v"(ch[1])::"memory");
    else if (nch == 4) asm volatile("" : "+v"(ch[0]), "+v"(ch[1]), "+v"(ch[2]), "+v"(ch[3])::"memory");
    else if (g < 31)
      asm volatile("" : "+v"(ch[0]), "+v"(ch[1]), "+v"(ch[2]), "+v"(ch[3]), "+v"(ch[4]), "+v"(ch[5]), "+v"(ch[6]),
                   "+v"(ch[7])::"memory");
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) y[i] = ch[i];
}

// min(x, x of a DPP partner lane); s_nop 1 gives the two wait states a DPP read of a just-written VGPR needs
#define KV800_MIN_DPP(x, ctrl)                                                                                \
  ({                                                                                                          \
    float r_;                                                                                                 \
    asm("s_nop 1\n\tv_min_f32_dpp %0, %1, %1 " ctrl " row_mask:0xf bank_mask:0xf" : "=v"(r_) : "v"(x));     \
    r_;                                                                                                       \
  })

// min over each 16-lane row, the result in every lane of the row (quad swaps, then half-row and row mirrors)
__device__ __forceinline__ float row_min16(float x) {
  x = KV800_MIN_DPP(x, "quad_perm:[1,0,3,2]");
  x = KV800_MIN_DPP(x, "quad_perm:[2,3,0,1]");
  x = KV800_MIN_DPP(x, "row_half_mirror");
  x = KV800_MIN_DPP(x, "row_mirror");
  return x;
}

// Scales of one token's V rows from the 8 chain outputs y each lane holds (lane 16 hh + jj: row hh): per 2-head group g
// (lanes 32 g .. 32 g + 31, 256 outputs) the min and max through a 16-row swap -- afterwards rows 0 / 1 hold group
// 0's min / -max partials (lanes l, l + 16 combined), rows 2 / 3 group 1's -- and DPP row reductions; lanes q = 0..3
// then encode lo (q even) or max(hi - lo, 1e-8) (q odd) of group q >> 1 in one pass. b8 is that byte (lanes 0..3);
// lof, scf are the lane's group's decoded lo and scale, den = max(scf, 1e-8) the quantizer's divisor.
struct VScales { uint32_t b8; float lof, scf, den; };
__device__ __forceinline__ VScales v_scales(const float (&y)[8], int lane) {
  const int q = lane & 3, g = lane >> 5;
  const float mn = fminf(fminf(fminf(y[0], y[1]), fminf(y[2], y[3])), fminf(fminf(y[4], y[5]), fminf(y[6], y[7])));
  const float mx = fmaxf(fmaxf(fmaxf(y[0], y[1]), fmaxf(y[2], y[3])), fmaxf(fmaxf(y[4], y[5]), fmaxf(y[6], y[7])));
  const auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(mn), __float_as_uint(-mx), false, false);
  const float red = row_min16(vmin(__uint_as_float(sw[0]), __uint_as_float(sw[1])));
  const float lo0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(red), 0));
  const float hi0 = -__int_as_float(__builtin_amdgcn_readlane(__float_as_int(red), 16));
  const float lo1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(red), 32));
  const float hi1 = -__int_as_float(__builtin_amdgcn_readlane(__float_as_int(red), 48));
  const float glo = (q & 2) ? lo1 : lo0, ghi = (q & 2) ? hi1 : hi0;
  const uint32_t b8 = f8e((q & 1) ? clamp_min_1e8(__fsub_rn(ghi, glo)) : glo);
  const float dec = f8d(b8);
  const float lof0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(dec), 0));
  const float scf0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(dec), 1));
  const float lof1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(dec), 2));
  const float scf1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(dec), 3));
  const float scf = g ? scf1 : scf0;
  return VScales{b8, g ? lof1 : lof0, scf, clamp_min_1e8(scf)};
}

// V bits and scales of tokens [t0, t0 + VT * QW) of one sub-block: wave w takes VT consecutive tokens, one token (its
// 4 head rows) per step. Each lane loads 16 bytes of the token's rows (head hh, dims 8 jj .. 8 jj + 7), two tokens
// ahead; the wave writes them as floats into its own LDS rows, and each lane runs its row's 8-output chain from there.
// Per (token, 2-head group) -- lanes 32 g .. 32 g + 31 -- the min / max of the 256 outputs go through a 16-row swap and
// DPP row reductions; the token's four scale bytes (lo and scale of each group) are encoded by lanes 0..3 at once.
// bit = rne(fl(d / den)) >= 1 with d = fl(y - lo) is evaluated without the division as d > den / 2: a float d above
// den / 2 exceeds it by at least an ulp of den / 2, so d / den > 1/2 + 2^-25 and the quotient rounds above 1/2; at
// d = den / 2 it is 1/2, which rounds to 0 (den >= 1e-8 is normal; a NaN den or d gives 0 both ways).
constexpr int VSPLIT = 4, VTOK = BLK / VSPLIT, VTPW = VTOK / QW;
constexpr int VROW = 132;   // floats per staged row: the 4 rows of a token start on different LDS banks
constexpr int VLDS_BYTES = QW * 4 * VROW * 4;

template <int VT, typename Src>
__device__ void quantize_v(const Src& src, uint8_t* __restrict__ out, int t0, char* lds) {
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int tw = t0 + VT * w;                    // this wave's first token
  const int hh = lane >> 4, jj = lane & 15;      // head row and code byte of this lane
  float* xrow = reinterpret_cast<float*>(lds) + (w * 4 + hh) * VROW;
  auto fetch = [&](int t) { return *reinterpret_cast<const uint4*>(src.vrow(t, hh) + 8 * jj); };
  uint4 pf0 = fetch(tw), pf1 = VT > 1 ? fetch(tw + 1) : pf0;
  float hl[16];
  hadamard_low(hl, jj);
  const int q = lane & 3;
#pragma unroll 1
  for (int tt = 0; tt < VT; ++tt) {
    const int t = tw + tt;
    // token t's rows -> LDS (a wave's LDS instructions execute in order: these stores follow the previous token's
    // reads and precede this token's)
    float4* dst = reinterpret_cast<float4*>(xrow + 8 * jj);
    dst[0] = make_float4(bf2f_lo(pf0.x), bf2f_hi(pf0.x), bf2f_lo(pf0.y), bf2f_hi(pf0.y));
    dst[1] = make_float4(bf2f_lo(pf0.z), bf2f_hi(pf0.z), bf2f_lo(pf0.w), bf2f_hi(pf0.w));
    pf0 = pf1;
    if (tt + 2 < VT) pf1 = fetch(t + 2);
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    float y[8];
    hadamard_row8(xrow, hl, y);

    const VScales sc = v_scales(y, lane);
    if (lane < 4) out[((q & 1) ? VSC_O : VLO_O) + t * 2 + (q >> 1)] = (uint8_t)sc.b8;
    const float half = sc.den * 0.5f;
    uint32_t byte = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) byte |= (__fsub_rn(y[i], sc.lof) > half) ? (1u << i) : 0u;
    out[VB_O + t * 64 + lane] = (uint8_t)byte;
  }
}

// A quantize grid holds, per sub-block, 4 K workgroups (one per head: all 256 tokens per channel, each row read once)
// followed in the grid by VSPLIT V workgroups (V is independent per token). Both passes fit 72 VGPRs and 39 KB of LDS,
// so 7 waves per SIMD run and the K workgroups' memory latency overlaps the V workgroups' fma chains. Workgroup
// i < 4 units is the K pass of unit i / 4, head i % 4; i >= 4 units is the V pass of unit (i - 4 units) / VSPLIT, token
// range (i - 4 units) % VSPLIT.
constexpr int QLDS_BYTES = (int)sizeof(QuantLds) > VLDS_BYTES ? (int)sizeof(QuantLds) : VLDS_BYTES;
static_assert(sizeof(QuantLds1) <= (size_t)QLDS_BYTES, "per-head K pass LDS");

// kpass: part = the head of the per-head K pass; else the V token range
template <typename Src>
__device__ __forceinline__ void quantize_part(const Src& src, uint8_t* __restrict__ out, char* lds, bool kpass, int part) {
  if (kpass) quantize_k1(src, out, lds, part);
  else quantize_v<VTPW>(src, out, part * VTOK, lds);
}

__global__ void __launch_bounds__(QTHREADS) quantize_dense_kernel(const uint16_t* __restrict__ k,
                                                                   const uint16_t* __restrict__ v,
                                                                   uint8_t* __restrict__ out, int64_t M) {
  __shared__ __align__(16) char lds[QLDS_BYTES];
  const int64_t i = blockIdx.x;
  const bool kpass = i < 4 * M;
  const int64_t m = kpass ? i / 4 : (i - 4 * M) / VSPLIT;
  quantize_part(DenseSrc{k, v, m}, out + m * SUB, lds, kpass, kpass ? (int)(i % 4) : (int)((i - 4 * M) % VSPLIT));
}

__global__ void __launch_bounds__(QTHREADS) flush_kernel(const uint16_t* __restrict__ ep, const int64_t* __restrict__ eoff,
                                                         int64_t es, int64_t ebs, int64_t e_hs, int64_t e_ts, int64_t e_v,
                                                         uint8_t* __restrict__ qpool, const int64_t* __restrict__ qbt,
                                                         int64_t qs, int64_t bsq, int64_t qs0,
                                                         const int32_t* __restrict__ nq_prev,
                                                         const int32_t* __restrict__ nq_new, int64_t R, int max_new) {
  __shared__ __align__(16) char lds[QLDS_BYTES];
  __shared__ int64_t rowtab[BLK];
  const int64_t units = R * max_new, i = blockIdx.x;
  const bool kpass = i < 4 * units;
  const int64_t unit = kpass ? i / 4 : (i - 4 * units) / VSPLIT;
  const int64_t r = unit / max_new;
  const int j = nq_prev[r] + (int)(unit % max_new);
  if (j >= nq_new[r]) return;   // uniform over the workgroup
  const int64_t tok0 = (int64_t)j * BLK;
  uint8_t* dst = qpool + qbt[r * qs + tok0 / bsq] * qs0 + ((tok0 % bsq) / BLK) * SUB;
  PagedSrc src{ep, eoff + r * es, ebs, e_hs, e_ts, e_v, tok0};
  src.prepare(rowtab);
  quantize_part(src, dst, lds, kpass, kpass ? (int)(i % 4) : (int)((i - 4 * units) % VSPLIT));
}

// ---------------------------------------------------------------- latency-oriented flush (decode steps)
// A decode step flushes one or two sub-blocks per layer, so the flush costs one sub-block's latency, not throughput.
// Same code as the throughput flush, with finer work: one token per V wave (32 V workgroups per sub-block instead of 4
// of 64 tokens) and the K rows read 16 at a time (4 dependent round trips instead of 8).
constexpr int LSPLIT = BLK / QW;   // V workgroups per sub-block in the latency flush: one token per wave

__global__ void __launch_bounds__(QTHREADS) flush_lat_kernel(const uint16_t* __restrict__ ep,
                                                             const int64_t* __restrict__ eoff, int64_t es, int64_t ebs,
                                                             int64_t e_hs, int64_t e_ts, int64_t e_v,
                                                             uint8_t* __restrict__ qpool, const int64_t* __restrict__ qbt,
                                                             int64_t qs, int64_t bsq, int64_t qs0,
                                                             const int32_t* __restrict__ nq_prev,
                                                             const int32_t* __restrict__ nq_new, int64_t R, int max_new) {
  __shared__ __align__(16) char lds[QLDS_BYTES];
  __shared__ int64_t rowtab[BLK];
  const int64_t units = R * max_new, i = blockIdx.x;
  const bool kpass = i < units;
  const int64_t unit = kpass ? i : (i - units) / LSPLIT;
  const int64_t r = unit / max_new;
  const int j = nq_prev[r] + (int)(unit % max_new);
  if (j >= nq_new[r]) return;   // uniform over the workgroup
  const int64_t tok0 = (int64_t)j * BLK;
  uint8_t* dst = qpool + qbt[r * qs + tok0 / bsq] * qs0 + ((tok0 % bsq) / BLK) * SUB;
  PagedSrc src{ep, eoff + r * es, ebs, e_hs, e_ts, e_v, tok0};
  src.prepare(rowtab);
  if (kpass) quantize_k<PagedSrc, 16>(src, dst, lds);
  else quantize_v<1>(src, dst, (int)((i - units) % LSPLIT) * QW, lds);
}

// ---------------------------------------------------------------- dequantize (kv800.py:79-92)
__global__ void __launch_bounds__(256) dequant_kernel(const uint8_t* __restrict__ sb, uint16_t* __restrict__ kout,
                                                      float* __restrict__ vout) {
  __shared__ __align__(16) float xbuf[4][4 * VROW];   // per wave: one token's 4 V rows
  const int64_t m = blockIdx.x;
  const uint8_t* s = sb + m * SUB;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  // K: bf16(code * ksc + klo) (product and sum rounded separately, as the reference's torch ops)
  for (int i = tid; i < BLK * 512 / 8; i += 256) {
    const int t = i / 64, hc0 = (i % 64) * 8, hh = hc0 >> 7, d0 = hc0 & 127;
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
      uint32_t pr = 0;
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int d = d0 + e + u;
        const uint32_t code = (s[KC_O + (t * 4 + hh) * 32 + (d & 31)] >> (2 * (d >> 5))) & 3u;
        const float kv = __fadd_rn(__fmul_rn((float)code, f8d(s[KSC_O + hh * 128 + d])), f8d(s[KLO_O + hh * 128 + d]));
        pr |= f2bf(kv) << (16 * u);
      }
      o[e >> 1] = pr;
    }
    *reinterpret_cast<uint4*>(kout + (m * BLK + t) * 512 + hc0) = make_uint4(o[0], o[1], o[2], o[3]);
  }
  // V: (bit * vsc + vlo) @ H, wave w = tokens 64w .. 64w + 63, per token its 4 head rows staged in the wave's LDS
  // rows; lane 16 hh + jj builds dims 8 jj .. 8 jj + 7 of row hh and gets dims jj + 16 i back from the chain
  float hl[16];
  const int hh = lane >> 4, jj = lane & 15;
  hadamard_low(hl, jj);
  float* xrow = &xbuf[w][hh * VROW];
  for (int tt = 0; tt < 64; ++tt) {
    const int t = 64 * w + tt;
    {
      const float vsc = f8d(s[VSC_O + t * 2 + (hh >> 1)]), vlo = f8d(s[VLO_O + t * 2 + (hh >> 1)]);
      const uint8_t* vb = s + VB_O + (t * 4 + hh) * 16;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int d = 8 * jj + e;
        const float bit = (float)((vb[d & 15] >> (d >> 4)) & 1u);
        xrow[d] = __fadd_rn(__fmul_rn(bit, vsc), vlo);
      }
    }
    __builtin_amdgcn_wave_barrier();   // a wave's LDS instructions run in order: this token's rows, then its reads
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    float y[8];
    hadamard_row8(xrow, hl, y);
    float* vo = vout + ((m * BLK + t) * 4 + hh) * 128 + jj;
#pragma unroll
    for (int i = 0; i < 8; ++i) vo[16 * i] = y[i];
  }
}


// ---------------------------------------------------------------- training fake quantization (train.py:82-100)
// fake_quant_k: x (G, 256, C) fp32 -> c * sc8 + lo8 per (group, channel), the K path of the quantizer on fp32 input
// (the product and the sum rounded separately, as torch's elementwise ops). One thread per channel, 256 channels per
// workgroup: the 256 tokens are read twice (min / max, then codes; the second pass hits L2), coalesced along C.
__global__ void __launch_bounds__(256) fake_quant_k_kernel(const float* __restrict__ x, int64_t C,
                                                           float* __restrict__ out) {
  const int64_t g = blockIdx.y, c = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (c >= C) return;
  const float* xg = x + g * BLK * C + c;
  float lo = INFINITY, hi = -INFINITY;
#pragma unroll 8
  for (int t = 0; t < BLK; ++t) {
    const float v = xg[(int64_t)t * C];
    lo = fminf(lo, v);
    hi = fmaxf(hi, v);
  }
  const float lof = f8d(f8e(lo));
  const float scf = f8d(f8e(clamp_min_1e8(__fdiv_rn(__fsub_rn(hi, lo), 3.0f))));
  const float den = clamp_min_1e8(scf);
  float* og = out + g * BLK * C + c;
#pragma unroll 8
  for (int t = 0; t < BLK; ++t) {
    float code = __builtin_rintf(__fdiv_rn(__fsub_rn(xg[(int64_t)t * C], lof), den));
    code = fminf(fmaxf(code, 0.f), 3.f);
    og[(int64_t)t * C] = __fadd_rn(__fmul_rn(code, scf), lof);
  }
}

// fake_quant_v: v (N, 4, 128) fp32 -> per token y = v H (the quantizer's sequential fma chain), one bit per dim with
// fp8 lo / scale per pair of heads, then (bit * sc8 + lo8) H with the dequantizer's chain: the V value of a
// quantize -> dequantize round trip. One wave per token at a time, the token's rows staged in LDS; lane 16 hh + jj
// holds dims jj + 16 i of row hh in both chains (the quantizer's scales and bit test as in quantize_v).
constexpr int FQV_TPW = 8;   // tokens per wave
__global__ void __launch_bounds__(256) fake_quant_v_kernel(const float* __restrict__ v, int64_t N,
                                                           float* __restrict__ out) {
  __shared__ __align__(16) float xb[4][4 * VROW];   // per wave: the token's 4 rows (v, then the dequantized values)
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int hh = lane >> 4, jj = lane & 15;
  float hl[16];
  hadamard_low(hl, jj);
  float* xrow = &xb[w][hh * VROW];
  const int64_t t0 = ((int64_t)blockIdx.x * 4 + w) * FQV_TPW;
#pragma unroll 1
  for (int tt = 0; tt < FQV_TPW; ++tt) {
    const int64_t t = t0 + tt;
    if (t >= N) break;   // uniform over the wave
    const float4* src = reinterpret_cast<const float4*>(v + (t * 4 + hh) * 128 + 8 * jj);
    const float4 a = src[0], b = src[1];
    *reinterpret_cast<float4*>(xrow + 8 * jj) = a;
    *reinterpret_cast<float4*>(xrow + 8 * jj + 4) = b;
    __builtin_amdgcn_wave_barrier();   // a wave's LDS instructions run in order
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    float y[8];
    hadamard_row8(xrow, hl, y);
    const VScales sc = v_scales(y, lane);
    const float half = sc.den * 0.5f;
    float z[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
      z[i] = __fadd_rn(__fmul_rn((__fsub_rn(y[i], sc.lof) > half) ? 1.f : 0.f, sc.scf), sc.lof);
    __builtin_amdgcn_wave_barrier();   // every lane has read the v rows
#pragma unroll
    for (int i = 0; i < 8; ++i) xrow[jj + 16 * i] = z[i];
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    hadamard_row8(xrow, hl, y);
#pragma unroll
    for (int i = 0; i < 8; ++i) out[(t * 4 + hh) * 128 + jj + 16 * i] = y[i];
    __builtin_amdgcn_wave_barrier();   // the next token's rows overwrite the staged rows
  }
}


// ---------------------------------------------------------------- prefill history (vllm_attn.py:160-163, 351-380)
// Row r's positions [0, N[r]) as contiguous bf16 K (rotated when cos_t != null) and V at output rows out_off[r] + p:
// positions below 256 NQ[r] come from sub-block p / 256 (K = bf16(code ksc + klo), V = (bit vsc + vlo) H by the
// dequantizer's fp32 chain, then bf16: dequantize_blocks, kv800.py:79-92), the others from the exact pages. RoPE is the
// reference's fp32 kf c + rotate_half(kf) s over the 128-wide tables (cos32 | 1 | cos32 | 1), (sin32 | 0 | sin32 | 0),
// each product and the sum rounded once, then bf16. Unreadable rows (offsets outside their pool, positions past the
// rope table) are written as zeros. One workgroup per (hpos-position tile, row): hpos = 64, a quarter of a sub-block,
// so that the V chain (one wave per token at a time) runs at eight waves per SIMD on a long prefill, or 16 or 4 when
// 64 gives fewer than 1,024 workgroups (a single row). hpos divides 256, so a tile never straddles a sub-block; the
// outputs do not depend on it.
__device__ __forceinline__ void rope8(float (&a)[8], float (&b)[8], const uint16_t* cs, const uint16_t* sn, bool rope) {
  // a = dims d0 .. d0 + 7, b = dims d0 + 64 .. d0 + 71; rope: d0 < 32 (cs / sn the tables' entries d0 ..), else the
  // unrotated dims, for which the table holds cos 1, sin 0
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float c = rope ? bf2f(cs[e]) : 1.0f, s = rope ? bf2f(sn[e]) : 0.0f;
    const float x = a[e], y = b[e];
    a[e] = __fadd_rn(__fmul_rn(x, c), __fmul_rn(-y, s));
    b[e] = __fadd_rn(__fmul_rn(y, c), __fmul_rn(x, s));
  }
}
__device__ __forceinline__ uint4 pack_bf16x8(const float (&x)[8]) {
  return make_uint4(f2bf(x[0]) | (f2bf(x[1]) << 16), f2bf(x[2]) | (f2bf(x[3]) << 16), f2bf(x[4]) | (f2bf(x[5]) << 16),
                    f2bf(x[6]) | (f2bf(x[7]) << 16));
}

// positions per history workgroup: a quarter of a sub-block, cut by 4 (down to 4 positions, one token per wave)
// while the rows give fewer than four workgroups per CU (a single long row: the V chain then runs at four waves per
// SIMD instead of one)
constexpr int HPOS = 64, HPOS_MIN = 4, HPOS_MIN_GROUPS = 1024;
__global__ void __launch_bounds__(256) history_kernel(kv800_paged_t P, const uint16_t* __restrict__ cos_t,
                                                      const uint16_t* __restrict__ sin_t, int64_t rope_rows,
                                                      int64_t qpool_bytes, int64_t epool_elems,
                                                      const int64_t* __restrict__ out_off, uint16_t* __restrict__ kout,
                                                      uint16_t* __restrict__ vout, int hpos) {
  __shared__ __align__(16) float xbuf[4][4 * VROW];   // per wave: one token's 4 dequantized V rows
  __shared__ float klo_s[512], ksc_s[512];
  const int r = blockIdx.y, tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int n = P.N[r], p0 = blockIdx.x * hpos;
  if (p0 >= n) return;   // uniform over the workgroup
  const int cnt = min(hpos, n - p0);
  const int sb = p0 / BLK, to = p0 - sb * BLK;   // the positions' sub-block and the first one's token in it
  const int64_t ob = out_off[r] + p0;
  const bool rot = cos_t != nullptr;
  const int nq = min((int64_t)max(P.NQ[r], 0), P.boff_stride);
  const uint4 zero4 = make_uint4(0, 0, 0, 0);
  if (sb < nq) {
    const int64_t base = P.boff[(int64_t)r * P.boff_stride + sb];
    const bool ok = base >= 0 && base + SUB <= qpool_bytes;   // uniform
    const uint8_t* s = P.qpool + (ok ? base : 0);
    if (ok)
      for (int i = tid; i < 512; i += 256) { klo_s[i] = f8d(s[KLO_O + i]); ksc_s[i] = f8d(s[KSC_O + i]); }
    __syncthreads();
    // K: unit u = (token t, head h, d0 = 8 (u % 8)): dims d0 .. d0 + 7 and d0 + 64 .. d0 + 71
    for (int u = tid; u < cnt * 32; u += 256) {
      const int t = u >> 5, h = (u >> 3) & 3, d0 = 8 * (u & 7);
      uint16_t* ko = kout + (ob + t) * 512 + h * 128 + d0;
      const int pos = p0 + t;
      if (!ok || (rot && pos >= rope_rows)) {
        *reinterpret_cast<uint4*>(ko) = zero4;
        *reinterpret_cast<uint4*>(ko + 64) = zero4;
        continue;
      }
      const uint2 by = *reinterpret_cast<const uint2*>(s + KC_O + ((to + t) * 4 + h) * 32 + (d0 & 31));
      const uint32_t bw[2] = {by.x, by.y};
      const int sa = 2 * (d0 >> 5), sb = sa + 4;   // code fields of dims d0 + e and d0 + 64 + e
      float a[8], b[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t byte = (bw[e >> 2] >> (8 * (e & 3))) & 0xFFu;
        const int ia = h * 128 + d0 + e, ib = ia + 64;
        a[e] = bf2f(f2bf(__fadd_rn(__fmul_rn((float)((byte >> sa) & 3u), ksc_s[ia]), klo_s[ia])));
        b[e] = bf2f(f2bf(__fadd_rn(__fmul_rn((float)((byte >> sb) & 3u), ksc_s[ib]), klo_s[ib])));
      }
      if (rot) rope8(a, b, cos_t + (int64_t)pos * 32 + d0, sin_t + (int64_t)pos * 32 + d0, d0 < 32);
      *reinterpret_cast<uint4*>(ko) = pack_bf16x8(a);
      *reinterpret_cast<uint4*>(ko + 64) = pack_bf16x8(b);
    }
    // V: wave w takes tokens w, w + 4, ...; lane 16 hh + jj builds dims 8 jj .. 8 jj + 7 of bit vsc + vlo for row hh,
    // then gets dims jj + 16 i of that row from the chain
    float hl[16];
    const int hh = lane >> 4, jj = lane & 15;
    hadamard_low(hl, jj);
    float* xrow = &xbuf[w][hh * VROW];
    for (int t = w; t < cnt; t += 4) {
      uint16_t* vo = vout + (ob + t) * 512;
      if (!ok) {
        for (int i = lane; i < 512; i += 64) vo[i] = 0;
        continue;
      }
      {
        const float vsc = f8d(s[VSC_O + (to + t) * 2 + (hh >> 1)]), vlo = f8d(s[VLO_O + (to + t) * 2 + (hh >> 1)]);
        const uint8_t* vb = s + VB_O + ((to + t) * 4 + hh) * 16;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int d = 8 * jj + e;
          const float bit = (float)((vb[d & 15] >> (d >> 4)) & 1u);
          xrow[d] = __fadd_rn(__fmul_rn(bit, vsc), vlo);
        }
      }
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      float y[8];
      hadamard_row8(xrow, hl, y);
#pragma unroll
      for (int i = 0; i < 8; ++i) vo[hh * 128 + jj + 16 * i] = (uint16_t)f2bf(y[i]);
    }
    return;
  }
  // exact positions: unit u = (token t, head h, d0), K rotated, V copied
  const int64_t* et = P.eoff + (int64_t)r * P.eoff_stride;
  for (int u = tid; u < cnt * 32; u += 256) {
    const int t = u >> 5, h = (u >> 3) & 3, d0 = 8 * (u & 7);
    const int pos = p0 + t;
    uint16_t* ko = kout + (ob + t) * 512 + h * 128 + d0;
    uint16_t* vo = vout + (ob + t) * 512 + h * 128 + d0;
    const int64_t pg = pos / P.ebs;
    const int64_t eb = pg < P.eoff_stride ? et[pg] : -1;
    const int64_t kr = eb + h * P.e_hs + (pos - pg * P.ebs) * P.e_ts, vr = kr + P.e_v;
    if (eb < 0 || kr < 0 || vr < 0 || kr + 128 > epool_elems || vr + 128 > epool_elems || (rot && pos >= rope_rows)) {
      *reinterpret_cast<uint4*>(ko) = zero4; *reinterpret_cast<uint4*>(ko + 64) = zero4;
      *reinterpret_cast<uint4*>(vo) = zero4; *reinterpret_cast<uint4*>(vo + 64) = zero4;
      continue;
    }
    const uint4 k0 = *reinterpret_cast<const uint4*>(P.epool + kr + d0);
    const uint4 k1 = *reinterpret_cast<const uint4*>(P.epool + kr + d0 + 64);
    *reinterpret_cast<uint4*>(vo) = *reinterpret_cast<const uint4*>(P.epool + vr + d0);
    *reinterpret_cast<uint4*>(vo + 64) = *reinterpret_cast<const uint4*>(P.epool + vr + d0 + 64);
    if (!rot) {
      *reinterpret_cast<uint4*>(ko) = k0;
      *reinterpret_cast<uint4*>(ko + 64) = k1;
      continue;
    }
    const uint32_t wa[4] = {k0.x, k0.y, k0.z, k0.w}, wb[4] = {k1.x, k1.y, k1.z, k1.w};
    float a[8], b[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      a[e] = (e & 1) ? bf2f_hi(wa[e >> 1]) : bf2f_lo(wa[e >> 1]);
      b[e] = (e & 1) ? bf2f_hi(wb[e >> 1]) : bf2f_lo(wb[e >> 1]);
    }
    rope8(a, b, cos_t + (int64_t)pos * 32 + d0, sin_t + (int64_t)pos * 32 + d0, d0 < 32);
    *reinterpret_cast<uint4*>(ko) = pack_bf16x8(a);
    *reinterpret_cast<uint4*>(ko + 64) = pack_bf16x8(b);
  }
}

}  // namespace
}  // namespace kv800

using namespace kv800;

extern "C" {

int kv800_hip_version(void) { return 100; }

const char* kv800_hip_last_error(void) { return g_err; }

int kv800_hip_quantize_blocks(const uint16_t* k, const uint16_t* v, int64_t M, uint8_t* out, void* stream) {
  g_err[0] = 0;
  KV800_REQUIRE(M >= 0, "quantize_blocks: M = %lld < 0", (long long)M);
  if (M == 0) return KV800_OK;
  KV800_REQUIRE(k && v && out, "quantize_blocks: null pointer");
  KV800_REQUIRE(M * (4 + VSPLIT) <= 0x7FFFFFFF, "quantize_blocks: M = %lld too large", (long long)M);
  KV800_REQUIRE(((uintptr_t)k % 16) == 0 && ((uintptr_t)v % 16) == 0 && ((uintptr_t)out % 8) == 0,
                "quantize_blocks: k / v must be 16-byte aligned and out 8-byte aligned");
  hipLaunchKernelGGL(quantize_dense_kernel, dim3((unsigned)(M * (4 + VSPLIT))), dim3(QTHREADS), 0, (hipStream_t)stream, k,
                     v, out, M);
  return check_launch("quantize_blocks");
}

int kv800_hip_flush(const uint16_t* epool, const int64_t* eoff, int64_t eoff_stride, int64_t ebs, int64_t e_hs,
                    int64_t e_ts, int64_t e_v, uint8_t* qpool, const int64_t* qbt, int64_t qbt_stride, int64_t bsq,
                    int64_t qs0, const int32_t* nq_prev, const int32_t* nq_new, int64_t R, int64_t max_new,
                    void* stream) {
  g_err[0] = 0;
  KV800_REQUIRE(R >= 0 && max_new >= 0, "flush: R and max_new must be >= 0");
  if (R == 0 || max_new == 0) return KV800_OK;
  KV800_REQUIRE(epool && eoff && qpool && qbt && nq_prev && nq_new, "flush: null pointer");
  KV800_REQUIRE(ebs > 0 && bsq > 0 && bsq % BLK == 0, "flush: ebs must be > 0 and bsq a positive multiple of 256");
  KV800_REQUIRE(e_hs % 8 == 0 && e_ts % 8 == 0 && e_v % 8 == 0 && ((uintptr_t)epool % 16) == 0,
                "flush: exact-pool strides must be multiples of 8 elements and the pool 16-byte aligned");
  KV800_REQUIRE(R * max_new * (4 + VSPLIT) <= 0x7FFFFFFF, "flush: grid too large");
  hipLaunchKernelGGL(flush_kernel, dim3((unsigned)(R * max_new * (4 + VSPLIT))), dim3(QTHREADS), 0, (hipStream_t)stream,
                     epool, eoff, eoff_stride, ebs, e_hs, e_ts, e_v, qpool, qbt, qbt_stride, bsq, qs0, nq_prev, nq_new, R,
                     (int)max_new);
  return check_launch("flush");
}

int kv800_hip_flush_latency(const uint16_t* epool, const int64_t* eoff, int64_t eoff_stride, int64_t ebs, int64_t e_hs,
                            int64_t e_ts, int64_t e_v, uint8_t* qpool, const int64_t* qbt, int64_t qbt_stride,
                            int64_t bsq, int64_t qs0, const int32_t* nq_prev, const int32_t* nq_new, int64_t R,
                            int64_t max_new, void* stream) {
  g_err[0] = 0;
  KV800_REQUIRE(R >= 0 && max_new >= 0, "flush_latency: R and max_new must be >= 0");
  if (R == 0 || max_new == 0) return KV800_OK;
  KV800_REQUIRE(epool && eoff && qpool && qbt && nq_prev && nq_new, "flush_latency: null pointer");
  KV800_REQUIRE(ebs > 0 && bsq > 0 && bsq % BLK == 0, "flush_latency: ebs must be > 0 and bsq a positive multiple of 256");
  KV800_REQUIRE(e_hs % 8 == 0 && e_ts % 8 == 0 && e_v % 8 == 0 && ((uintptr_t)epool % 16) == 0,
                "flush_latency: exact-pool strides must be multiples of 8 elements and the pool 16-byte aligned");
  KV800_REQUIRE(R * max_new * (1 + LSPLIT) <= 0x7FFFFFFF, "flush_latency: grid too large");
  hipLaunchKernelGGL(flush_lat_kernel, dim3((unsigned)(R * max_new * (1 + LSPLIT))), dim3(QTHREADS), 0,
                     (hipStream_t)stream, epool, eoff, eoff_stride, ebs, e_hs, e_ts, e_v, qpool, qbt, qbt_stride, bsq,
                     qs0, nq_prev, nq_new, R, (int)max_new);
  return check_launch("flush_latency");
}

int kv800_hip_dequantize_blocks(const uint8_t* sb, int64_t M, uint16_t* k_out, float* v_out, void* stream) {
  g_err[0] = 0;
  KV800_REQUIRE(M >= 0, "dequantize_blocks: M = %lld < 0", (long long)M);
  if (M == 0) return KV800_OK;
  KV800_REQUIRE(sb && k_out && v_out, "dequantize_blocks: null pointer");
  KV800_REQUIRE(M <= 0x7FFFFFFF, "dequantize_blocks: M too large");
  KV800_REQUIRE(((uintptr_t)k_out % 16) == 0, "dequantize_blocks: k_out must be 16-byte aligned");
  hipLaunchKernelGGL(dequant_kernel, dim3((unsigned)M), dim3(256), 0, (hipStream_t)stream, sb, k_out, v_out);
  return check_launch("dequantize_blocks");
}

int kv800_hip_fake_quant_k(const float* x, int64_t G, int64_t C, float* out, void* stream) {
  g_err[0] = 0;
  KV800_REQUIRE(G >= 0 && C >= 0, "fake_quant_k: G and C must be >= 0");
  if (G == 0 || C == 0) return KV800_OK;
  KV800_REQUIRE(x && out, "fake_quant_k: null pointer");
  KV800_REQUIRE(G <= 65535 && (C + 255) / 256 <= 0x7FFFFFFF, "fake_quant_k: at most 65535 groups per call");
  hipLaunchKernelGGL(fake_quant_k_kernel, dim3((unsigned)((C + 255) / 256), (unsigned)G), dim3(256), 0,
                     (hipStream_t)stream, x, C, out);
  return check_launch("fake_quant_k");
}

int kv800_hip_fake_quant_v(const float* v, int64_t N, float* out, void* stream) {
  g_err[0] = 0;
  KV800_REQUIRE(N >= 0, "fake_quant_v: N < 0");
  if (N == 0) return KV800_OK;
  KV800_REQUIRE(v && out, "fake_quant_v: null pointer");
  KV800_REQUIRE(((uintptr_t)v % 16) == 0, "fake_quant_v: v must be 16-byte aligned");
  const int64_t nb = (N + 4 * FQV_TPW - 1) / (4 * FQV_TPW);
  KV800_REQUIRE(nb <= 0x7FFFFFFF, "fake_quant_v: N too large");
  hipLaunchKernelGGL(fake_quant_v_kernel, dim3((unsigned)nb), dim3(256), 0, (hipStream_t)stream, v, N, out);
  return check_launch("fake_quant_v");
}

int kv800_hip_history(const kv800_paged_t* P, int64_t R, int64_t max_n, const uint16_t* cos_t, const uint16_t* sin_t,
                       int64_t rope_rows, int64_t qpool_bytes, int64_t epool_elems, const int64_t* out_off,
                       uint16_t* k_out, uint16_t* v_out, void* stream) {
  g_err[0] = 0;
  KV800_REQUIRE(P && R >= 0 && max_n >= 0, "history: bad arguments");
  if (R == 0 || max_n == 0) return KV800_OK;
  KV800_REQUIRE(P->N && P->NQ && P->epool && P->eoff && out_off && k_out && v_out, "history: null pointer");
  KV800_REQUIRE(!cos_t == !sin_t, "history: cos_t and sin_t go together");
  KV800_REQUIRE(P->ebs > 0 && P->e_hs % 8 == 0 && P->e_ts % 8 == 0 && P->e_v % 8 == 0 && ((uintptr_t)P->epool % 16) == 0,
                "history: exact strides must be multiples of 8 elements and the pool 16-byte aligned");
  KV800_REQUIRE(P->boff_stride == 0 || (P->qpool && P->boff), "history: quantized rows need qpool and boff");
  KV800_REQUIRE(((uintptr_t)k_out % 16) == 0 && ((uintptr_t)v_out % 16) == 0, "history: outputs must be 16-byte aligned");
  KV800_REQUIRE(R <= 65535, "history: at most 65535 rows per call");
  int hpos = HPOS;
  while (hpos > HPOS_MIN && (max_n + hpos - 1) / hpos * R < HPOS_MIN_GROUPS) hpos /= 4;
  const int64_t tiles = (max_n + hpos - 1) / hpos;
  KV800_REQUIRE(tiles <= 0x7FFFFFFF, "history: max_n too large");
  hipLaunchKernelGGL(history_kernel, dim3((unsigned)tiles, (unsigned)R), dim3(256), 0, (hipStream_t)stream, *P, cos_t,
                     sin_t, rope_rows, qpool_bytes, epool_elems, out_off, k_out, v_out, hpos);
  return check_launch("history");
}

}  // extern "C"
