// kv800_decode.hip -- paged split-K decode attention over the 800h cache for gfx950, and its C-ABI entry points.
//
// Semantics (kv800.py:120-236, kv800_sycl.sycl:48-504, torch_decode.py:16-80): for each row b, 16 query rows over
// 4 KV heads (GQA 4), head_dim 128, scores q . RoPE(K) with RoPE on the dim pairs (d, d + 64), d < 32, fp32 online
// softmax in log2 units (scale = log2(e) / sqrt(128)); flushed sub-blocks contribute 2-bit K and 1-bit
// Hadamard-domain V, the exact tail / sinks bf16 K (rotated, rounded to bf16) and V; splits are merged by
// log-sum-exp, with the 128-point Hadamard applied once to the merged quantized part.
//
// Kernels
//   rope_table_kernel   bf16 (cos, sin) tables -> packed fp16 pairs (exact for every table value above 2^-17).
//   decode_quant_kernel one workgroup (4 waves) per (row b, split s); each wave owns whole 256-token sub-blocks,
//                       32 tokens (one chunk) at a time, the next chunk's bytes prefetched into registers.
//     QK on MFMA f32_16x16x32_f16, N = the 16 query rows. With the 2-bit codes c as exact fp16 features (one
//       e2m1 -> fp16 conversion per byte) and per-channel k = klo + ksc c, RoPE is moved onto exact fp16 features:
//         rope dims: (cos c0, sin c0, cos c2, sin c2) x weights (q0 S0, q2 S0, q2 S2, -q0 S2), S = ksc scale
//         nope dims: (c1, c3)                         x weights (q1 S1, q3 S3)
//         klo part : (cos, sin) of the position        x weights (q0 T0 + q2 T2, q2 T0 - q0 T2), T = klo
//       and the per-row constant sum(q1 T1 + q3 T3) initialises the accumulator.
//       Rope / nope MFMAs take M = 16 (token, head) rows -- 4 tokens x the 4 KV heads -- so every weight register is
//       dense (query row n applies head n / 4's scales) and only the output rows of head n / 4 are kept; the klo part
//       takes M = 16 tokens (head-independent features, weights from head n / 4). Weights are rebuilt per sub-block.
//     PV on the same MFMA: M = 16 dims (one bit plane), N = the 16 rows, K = 32 tokens. The bit feature is the
//       fp16 subnormal bit 2^(i - 24) (one AND per two tokens; MFMA keeps fp16 subnormal inputs exactly), the
//       weights fp16(p vsc) masked to the head's rows; plane i is scaled back by 2^(24 - i) at the end.
//     Softmax with a lazy running max (rescale only when a tile max exceeds it by more than 8 log2 units).
//   decode_exact_kernel one workgroup per row b, one wave per KV head (the exact-tail workgroups of the quantized
//                       grid: one per (row, KV head), its 4 waves taking turns over the chunks): sinks + exact
//                       positions in 32-token chunks (loads one chunk ahead), QK on v_dot2 bf16 pairs, PV fp32; the
//                       fused variant also merges the quantized splits of its rows.
//   decode_merge_kernel one workgroup per row b: LSE merge + in-register FWHT (staged path).
#include <math.h>

#include "kv800_common.h"
#include "../../include/kv800_hip.h"

namespace kv800 {
namespace {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4v __attribute__((ext_vector_type(4)));

constexpr float NEG_BIG = -1e30f;
constexpr float LAZY = 8.f;   // log2 units a tile max may exceed the running max before the state is rescaled

__device__ __forceinline__ uint32_t hbits(h2 x) { return __builtin_bit_cast(uint32_t, x); }
__device__ __forceinline__ h2 as_h2(uint32_t x) { return __builtin_bit_cast(h2, x); }
__device__ __forceinline__ h8 pack8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  u4v v = {a, b, c, d};
  return __builtin_bit_cast(h8, v);
}
__device__ __forceinline__ f4 mfma16(h8 a, h8 b, f4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }
__device__ __forceinline__ uint32_t pk2(float a, float b) {   // two floats -> packed fp16 (round to nearest even)
  h2 v = {(_Float16)a, (_Float16)b};
  return hbits(v);
}

// Values of the lanes 16 (32) apart without an LDS round trip: v_permlane16_swap (v_permlane32_swap) on two copies of
// x leaves the even 16-lane row (lower half) in .x and the odd row (upper half) in .y, in both lanes of each pair, so
// combining .x and .y gives the pair the same result. All 64 lanes must be active.
__device__ __forceinline__ float2 rows16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return make_float2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float2 halves32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return make_float2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum4rows(float x) {   // sum over lanes l, l ^ 16, l ^ 32, l ^ 48
  float2 p = rows16(x);
  p = halves32(p.x + p.y);
  return p.x + p.y;
}
__device__ __forceinline__ float max4rows(float x) {
  float2 p = rows16(x);
  p = halves32(fmaxf(p.x, p.y));
  return fmaxf(p.x, p.y);
}

// Four fp8 e4m3fn bytes of w -> floats (byte i -> o[i]) with the hardware conversion: gfx950 converts the OCP e4m3
// format, the same as torch's float8_e4m3fn, exactly; the NaN bytes 0x7F / 0xFF give NaN as torch's .float() does
// (kv800.py:84-91; the quantizer writes them only for scales beyond +-464).
__device__ __forceinline__ void f8x4(uint32_t w, float* o) {
  const auto a = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false), b = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
  o[0] = a[0]; o[1] = a[1]; o[2] = b[0]; o[3] = b[1];
}

// ---------------------------------------------------------------- rope table
__global__ void rope_table_kernel(const uint16_t* __restrict__ cos_t, const uint16_t* __restrict__ sin_t, int64_t n,
                                  uint32_t* __restrict__ cs16) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  cs16[i] = pk2(bf2f(cos_t[i]), bf2f(sin_t[i]));
}

// ---------------------------------------------------------------- exact tail + sinks
// A workgroup of 4 waves takes NH KV heads of one row b (query rows 4 h .. 4 h + 3 of head h): NH = 4, one wave per
// head; NH = 1, the 4 waves take the head's 32-token chunks in turn (wave w: chunks w, w + 4, ...) and merge their
// states at the end. The tokens are the row's sinks, then its exact positions. Both products run on MFMA
// f32_16x16x32_bf16 with a 32-token chunk as two 16-token tiles u; lane (g, n) = (lane / 16, lane % 16):
// - QK: A = the tile's K rows (row n = token 16 u + n; k-step s = dims 32 s + 8 g .. + 7), B = q (column n < 8 =
//   query row n % 4, zero above). The RoPE pairs (j, j + 64), j < 32, are rotated in fp32 and rounded to bf16 by one
//   packed convert (RNE, as kv800.py:182-183); the NoPE dims go in as stored. Score register i of tile u in lane
//   (g, n) is token 16 u + 4 g + i, column n.
// - softmax: fp32, log2 units, with a lazy running max (rescale only when a chunk max exceeds it by more than LAZY).
// - PV: A = V^T (row = dim; K = the 8 tokens 4 g .. 4 g + 3, 16 + 4 g .. + 3 whose scores the lane holds), read by
//   ds_read_b64_tr_b16 from the wave's LDS copy of the chunk's V rows; B = the weights in bf16, hi = bf16(p) in
//   columns 0..3 and lo = bf16(p - hi) in the duplicate columns 4..7, so hi + lo carries p to ~16 bits.
// A wave requests its next chunk's K, V and rope rows before computing the current one; the row's page-table entries
// sit in LDS, so no load inside the loop waits on another.
typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
typedef __bf16 b8 __attribute__((ext_vector_type(8)));
typedef short s4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s4 lds_s4;
constexpr int XCH = 32;                // tokens per chunk
constexpr int XPG = 64;                // page-table entries of the row kept in LDS (later pages are read from memory)
constexpr int XVROW = 144;             // bf16 per staged V row: 128 + 16 padding spreads a tile's rows over the banks
constexpr int XTROW = 132;             // floats per row of the end-of-row column dump
struct XLds {
  int64_t pg[XPG];                     // element offsets of the row's exact pages, from page lo_e / ebs on
  uint16_t v[4][XCH][XVROW];           // each wave's copy of its chunk's V rows; at the end its columns and (m, l)
  u4v qb[4][4][64];                    // each wave's QK B operand: k-step s of lane l in qb[w][s][l]
  float fm[4][4], fl[4][4];            // NH = 1: each wave's m and l of rows 0..3
  float facc[4][4][128];               // NH = 1: each wave's accumulators of rows 0..3
};
static_assert(sizeof(float) * (8 * XTROW + 8) <= sizeof(uint16_t) * XCH * XVROW, "column dump must fit the V copy");
struct XChunk {                        // one chunk's data in registers; lane (g, r): token 16 u + r of tile u
  u4v k[2][4];                         // K dims 32 s + 8 g .. + 7
  u4v v[2][4];                         // V dims 32 s + 8 g .. + 7
  u4v c[2], s[2];                      // cos / sin of channels 8 g .. + 7 at the token's position
  uint32_t ok;                         // chunk tokens with K, V and rope rows (bit t = chunk token t)
};
__device__ __forceinline__ float bf_elem(const u4v& x, int e) {   // bf16 element e < 8 of x as a float
  const uint32_t w = x[e >> 1];
  return __uint_as_float((e & 1) ? (w & 0xFFFF0000u) : (w << 16));
}
__device__ __forceinline__ uint32_t bfpk(float a, float b) {   // two floats -> packed bf16 (round to nearest even)
  const bf2 v = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ b8 as_b8(const u4v& x) { return __builtin_bit_cast(b8, x); }
__device__ __forceinline__ f4 mfma_bf(b8 a, b8 b, f4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0); }

// MERGE = false: writes the exact partial (m, l, acc) of the heads' rows into partial slot xslot.
// MERGE = true : instead merges it with the ns quantized partials of those rows (slots b (ns + 1) + s, written before
//                on the same stream) and writes the bf16 output rows, as decode_merge_kernel does for all 16 rows.
template <int NH, bool MERGE>
__device__ __forceinline__ void exact_row(XLds& X, const int b, const int h0, const kv800_paged_t& P,
                                          const uint16_t* __restrict__ q,
                                          const uint16_t* __restrict__ cos_t, const uint16_t* __restrict__ sin_t,
                                          int64_t rope_rows, int64_t epool_elems, int64_t sink_elems,
                                          float* __restrict__ mo, float* __restrict__ lo_out, float* __restrict__ ao,
                                          int ns, int64_t xslot, float scale, int nsink, uint16_t* __restrict__ out) {
  static_assert(NH == 1 || NH == 4, "a workgroup takes one KV head or all four");
  constexpr int WPH = 4 / NH;          // waves per head
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, g = lane >> 4, r16 = lane & 15;
  const int hl = w / WPH, ph = w % WPH, h = h0 + hl;   // head slot, chunk phase, KV head
  const int n = P.N[b];
  int lo_e = P.NQ[b] * BLK;
  if (P.win > 0) lo_e = max(lo_e, n - (int)P.win);
  lo_e = max(lo_e, 0);
  const int cnt = (nsink > 0) ? max(0, min(min(nsink, lo_e), n)) : 0;
  const int T = cnt + max(0, n - lo_e);
  const int64_t* et = P.eoff + (int64_t)b * P.eoff_stride;
  const int64_t p0 = lo_e / P.ebs;
  if (tid < XPG) X.pg[tid] = (p0 + tid < P.eoff_stride) ? et[p0 + tid] : -1;
  // q as the QK B operand: column r16 < 8 holds query row 4 h + r16 % 4, dims 32 s + 8 g .. + 7 in k-step s (kept in
  // LDS and read per chunk: 16 registers fewer across the loop)
  {
    const uint16_t* qr = q + ((int64_t)b * 16 + 4 * h + (r16 & 3)) * 128 + 8 * g;
#pragma unroll
    for (int s = 0; s < 4; ++s)
      X.qb[w][s][lane] = (r16 < 8) ? *reinterpret_cast<const u4v*>(qr + 32 * s) : u4v{0u, 0u, 0u, 0u};
  }
  const int64_t sko = cnt ? P.skoff[b] : 0, svo = cnt ? P.svoff[b] : 0;
  __syncthreads();

  // element offsets of token i's K and V rows (sink or exact page), its position; -1 if out of range
  auto rows = [&](int i, int64_t& ko, int64_t& vo, int& pos) {
    if (i < cnt) {
      pos = i;
      ko = sko + ((int64_t)i * 4 + h) * 128;
      vo = svo + ((int64_t)i * 4 + h) * 128;
      if (ko < 0 || vo < 0 || ko + 128 > sink_elems || vo + 128 > sink_elems) ko = vo = -1;
    } else {
      pos = lo_e + (i - cnt);
      const int64_t pg = pos / P.ebs, pi = pg - p0;
      int64_t base = -1;
      if (pi < XPG) base = X.pg[pi];
      else if (pg < P.eoff_stride) base = et[pg];
      ko = base + h * P.e_hs + (pos - pg * P.ebs) * P.e_ts;
      vo = ko + P.e_v;
      if (base < 0 || ko < 0 || ko + 128 > epool_elems || vo + 128 > epool_elems) ko = vo = -1;
    }
  };
  // lanes without a token read the row's first query row instead (finite data: its scores are masked and its
  // weights are zero, so nothing of it reaches the output), which keeps every load unconditional
  const uint16_t* qf = q + (int64_t)b * 16 * 128 + 8 * g;
  auto load = [&](int c0, XChunk& C) {
    uint32_t okm = 0;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int t = c0 + 16 * u + r16;
      int64_t ko = -1, vo = -1;
      int pos = 0;
      if (t < T) rows(t, ko, vo, pos);
      const bool ok = t < T && ko >= 0 && pos < rope_rows;   // rows() sets ko and vo out of range together
      const uint16_t *kr = qf, *vr = qf, *cr = qf, *sr = qf;
      if (ok) {
        kr = ((t < cnt) ? P.sk : P.epool) + ko + 8 * g;
        vr = ((t < cnt) ? P.sv : P.epool) + vo + 8 * g;
        cr = cos_t + (int64_t)pos * 32 + 8 * g;
        sr = sin_t + (int64_t)pos * 32 + 8 * g;
      }
#pragma unroll
      for (int s = 0; s < 4; ++s) C.k[u][s] = *reinterpret_cast<const u4v*>(kr + 32 * s);
      C.c[u] = *reinterpret_cast<const u4v*>(cr);
      C.s[u] = *reinterpret_cast<const u4v*>(sr);
#pragma unroll
      for (int s = 0; s < 4; ++s) C.v[u][s] = *reinterpret_cast<const u4v*>(vr + 32 * s);
      okm |= ((uint32_t)__ballot(ok) & 0xFFFFu) << (16 * u);
    }
    C.ok = okm;
  };

  uint16_t (*Vs)[XVROW] = X.v[w];
  float m = NEG_BIG, lsum = 0.f;      // column r16's running max; this lane's share of its weight sum
  f4 acc[8];                          // dims 16 j + 4 g + i of column r16
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = f4{0.f, 0.f, 0.f, 0.f};
  // the chunk's V rows into the wave's LDS rows (row = chunk token; the previous chunk's reads are issued before)
  auto stage = [&](const XChunk& C) {
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int s = 0; s < 4; ++s) *reinterpret_cast<u4v*>(&Vs[16 * u + r16][32 * s + 8 * g]) = C.v[u][s];
  };
  auto qk = [&](const XChunk& C, f4 (&sc)[2]) {
    asm volatile("" ::: "memory");   // keeps the q reads in the loop
    u4v qb[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) qb[s] = X.qb[w][s][lane];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      u4v a0, a2;   // rotated dims 8 g .. + 7 and 64 + 8 g .. + 7, bf16
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        float r0[2], r2[2];
#pragma unroll
        for (int d = 0; d < 2; ++d) {
#pragma clang fp contract(off)   // products rounded before the sum, as torch_decode.py:22-23 evaluates them
          const float k0 = bf_elem(C.k[u][0], e + d), k2 = bf_elem(C.k[u][2], e + d);
          const float cs = bf_elem(C.c[u], e + d), sn = bf_elem(C.s[u], e + d);
          r0[d] = k0 * cs - k2 * sn;
          r2[d] = k2 * cs + k0 * sn;
        }
        a0[e >> 1] = bfpk(r0[0], r0[1]);
        a2[e >> 1] = bfpk(r2[0], r2[1]);
        __builtin_amdgcn_sched_barrier(0);   // one channel pair's temporaries at a time
      }
      f4 x = {0.f, 0.f, 0.f, 0.f};
      x = mfma_bf(as_b8(a0), as_b8(qb[0]), x);
      x = mfma_bf(as_b8(C.k[u][1]), as_b8(qb[1]), x);
      x = mfma_bf(as_b8(a2), as_b8(qb[2]), x);
      x = mfma_bf(as_b8(C.k[u][3]), as_b8(qb[3]), x);
      sc[u] = x;
    }
  };
  auto pv = [&](const XChunk& C, const f4 (&sc)[2]) {
    const uint32_t tb = C.ok >> (4 * g);   // bit 16 u + i: token 16 u + 4 g + i
    float xs[2][4], cm = -INFINITY;
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        xs[u][i] = ((tb >> (16 * u + i)) & 1u) ? sc[u][i] * scale : -INFINITY;
        cm = fmaxf(cm, xs[u][i]);
      }
    cm = max4rows(cm);
    if (__ballot(cm > m + LAZY)) {
      const float mn = fmaxf(m, cm), al = __builtin_amdgcn_exp2f(m - mn);
      m = mn;
      lsum *= al;
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] *= al;
    }
    u4v bp;   // weights of the lane's 8 tokens in K order, column r16: hi (r16 < 4), lo (4 <= r16 < 8), 0 above
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int u = k >> 1, i = 2 * (k & 1);
      const float pa = __builtin_amdgcn_exp2f(xs[u][i] - m), pb = __builtin_amdgcn_exp2f(xs[u][i + 1] - m);
      lsum += pa + pb;
      const uint32_t hi = bfpk(pa, pb);
      const uint32_t lo = bfpk(pa - __uint_as_float(hi << 16), pb - __uint_as_float(hi & 0xFFFF0000u));
      bp[k] = (r16 < 4) ? hi : ((r16 < 8) ? lo : 0u);
    }
    asm volatile("" ::: "memory");   // the staged V rows are written before the transposed reads
    const int vrow = 4 * g + (r16 >> 2), vcol = 4 * (r16 & 3);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const s4 t0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)&Vs[vrow][16 * j + vcol]);
      const s4 t1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)&Vs[vrow + 16][16 * j + vcol]);
      const u4v av = {__builtin_bit_cast(uint32_t, __builtin_shufflevector(t0, t0, 0, 1)),
                      __builtin_bit_cast(uint32_t, __builtin_shufflevector(t0, t0, 2, 3)),
                      __builtin_bit_cast(uint32_t, __builtin_shufflevector(t1, t1, 0, 1)),
                      __builtin_bit_cast(uint32_t, __builtin_shufflevector(t1, t1, 2, 3))};
      acc[j] = mfma_bf(as_b8(av), as_b8(bp), acc[j]);
    }
    asm volatile("" ::: "memory");   // and read before the next chunk's rows overwrite them
  };
  constexpr int STEP = WPH * XCH;     // tokens between this wave's chunks
  if (ph * XCH < T) {
    XChunk A, Bc;
    f4 sc[2];
    load(ph * XCH, A);
    // two chunk buffers, each loaded one chunk ahead of its use; the loads are unconditional (past the row they
    // request nothing and give zeros), so neither buffer's old contents stay live across the loop
    for (int c0 = ph * XCH;;) {
      load(c0 + STEP, Bc);
      stage(A);
      qk(A, sc);
      pv(A, sc);
      c0 += STEP;
      if (c0 >= T) break;
      load(c0 + STEP, A);
      stage(Bc);
      qk(Bc, sc);
      pv(Bc, sc);
      c0 += STEP;
      if (c0 >= T) break;
    }
  }

  // ---- columns -> rows: row r = column r (hi) + column r + 4 (lo); lane owns dims 2 lane, 2 lane + 1 of each row
  lsum = sum4rows(lsum);
  float* Tc = reinterpret_cast<float*>(&Vs[0][0]);   // [8][XTROW] columns, then m and l of rows 0..3
  if (r16 < 8) {
#pragma unroll
    for (int j = 0; j < 8; ++j) *reinterpret_cast<f4*>(Tc + r16 * XTROW + 16 * j + 4 * g) = acc[j];
  }
  if (lane < 4) { Tc[8 * XTROW + lane] = m; Tc[8 * XTROW + 4 + lane] = lsum; }
  __builtin_amdgcn_wave_barrier();
  asm volatile("" ::: "memory");
  const int dd = 2 * lane;
  float mr[4], Lr[4], ar[4][2];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float2 hi2 = *reinterpret_cast<const float2*>(Tc + r * XTROW + dd);
    const float2 lo2 = *reinterpret_cast<const float2*>(Tc + (r + 4) * XTROW + dd);
    ar[r][0] = hi2.x + lo2.x;
    ar[r][1] = hi2.y + lo2.y;
    mr[r] = Tc[8 * XTROW + r];
    Lr[r] = Tc[8 * XTROW + 4 + r];
  }
  // (m, l, o0, o1) of query row 4 h + r of this row b -> its partial slot, or merged with the quantized partials
  auto emit = [&](int r, float M, float L, float o0, float o1) {
    if constexpr (!MERGE) {
      const int64_t row = xslot * 16 + h * 4 + r;
      if (lane == 0) { mo[row] = M; lo_out[row] = L; }
      *reinterpret_cast<float2*>(ao + row * 128 + dd) = make_float2(o0, o1);
    } else {
      const int64_t rq = (int64_t)b * (ns + 1) * 16 + h * 4 + r;   // row of split 0; split s adds 16 s
      // splits are visited 8 at a time with all of their loads issued together
      float Mq = M;
      for (int s0 = 0; s0 < ns; s0 += 8) {
        float mv[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) mv[k] = (s0 + k < ns) ? mo[rq + 16 * (s0 + k)] : NEG_BIG;
#pragma unroll
        for (int k = 0; k < 8; ++k) Mq = fmaxf(Mq, mv[k]);
      }
      const float we = exp2f(M - Mq);
      float Lt = L * we, x0 = 0.f, x1 = 0.f;
      for (int s0 = 0; s0 < ns; s0 += 8) {
        float mv[8], lv[8];
        float2 av[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const bool in = s0 + k < ns;
          const int64_t row = rq + 16 * (in ? s0 + k : 0);
          mv[k] = in ? mo[row] : NEG_BIG;
          lv[k] = lo_out[row];
          av[k] = *reinterpret_cast<const float2*>(ao + row * 128 + dd);
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const float wq = exp2f(mv[k] - Mq);   // 0 for the padding entries
          Lt += wq * lv[k];
          x0 += wq * av[k].x;
          x1 += wq * av[k].y;
        }
      }
      // y = H x over the 128 dims: bit 0 of the dim in-lane, bits 1..6 across the wave's lanes
      {
        const float a = x0, c = x1;
        x0 = a + c;
        x1 = a - c;
      }
#pragma unroll
      for (int k = 0; k < 6; ++k) {
        const int msk = 1 << k;
        const float p0 = __shfl_xor(x0, msk), p1 = __shfl_xor(x1, msk);
        x0 = (lane & msk) ? p0 - x0 : x0 + p0;
        x1 = (lane & msk) ? p1 - x1 : x1 + p1;
      }
      const float hn = __uint_as_float(0x3DB504F3u);
      float y0 = (ns > 0 ? x0 * hn : 0.f) + o0 * we;
      float y1 = (ns > 0 ? x1 * hn : 0.f) + o1 * we;
      y0 = Lt > 0.f ? y0 / Lt : 0.f;
      y1 = Lt > 0.f ? y1 / Lt : 0.f;
      *reinterpret_cast<uint32_t*>(out + ((int64_t)b * 16 + h * 4 + r) * 128 + dd) = f2bf(y0) | (f2bf(y1) << 16);
    }
  };
  if constexpr (NH == 4) {
#pragma unroll
    for (int r = 0; r < 4; ++r) emit(r, mr[r], Lr[r], ar[r][0], ar[r][1]);
  } else {   // the 4 waves' states of each row, merged by wave r for row r
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if (lane == 0) { X.fm[w][r] = mr[r]; X.fl[w][r] = Lr[r]; }
      *reinterpret_cast<float2*>(&X.facc[w][r][dd]) = make_float2(ar[r][0], ar[r][1]);
    }
    __syncthreads();
    const int r = w;
    float M = NEG_BIG;
#pragma unroll
    for (int ww = 0; ww < 4; ++ww) M = fmaxf(M, X.fm[ww][r]);
    float L = 0.f, o0 = 0.f, o1 = 0.f;
#pragma unroll
    for (int ww = 0; ww < 4; ++ww) {
      const float sc = exp2f(X.fm[ww][r] - M);
      const float2 a = *reinterpret_cast<const float2*>(&X.facc[ww][r][dd]);
      L += sc * X.fl[ww][r];
      o0 += sc * a.x;
      o1 += sc * a.y;
    }
    emit(r, M, L, o0, o1);
  }
}

// KV heads per workgroup of the fused exact kernel (window layers) and of the exact-tail workgroups of the quantized
// grid, which must finish early to free their CUs for the split work. The standalone partial-writing variant uses the
// tails' split, so its partials are bit-identical to the ones the quantized grid computes in-grid.
constexpr int XNH = 4, XNH_TAIL = 1;
template <bool MERGE> constexpr int exact_nh() { return MERGE ? XNH : XNH_TAIL; }

template <bool MERGE>
__global__ void __launch_bounds__(256)
decode_exact_kernel(kv800_paged_t P, const uint16_t* __restrict__ q, const uint16_t* __restrict__ cos_t,
                    const uint16_t* __restrict__ sin_t, int64_t rope_rows, int64_t epool_elems, int64_t sink_elems,
                    float* __restrict__ mo, float* __restrict__ lo_out, float* __restrict__ ao, int ns, float scale,
                    int nsink, uint16_t* __restrict__ out) {
  __shared__ XLds X;
  constexpr int NH = exact_nh<MERGE>(), G = 4 / NH;   // KV heads per workgroup, workgroups per row
  const int b = blockIdx.x / G;
  exact_row<NH, MERGE>(X, b, (blockIdx.x % G) * NH, P, q, cos_t, sin_t, rope_rows, epool_elems, sink_elems, mo,
                        lo_out, ao, ns, (int64_t)b * (ns + 1) + ns, scale, nsink, out);
}

// ---------------------------------------------------------------- quantized sub-blocks
constexpr int QWAVES = 4;
constexpr int64_t BAL_CHUNK = 16, BAL_GROUPS = 1536;   // balanced schedule: sub-blocks per workgroup, most workgroups
// LDS row strides are padded (132 floats, 272 floats, 9 x 16 bytes) so that the 16 lanes of a lane group, which read
// 16 different rows at the same column, fall into distinct banks; the vb chunk is XOR-swizzled instead (below).
constexpr int QROW = 132, HROW = 132, VROW = 272, CSP = 9;
struct QWaveLds {
  float vs[2][VROW];          // decoded vsc per (head group, token)
  float vl[2][VROW];          // decoded vlo
  u4v vb[2][32 * 4];          // vb bytes of a 32-token chunk (double buffer), 16-byte pieces placed by vb_at
  u4v cs[2][32 * CSP];         // fp16 (cos, sin) rows of the chunk's 32 positions (double buffer), placed by cs_at
};
struct QLds {
  float q[16][QROW];
  QWaveLds wv[QWAVES];
};
// Per-sub-block scale staging, scale * ksc and klo as [head][channel] floats, lives in the wave's second
// rope buffer: it is read only while the weights are built, before chunk 1 (the first user of that buffer) is stored,
// and a wave's LDS instructions execute in order. This keeps a workgroup under 80 KB (two per CU).
constexpr int SCALE_FLOATS = 8 * HROW;
static_assert(SCALE_FLOATS * 4 <= (int)sizeof(u4v) * 32 * CSP, "scale staging must fit one rope buffer");
struct QFinLds {              // end-of-split merge of the 4 waves (reuses the LDS)
  float m[QWAVES][16], l[QWAVES][16], lv[QWAVES][16];
  float acc[QWAVES][16][QROW];
};
// 16-byte slot of (token t of the chunk, piece k = head) in a vb chunk buffer: piece k of token t is stored at slot
// k ^ ((t >> 2) & 3) of the token's 4, so the four lane groups (tokens 4 g + ...) read four different banks
__device__ __forceinline__ int vb_at(int t, int k) { return 4 * t + (k ^ ((t >> 2) & 3)); }
// 16-byte slot of piece p (dwords 4 p .. 4 p + 3) of rope row r in a chunk buffer: rows are padded to 9 slots and the
// pieces of rows with (r / 4) odd are swapped in pairs, so the 16 (row, piece) pairs a rope / nope read touches
// (4 tokens x 4 lane groups) cover all 16 bank quads
__device__ __forceinline__ int cs_at(int r, int p) { return r * CSP + (p ^ ((r >> 2) & 1)); }

// rope + nope features of one kc dword x (channels e = 0..3 of the lane's 8, one byte each holding the codes
// c0 | c1 << 2 | c2 << 4 | c3 << 6 of dims j, j + 32, j + 64, j + 96; cos / sin of channel e in cs4) against weight
// blocks w0 (channels 0, 1), w1 (channels 2, 3) and wn (nope, channels 0..3). A byte masked to bits 0-1 | 4-5 is two
// e2m1 nibbles whose values are c0 / 2 and c2 / 2; v_cvt_scalef32_pk_f16_fp4 with scale 2 turns it into the exact
// fp16 pair (c0, c2) in one instruction (its scale applies the exponent only), and bits 2-3 | 6-7 shifted down give
// (c1, c3) the same way.
template <int E>
__device__ __forceinline__ h2 codes2(uint32_t m) { return __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(m, 2.0f, E); }

__device__ __forceinline__ f4 rope_nope(uint32_t x, u4v cs4, h8 w0, h8 w1, h8 wn, f4 a) {
  const uint32_t m02 = x & 0x33333333u, m13 = (x >> 2) & 0x33333333u;
  const h2 F[4] = {codes2<0>(m02), codes2<1>(m02), codes2<2>(m02), codes2<3>(m02)};   // (c0, c2) of channel e
  const uint32_t f13[4] = {hbits(codes2<0>(m13)), hbits(codes2<1>(m13)), hbits(codes2<2>(m13)),
                           hbits(codes2<3>(m13))};                                  // (c1, c3) of channel e
  const uint32_t csv[4] = {cs4.x, cs4.y, cs4.z, cs4.w};
  uint32_t ga[4], gb[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const h2 CS = as_h2(csv[e]);
    ga[e] = hbits(CS * h2{F[e].x, F[e].x});   // (cos c0, sin c0)
    gb[e] = hbits(CS * h2{F[e].y, F[e].y});   // (cos c2, sin c2)
  }
  a = mfma16(pack8(ga[0], gb[0], ga[1], gb[1]), w0, a);
  a = mfma16(pack8(ga[2], gb[2], ga[3], gb[3]), w1, a);
  return mfma16(pack8(f13[0], f13[1], f13[2], f13[3]), wn, a);
}
static_assert(sizeof(QFinLds) <= sizeof(QLds), "fin scratch must fit");

// Exact-tail work carried by the quantized-split grid: workgroups [0, nexact) each run the exact tail of one row's
// KV head(s) (its exact partial slot, as decode_exact_kernel<false>) before the split workgroups, so their memory
// latency overlaps the splits' VALU work on the same CUs instead of following it.
struct ExactArgs {
  kv800_paged_t P;
  const uint16_t* cos_t;
  const uint16_t* sin_t;
  int64_t rope_rows, epool_elems, sink_elems;
  int64_t xs0, xst;   // exact partial of row b in slot xs0 + b xst
  int nexact, nsink;
};

// Balanced schedule (groups > 0): the B rows' sub-blocks in quads of 4 (one per wave; a row's last quad may be
// partial), q_b quads in row b, T = sum q_b. With C = ceil(T / groups), row b is cut into n_b = ceil(q_b / C) slices of
// at most C quads, and the slices of all rows are laid end to end: row b's at workgroup indices [pre[b], pre[b + 1]).
// Workgroup g takes one slice and writes its partial to slot g; sum n_b <= T / C + B <= groups + B, so the grid has
// groups + B workgroups and the ones past the last slice return at once. The exact partial of row b is slot
// groups + B + b. groups = 0: the fixed (row, split) grid, split s of row b in slot b (ns + 1) + s, the exact partial
// in slot b (ns + 1) + ns (the reference's partial layout).
struct Sched {
  int32_t* pre;         // pre[0 .. B]: written by workgroup 0 of the decode grid, read by the merge
  int groups, B, cap;   // cap: sub-blocks per row are clamped to [0, cap]
};

// The decode grid's workgroups each scan NQ themselves: thread t owns rows [t k, t k + k), k = ceil(B / 256), reads
// their counts once (into registers, up to RREG rows, i.e. B <= 1024; later rows are read again) and takes part in
// two block-wide scans, of the quads (for T) and of the slices.
constexpr int RREG = 4;
struct RowTab {
  int wsum[4];
  int b, pb, nsb;       // the row of this workgroup's slice, its first slice index, its clamped sub-block count
};
struct RowCache {       // this thread's rows [r0, r1) and their clamped sub-block counts
  int r0, r1;
  int v[RREG];
};
__device__ __forceinline__ void load_rows(const int32_t* __restrict__ nq, const Sched& S, RowCache& C) {
  const int k = (S.B + 255) >> 8;
  C.r0 = min((int)threadIdx.x * k, S.B);
  C.r1 = min(C.r0 + k, S.B);
#pragma unroll
  for (int i = 0; i < RREG; ++i) C.v[i] = (C.r0 + i < C.r1) ? min(max(nq[C.r0 + i], 0), S.cap) : 0;
}
__device__ __forceinline__ int nsb_of(const int32_t* __restrict__ nq, const Sched& S, const RowCache& C, int i) {
  int x = 0;
#pragma unroll
  for (int k = 0; k < RREG; ++k)
    if (k == i) x = C.v[k];
  return i < RREG ? x : min(max(nq[C.r0 + i], 0), S.cap);
}
__device__ __forceinline__ int quads_of(int nsb) { return (nsb + QWAVES - 1) / QWAVES; }
__device__ __forceinline__ int slices_of(int quads, int C) { return (quads + C - 1) / C; }
// Exclusive prefix of v over the workgroup's threads (in thread order); *total = the sum over all threads.
__device__ __forceinline__ int block_scan(int v, RowTab& R, int* total) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  int x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int t = __shfl_up(x, o);
    if (lane >= o) x += t;
  }
  __syncthreads();   // earlier readers of R.wsum are done
  if (lane == 63) R.wsum[w] = x;
  __syncthreads();
  int add = 0;
  for (int ww = 0; ww < w; ++ww) add += R.wsum[ww];
  *total = R.wsum[0] + R.wsum[1] + R.wsum[2] + R.wsum[3];
  return add + x - v;
}
static_assert(sizeof(XLds) <= sizeof(QLds), "exact-tail scratch must fit the split workgroup's LDS");

// Attention of row b's 16 query rows over its sub-blocks [j0, j1): wave w takes j0 + w, then every 4th.
// The workgroup's partial (m, l, acc in the Hadamard domain) goes to partial rows prow .. prow + 15.
__device__ __forceinline__ void quant_span(char* lds_raw, const uint16_t* __restrict__ q,
                                           const uint8_t* __restrict__ qpool, int64_t qpool_bytes,
                                           const int64_t* __restrict__ boff, int64_t bstride,
                                           const uint32_t* __restrict__ cs16, int64_t rope_rows, float* __restrict__ mo,
                                           float* __restrict__ lo_out, float* __restrict__ ao, float scale, const int b,
                                           const int j0, const int j1, const int64_t prow) {
  QLds& L = *reinterpret_cast<QLds*>(lds_raw);
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, n = lane & 15, hn = n >> 2;
  QWaveLds& W = L.wv[w];
  float* const s4w = reinterpret_cast<float*>(W.cs[1]);   // scale staging (see SCALE_FLOATS)
  float* const tpw = s4w + 4 * HROW;
  // kc bytes a lane reads for token group tg of a 16-token tile: token 4 (n / 4) + tg, head n % 4, channels 8 g .. + 7
  const int kofs = (n >> 2) * 512 + (n & 3) * 32 + 8 * g;

  for (int i = tid; i < 16 * 128; i += 256) L.q[i >> 7][i & 127] = bf2f(q[(int64_t)b * 2048 + i]);   // padded rows
  __syncthreads();

  float m = NEG_BIG, lsum = 0.f, lvs = 0.f;
  f4 acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = f4{0.f, 0.f, 0.f, 0.f};

  for (int jb = j0 + w; jb < j1; jb += QWAVES) {
    const int64_t base = boff[(int64_t)b * bstride + jb];
    if (base < 0 || base + SUB > qpool_bytes || (int64_t)(jb + 1) * BLK > rope_rows) continue;   // guard
    const uint8_t* sb = qpool + base;
    const uint32_t* csb = cs16 + (int64_t)jb * BLK * 32;

    // ---- stage per-sub-block scales as floats: S = scale ksc, T = klo per (head, channel); vlo / vsc
    {
      const uint2 lo2 = *reinterpret_cast<const uint2*>(sb + KLO_O + 8 * lane);   // channels 8 lane .. 8 lane + 7
      const uint2 sc2 = *reinterpret_cast<const uint2*>(sb + KSC_O + 8 * lane);
      float ksc[8], klo[8];
      f8x4(sc2.x, ksc); f8x4(sc2.y, ksc + 4);
      f8x4(lo2.x, klo); f8x4(lo2.y, klo + 4);
      const int ho = (lane >> 4) * HROW + 8 * (lane & 15);   // head lane / 16, channels 8 (lane % 16) ..
      // k = klo + ksc * code: the weights act on the integer code features
      *reinterpret_cast<float4*>(s4w + ho) = make_float4(scale * ksc[0], scale * ksc[1], scale * ksc[2], scale * ksc[3]);
      *reinterpret_cast<float4*>(s4w + ho + 4) = make_float4(scale * ksc[4], scale * ksc[5], scale * ksc[6], scale * ksc[7]);
      *reinterpret_cast<float4*>(tpw + ho) = make_float4(klo[0], klo[1], klo[2], klo[3]);
      *reinterpret_cast<float4*>(tpw + ho + 4) = make_float4(klo[4], klo[5], klo[6], klo[7]);
    }
    {
      const uint2 vl2 = *reinterpret_cast<const uint2*>(sb + VLO_O + 8 * lane);   // bytes 8 lane .. 8 lane + 7
      const uint2 vs2 = *reinterpret_cast<const uint2*>(sb + VSC_O + 8 * lane);
      // byte 8 lane + e -> token 4 lane + e / 2, head group e & 1
      float vl[8], vs[8];
      f8x4(vl2.x, vl); f8x4(vl2.y, vl + 4);
      f8x4(vs2.x, vs); f8x4(vs2.y, vs + 4);
      *reinterpret_cast<float4*>(&W.vl[0][4 * lane]) = make_float4(vl[0], vl[2], vl[4], vl[6]);
      *reinterpret_cast<float4*>(&W.vl[1][4 * lane]) = make_float4(vl[1], vl[3], vl[5], vl[7]);
      *reinterpret_cast<float4*>(&W.vs[0][4 * lane]) = make_float4(vs[0], vs[2], vs[4], vs[6]);
      *reinterpret_cast<float4*>(&W.vs[1][4 * lane]) = make_float4(vs[1], vs[3], vs[5], vs[7]);
    }
    // ---- prefetch chunk 0 (vb bytes, rope rows, kc rows of tiles 0 / 1)
    u4v vbn0 = *reinterpret_cast<const u4v*>(sb + VB_O + 32 * lane);
    u4v vbn1 = *reinterpret_cast<const u4v*>(sb + VB_O + 32 * lane + 16);
    u4v csn[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) csn[u] = *reinterpret_cast<const u4v*>(csb + 256 * u + 4 * lane);
    const uint8_t* kcb = sb + KC_O + kofs;
    uint2 kn[2][4];
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int tg = 0; tg < 4; ++tg) kn[u][tg] = *reinterpret_cast<const uint2*>(kcb + (16 * u + tg) * 128);
    __builtin_amdgcn_wave_barrier();

    // ---- weights of this sub-block (B operands), scaled by `scale` so the accumulator is in log2 units.
    // Rope / nope MFMAs: lane (g, n) holds the weights of query row n (head hn's scales) for channels 8 g .. 8 g + 7:
    // block r < 4 = channels 8 g + 2 r, + 1 (4 rope features each), nope block p = channels 8 g + 4 p .. + 3.
    const float* qn = L.q[n];
    const float* sh = s4w + hn * HROW;
    const float* tpn = tpw + hn * HROW;
    h8 wr[4], wnp[2], wt[2];
    {
      float q0[8], q1[8], q2[8], q3[8], s0[8], s1[8], s2[8], s3[8];
      auto ld8 = [](const float* p, float* o) {
        const float4 x = *reinterpret_cast<const float4*>(p), y = *reinterpret_cast<const float4*>(p + 4);
        o[0] = x.x; o[1] = x.y; o[2] = x.z; o[3] = x.w; o[4] = y.x; o[5] = y.y; o[6] = y.z; o[7] = y.w;
      };
      ld8(qn + 8 * g, q0); ld8(qn + 32 + 8 * g, q1); ld8(qn + 64 + 8 * g, q2); ld8(qn + 96 + 8 * g, q3);
      ld8(sh + 8 * g, s0); ld8(sh + 32 + 8 * g, s1); ld8(sh + 64 + 8 * g, s2); ld8(sh + 96 + 8 * g, s3);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int e0 = 2 * r, e1 = 2 * r + 1;
        wr[r] = pack8(pk2(q0[e0] * s0[e0], q2[e0] * s0[e0]), pk2(q2[e0] * s2[e0], -q0[e0] * s2[e0]),
                      pk2(q0[e1] * s0[e1], q2[e1] * s0[e1]), pk2(q2[e1] * s2[e1], -q0[e1] * s2[e1]));
      }
#pragma unroll
      for (int pq = 0; pq < 2; ++pq) {
        const int e = 4 * pq;
        wnp[pq] = pack8(pk2(q1[e] * s1[e], q3[e] * s3[e]), pk2(q1[e + 1] * s1[e + 1], q3[e + 1] * s3[e + 1]),
                        pk2(q1[e + 2] * s1[e + 2], q3[e + 2] * s3[e + 2]), pk2(q1[e + 3] * s1[e + 3], q3[e + 3] * s3[e + 3]));
      }
    }
    // table part (all 16 rows, dense): lane (g, n) channels 16 kk + 4 g .. + 3, features (cos, sin)
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const int jc = 16 * kk + 4 * g;
      const float4 q0 = *reinterpret_cast<const float4*>(qn + jc), q2 = *reinterpret_cast<const float4*>(qn + 64 + jc);
      const float4 T0 = *reinterpret_cast<const float4*>(tpn + jc), T2 = *reinterpret_cast<const float4*>(tpn + 64 + jc);
      const float a0[4] = {q0.x, q0.y, q0.z, q0.w}, a2[4] = {q2.x, q2.y, q2.z, q2.w};
      const float t0[4] = {T0.x, T0.y, T0.z, T0.w}, t2[4] = {T2.x, T2.y, T2.z, T2.w};
      uint32_t ht[4];
#pragma unroll
      for (int u = 0; u < 4; ++u)
        ht[u] = pk2(scale * (a0[u] * t0[u] + a2[u] * t2[u]), scale * (a2[u] * t0[u] - a0[u] * t2[u]));
      wt[kk] = pack8(ht[0], ht[1], ht[2], ht[3]);
    }
    float c13 = 0.f;
    {
      const float4 q1a = *reinterpret_cast<const float4*>(qn + 32 + 8 * g), q1b = *reinterpret_cast<const float4*>(qn + 36 + 8 * g);
      const float4 q3a = *reinterpret_cast<const float4*>(qn + 96 + 8 * g), q3b = *reinterpret_cast<const float4*>(qn + 100 + 8 * g);
      const float4 t1a = *reinterpret_cast<const float4*>(tpn + 32 + 8 * g), t1b = *reinterpret_cast<const float4*>(tpn + 36 + 8 * g);
      const float4 t3a = *reinterpret_cast<const float4*>(tpn + 96 + 8 * g), t3b = *reinterpret_cast<const float4*>(tpn + 100 + 8 * g);
      c13 = q1a.x * t1a.x + q1a.y * t1a.y + q1a.z * t1a.z + q1a.w * t1a.w + q1b.x * t1b.x + q1b.y * t1b.y + q1b.z * t1b.z +
            q1b.w * t1b.w + q3a.x * t3a.x + q3a.y * t3a.y + q3a.z * t3a.z + q3a.w * t3a.w + q3b.x * t3b.x +
            q3b.y * t3b.y + q3b.z * t3b.z + q3b.w * t3b.w;
    }
    c13 = sum4rows(c13) * scale;
    asm volatile("" ::: "memory");   // the scale staging reads above stay before the chunk stores below

    // ---- 8 chunks of 32 tokens (2 QK tiles + 1 PV step)
#pragma unroll 2
    for (int c = 0; c < 8; ++c) {
      const int cb = c & 1;   // constant in each of the two unrolled copies
      // lane holds token lane / 2, pieces 2 (lane % 2) and 2 (lane % 2) + 1; rope dwords 256 u + 4 lane
      W.vb[cb][vb_at(lane >> 1, 2 * (lane & 1))] = vbn0;
      W.vb[cb][vb_at(lane >> 1, 2 * (lane & 1) + 1)] = vbn1;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int r = 8 * u + (lane >> 3);
        W.cs[cb][cs_at(r, lane & 7)] = csn[u];
      }
      uint2 kc[2][4];
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int tg = 0; tg < 4; ++tg) kc[u][tg] = kn[u][tg];
      if (c + 1 < 8) {   // prefetch the next chunk
        const uint8_t* vbp = sb + VB_O + (c + 1) * 32 * 64 + 32 * lane;
        vbn0 = *reinterpret_cast<const u4v*>(vbp);
        vbn1 = *reinterpret_cast<const u4v*>(vbp + 16);
        const uint32_t* csp = csb + (c + 1) * 32 * 32;
#pragma unroll
        for (int u = 0; u < 4; ++u) csn[u] = *reinterpret_cast<const u4v*>(csp + 256 * u + 4 * lane);
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
          for (int tg = 0; tg < 4; ++tg)
            kn[u][tg] = *reinterpret_cast<const uint2*>(kcb + (32 * (c + 1) + 16 * u + tg) * 128);
      }
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");

      // Wave priority by phase: the QK features (LDS reads feeding VALU feeding MFMA) go first, the softmax next, PV
      // last, so that of the SIMD's two waves the one still in QK wins the issue slots over one already in PV, whose
      // MFMA chain then overlaps it; measured 3-4 % faster than equal priority.
      __builtin_amdgcn_s_setprio(2);
      f4 sacc2[2];   // lane (g, n) register i: score of token 32 c + 16 u + 4 g + i, query row n
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        // table part: A row n = token 16 u + n
        const int trow = 16 * u + n;
        f4 tacc = {c13, c13, c13, c13};
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          const u4v t4 = W.cs[cb][cs_at(trow, 4 * kk + g)];
          tacc = mfma16(__builtin_bit_cast(h8, t4), wt[kk], tacc);
        }
        // rope / nope part, 4 token groups: A row n = (token 16 u + 4 (n / 4) + tg, head n % 4); the result for query
        // row n sits in output register n / 4 (the output rows of other heads are discarded)
#pragma unroll
        for (int tg = 0; tg < 4; ++tg) {
          const int tok = 16 * u + 4 * (n >> 2) + tg;
          const u4v cA = W.cs[cb][cs_at(tok, 2 * g)];
          const u4v cB = W.cs[cb][cs_at(tok, 2 * g + 1)];
          f4 a = {0.f, 0.f, 0.f, 0.f};
          a = rope_nope(kc[u][tg].x, cA, wr[0], wr[1], wnp[0], a);
          a = rope_nope(kc[u][tg].y, cB, wr[2], wr[3], wnp[1], a);
          const float lo = (hn & 1) ? a[1] : a[0], hi = (hn & 1) ? a[3] : a[2];
          sacc2[u][tg] = tacc[tg] + ((hn & 2) ? hi : lo);
        }
      }
      __builtin_amdgcn_s_setprio(1);
      // ---- online softmax over the chunk's 32 tokens (lazy max); row = column n, tokens 4 g + i of each tile
      float tmax = fmaxf(fmaxf(fmaxf(sacc2[0][0], sacc2[0][1]), fmaxf(sacc2[0][2], sacc2[0][3])),
                         fmaxf(fmaxf(sacc2[1][0], sacc2[1][1]), fmaxf(sacc2[1][2], sacc2[1][3])));
      tmax = max4rows(tmax);
      if (__any(tmax > m + LAZY)) {
        const float mn = fmaxf(m, tmax);
        const float al = __builtin_amdgcn_exp2f(m - mn);   // v_exp_f32; tiny results flush to 0
        m = mn; lsum *= al; lvs *= al;
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] *= al;
      }
      uint32_t bpv[4];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const f4 sacc = sacc2[u];
        const int t0 = 32 * c + 16 * u + 4 * g;
        const float4 vs4 = *reinterpret_cast<const float4*>(&W.vs[n >> 3][t0]);
        const float4 vl4 = *reinterpret_cast<const float4*>(&W.vl[n >> 3][t0]);
        const float p0 = __builtin_amdgcn_exp2f(sacc[0] - m), p1 = __builtin_amdgcn_exp2f(sacc[1] - m);
        const float p2 = __builtin_amdgcn_exp2f(sacc[2] - m), p3 = __builtin_amdgcn_exp2f(sacc[3] - m);
        lsum += (p0 + p1) + (p2 + p3);
        lvs += (p0 * vl4.x + p1 * vl4.y) + (p2 * vl4.z + p3 * vl4.w);
        const h2 w01 = {(_Float16)(p0 * vs4.x), (_Float16)(p1 * vs4.y)};
        const h2 w23 = {(_Float16)(p2 * vs4.z), (_Float16)(p3 * vs4.w)};
        bpv[2 * u] = hbits(w01);
        bpv[2 * u + 1] = hbits(w23);
      }
      __builtin_amdgcn_s_setprio(0);
      // ---- PV: per head hh, plane i. Lane (g, jj = n): bytes jj of tokens 32 c + {4 g + (0..3), 16 + 4 g + (0..3)}
      const uint8_t* vbc = reinterpret_cast<const uint8_t*>(W.vb[cb]);
#pragma unroll
      for (int hh = 0; hh < 4; ++hh) {
        const bool mine = (hn == hh);
        const h8 B = mine ? pack8(bpv[0], bpv[1], bpv[2], bpv[3]) : pack8(0u, 0u, 0u, 0u);
        uint32_t D[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int ta = 16 * (v >> 1) + 4 * g + 2 * (v & 1);
          D[v] = (uint32_t)vbc[16 * vb_at(ta, hh) + n] | ((uint32_t)vbc[16 * vb_at(ta + 1, hh) + n] << 16);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const uint32_t msk = (1u << i) | (1u << (16 + i));
          const h8 A = pack8(D[0] & msk, D[1] & msk, D[2] & msk, D[3] & msk);
          acc[i] = mfma16(A, B, acc[i]);
        }
      }
    }
  }

  // ---- combine the 4 waves of the split
  lsum = sum4rows(lsum);
  lvs = sum4rows(lvs);
  __syncthreads();
  QFinLds& F = *reinterpret_cast<QFinLds*>(lds_raw);
  if (g == 0) { F.m[w][n] = m; F.l[w][n] = lsum; F.lv[w][n] = lvs; }
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) F.acc[w][n][16 * i + 4 * g + r] = acc[i][r];
  __syncthreads();
  // thread -> (row rr = tid / 16, dims 8 (tid % 16) .. + 7)
  const int rr = tid >> 4, d0 = 8 * (tid & 15);
  float M = NEG_BIG;
#pragma unroll
  for (int ww = 0; ww < QWAVES; ++ww) M = fmaxf(M, F.m[ww][rr]);
  float Ls = 0.f, LV = 0.f, o[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
  for (int ww = 0; ww < QWAVES; ++ww) {
    const float sc = exp2f(F.m[ww][rr] - M);
    Ls += sc * F.l[ww][rr]; LV += sc * F.lv[ww][rr];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] += sc * F.acc[ww][rr][d0 + e];
  }
  const int64_t row = prow + rr;
  if ((tid & 15) == 0) { mo[row] = M; lo_out[row] = Ls; }
  const float pscale = __uint_as_float((uint32_t)(127 + 24 - (d0 >> 4)) << 23);   // 2^(24 - i), plane i = d / 16
  float4 r0, r1;
  r0.x = o[0] * pscale + LV; r0.y = o[1] * pscale + LV; r0.z = o[2] * pscale + LV; r0.w = o[3] * pscale + LV;
  r1.x = o[4] * pscale + LV; r1.y = o[5] * pscale + LV; r1.z = o[6] * pscale + LV; r1.w = o[7] * pscale + LV;
  *reinterpret_cast<float4*>(ao + row * 128 + d0) = r0;
  *reinterpret_cast<float4*>(ao + row * 128 + d0 + 4) = r1;
}

__global__ void __launch_bounds__(256, 2)
decode_quant_kernel(const uint16_t* __restrict__ q, const uint8_t* __restrict__ qpool, int64_t qpool_bytes,
                    const int64_t* __restrict__ boff, int64_t bstride, const int32_t* __restrict__ nq,
                    const uint32_t* __restrict__ cs16, int64_t rope_rows, float* __restrict__ mo,
                    float* __restrict__ lo_out, float* __restrict__ ao, int ns, int spb, float scale, ExactArgs X,
                    Sched S) {
  __shared__ __align__(16) char lds_raw[sizeof(QLds)];
  if ((int)blockIdx.x < X.nexact) {
    constexpr int G = 4 / XNH_TAIL;   // workgroups per row
    const int b = (int)blockIdx.x / G;
    exact_row<XNH_TAIL, false>(*reinterpret_cast<XLds*>(lds_raw), b, ((int)blockIdx.x % G) * XNH_TAIL, X.P, q, X.cos_t,
                               X.sin_t, X.rope_rows, X.epool_elems, X.sink_elems, mo, lo_out, ao, ns,
                               X.xs0 + b * X.xst, scale, X.nsink, nullptr);
    return;
  }
  const int blk = (int)blockIdx.x - X.nexact;
  // fixed grid: (row b, split s); balanced: slice blk (one row's quads [c0, c1))
  int b, j0, j1;
  int64_t prow;
  if (S.groups == 0) {
    b = blk / ns;
    const int s = blk % ns;
    j0 = s * spb;
    j1 = min(min((s + 1) * spb, nq[b]), (int)min(bstride, (int64_t)INT32_MAX));
    prow = ((int64_t)b * (ns + 1) + s) * 16;
  } else {
    __shared__ RowTab R;
    RowCache RC;
    load_rows(nq, S, RC);
    int qsum = 0;
    for (int i = 0; i < RC.r1 - RC.r0; ++i) qsum += quads_of(nsb_of(nq, S, RC, i));
    int T;
    block_scan(qsum, R, &T);
    if (T <= 0) {   // no quantized work in any row
      if (blk == 0)
        for (int r = threadIdx.x; r <= S.B; r += 256) S.pre[r] = 0;
      return;
    }
    const int C = (T + S.groups - 1) / S.groups;
    int nsl = 0;
    for (int i = 0; i < RC.r1 - RC.r0; ++i) nsl += slices_of(quads_of(nsb_of(nq, S, RC, i)), C);
    int G2;
    int p = block_scan(nsl, R, &G2);
    if (blk == 0) {   // pre[0 .. B] for the merge
      if (threadIdx.x == 0) S.pre[0] = 0;
      int pp = p;
      for (int i = 0; i < RC.r1 - RC.r0; ++i) {
        pp += slices_of(quads_of(nsb_of(nq, S, RC, i)), C);
        S.pre[RC.r0 + i + 1] = pp;
      }
    }
    if (blk >= G2) return;   // past the last slice (uniform over the workgroup)
    for (int i = 0; i < RC.r1 - RC.r0; ++i) {   // exactly one thread owns the row of slice blk
      const int nb = nsb_of(nq, S, RC, i), n = slices_of(quads_of(nb), C);
      if (p <= blk && blk < p + n) { R.b = RC.r0 + i; R.pb = p; R.nsb = nb; }
      p += n;
    }
    __syncthreads();
    b = __builtin_amdgcn_readfirstlane(R.b);
    const int k = blk - __builtin_amdgcn_readfirstlane(R.pb), nb = __builtin_amdgcn_readfirstlane(R.nsb);
    j0 = QWAVES * C * k;
    j1 = min(QWAVES * C * (k + 1), nb);
    prow = (int64_t)blk * 16;
  }
  quant_span(lds_raw, q, qpool, qpool_bytes, boff, bstride, cs16, rope_rows, mo, lo_out, ao, scale, b, j0, j1, prow);
}


// ---------------------------------------------------------------- split merge
__global__ void __launch_bounds__(256)
decode_merge_kernel(const float* __restrict__ mo, const float* __restrict__ lo, const float* __restrict__ ao, int ns,
                    Sched S, uint16_t* __restrict__ out) {
  const int b = blockIdx.x, tid = threadIdx.x, r = tid >> 4, l16 = tid & 15;
  // row b's quantized partials: slots first .. first + ns - 1; its exact partial: slot xs
  int64_t first = (int64_t)b * (ns + 1), xs = first + ns;
  if (S.groups > 0) {   // row b's slices are workgroups [pre[b], pre[b + 1]), one partial each
    first = S.pre[b];
    ns = S.pre[b + 1] - S.pre[b];
    xs = (int64_t)S.groups + S.B + b;
  }
  const int64_t r0 = first * 16 + r;   // row of the first quantized partial; the next adds 16
  // one pass with a running max: each batch of 4 partials (m, l, acc) is requested together, the exact partial with
  // the first batch, so the row waits on one memory round trip per batch
  const int64_t xrow = xs * 16 + r;
  float M = mo[xrow];
  const float xl = lo[xrow];
  const float4 xa0 = *reinterpret_cast<const float4*>(ao + xrow * 128 + 8 * l16);
  const float4 xa1 = *reinterpret_cast<const float4*>(ao + xrow * 128 + 8 * l16 + 4);
  const float Mx = M;
  float Ls = 0.f, xq[8] = {0, 0, 0, 0, 0, 0, 0, 0}, xe[8];
  for (int s0 = 0; s0 < ns; s0 += 4) {   // quantized splits
    float mv[4], lv[4];
    float4 a0[4], a1[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const bool in = s0 + k < ns;
      const int64_t row = r0 + 16 * (in ? s0 + k : 0);
      mv[k] = in ? mo[row] : NEG_BIG;
      lv[k] = lo[row];
      a0[k] = *reinterpret_cast<const float4*>(ao + row * 128 + 8 * l16);
      a1[k] = *reinterpret_cast<const float4*>(ao + row * 128 + 8 * l16 + 4);
    }
    const float Mn = fmaxf(fmaxf(M, fmaxf(mv[0], mv[1])), fmaxf(mv[2], mv[3]));
    const float al = exp2f(M - Mn);   // rescales what the earlier batches added
    M = Mn;
    Ls *= al;
#pragma unroll
    for (int e = 0; e < 8; ++e) xq[e] *= al;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float wgt = exp2f(mv[k] - M);   // 0 for the padding entries
      const float a[8] = {a0[k].x, a0[k].y, a0[k].z, a0[k].w, a1[k].x, a1[k].y, a1[k].z, a1[k].w};
      Ls += wgt * lv[k];
#pragma unroll
      for (int e = 0; e < 8; ++e) xq[e] += wgt * a[e];
    }
  }
  {   // exact partial
    const float wgt = exp2f(Mx - M);
    Ls += wgt * xl;
    const float a[8] = {xa0.x, xa0.y, xa0.z, xa0.w, xa1.x, xa1.y, xa1.z, xa1.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) xe[e] = wgt * a[e];
  }
  if (ns > 0) {   // y = H x, d = 8 l16 + e: three in-lane stages, four across the 16-lane group
#pragma unroll
    for (int k = 0; k < 3; ++k)
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (!(e & (1 << k))) {
          const float a = xq[e], c = xq[e | (1 << k)];
          xq[e] = a + c; xq[e | (1 << k)] = a - c;
        }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int msk = 1 << k;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float pv = __shfl_xor(xq[e], msk);
        xq[e] = (l16 & msk) ? pv - xq[e] : xq[e] + pv;
      }
    }
  }
  const float hn = __uint_as_float(0x3DB504F3u);
  uint32_t o[4];
#pragma unroll
  for (int e = 0; e < 8; e += 2) {
    float y0 = (ns > 0 ? xq[e] * hn : 0.f) + xe[e];
    float y1 = (ns > 0 ? xq[e + 1] * hn : 0.f) + xe[e + 1];
    y0 = Ls > 0.f ? y0 / Ls : 0.f;
    y1 = Ls > 0.f ? y1 / Ls : 0.f;
    o[e >> 1] = f2bf(y0) | (f2bf(y1) << 16);
  }
  *reinterpret_cast<uint4*>(out + ((int64_t)b * 16 + r) * 128 + 8 * l16) = make_uint4(o[0], o[1], o[2], o[3]);
}

int64_t align256(int64_t x) { return (x + 255) & ~(int64_t)255; }

// Validates the exact-tail arguments (for the standalone kernel and for the exact workgroups of the split grid);
// sets *nsink.
int check_exact(const kv800_paged_t* P, const uint16_t* q, const uint16_t* cos_t, const uint16_t* sin_t,
                int64_t epool_elems, float* mo, float* lo, float* ao, int64_t B, int64_t ns, uint16_t* out,
                int* nsink) {
  KV800_REQUIRE(P && B >= 0 && ns >= 0, "decode_exact: bad arguments");
  KV800_REQUIRE(q && cos_t && sin_t && mo && lo && ao && P->epool && P->eoff && P->N && P->NQ,
                "decode_exact: null pointer");
  KV800_REQUIRE(P->ebs > 0 && P->win >= 0, "decode_exact: ebs must be > 0");
  KV800_REQUIRE(P->e_hs % 8 == 0 && P->e_ts % 8 == 0 && ((uintptr_t)P->epool % 16) == 0,
                "decode_exact: exact strides must be multiples of 8 elements and the pool 16-byte aligned");
  *nsink = P->sk ? NSINK : 0;
  KV800_REQUIRE(!*nsink || (P->sv && P->skoff && P->svoff), "decode_exact: sinks need sv, skoff and svoff");
  KV800_REQUIRE(B * 4 <= 0x7FFFFFFF, "decode_exact: grid too large");
  KV800_REQUIRE(!out || ((uintptr_t)out % 4) == 0, "decode: out must be 4-byte aligned");
  KV800_REQUIRE(epool_elems >= 128, "decode_exact: the exact pool must hold at least one 128-element row");
  return KV800_OK;
}

// Launches decode_exact_kernel; with out != null the fused variant that also merges the quantized splits and writes
// the bf16 rows.
int launch_exact(const kv800_paged_t* P, const uint16_t* q, const uint16_t* cos_t, const uint16_t* sin_t,
                 int64_t rope_rows, int64_t epool_elems, int64_t sink_elems, float* mo, float* lo, float* ao, int64_t B,
                 int64_t ns, float scale, uint16_t* out, void* stream) {
  if (B == 0) return KV800_OK;
  int nsink = 0, rc;
  if ((rc = check_exact(P, q, cos_t, sin_t, epool_elems, mo, lo, ao, B, ns, out, &nsink)) != KV800_OK) return rc;
  const unsigned grid = (unsigned)(B * (4 / (out ? exact_nh<true>() : exact_nh<false>())));
  if (out)
    hipLaunchKernelGGL(decode_exact_kernel<true>, dim3(grid), dim3(256), 0, (hipStream_t)stream, *P, q, cos_t, sin_t,
                       rope_rows, epool_elems, sink_elems, mo, lo, ao, (int)ns, scale, nsink, out);
  else
    hipLaunchKernelGGL(decode_exact_kernel<false>, dim3(grid), dim3(256), 0, (hipStream_t)stream, *P, q, cos_t, sin_t,
                       rope_rows, epool_elems, sink_elems, mo, lo, ao, (int)ns, scale, nsink, (uint16_t*)nullptr);
  return check_launch(out ? "decode_exact_merge" : "decode_exact");
}

// Launches the quantized-split grid; xa != null adds the exact-tail workgroups (arguments checked by
// check_exact).
int launch_quant(const uint16_t* q, const uint8_t* qpool, int64_t qpool_bytes, const int64_t* boff,
                 int64_t boff_stride, const int32_t* nq, const uint32_t* cs16, int64_t rope_rows, float* mo, float* lo,
                 float* ao, int64_t B, int64_t ns, int64_t spb, float scale, const ExactArgs* xa, Sched S,
                 void* stream) {
  KV800_REQUIRE(B >= 0 && ns >= 0 && spb >= 1, "decode_quant: need B >= 0, ns >= 0, spb >= 1");
  if (B == 0 || ns == 0) return KV800_OK;
  KV800_REQUIRE(q && qpool && boff && nq && cs16 && mo && lo && ao, "decode_quant: null pointer");
  const int64_t nwork = S.groups ? S.groups + B : B * ns;
  KV800_REQUIRE(nwork + B * 4 <= 0x7FFFFFFF && ns * spb <= 0x7FFFFFFF, "decode_quant: grid too large");
  KV800_REQUIRE(((uintptr_t)qpool % 16) == 0 && ((uintptr_t)cs16 % 16) == 0 && ((uintptr_t)ao % 16) == 0,
                "decode_quant: qpool / cs16 / ao must be 16-byte aligned");
  ExactArgs X{};
  if (xa) X = *xa;
  else X.nexact = 0;
  hipLaunchKernelGGL(decode_quant_kernel, dim3((unsigned)(nwork + X.nexact)), dim3(256), 0, (hipStream_t)stream, q,
                     qpool, qpool_bytes, boff, boff_stride, nq, cs16, rope_rows, mo, lo, ao, (int)ns, (int)spb, scale, X,
                     S);
  return check_launch(xa ? "decode_quant_exact" : "decode_quant");
}

}  // namespace
}  // namespace kv800

using namespace kv800;

extern "C" {

int kv800_hip_rope_table(const uint16_t* cos_t, const uint16_t* sin_t, int64_t P, uint32_t* cs16, void* stream) {
  KV800_REQUIRE(P >= 0, "rope_table: P < 0");
  if (P == 0) return KV800_OK;
  KV800_REQUIRE(cos_t && sin_t && cs16, "rope_table: null pointer");
  const int64_t n = P * 32;
  hipLaunchKernelGGL(rope_table_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, cos_t,
                     sin_t, n, cs16);
  return check_launch("rope_table");
}

int kv800_hip_plan(int64_t B, int64_t nqmax, int64_t* ns, int64_t* spb) {
  KV800_REQUIRE(B >= 0 && nqmax >= 0 && ns && spb, "plan: bad arguments");
  if (nqmax == 0 || B == 0) { *ns = 0; *spb = 1; return KV800_OK; }
  // ~512 workgroups (2 per CU), each wave owning whole sub-blocks
  const int64_t want = (512 + B - 1) / B;
  const int64_t cap = (nqmax + QWAVES - 1) / QWAVES;
  int64_t n_s = want < cap ? want : cap;
  if (n_s < 1) n_s = 1;
  const int64_t sp = (nqmax + n_s - 1) / n_s;
  *spb = sp;
  *ns = (nqmax + sp - 1) / sp;
  return KV800_OK;
}

int kv800_hip_decode_quant_sized(const uint16_t* q, const uint8_t* qpool, int64_t qpool_bytes, const int64_t* boff,
                                 int64_t boff_stride, const int32_t* nq, const uint32_t* cs16, int64_t rope_rows,
                                 float* mo, float* lo, float* ao, int64_t B, int64_t ns, int64_t spb, float scale,
                                 void* stream) {
  return launch_quant(q, qpool, qpool_bytes, boff, boff_stride, nq, cs16, rope_rows, mo, lo, ao, B, ns, spb, scale,
                      nullptr, Sched{nullptr, 0, (int)B, 0}, stream);
}

int kv800_hip_decode_quant(const uint16_t* q, const uint8_t* qpool, const int64_t* boff, int64_t boff_stride,
                           const int32_t* nq, const uint32_t* cs16, float* mo, float* lo, float* ao, int64_t B,
                           int64_t ns, int64_t spb, float scale, void* stream) {
  return kv800_hip_decode_quant_sized(q, qpool, INT64_MAX / 2, boff, boff_stride, nq, cs16, INT64_MAX / 2, mo, lo, ao,
                                      B, ns, spb, scale, stream);
}

int kv800_hip_decode_exact_sized(const kv800_paged_t* P, const uint16_t* q, const uint16_t* cos_t,
                                 const uint16_t* sin_t, int64_t rope_rows, int64_t epool_elems, int64_t sink_elems,
                                 float* mo, float* lo, float* ao, int64_t B, int64_t ns, float scale, void* stream) {
  return launch_exact(P, q, cos_t, sin_t, rope_rows, epool_elems, sink_elems, mo, lo, ao, B, ns, scale, nullptr, stream);
}

int kv800_hip_decode_exact(const kv800_paged_t* P, const uint16_t* q, const uint16_t* cos_t, const uint16_t* sin_t,
                           float* mo, float* lo, float* ao, int64_t B, int64_t ns, float scale, void* stream) {
  return kv800_hip_decode_exact_sized(P, q, cos_t, sin_t, INT64_MAX / 2, INT64_MAX / 2, INT64_MAX / 2, mo, lo, ao, B, ns,
                                      scale, stream);
}

int kv800_hip_decode_merge(const float* mo, const float* lo, const float* ao, int64_t B, int64_t ns, uint16_t* out,
                           void* stream) {
  KV800_REQUIRE(B >= 0 && ns >= 0, "decode_merge: bad arguments");
  if (B == 0) return KV800_OK;
  KV800_REQUIRE(mo && lo && ao && out, "decode_merge: null pointer");
  KV800_REQUIRE(((uintptr_t)ao % 16) == 0 && ((uintptr_t)out % 16) == 0, "decode_merge: ao / out must be 16-byte aligned");
  hipLaunchKernelGGL(decode_merge_kernel, dim3((unsigned)B), dim3(256), 0, (hipStream_t)stream, mo, lo, ao, (int)ns,
                     Sched{nullptr, 0, (int)B, 0}, out);
  return check_launch("decode_merge");
}

int64_t kv800_hip_decode_workspace(int64_t B, int64_t ns, int64_t rope_rows) {
  const int64_t S = ns + 1;
  return align256(B * S * 16 * 4) * 2 + align256(B * S * 16 * 128 * 4) + align256(rope_rows * 32 * 4);
}

int64_t kv800_hip_decode_workspace_balanced(int64_t B, int64_t groups, int64_t rope_rows) {
  const int64_t S = 2 * B + groups;
  return align256(S * 16 * 4) * 2 + align256(S * 16 * 128 * 4) + align256((B + 1) * 4) + align256(rope_rows * 32 * 4);
}

int kv800_hip_plan_balanced(int64_t B, int64_t nqmax, int64_t* groups) {
  KV800_REQUIRE(B >= 0 && nqmax >= 0 && groups, "plan_balanced: bad arguments");
  // about BAL_CHUNK sub-blocks per workgroup (at most BAL_GROUPS workgroups) at the batch's largest size B * nqmax;
  // ragged batches hold fewer sub-blocks, and each workgroup then takes proportionally fewer
  const int64_t want = (B * ((nqmax + QWAVES - 1) / QWAVES) * QWAVES + BAL_CHUNK - 1) / BAL_CHUNK;
  *groups = want < 1 ? 1 : want > BAL_GROUPS ? BAL_GROUPS : want;
  return KV800_OK;
}

int kv800_hip_decode_sized(const kv800_paged_t* P, const uint16_t* q, int64_t B, const uint16_t* cos_t,
                           const uint16_t* sin_t, int64_t rope_rows, const uint32_t* cs16, int64_t qpool_bytes,
                           int64_t epool_elems, int64_t sink_elems, uint16_t* out, void* workspace,
                           int64_t workspace_bytes, int64_t spb, void* stream) {
  KV800_REQUIRE(P && B >= 0, "decode: bad arguments");
  if (B == 0) return KV800_OK;
  KV800_REQUIRE(q && out && workspace && cos_t && sin_t, "decode: null pointer");
  const int64_t nqmax = P->win ? 0 : P->nqmax;
  KV800_REQUIRE(nqmax >= 0, "decode: nqmax < 0");
  KV800_REQUIRE(!nqmax || (P->qpool && P->boff && nqmax <= P->boff_stride), "decode: nqmax exceeds the boff table");
  const int64_t rows = nqmax * BLK;
  KV800_REQUIRE(rows <= rope_rows, "decode: rope tables hold %lld rows, the quantized part needs %lld",
                (long long)rope_rows, (long long)rows);
  KV800_REQUIRE(((uintptr_t)workspace % 256) == 0, "decode: workspace must be 256-byte aligned");
  const float scale = (float)(1.4426950408889634 / sqrt(128.0));
  char* ws = (char*)workspace;
  int rc;
  if (!nqmax) {
    // no quantized part (window layers): exact tail + sinks fused with the merge (one launch writes the bf16 rows)
    const int64_t need = kv800_hip_decode_workspace(B, 0, 0);
    KV800_REQUIRE(workspace_bytes >= need, "decode: workspace of %lld bytes, need %lld", (long long)workspace_bytes,
                  (long long)need);
    float* mo = (float*)ws;
    float* lo = (float*)(ws + align256(B * 16 * 4));
    float* ao = (float*)(ws + 2 * align256(B * 16 * 4));
    return launch_exact(P, q, cos_t, sin_t, rope_rows, epool_elems, sink_elems, mo, lo, ao, B, 0, scale, out, stream);
  }
  // spb > 0: fixed (row, split) grid of spb sub-blocks per split; spb == 0: balanced schedule with the library's group
  // count; spb < 0: balanced schedule with -spb groups
  Sched S{nullptr, 0, (int)B, (int)nqmax};
  int64_t ns, sp, slots;
  if (spb > 0) {
    sp = spb;
    ns = (nqmax + sp - 1) / sp;
    slots = B * (ns + 1);
  } else {
    int64_t G = -spb;
    if (!G && (rc = kv800_hip_plan_balanced(B, nqmax, &G)) != KV800_OK) return rc;
    KV800_REQUIRE(B * nqmax < 0x7FFFFFFF - G && B < 0x7FFFFFFF / 2 - G, "decode: batch too large for the balanced schedule");
    S.groups = (int)G;
    ns = 1;
    sp = nqmax;
    slots = 2 * B + G;
  }
  const int64_t need = S.groups ? kv800_hip_decode_workspace_balanced(B, S.groups, cs16 ? 0 : rows)
                                : kv800_hip_decode_workspace(B, ns, cs16 ? 0 : rows);
  KV800_REQUIRE(workspace_bytes >= need, "decode: workspace of %lld bytes, need %lld", (long long)workspace_bytes,
                (long long)need);
  float* mo = (float*)ws;
  float* lo = (float*)(ws + align256(slots * 16 * 4));
  float* ao = (float*)(ws + 2 * align256(slots * 16 * 4));
  char* tail = ws + 2 * align256(slots * 16 * 4) + align256(slots * 16 * 128 * 4);
  if (S.groups) {
    S.pre = (int32_t*)tail;
    tail += align256((B + 1) * 4);
  }
  uint32_t* cst = (uint32_t*)tail;
  if (!cs16) {
    if ((rc = kv800_hip_rope_table(cos_t, sin_t, rows, cst, stream)) != KV800_OK) return rc;
    cs16 = cst;
  }
  // quantized work and the exact tail in one grid, then the merge
  ExactArgs X{};
  X.P = *P; X.cos_t = cos_t; X.sin_t = sin_t; X.rope_rows = rope_rows; X.epool_elems = epool_elems;
  X.sink_elems = sink_elems; X.nexact = (int)(B * (4 / XNH_TAIL));
  X.xs0 = S.groups ? B + S.groups : ns;
  X.xst = S.groups ? 1 : ns + 1;
  if ((rc = check_exact(P, q, cos_t, sin_t, epool_elems, mo, lo, ao, B, ns, out, &X.nsink)) != KV800_OK) return rc;
  if ((rc = launch_quant(q, P->qpool, qpool_bytes, P->boff, P->boff_stride, P->NQ, cs16, rows, mo, lo, ao, B, ns, sp,
                         scale, &X, S, stream)) != KV800_OK)
    return rc;
  KV800_REQUIRE(((uintptr_t)ao % 16) == 0 && ((uintptr_t)out % 16) == 0, "decode_merge: ao / out must be 16-byte aligned");
  hipLaunchKernelGGL(decode_merge_kernel, dim3((unsigned)B), dim3(256), 0, (hipStream_t)stream, mo, lo, ao, (int)ns, S,
                     out);
  return check_launch("decode_merge");
}

int kv800_hip_decode(const kv800_paged_t* P, const uint16_t* q, int64_t B, const uint16_t* cos_t,
                     const uint16_t* sin_t, const uint32_t* cs16, uint16_t* out, void* workspace,
                     int64_t workspace_bytes, int64_t spb, void* stream) {
  const int64_t rows = P ? (P->win ? 0 : P->nqmax) * BLK : 0;
  return kv800_hip_decode_sized(P, q, B, cos_t, sin_t, rows > 0 ? rows : INT64_MAX / 2, cs16, INT64_MAX / 2,
                                INT64_MAX / 2, INT64_MAX / 2, out, workspace, workspace_bytes, spb, stream);
}

}  // extern "C"
