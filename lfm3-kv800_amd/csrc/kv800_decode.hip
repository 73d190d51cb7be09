// kv800_decode.hip -- paged split-K decode attention over the 800h cache for gfx950, and its C-ABI entry points.
//
// Semantics (kv800.py:120-236, kv800_sycl.sycl:48-504, torch_decode.py:16-80): for each row b, 16 query rows over
// 4 KV heads (GQA 4), head_dim 128, scores q . RoPE(K) with RoPE on the dim pairs (d, d + 64), d < 32, fp32 online
// softmax in log2 units (scale = log2(e) / sqrt(128)); flushed sub-blocks contribute 2-bit K and 1-bit
// Hadamard-domain V, the exact tail / sinks bf16 K (rotated, rounded to bf16) and V; splits are merged by
// log-sum-exp, with the 128-point Hadamard applied once to the merged quantized part.
//
// Kernels
//   rope_table_kernel   bf16 (cos, sin) tables -> packed bf16 (cos, sin) pairs, one dword per (position, channel).
//   decode_quant_kernel one workgroup (4 waves) per span of one row's sub-blocks (a (row, split) of the fixed grid or
//                       a slice of the balanced schedule); the 4 waves share each sub-block, 64 tokens each, as
//                       32-token chunks whose bytes are prefetched one chunk ahead. Keys are formed exactly as
//                       torch_decode forms them (bf16 dequantized K from per-sub-block LDS code tables, RoPE in fp32
//                       rounded to bf16 again), QK on bf16 MFMA with exact products, PV on fp16 MFMA over the 1-bit
//                       Hadamard-domain planes (details at quant_span).
//   decode_exact_kernel one workgroup per row b, one wave per KV head (the exact-tail workgroups of the quantized
//                       grid: one per (row, KV head), its 4 waves taking turns over the chunks): sinks + exact
//                       positions in 32-token chunks (loads one chunk ahead), QK and PV on bf16 MFMA; the fused
//                       variant also merges the quantized splits of its rows.
//   decode_merge_kernel 1, 4 or 16 query heads of a row per workgroup: LSE merge of the partials (a row's many
//                       partials shared out over up to 16 lane groups per head, then combined), in-register FWHT,
//                       bf16 out.
#include <math.h>

#include <mutex>

#include "kv800_common.h"
#include "../../include/kv800_hip.h"

namespace kv800 {
namespace {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4v __attribute__((ext_vector_type(4)));
typedef int i2v __attribute__((ext_vector_type(2)));

constexpr float NEG_BIG = -1e30f;
constexpr float LAZY = 8.f;   // log2 units a tile max may exceed the running max before the state is rescaled

__device__ __forceinline__ uint32_t hbits(h2 x) { return __builtin_bit_cast(uint32_t, x); }
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
  p = halves32(vmax(p.x, p.y));
  return vmax(p.x, p.y);
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
                                  uint32_t* __restrict__ cs2) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  cs2[i] = (uint32_t)cos_t[i] | ((uint32_t)sin_t[i] << 16);
}

// ---------------------------------------------------------------- exact tail + sinks
// A workgroup takes one KV head h of one row b (query rows 4 h .. 4 h + 3): with NW = 4 waves, the waves take the
// head's 32-token chunks in turn (wave w: chunks w, w + 4, ...) and merge their states at the end; with NW = 1, its
// one wave takes every chunk. The tokens are the row's sinks, then its exact positions. Both products run on MFMA
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
template <int NW>                      // NW waves per workgroup
struct XLdsT {
  int64_t pg[XPG];                     // element offsets of the row's exact pages, from page lo_e / ebs on
  uint16_t v[NW][XCH][XVROW];          // each wave's copy of its chunk's V rows; at the end its columns and (m, l)
  u4v qb[NW][4][64];                   // each wave's QK B operand: k-step s of lane l in qb[w][s][l]
  float fm[NW][4], fl[NW][4];          // 4 waves on one head: each wave's m and l of rows 0..3
  float facc[NW][4][128];              // 4 waves on one head: each wave's accumulators of rows 0..3
};
typedef XLdsT<4> XLds;
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
template <bool MERGE, int NW>
__device__ __forceinline__ void exact_row(XLdsT<NW>& X, const int b, const int h0, const kv800_paged_t& P,
                                          const uint16_t* __restrict__ q,
                                          const uint16_t* __restrict__ cos_t, const uint16_t* __restrict__ sin_t,
                                          int64_t rope_rows, int64_t epool_elems, int64_t sink_elems,
                                          float* __restrict__ mo, float* __restrict__ lo_out, float* __restrict__ ao,
                                          int ns, int64_t xslot, float scale, int nsink, uint16_t* __restrict__ out) {
  static_assert(NW == 1 || NW == 4, "a workgroup of 1 or 4 waves takes one KV head");
  constexpr int WPH = NW;              // waves per head
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, g = lane >> 4, r16 = lane & 15;
  const int ph = w, h = h0;            // chunk phase, KV head
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
  if constexpr (WPH == 1) {
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
    for (int ww = 0; ww < NW; ++ww) M = fmaxf(M, X.fm[ww][r]);
    float L = 0.f, o0 = 0.f, o1 = 0.f;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) {
      const float sc = exp2f(X.fm[ww][r] - M);
      const float2 a = *reinterpret_cast<const float2*>(&X.facc[ww][r][dd]);
      L += sc * X.fl[ww][r];
      o0 += sc * a.x;
      o1 += sc * a.y;
    }
    emit(r, M, L, o0, o1);
  }
}

// The exact-tail workgroups of the quantized grid take NW = 4 (a tail must finish early to free its CU for the split
// work); the standalone partial-writing variant does the same, so its partials are bit-identical to the ones the
// quantized grid computes in-grid. The fused exact kernel (window layers) takes NW = 4 while its 4 B workgroups fit
// one round of resident workgroups (more waves on each head's chunks) and NW = 1 beyond: 4 B one-wave workgroups,
// up to 8 resident per CU, spread the (row, head) streams over the CUs in units of one stream. MI355X, window 256 + 4
// sinks at 32K: B = 64 / 96 / 128 take 14.0 / 19.0 / 19.6 us with NW = 4; B = 192 / 256 / 320 / 398 take 23.5 /
// 25.5 / 33.1 / 42.6 us with NW = 1, against 23.5 / 25.5 / 42.2 / 43.4 us with one 4-wave workgroup per row (one
// wave per head), whose 398 workgroups left 142 CUs with two rows and the rest with one.
template <bool MERGE, int NW>
__global__ void __launch_bounds__(64 * NW)
decode_exact_kernel(kv800_paged_t P, const uint16_t* __restrict__ q, const uint16_t* __restrict__ cos_t,
                    const uint16_t* __restrict__ sin_t, int64_t rope_rows, int64_t epool_elems, int64_t sink_elems,
                    float* __restrict__ mo, float* __restrict__ lo_out, float* __restrict__ ao, int ns, float scale,
                    int nsink, uint16_t* __restrict__ out) {
  __shared__ XLdsT<NW> X;
  const int b = blockIdx.x / 4;   // 4 workgroups per row, one per KV head
  exact_row<MERGE, NW>(X, b, blockIdx.x % 4, P, q, cos_t, sin_t, rope_rows, epool_elems, sink_elems, mo,
                        lo_out, ao, ns, (int64_t)b * (ns + 1) + ns, scale, nsink, out);
}

// ---------------------------------------------------------------- quantized sub-blocks
// A workgroup of 4 waves takes one row's sub-blocks [j0, j1) in order; the 4 waves share each sub-block, wave w taking
// its tokens 64 w .. 64 w + 63 as two 32-token chunks. Per chunk, lane (g, n) = (lane / 16, lane % 16):
// - K as torch_decode sees it (torch_decode.py:16-24, 54; kv800.py:79-86): every element of the dequantized K is
//   bf16(code * ksc + klo), 4 values per (head, dim) and sub-block, and the RoPE pairs (j, j + 64), j < 32, are rotated
//   in fp32 and rounded to bf16 again. Per sub-block the workgroup writes one 16-entry table per (head, channel j, kind)
//   into LDS: kind rope holds (bf16 K of dim j for code c0, of dim j + 64 for code c2) at entry (c0, c2); kind nope
//   (dims j + 32, j + 96) at (c1, c3). A kc byte c0 | c1 << 2 | c2 << 4 | c3 << 6 thus gives both pairs of its channel
//   with two lookups (one v_perm each to form the LDS address); a rope pair (k0, k2) is rotated by two v_dot2_f32_bf16
//   against the position's (cos, sin) and rounded by v_cvt_pk_bf16_f32, so the MFMA operands are exactly torch_decode's
//   rotated bf16 keys.
// - QK on MFMA f32_16x16x32_bf16: A = 16 tokens (row n = token n of the tile) x 32 K-elements of one KV head h
//   (lane group g: channels 8 g .. 8 g + 7, their rope pairs (dim j, dim j + 64) in two k-steps and nope pairs
//   (j + 32, j + 96) in two more), B = q (column n = query row n, the same K order), so products are exact and sums
//   fp32. Column n is meaningful for head h = n / 4 only; lane (g, n) keeps head n / 4's scores of tokens 4 g .. 4 g + 3.
// - softmax: fp32, log2 units, exact running max (the state is rescaled when a chunk max exceeds it): the largest
//   score's p is exactly 1, so its P.V weight is its vsc, exactly.
// - PV on MFMA f32_16x16x32_f16 in the Hadamard domain (kv800.py:157-168): A = 16 dims of one bit plane x the lane
//   group's 8 tokens, read by one ds_read_b64_tr_b8 per head from the wave's LDS copy of the chunk's vb bytes; a bit
//   becomes the fp16 subnormal 2^(i - 24) by one AND per two tokens; B = the weights fp16(p vsc) in head h's columns.
//   Plane i is scaled back by 2^(24 - i) at the end; sum p vlo is kept per row.
// The table lookups of one instruction touch 4 tables (one per lane group) whose entries sit in disjoint LDS banks.
constexpr int QWAVES = 4;
constexpr float QLAZY = 0.f;   // rescale threshold (log2 units): p <= 2^QLAZY, and p vsc <= 448 stays far below 65,504
constexpr int64_t BAL_CHUNK = 4, BAL_ROUNDS = 1;    // balanced schedule: sub-blocks per workgroup, most rounds
constexpr int LUT_WORDS = 64 * 64;                     // 64 blocks of 64 dwords: (kind, head, channel quad, channel)
constexpr int QROW = 132;
constexpr int VBH = 34;        // staged vb rows per head: 32 + 2 of padding put head h + 2 16 banks away from head h
struct QWaveLds {
  u4v vb[4 * VBH];             // the chunk's vb bytes: the 16-byte row of (head h, slot) at vb[VBH h + slot]
  float vs[2][64], vl[2][64];  // decoded vsc / vlo of the wave's 64 tokens, per head group
};
struct QLds {
  uint32_t lut[QWAVES][LUT_WORDS];  // each wave's code tables of the sub-block it is in
  QWaveLds wv[QWAVES];
};
struct QFinLds {               // end-of-span merge of the 4 waves (reuses the LDS)
  float m[QWAVES][16], l[QWAVES][16], lv[QWAVES][16];
  float acc[QWAVES][16][QROW];
};
static_assert(sizeof(QFinLds) <= sizeof(QLds), "fin scratch must fit");

// Slot of chunk token t in the staged vb rows: slot 8 g + k holds token 4 g + k (k < 4) or 16 + 4 g + k - 4, the 8
// tokens of lane group g in the K order of the PV MFMA (the tokens whose scores the group's lanes hold).
__device__ __forceinline__ int vb_slot(int t) { return 8 * ((t >> 2) & 3) + 4 * (t >> 4) + (t & 3); }

// RoPE of four channels' dequantized key pairs k[e] = (k0, k2) (bf16 lo / hi) against cs[e] = (cos, sin) and
// sw[e] = (sin, cos): r[e] = (bf16(k0 cos - k2 sin), bf16(k2 cos + k0 sin)), torch_decode.py:22-24. Each sum comes from
// one v_dot2_f32_bf16 (exact bf16 products; the hardware sum is within one fp32 ulp of the rounded exact sum, which
// changes the bf16 rounding that follows only for values within that ulp of a bf16 rounding boundary) and the pair is
// rounded by v_cvt_pk_bf16_f32 (RNE). The compiler does not see inside the block, so the block keeps the hazards of the
// dot instructions itself: every v_cvt reads dot results written at least three instructions earlier, and the
// leading / trailing s_nop cover a VALU write of an input just before and an MFMA read of an output just after.
__device__ __forceinline__ void rope4(const uint32_t (&k)[4], const uint32_t (&cs)[4], const uint32_t (&sw)[4],
                                      uint32_t (&r)[4]) {
  uint32_t t0, t1, t2, t3;
  asm("s_nop 1\n"
      "v_dot2_f32_bf16 %0, %8, %12, 0 neg_hi:[0,1,0]\n"
      "v_dot2_f32_bf16 %4, %8, %16, 0\n"
      "v_dot2_f32_bf16 %1, %9, %13, 0 neg_hi:[0,1,0]\n"
      "v_dot2_f32_bf16 %5, %9, %17, 0\n"
      "v_dot2_f32_bf16 %2, %10, %14, 0 neg_hi:[0,1,0]\n"
      "v_dot2_f32_bf16 %6, %10, %18, 0\n"
      "v_dot2_f32_bf16 %3, %11, %15, 0 neg_hi:[0,1,0]\n"
      "v_dot2_f32_bf16 %7, %11, %19, 0\n"
      "v_cvt_pk_bf16_f32 %0, %0, %4\n"
      "v_cvt_pk_bf16_f32 %1, %1, %5\n"
      "v_cvt_pk_bf16_f32 %2, %2, %6\n"
      "v_cvt_pk_bf16_f32 %3, %3, %7\n"
      "s_nop 1"
      : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3]), "=&v"(t0), "=&v"(t1), "=&v"(t2), "=&v"(t3)
      : "v"(k[0]), "v"(k[1]), "v"(k[2]), "v"(k[3]), "v"(cs[0]), "v"(cs[1]), "v"(cs[2]), "v"(cs[3]), "v"(sw[0]),
        "v"(sw[1]), "v"(sw[2]), "v"(sw[3]));
}
__device__ __forceinline__ b8 pack8b(const uint32_t (&x)[4]) { return as_b8(u4v{x[0], x[1], x[2], x[3]}); }

// The K scale bytes of the 4 tables lane l builds, t = 4 l + e (kind t >> 7 = l >> 5, head (t >> 5) & 3, channel
// t & 31 = 4 (l & 7) + e): klo / ksc of the tables' two dims (kind 0: dims j, j + 64; kind 1: j + 32, j + 96) for 4
// consecutive channels, one aligned dword each, byte e for table e (combined only when the tables are built, a
// pair of chunks after they are issued).
struct TabWords { uint32_t la, lb, sa, sb; };
// Sub-block reads go through a buffer resource of the sub-block (base and size in SGPRs, built per sub-block by
// scalar instructions): each load's address is a lane constant plus a wave-uniform SGPR offset plus its immediate, so
// no per-lane address arithmetic runs per chunk, and a read past the 51,200 bytes returns zeros.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr int RSRC_WORD3 = 0x00020000;   // raw (untyped, unswizzled) buffer access on gfx9-family parts
__device__ __forceinline__ rsrc_t sub_rsrc(const uint8_t* sb) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(sb), (short)0, SUB, RSRC_WORD3);
}
__device__ __forceinline__ TabWords table_words(rsrc_t rs, int lane) {
  const int o = 128 * ((lane >> 3) & 3) + 32 * (lane >> 5) + 4 * (lane & 7);
  return TabWords{__builtin_amdgcn_raw_buffer_load_b32(rs, o, KLO_O, 0),
                  __builtin_amdgcn_raw_buffer_load_b32(rs, o + 64, KLO_O, 0),
                  __builtin_amdgcn_raw_buffer_load_b32(rs, o, KSC_O, 0),
                  __builtin_amdgcn_raw_buffer_load_b32(rs, o + 64, KSC_O, 0)};
}
// Table t of a wave's LUT: entry (ca, cb) = bf16(ca ksc_a + klo_a) | bf16(cb ksc_b + klo_b) << 16 (kv800.py:84-86:
// the product is exact in fp32, so the fused multiply-add rounds where torch's add does). Channel j = 8 g + 4 d + e of
// (kind, head h) has its table in the 256-byte block ((kind 4 + h) 2 + d) 4 + e, entry (ca, cb) at byte
// 4 ca + 16 g + 64 cb: the four lane groups' tables of one (kind, h, d, e) interleave in one block, so a lookup's
// address is the masked kc byte (4 ca + 64 cb, code_lookup) or'ed with the lane's 16 g and the wave's LUT base, and
// its block is the instruction's immediate offset. Lane group g's 16 entries sit in banks 4 g .. 4 g + 3 and
// 16 + 4 g .. + 3 of the 32: the two groups of a half-wave never meet; within a group, entries whose cb differ by 2
// share a bank.
__device__ __forceinline__ void lut_build4(uint32_t* lut, int lane, const TabWords& tw) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t sel = 0x0C0C0000u | ((uint32_t)(4 + e) << 8) | (uint32_t)e;
    const uint32_t x = __builtin_amdgcn_perm(tw.lb, tw.la, sel) | (__builtin_amdgcn_perm(tw.sb, tw.sa, sel) << 16);
    float v[4];
    f8x4(x, v);   // klo_a, klo_b, ksc_a, ksc_b
    const int t = 4 * lane + e, kind = t >> 7, h = (t >> 5) & 3, j = t & 31, g = j >> 3, d = (j >> 2) & 1;
    uint32_t pa[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) pa[c] = bfpk(fmaf((float)c, v[2], v[0]), fmaf((float)c, v[3], v[1]));
    uint32_t* tab = lut + 64 * (((kind * 4 + h) * 2 + d) * 4 + e) + 4 * g;
    // row cb (entries ca = 0..3) at dword 16 cb; write k stores row (k + d) & 3: the 8 lanes of one 128-byte write
    // cycle (same kind, head and e; d = lane & 1, g = (lane & 7) >> 1) then cover the 32 banks once
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int cb = (k + d) & 3;
      const uint32_t hi = (cb & 2 ? (cb & 1 ? pa[3] : pa[2]) : (cb & 1 ? pa[1] : pa[0])) & 0xFFFF0000u;
      *reinterpret_cast<u4v*>(tab + 16 * cb) =
          u4v{(pa[0] & 0xFFFFu) | hi, (pa[1] & 0xFFFFu) | hi, (pa[2] & 0xFFFFu) | hi, (pa[3] & 0xFFFFu) | hi};
    }
  }
}
// Byte E of x, zero-extended, or'ed with base: one v_or_b32_sdwa (the compiler forms it from two instructions).
template <int E>
__device__ __forceinline__ uint32_t byte_or(uint32_t x, uint32_t base) {
  uint32_t r;
  asm("v_or_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_%c3 src1_sel:DWORD"
      : "=v"(r) : "v"(x), "v"(base), "n"(E));
  return r;
}
// vlo / vsc bytes of token t (both head groups)
__device__ __forceinline__ uint32_t scale_bytes(rsrc_t rs, int t0, int lane) {   // token t0 + lane
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rs, 2 * lane, VLO_O + 2 * t0, 0) |
         ((uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rs, 2 * lane, VSC_O + 2 * t0, 0) << 16);
}

struct QChunk {                // one chunk's data in registers
  uint2 kc[2][4];              // [tile u][head h]: kc bytes of token 16 u + n, channels 8 g .. 8 g + 7
  u4v cs[2][2];                // [tile u][d]: (cos, sin) bf16 pairs of channels 8 g + 4 d .. + 3 at the token's position
  u4v vb[2];                   // vb bytes 32 lane .. 32 lane + 31 of the chunk: token lane / 2, heads 2 (lane % 2), + 1
};
// rs: the sub-block; rc: the rope pair table, cpos: the sub-block's first position (token t0 of the sub-block is
// at position cpos + t0)
__device__ __forceinline__ void qload(QChunk& C, rsrc_t rs, rsrc_t rc, int cpos, int t0, int lane) {
  const int g = lane >> 4, n = lane & 15;
  const int ok = n * 128 + 8 * g, oc = n * 128 + 32 * g;   // lane parts of the kc and pair-table offsets
#pragma unroll
  for (int u = 0; u < 2; ++u) {
#pragma unroll
    for (int h = 0; h < 4; ++h)
      C.kc[u][h] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rs, ok + 2048 * u + 32 * h,
                                                                                   KC_O + t0 * 128, 0));
    C.cs[u][0] = __builtin_bit_cast(u4v, __builtin_amdgcn_raw_buffer_load_b128(rc, oc + 2048 * u, (cpos + t0) * 128, 0));
    C.cs[u][1] = __builtin_bit_cast(u4v, __builtin_amdgcn_raw_buffer_load_b128(rc, oc + 2048 * u + 16,
                                                                               (cpos + t0) * 128, 0));
  }
  C.vb[0] = __builtin_bit_cast(u4v, __builtin_amdgcn_raw_buffer_load_b128(rs, 32 * lane, VB_O + t0 * 64, 0));
  C.vb[1] = __builtin_bit_cast(u4v, __builtin_amdgcn_raw_buffer_load_b128(rs, 32 * lane + 16, VB_O + t0 * 64, 0));
}

static_assert(sizeof(XLds) <= 65536, "exact-tail scratch too large");

// Attention of row b's 16 query rows over its sub-blocks [j0, j1). The workgroup's partial (m, l, acc in the Hadamard
// domain) goes to partial rows prow .. prow + 15. A sub-block whose offset falls outside the pool (or whose positions
// fall outside the rope table) is skipped; its loads read the pool's first sub-block instead (the host requires the
// pool to hold one).
__device__ __forceinline__ void quant_span(char* lds_raw, const uint16_t* __restrict__ q,
                                           const uint8_t* __restrict__ qpool, int64_t qpool_bytes,
                                           const int64_t* __restrict__ boff, int64_t bstride,
                                           const uint32_t* __restrict__ cs2, int64_t rope_rows, float* __restrict__ mo,
                                           float* __restrict__ lo_out, float* __restrict__ ao, float scale, const int b,
                                           const int j0, const int j1, const int64_t prow) {
  QLds& L = *reinterpret_cast<QLds*>(lds_raw);
  // the wave index as a scalar: the span's sub-block offsets, buffer resources and loop bounds stay in SGPRs
  const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int g = lane >> 4, n = lane & 15, hn = n >> 2;
  QWaveLds& W = L.wv[w];
  const char* lutc = reinterpret_cast<const char*>(&L.lut[0][0]);

  // q as the QK B operands: k-step d (rope) = (q[j], q[j + 64]) pairs, k-step 2 + d (nope) = (q[j + 32], q[j + 96]),
  // j = 8 g + 4 d + e in register e
  b8 bq[4];
  {
    const uint16_t* qr = q + ((int64_t)b * 16 + n) * 128 + 8 * g;
    const u4v Q0 = *reinterpret_cast<const u4v*>(qr), Q1 = *reinterpret_cast<const u4v*>(qr + 32);
    const u4v Q2 = *reinterpret_cast<const u4v*>(qr + 64), Q3 = *reinterpret_cast<const u4v*>(qr + 96);
    auto el = [](const u4v& Q, int i) -> uint32_t { return (Q[i >> 1] >> (16 * (i & 1))) & 0xFFFFu; };
#pragma unroll
    for (int d = 0; d < 2; ++d) {
      uint32_t r[4], p[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        r[e] = el(Q0, 4 * d + e) | (el(Q2, 4 * d + e) << 16);
        p[e] = el(Q1, 4 * d + e) | (el(Q3, 4 * d + e) << 16);
      }
      bq[d] = pack8b(r);
      bq[2 + d] = pack8b(p);
    }
  }

  float m = NEG_BIG, lsum = 0.f, lvs = 0.f;
  f4 acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = f4{0.f, 0.f, 0.f, 0.f};

  auto stage_scales = [&](uint32_t x) {
    float v[4];
    f8x4(x, v);
    W.vl[0][lane] = v[0]; W.vl[1][lane] = v[1]; W.vs[0][lane] = v[2]; W.vs[1][lane] = v[3];
  };

  // One chunk of 32 tokens (tokens 64 w + 32 cc ..) of the current sub-block.
  auto chunk = [&](const QChunk& C, int cc, uint32_t kg) {
    {   // the chunk's vb rows into the wave's LDS copy (the previous chunk's reads were issued before)
      const int t = lane >> 1, s = vb_slot(t), h0 = 2 * (lane & 1);
      asm volatile("" ::: "memory");
      W.vb[VBH * h0 + s] = C.vb[0];
      W.vb[VBH * (h0 + 1) + s] = C.vb[1];
      asm volatile("" ::: "memory");
    }
    // QK in 8 steps (head h, kc dword d), both tiles per step; each step's table reads are issued one step ahead. The
    // lane keeps only its own head's scores: after head h's two k-step pairs, column n's values move to sv when h == hn.
    f4 qa[2];
    float sv[2][4];   // raw scores (scale > 0 is applied inside the exponent)
    uint32_t kk[3][2][4], an[3][2][4];   // [step % 3][tile][e]
    auto lookup = [&](const int st, const int pb) {
      const int h = st >> 1, d = st & 1;
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const uint32_t x = d ? C.kc[u][h].y : C.kc[u][h].x;
        // byte e of xr: 4 c0 + 64 c2 (rope), of xn: 4 c1 + 64 c3 (nope); with kg (wave base + 16 g) the entry's
        // address; the table's block (kind, h, d, e) is the immediate offset
        const uint32_t xr = (x << 2) & 0xCCCCCCCCu, xn = x & 0xCCCCCCCCu;
        const char* br = lutc + 256 * ((h * 2 + d) * 4);
        const char* bn = lutc + 256 * (((4 + h) * 2 + d) * 4);
        kk[pb][u][0] = *reinterpret_cast<const uint32_t*>(br + byte_or<0>(xr, kg));
        an[pb][u][0] = *reinterpret_cast<const uint32_t*>(bn + byte_or<0>(xn, kg));
        kk[pb][u][1] = *reinterpret_cast<const uint32_t*>(br + 256 + byte_or<1>(xr, kg));
        an[pb][u][1] = *reinterpret_cast<const uint32_t*>(bn + 256 + byte_or<1>(xn, kg));
        kk[pb][u][2] = *reinterpret_cast<const uint32_t*>(br + 512 + byte_or<2>(xr, kg));
        an[pb][u][2] = *reinterpret_cast<const uint32_t*>(bn + 512 + byte_or<2>(xn, kg));
        kk[pb][u][3] = *reinterpret_cast<const uint32_t*>(br + 768 + byte_or<3>(xr, kg));
        an[pb][u][3] = *reinterpret_cast<const uint32_t*>(bn + 768 + byte_or<3>(xn, kg));
      }
    };
    // wave priority by phase: of a SIMD's two waves, the one in its LDS -> VALU -> MFMA QK chain (3) or softmax (2)
    // wins the issue slots over one in PV (0), whose MFMA chain then runs under it
    __builtin_amdgcn_s_setprio(3);
    lookup(0, 0);
    lookup(1, 1);
#pragma unroll
    for (int st = 0; st < 8; ++st) {
      if (st + 2 < 8) lookup(st + 2, (st + 2) % 3);
      const int h = st >> 1, d = st & 1, pb = st % 3;
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        uint32_t c4[4], s4[4], ar[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          c4[e] = C.cs[u][d][e];
          s4[e] = __builtin_amdgcn_alignbit(C.cs[u][d][e], C.cs[u][d][e], 16);
        }
        rope4(kk[pb][u], c4, s4, ar);
        const f4 z = (d == 0) ? f4{0.f, 0.f, 0.f, 0.f} : qa[u];
        qa[u] = mfma_bf(pack8b(ar), bq[d], z);
        qa[u] = mfma_bf(pack8b(an[pb][u]), bq[2 + d], qa[u]);
        if (d == 1) {
#pragma unroll
          for (int i = 0; i < 4; ++i) sv[u][i] = (h == 0 || hn == h) ? qa[u][i] : sv[u][i];
        }
      }
    }
    __builtin_amdgcn_s_setprio(2);
    // ---- online softmax over the chunk's 32 tokens; row = column n, tokens 4 g + i of each tile
    float tmax = vmax3(vmax3(sv[0][0], sv[0][1], sv[0][2]), vmax3(sv[0][3], sv[1][0], sv[1][1]),
                       vmax(sv[1][2], sv[1][3]));
    tmax = max4rows(tmax) * scale;
    if (__any(tmax > m + QLAZY)) {   // a chunk max above the running max: rescale (a wave-uniform branch)
      const float mn = fmaxf(m, tmax);
      const float al = __builtin_amdgcn_exp2f(m - mn);   // v_exp_f32; tiny results flush to 0
      m = mn; lsum *= al; lvs *= al;
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] *= al;
    }
    float wt[2][4];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int t0 = 32 * cc + 16 * u + 4 * g;
      const float4 vs4 = *reinterpret_cast<const float4*>(&W.vs[n >> 3][t0]);
      const float4 vl4 = *reinterpret_cast<const float4*>(&W.vl[n >> 3][t0]);
      const float p0 = __builtin_amdgcn_exp2f(fmaf(sv[u][0], scale, -m));
      const float p1 = __builtin_amdgcn_exp2f(fmaf(sv[u][1], scale, -m));
      const float p2 = __builtin_amdgcn_exp2f(fmaf(sv[u][2], scale, -m));
      const float p3 = __builtin_amdgcn_exp2f(fmaf(sv[u][3], scale, -m));
      lsum += (p0 + p1) + (p2 + p3);
      lvs += (p0 * vl4.x + p1 * vl4.y) + (p2 * vl4.z + p3 * vl4.w);
      wt[u][0] = p0 * vs4.x; wt[u][1] = p1 * vs4.y; wt[u][2] = p2 * vs4.z; wt[u][3] = p3 * vs4.w;
    }
    // B in the K order of the A registers: (k0, k2), (k1, k3), (k4, k6), (k5, k7), token k of the group = slot 8 g + k
    const h8 Bw = pack8(pk2(wt[0][0], wt[0][2]), pk2(wt[0][1], wt[0][3]), pk2(wt[1][0], wt[1][2]), pk2(wt[1][1], wt[1][3]));
    __builtin_amdgcn_s_setprio(0);
    // ---- PV per head: A row n = dim n of plane i, bytes of the group's 8 tokens by one transposed read
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      const h8 B = (hn == h) ? Bw : pack8(0u, 0u, 0u, 0u);
      typedef __attribute__((address_space(3))) i2v lds_i2;
      const i2v X = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
          (lds_i2*)(reinterpret_cast<char*>(W.vb) + (h * VBH + 8 * g) * 16 + 8 * n));
      const uint32_t x0 = (uint32_t)X.x, x1 = (uint32_t)X.x >> 8, x2 = (uint32_t)X.y, x3 = (uint32_t)X.y >> 8;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t msk = (1u << i) | (1u << (16 + i));
        acc[i] = mfma16(pack8(x0 & msk, x1 & msk, x2 & msk, x3 & msk), B, acc[i]);
      }
    }
    asm volatile("" ::: "memory");   // the transposed reads stay before the next chunk's staging
  };

  if (j0 < j1) {
    // The span's 4 (j1 - j0) pairs of 32-token chunks: wave w takes pairs [len w, len (w + 1)), pair P being tokens
    // 64 (P % 4) .. + 63 of sub-block j0 + P / 4. The wave builds its own code tables for each sub-block it enters,
    // so the waves never wait for each other until the span's end.
    const int64_t* brow = boff + (int64_t)b * bstride;
    auto sanitize = [&](int64_t raw, int jb) -> int64_t {
      return (raw < 0 || raw > qpool_bytes - SUB || (int64_t)(jb + 1) * BLK > rope_rows) ? -1 : raw;
    };
    const int len = j1 - j0, P0 = len * w, P1 = P0 + len;
    int jb = j0 + P0 / 4, pin = P0 % 4;
    int64_t base = sanitize(brow[jb], jb);
    int64_t nraw = brow[min(jb + 1, j1 - 1)];   // the next sub-block's offset, loaded a sub-block ahead of its use
    const uint8_t* sb = qpool + (base < 0 ? 0 : base);
    rsrc_t rs = sub_rsrc(sb);
    const rsrc_t rc = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(cs2), (short)0,
                                                        (int)min(rope_rows * 128, (int64_t)INT32_MAX), RSRC_WORD3);
    int cpos = base < 0 ? 0 : jb * BLK;
    uint32_t* lut = L.lut[w];
    const uint32_t kg = (uint32_t)w * (LUT_WORDS * 4) + 16u * (uint32_t)g;   // the wave's LUT and the lane group
    QChunk C0, C1;
    qload(C0, rs, rc, cpos, 64 * pin, lane);
    lut_build4(lut, lane, table_words(rs, lane));
    stage_scales(scale_bytes(rs, 64 * pin, lane));
    for (int P = P0; P < P1; ++P) {
      const bool more = P + 1 < P1, cross = more && pin == 3;   // the next pair is in the next sub-block
      const int njb = cross ? jb + 1 : jb, npin = cross ? 0 : (pin + 1) & 3;
      int64_t nbase = base;
      rsrc_t nrs = rs;
      int ncpos = cpos;
      if (cross) {
        nbase = sanitize(nraw, njb);
        nrs = sub_rsrc(qpool + (nbase < 0 ? 0 : nbase));
        ncpos = nbase < 0 ? 0 : njb * BLK;
        nraw = brow[min(njb + 1, j1 - 1)];
      }
      // the next sub-block's table words (used after this pair's chunks) and the next pair's scale bytes
      const TabWords ntw = table_words(nrs, lane);
      const uint32_t nsc = scale_bytes(nrs, 64 * npin, lane);
      qload(C1, rs, rc, cpos, 64 * pin + 32, lane);
      if (base >= 0) chunk(C0, 0, kg);
      qload(C0, nrs, rc, ncpos, 64 * npin, lane);
      if (base >= 0) chunk(C1, 1, kg);
      if (more) {   // the wave's own LDS: its lookups and scale reads of this pair were issued before these writes
        if (cross) lut_build4(lut, lane, ntw);
        stage_scales(nsc);
      }
      jb = njb;
      pin = npin;
      base = nbase;
      rs = nrs;
      cpos = ncpos;
    }
  }  // ---- combine the 4 waves of the span
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

// Exact-tail work carried by the quantized-split grid: the workgroups after the split workgroups, [nwork, nwork +
// nexact), each run the exact tail of one row's KV head(s) (its exact partial slot, as decode_exact_kernel<false>).
// Placed last, they take the slots the split workgroups free as they finish: placed first, they would hold half of
// the CUs' workgroup slots for their latency-bound few microseconds while the split workgroups queued behind them,
// whose one round of resident workgroups then ended that much later.
struct ExactArgs {
  kv800_paged_t P;
  const uint16_t* cos_t;
  const uint16_t* sin_t;
  int64_t rope_rows, epool_elems, sink_elems;
  int64_t xs0, xst;   // exact partial of row b in slot xs0 + b xst
  int nexact, nsink;
};

// Balanced schedule (groups > 0): the B rows' sub-blocks laid end to end, q_b sub-blocks in row b (clamped to
// [0, cap]), T = sum q_b, C = ceil(T / groups). Two cuts of that list into pieces of at most C sub-blocks, the one
// needing fewer rounds of resident workgroups taken (ties: row-wise):
//   row-wise: row b is cut into ceil(q_b / C) slices, the slices of all rows laid end to end; workgroup g takes
//     slice g (one row) and writes its partial to slot g. sum ceil(q_b / C) <= T / C + B <= groups + B, so the grid
//     has groups + B workgroups and the ones past the last slice return at once.
//   list-wise: workgroup g takes the list's sub-blocks [g C, (g + 1) C), which may end in a later row than they
//     start; it attends each row segment in turn and writes one partial per segment, the first to slot g, each later
//     one (which starts a row b) to slot groups + b, since no other workgroup enters row b from an earlier row. Every
//     workgroup but the last has exactly C sub-blocks, however ragged the rows are.
// Uniform rows whose count divides into whole rounds (64 x 127 sub-blocks: 8 slices of 16 a row, 512 workgroups,
// one round) keep one segment per workgroup; otherwise the list-wise cut avoids a nearly empty last round (398 x 127
// sub-blocks over 512 workgroups: 796 row-wise slices of 99 would take 2 rounds, the list-wise cut's 511 pieces of
// 99 take one). The exact partial of row b is
// slot groups + B + b. groups = 0: the fixed (row, split) grid, split s of row b in slot b (ns + 1) + s, the exact
// partial in slot b (ns + 1) + ns (the reference's partial layout).
struct Sched {
  int32_t* pre;         // pre[0 .. B + 1], written by workgroup 0 of the decode grid for the merge: the row-wise cut's
                        // slices before each row and pre[B + 1] = -C, or the list's sub-blocks before each row and
                        // pre[B + 1] = C
  int groups, B, cap;   // cap: sub-blocks per row are clamped to [0, cap]
  int res;              // workgroups of the grid resident at once (one round)
};

// The decode grid's workgroups each scan NQ themselves: thread t owns rows [t k, t k + k), k = ceil(B / 256), reads
// their counts once (into registers, up to RREG rows, i.e. B <= 1024; later rows are read again) and takes part in
// two block-wide scans, of the sub-blocks (for T) and of the slices.
constexpr int RREG = 4;
struct RowTab {
  int wsum[4];
  int b, pb, nsb, s1;   // the row of the current segment, its first sub-block in the list, its clamped sub-block
                        // count; the end of the workgroup's sub-blocks in the list
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
// Exclusive prefix of v over the workgroup's threads (in thread order); *total = the sum over all threads.
__device__ __forceinline__ int slices_of(int nsb, int C) { return (nsb + C - 1) / C; }
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

constexpr int QLDS_BYTES = sizeof(QLds) > sizeof(XLds) ? (int)sizeof(QLds) : (int)sizeof(XLds);

__global__ void __launch_bounds__(256, 2)
decode_quant_kernel(const uint16_t* __restrict__ q, const uint8_t* __restrict__ qpool, int64_t qpool_bytes,
                    const int64_t* __restrict__ boff, int64_t bstride, const int32_t* __restrict__ nq,
                    const uint32_t* __restrict__ cs2, int64_t rope_rows, float* __restrict__ mo,
                    float* __restrict__ lo_out, float* __restrict__ ao, int ns, int spb, float scale, ExactArgs X,
                    Sched S) {
  __shared__ __align__(16) char lds_raw[QLDS_BYTES];
  const int nwork = (int)gridDim.x - X.nexact;
  if ((int)blockIdx.x >= nwork) {
    const int xb = (int)blockIdx.x - nwork, b = xb / 4;   // 4 workgroups per row, one per KV head
    exact_row<false, 4>(*reinterpret_cast<XLds*>(lds_raw), b, xb % 4, X.P, q, X.cos_t,
                               X.sin_t, X.rope_rows, X.epool_elems, X.sink_elems, mo, lo_out, ao, ns,
                               X.xs0 + b * X.xst, scale, X.nsink, nullptr);
    return;
  }
  const int blk = (int)blockIdx.x;
  int b, j0, j1;
  int64_t prow;
  bool rowwise = true;   // one span per workgroup (the fixed grid, the row-wise cut)
  __shared__ RowTab R;
  if (S.groups == 0) {   // fixed grid: (row b, split s)
    b = blk / ns;
    const int s = blk % ns;
    j0 = s * spb;
    j1 = min(min((s + 1) * spb, nq[b]), (int)min(bstride, (int64_t)INT32_MAX));
    prow = ((int64_t)b * (ns + 1) + s) * 16;
  } else {   // balanced: the row-wise or the list-wise cut of the rows' sub-blocks laid end to end
    RowCache RC;
    load_rows(nq, S, RC);
    int qsum = 0;
    for (int i = 0; i < RC.r1 - RC.r0; ++i) qsum += nsb_of(nq, S, RC, i);
    int T;
    const int p = block_scan(qsum, R, &T);   // sub-blocks of the rows before this thread's rows
    const int C = T > 0 ? (T + S.groups - 1) / S.groups : 1;
    int nsl = 0;
    for (int i = 0; i < RC.r1 - RC.r0; ++i) nsl += slices_of(nsb_of(nq, S, RC, i), C);
    int G1;
    const int ps = block_scan(nsl, R, &G1);  // row-wise slices of the rows before this thread's rows
    const int G2 = (T + C - 1) / C, res = max(S.res, 1);
    rowwise = (G1 + res - 1) / res <= (G2 + res - 1) / res;
    if (blk == 0) {   // pre[0 .. B + 1] for the merge
      if (threadIdx.x == 0) { S.pre[0] = 0; S.pre[S.B + 1] = rowwise ? -C : C; }
      int pp = rowwise ? ps : p;
      for (int i = 0; i < RC.r1 - RC.r0; ++i) {
        const int nb = nsb_of(nq, S, RC, i);
        pp += rowwise ? slices_of(nb, C) : nb;
        S.pre[RC.r0 + i + 1] = pp;
      }
    }
    if (rowwise) {   // slice blk: one row's sub-blocks [j0, j1)
      if (blk >= G1) return;   // past the last slice (uniform over the workgroup)
      int pp = ps;
      for (int i = 0; i < RC.r1 - RC.r0; ++i) {   // exactly one thread owns the row of slice blk
        const int nb = nsb_of(nq, S, RC, i), n = slices_of(nb, C);
        if (pp <= blk && blk < pp + n) { R.b = RC.r0 + i; R.pb = pp; R.nsb = nb; }
        pp += n;
      }
      __syncthreads();
      b = __builtin_amdgcn_readfirstlane(R.b);
      const int k = blk - __builtin_amdgcn_readfirstlane(R.pb);
      j0 = C * k;
      j1 = min(C * (k + 1), __builtin_amdgcn_readfirstlane(R.nsb));
    } else {   // sub-blocks [blk C, (blk + 1) C) of the list
      const int s0 = blk * C;
      if (s0 >= T) return;   // past the last sub-block (uniform over the workgroup)
      int pp = p;
      for (int i = 0; i < RC.r1 - RC.r0; ++i) {   // exactly one thread owns the row holding sub-block s0
        const int nb = nsb_of(nq, S, RC, i);
        if (pp <= s0 && s0 < pp + nb) { R.b = RC.r0 + i; R.pb = pp; R.nsb = nb; }
        pp += nb;
      }
      if (threadIdx.x == 0) R.s1 = min(T, s0 + C);
      __syncthreads();
      b = __builtin_amdgcn_readfirstlane(R.b);
      const int st = __builtin_amdgcn_readfirstlane(R.pb);
      j0 = s0 - st;
      j1 = min(__builtin_amdgcn_readfirstlane(R.nsb), __builtin_amdgcn_readfirstlane(R.s1) - st);
    }
    prow = (int64_t)blk * 16;
  }
  // one span per row segment; between spans the segment state lives in R, so that only the span's own arguments stay
  // in registers across it
  for (;;) {
    quant_span(lds_raw, q, qpool, qpool_bytes, boff, bstride, cs2, rope_rows, mo, lo_out, ao, scale, b, j0, j1, prow);
    if (rowwise) return;
    asm volatile("" ::: "memory");
    const int st = __builtin_amdgcn_readfirstlane(R.pb), nb = __builtin_amdgcn_readfirstlane(R.nsb);
    const int s1 = __builtin_amdgcn_readfirstlane(R.s1);
    if (st + nb >= s1) return;   // the segment reached the end of the workgroup's sub-blocks
    b = __builtin_amdgcn_readfirstlane(R.b);
    int nb2;
    do {   // the next row with sub-blocks (one exists: st + nb < s1 <= T)
      ++b;
      nb2 = min(max(nq[b], 0), S.cap);
    } while (nb2 == 0);
    __syncthreads();   // every wave has read R and is done with the span's end-of-span LDS
    if (threadIdx.x == 0) { R.b = b; R.pb = st + nb; R.nsb = nb2; }
    j0 = 0;
    j1 = min(nb2, s1 - (st + nb));
    prow = ((int64_t)S.groups + b) * 16;
  }
}


// ---------------------------------------------------------------- split merge
// HPW query heads of row b per workgroup (grid (B, 16 / HPW)), SG = 16 / HPW lane groups of 16 per head: the row's
// quantized partials are shared out over a head's SG groups (group k takes partials k, k + SG, ..., four per memory
// round trip), each keeping a running (M, L, x) of its share; with SG > 1 the first group of each head combines the
// states from LDS. Then the exact partial, the FWHT across the group's 16 lanes and the head's 128 bf16 outputs. Many
// partials per row (a small batch cut into many slices) take SG = 16, so a row waits on one or two round trips
// instead of one per four partials; large batches with a few partials per row take HPW = 16, one workgroup per row.
template <int HPW>
__global__ void __launch_bounds__(256)
decode_merge_kernel(const float* __restrict__ mo, const float* __restrict__ lo, const float* __restrict__ ao, int ns,
                    Sched S, uint16_t* __restrict__ out) {
  constexpr int SG = 16 / HPW;
  __shared__ float gm[SG > 1 ? 16 : 1], gl[SG > 1 ? 16 : 1];
  __shared__ __align__(16) float gx[SG > 1 ? 16 : 1][128];
  const int b = blockIdx.x, tid = threadIdx.x, r16 = tid >> 4, l16 = tid & 15;
  const int hl = r16 / SG, k = r16 % SG, hq = (int)blockIdx.y * HPW + hl;
  // row b's exact partial: slot xs, requested first (its slot needs no table); its quantized partials: slots
  // first .. first + ns - 1 (and slot extra)
  const int64_t xs = S.groups > 0 ? (int64_t)S.groups + S.B + b : (int64_t)b * (ns + 1) + ns;
  const int64_t xrow = xs * 16 + hq;
  const float Mx = mo[xrow], xl = lo[xrow];
  const float4 xa0 = *reinterpret_cast<const float4*>(ao + xrow * 128 + 8 * l16);
  const float4 xa1 = *reinterpret_cast<const float4*>(ao + xrow * 128 + 8 * l16 + 4);
  int64_t first = (int64_t)b * (ns + 1), extra = -1;
  if (S.groups > 0) {
    const int cut = S.pre[S.B + 1];
    if (cut < 0) {   // row-wise: row b's slices are workgroups [pre[b], pre[b + 1]), one partial each
      first = S.pre[b];
      ns = S.pre[b + 1] - S.pre[b];
    } else {         // list-wise: row b holds sub-blocks [st, st + nb) of the list, workgroup g took [g C, (g + 1) C)
      const int st = S.pre[b], nb = S.pre[b + 1] - st, C = cut;
      first = (st + C - 1) / C;                                     // the workgroups that start inside the row
      ns = nb > 0 ? (st + nb - 1) / C - (int)first + 1 : 0;
      if (nb > 0 && st % C != 0) extra = (int64_t)S.groups + b;     // the one that entered it from an earlier row
    }
  }
  // partial j < nt: slot first + j for j < ns, the entering workgroup's slot for j = ns
  const int nt = ns + (extra >= 0 ? 1 : 0);
  auto row_of = [&](int j) { return ((j < ns) ? first + j : extra) * 16 + hq; };
  float M = NEG_BIG, Ls = 0.f, xq[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int j0 = k; j0 < nt; j0 += 4 * SG) {   // group k: partials j0, j0 + SG, j0 + 2 SG, j0 + 3 SG
    float mv[4], lv[4];
    float4 a0[4], a1[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int j = j0 + SG * i;
      const bool in = j < nt;
      const int64_t row = row_of(in ? j : j0);   // past the end: a repeat of partial j0, weighted 0 below
      mv[i] = in ? mo[row] : NEG_BIG;
      lv[i] = lo[row];
      a0[i] = *reinterpret_cast<const float4*>(ao + row * 128 + 8 * l16);
      a1[i] = *reinterpret_cast<const float4*>(ao + row * 128 + 8 * l16 + 4);
    }
    const float Mn = fmaxf(fmaxf(M, fmaxf(mv[0], mv[1])), fmaxf(mv[2], mv[3]));
    const float al = exp2f(M - Mn);   // rescales what the earlier batches added
    M = Mn;
    Ls *= al;
#pragma unroll
    for (int e = 0; e < 8; ++e) xq[e] *= al;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float wgt = exp2f(mv[i] - M);   // 0 for the padding entries
      const float a[8] = {a0[i].x, a0[i].y, a0[i].z, a0[i].w, a1[i].x, a1[i].y, a1[i].z, a1[i].w};
      Ls += wgt * lv[i];
#pragma unroll
      for (int e = 0; e < 8; ++e) xq[e] += wgt * a[e];
    }
  }
  if (SG > 1) {   // the head's SG group states, combined by its first group
    if (l16 == 0) { gm[r16] = M; gl[r16] = Ls; }
    *reinterpret_cast<float4*>(&gx[r16][8 * l16]) = make_float4(xq[0], xq[1], xq[2], xq[3]);
    *reinterpret_cast<float4*>(&gx[r16][8 * l16 + 4]) = make_float4(xq[4], xq[5], xq[6], xq[7]);
    __syncthreads();
    if (k != 0) return;   // whole 16-lane rows leave; the FWHT below stays within each remaining row
    M = NEG_BIG;
#pragma unroll
    for (int kk = 0; kk < SG; ++kk) M = fmaxf(M, gm[hl * SG + kk]);
    Ls = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) xq[e] = 0.f;
#pragma unroll
    for (int kk = 0; kk < SG; ++kk) {
      const int rr = hl * SG + kk;
      const float wgt = exp2f(gm[rr] - M);   // 0 for groups without partials (their state is zero anyway)
      Ls += wgt * gl[rr];
      const float4 c0 = *reinterpret_cast<const float4*>(&gx[rr][8 * l16]);
      const float4 c1 = *reinterpret_cast<const float4*>(&gx[rr][8 * l16 + 4]);
      const float a[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) xq[e] += wgt * a[e];
    }
  }
  // the exact partial, relative to the larger max
  const float Mt = fmaxf(M, Mx);
  {
    const float al = exp2f(M - Mt);
    Ls *= al;
#pragma unroll
    for (int e = 0; e < 8; ++e) xq[e] *= al;
  }
  float xe[8];
  {
    const float wgt = exp2f(Mx - Mt);
    Ls += wgt * xl;
    const float a[8] = {xa0.x, xa0.y, xa0.z, xa0.w, xa1.x, xa1.y, xa1.z, xa1.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) xe[e] = wgt * a[e];
  }
  const bool anyq = nt > 0;
  if (anyq) {   // y = H x, d = 8 l16 + e: three in-lane stages, four across the 16-lane group
#pragma unroll
    for (int kk = 0; kk < 3; ++kk)
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (!(e & (1 << kk))) {
          const float a = xq[e], c = xq[e | (1 << kk)];
          xq[e] = a + c; xq[e | (1 << kk)] = a - c;
        }
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int msk = 1 << kk;
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
    float y0 = (anyq ? xq[e] * hn : 0.f) + xe[e];
    float y1 = (anyq ? xq[e + 1] * hn : 0.f) + xe[e + 1];
    y0 = Ls > 0.f ? y0 / Ls : 0.f;
    y1 = Ls > 0.f ? y1 / Ls : 0.f;
    o[e >> 1] = f2bf(y0) | (f2bf(y1) << 16);
  }
  *reinterpret_cast<uint4*>(out + ((int64_t)b * 16 + hq) * 128 + 8 * l16) = make_uint4(o[0], o[1], o[2], o[3]);
}

// Heads per merge workgroup for about p partials per row. Whole decode, same process, HIP events (balanced plan; C3
// rows of 32K for B <= 64, 4K-token rows above): B = 1 / 8 / 16 / 64 / 128 / 256 / 398 rows (127 / 64 / 32 / 8 / 4 /
// 2 / 1-2 partials a row) 18.8 / 34.8 / 47.4 / 142 / 56.6 / 100.1 / 154.1 us with 1 head per workgroup, 22.8 / 36.8 /
// 47.2 / 136.5 / 54.4 / 97.4 / 148.8 with 4, 35.9 / 44.1 / 51.1 / 139.9 / 53.7 / 95.3 / 145.8 with 16.
int merge_hpw(int64_t p) { return p >= 16 ? 1 : p >= 6 ? 4 : 16; }

// Launches the merge with hpw (1, 4 or 16) heads per workgroup.
int launch_merge(const float* mo, const float* lo, const float* ao, int ns, const Sched& S, int64_t B, uint16_t* out,
                 void* stream, int hpw) {
  if (hpw == 16)
    hipLaunchKernelGGL(decode_merge_kernel<16>, dim3((unsigned)B, 1), dim3(256), 0, (hipStream_t)stream, mo, lo, ao, ns,
                       S, out);
  else if (hpw == 4)
    hipLaunchKernelGGL(decode_merge_kernel<4>, dim3((unsigned)B, 4), dim3(256), 0, (hipStream_t)stream, mo, lo, ao, ns,
                       S, out);
  else
    hipLaunchKernelGGL(decode_merge_kernel<1>, dim3((unsigned)B, 16), dim3(256), 0, (hipStream_t)stream, mo, lo, ao, ns,
                       S, out);
  return check_launch("decode_merge");
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

// Launches decode_exact_kernel, one workgroup per (row, KV head); with out != null the fused variant that also merges
// the quantized splits and writes the bf16 rows, with nw (1 or 4) waves per workgroup (the partial-writing variant
// always takes 4, as the quantized grid's tails do).
int launch_exact(const kv800_paged_t* P, const uint16_t* q, const uint16_t* cos_t, const uint16_t* sin_t,
                 int64_t rope_rows, int64_t epool_elems, int64_t sink_elems, float* mo, float* lo, float* ao, int64_t B,
                 int64_t ns, float scale, uint16_t* out, int nw, void* stream) {
  if (B == 0) return KV800_OK;
  int nsink = 0, rc;
  if ((rc = check_exact(P, q, cos_t, sin_t, epool_elems, mo, lo, ao, B, ns, out, &nsink)) != KV800_OK) return rc;
  if (!out) nw = 4;
  KV800_REQUIRE(nw == 1 || nw == 4, "decode_exact: 1 or 4 waves per workgroup");
  const unsigned grid = (unsigned)(B * 4);
  if (out && nw == 1)
    hipLaunchKernelGGL((decode_exact_kernel<true, 1>), dim3(grid), dim3(64), 0, (hipStream_t)stream, *P, q, cos_t,
                       sin_t, rope_rows, epool_elems, sink_elems, mo, lo, ao, (int)ns, scale, nsink, out);
  else if (out)
    hipLaunchKernelGGL((decode_exact_kernel<true, 4>), dim3(grid), dim3(256), 0, (hipStream_t)stream, *P, q, cos_t,
                       sin_t, rope_rows, epool_elems, sink_elems, mo, lo, ao, (int)ns, scale, nsink, out);
  else
    hipLaunchKernelGGL((decode_exact_kernel<false, 4>), dim3(grid), dim3(256), 0, (hipStream_t)stream, *P, q,
                       cos_t, sin_t, rope_rows, epool_elems, sink_elems, mo, lo, ao, (int)ns, scale, nsink,
                       (uint16_t*)nullptr);
  return check_launch(out ? "decode_exact_merge" : "decode_exact");
}

// Launches the quantized-split grid; xa != null adds the exact-tail workgroups (arguments checked by
// check_exact).
int launch_quant(const uint16_t* q, const uint8_t* qpool, int64_t qpool_bytes, const int64_t* boff,
                 int64_t boff_stride, const int32_t* nq, const uint32_t* cs2, int64_t rope_rows, float* mo, float* lo,
                 float* ao, int64_t B, int64_t ns, int64_t spb, float scale, const ExactArgs* xa, Sched S,
                 void* stream) {
  KV800_REQUIRE(B >= 0 && ns >= 0 && spb >= 1, "decode_quant: need B >= 0, ns >= 0, spb >= 1");
  if (B == 0 || ns == 0) return KV800_OK;
  KV800_REQUIRE(q && qpool && boff && nq && cs2 && mo && lo && ao, "decode_quant: null pointer");
  KV800_REQUIRE(qpool_bytes >= SUB, "decode_quant: the quant pool must hold at least one sub-block");
  const int64_t nwork = S.groups ? S.groups + B : B * ns;
  KV800_REQUIRE(nwork + B * 4 <= 0x7FFFFFFF && ns * spb <= 0x7FFFFFFF, "decode_quant: grid too large");
  KV800_REQUIRE(((uintptr_t)qpool % 16) == 0 && ((uintptr_t)cs2 % 16) == 0 && ((uintptr_t)ao % 16) == 0,
                "decode_quant: qpool / cs2 / ao must be 16-byte aligned");
  ExactArgs X{};
  if (xa) X = *xa;
  else X.nexact = 0;
  hipLaunchKernelGGL(decode_quant_kernel, dim3((unsigned)(nwork + X.nexact)), dim3(256), 0, (hipStream_t)stream, q,
                     qpool, qpool_bytes, boff, boff_stride, nq, cs2, rope_rows, mo, lo, ao, (int)ns, (int)spb, scale, X,
                     S);
  return check_launch(xa ? "decode_quant_exact" : "decode_quant");
}

}  // namespace
}  // namespace kv800

using namespace kv800;

extern "C" {

int kv800_hip_rope_table(const uint16_t* cos_t, const uint16_t* sin_t, int64_t P, uint32_t* cs2, void* stream) {
  KV800_REQUIRE(P >= 0, "rope_table: P < 0");
  if (P == 0) return KV800_OK;
  KV800_REQUIRE(cos_t && sin_t && cs2, "rope_table: null pointer");
  const int64_t n = P * 32;
  hipLaunchKernelGGL(rope_table_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, cos_t,
                     sin_t, n, cs2);
  return check_launch("rope_table");
}

int kv800_hip_plan(int64_t B, int64_t nqmax, int64_t* ns, int64_t* spb) {
  KV800_REQUIRE(B >= 0 && nqmax >= 0 && ns && spb, "plan: bad arguments");
  if (nqmax == 0 || B == 0) { *ns = 0; *spb = 1; return KV800_OK; }
  // ~512 workgroups (2 per CU), each taking whole sub-blocks
  const int64_t want = (512 + B - 1) / B;
  const int64_t cap = nqmax;
  int64_t n_s = want < cap ? want : cap;
  if (n_s < 1) n_s = 1;
  const int64_t sp = (nqmax + n_s - 1) / n_s;
  *spb = sp;
  *ns = (nqmax + sp - 1) / sp;
  return KV800_OK;
}

int kv800_hip_decode_quant_sized(const uint16_t* q, const uint8_t* qpool, int64_t qpool_bytes, const int64_t* boff,
                                 int64_t boff_stride, const int32_t* nq, const uint32_t* cs2, int64_t rope_rows,
                                 float* mo, float* lo, float* ao, int64_t B, int64_t ns, int64_t spb, float scale,
                                 void* stream) {
  return launch_quant(q, qpool, qpool_bytes, boff, boff_stride, nq, cs2, rope_rows, mo, lo, ao, B, ns, spb, scale,
                      nullptr, Sched{nullptr, 0, (int)B, 0, 0}, stream);
}

int kv800_hip_decode_quant(const uint16_t* q, const uint8_t* qpool, const int64_t* boff, int64_t boff_stride,
                           const int32_t* nq, const uint32_t* cs2, float* mo, float* lo, float* ao, int64_t B,
                           int64_t ns, int64_t spb, float scale, void* stream) {
  return kv800_hip_decode_quant_sized(q, qpool, INT64_MAX / 2, boff, boff_stride, nq, cs2, INT64_MAX / 2, mo, lo, ao,
                                      B, ns, spb, scale, stream);
}

int kv800_hip_decode_exact_sized(const kv800_paged_t* P, const uint16_t* q, const uint16_t* cos_t,
                                 const uint16_t* sin_t, int64_t rope_rows, int64_t epool_elems, int64_t sink_elems,
                                 float* mo, float* lo, float* ao, int64_t B, int64_t ns, float scale, void* stream) {
  return launch_exact(P, q, cos_t, sin_t, rope_rows, epool_elems, sink_elems, mo, lo, ao, B, ns, scale, nullptr,
                      4, stream);
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
  return launch_merge(mo, lo, ao, (int)ns, Sched{nullptr, 0, (int)B, 0, 0}, B, out, stream, merge_hpw(ns + 1));
}

int64_t kv800_hip_decode_workspace(int64_t B, int64_t ns, int64_t rope_rows) {
  const int64_t S = ns + 1;
  return align256(B * S * 16 * 4) * 2 + align256(B * S * 16 * 128 * 4) + align256(rope_rows * 32 * 4);
}

// Workgroups of decode_quant_kernel resident at once on the current device (its CUs x the kernel's workgroups per
// CU), cached per device; 512 (MI355X: 256 CUs x 2) when the device cannot be queried.
static int64_t resident_groups() {
  static std::mutex mu;
  static int64_t cache[64] = {0};
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    (void)hipGetLastError();
    return 512;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (cache[dev] == 0) {
    int cu = 0, per = 0;
    if (hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, reinterpret_cast<const void*>(decode_quant_kernel), 256, 0) !=
            hipSuccess ||
        cu <= 0 || per <= 0) {
      (void)hipGetLastError();
      cache[dev] = 512;
    } else {
      cache[dev] = (int64_t)cu * per;
    }
  }
  return cache[dev];
}

int64_t kv800_hip_decode_workspace_balanced(int64_t B, int64_t groups, int64_t rope_rows) {
  const int64_t S = 2 * B + groups;
  return align256(S * 16 * 4) * 2 + align256(S * 16 * 128 * 4) + align256((B + 2) * 4) + align256(rope_rows * 32 * 4);
}

int kv800_hip_plan_balanced(int64_t B, int64_t nqmax, int64_t* groups) {
  KV800_REQUIRE(B >= 0 && nqmax >= 0 && groups, "plan_balanced: bad arguments");
  // about BAL_CHUNK sub-blocks per workgroup at the batch's largest size T = B * nqmax (ragged batches hold fewer
  // sub-blocks, and each workgroup then takes proportionally fewer), or 1 while T fills at most half a round of
  // resident workgroups and 2 while T / 2 fills at most one; beyond one round, whole rounds, at most BAL_ROUNDS (one:
  // longer spans in a single round measured faster than two or three rounds of shorter ones at 256-400 rows of up to
  // 32K tokens). Small batches are latency chains: at 32K tokens per row, B = 1 / 2 / 4 / 8 rows take
  // 19.2 / 23.0 / 30.0 / 34.9 us at 1 sub-block per workgroup, 23.2 / 23.2 / 25.7 / 35.0 at 2, 32.4 / 32.8 / 32.8 /
  // 34.6 at 4 (89-91 us at 16); from 16 rows on one round holds 4 or more per workgroup.
  const int64_t T = B * nqmax, res = resident_groups();
  const int64_t want = T <= res / 2 ? T : (T + 1) / 2 <= res ? (T + 1) / 2 : (T + BAL_CHUNK - 1) / BAL_CHUNK;
  *groups = want < 1 ? 1 : want <= res ? want : min((want + res - 1) / res, BAL_ROUNDS) * res;
  return KV800_OK;
}

int kv800_hip_decode_sized(const kv800_paged_t* P, const uint16_t* q, int64_t B, const uint16_t* cos_t,
                           const uint16_t* sin_t, int64_t rope_rows, const uint32_t* cs2, int64_t qpool_bytes,
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
    const int nw = 4 * B <= resident_groups() ? 4 : 1;
    return launch_exact(P, q, cos_t, sin_t, rope_rows, epool_elems, sink_elems, mo, lo, ao, B, 0, scale, out, nw,
                        stream);
  }
  // spb > 0: fixed (row, split) grid of spb sub-blocks per split; spb == 0: balanced schedule with the library's group
  // count; spb < 0: balanced schedule with -spb groups
  Sched S{nullptr, 0, (int)B, (int)nqmax, 0};
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
    S.res = (int)resident_groups();
    ns = 1;
    sp = nqmax;
    slots = 2 * B + G;
  }
  const int64_t need = S.groups ? kv800_hip_decode_workspace_balanced(B, S.groups, cs2 ? 0 : rows)
                                : kv800_hip_decode_workspace(B, ns, cs2 ? 0 : rows);
  KV800_REQUIRE(workspace_bytes >= need, "decode: workspace of %lld bytes, need %lld", (long long)workspace_bytes,
                (long long)need);
  float* mo = (float*)ws;
  float* lo = (float*)(ws + align256(slots * 16 * 4));
  float* ao = (float*)(ws + 2 * align256(slots * 16 * 4));
  char* tail = ws + 2 * align256(slots * 16 * 4) + align256(slots * 16 * 128 * 4);
  if (S.groups) {
    S.pre = (int32_t*)tail;
    tail += align256((B + 2) * 4);
  }
  uint32_t* cst = (uint32_t*)tail;
  if (!cs2) {
    if ((rc = kv800_hip_rope_table(cos_t, sin_t, rows, cst, stream)) != KV800_OK) return rc;
    cs2 = cst;
  }
  // quantized work and the exact tail in one grid, then the merge
  ExactArgs X{};
  X.P = *P; X.cos_t = cos_t; X.sin_t = sin_t; X.rope_rows = rope_rows; X.epool_elems = epool_elems;
  X.sink_elems = sink_elems; X.nexact = (int)(B * 4);
  X.xs0 = S.groups ? B + S.groups : ns;
  X.xst = S.groups ? 1 : ns + 1;
  if ((rc = check_exact(P, q, cos_t, sin_t, epool_elems, mo, lo, ao, B, ns, out, &X.nsink)) != KV800_OK) return rc;
  if ((rc = launch_quant(q, P->qpool, qpool_bytes, P->boff, P->boff_stride, P->NQ, cs2, rows, mo, lo, ao, B, ns, sp,
                         scale, &X, S, stream)) != KV800_OK)
    return rc;
  KV800_REQUIRE(((uintptr_t)ao % 16) == 0 && ((uintptr_t)out % 16) == 0, "decode_merge: ao / out must be 16-byte aligned");
  return launch_merge(mo, lo, ao, (int)ns, S, B, out, stream,
                      merge_hpw(S.groups ? (S.groups + B - 1) / B + 1 : ns + 1));   // partials per row, about
}

int kv800_hip_decode(const kv800_paged_t* P, const uint16_t* q, int64_t B, const uint16_t* cos_t,
                     const uint16_t* sin_t, const uint32_t* cs2, uint16_t* out, void* workspace,
                     int64_t workspace_bytes, int64_t spb, void* stream) {
  const int64_t rows = P ? (P->win ? 0 : P->nqmax) * BLK : 0;
  return kv800_hip_decode_sized(P, q, B, cos_t, sin_t, rows > 0 ? rows : INT64_MAX / 2, cs2, INT64_MAX / 2,
                                INT64_MAX / 2, INT64_MAX / 2, out, workspace, workspace_bytes, spb, stream);
}

}  // extern "C"

// ---------------------------------------------------------------- allocation-free decode
// Scratch of kv800_hip_decode_noalloc: the decode's split partials (m, l, acc), the balanced schedule's row offsets and,
// without a prebuilt pair table, the rope pair table live here instead of in a caller workspace. Every device the
// library runs on holds its own copy until the process ends. In host code `scratch` names a host-side stand-in: its
// device address is resolved per device with hipGetSymbolAddress and only that address is handed to the kernels.
static constexpr int64_t KV800_SCRATCH_BYTES = 32ll << 20;
static __device__ __align__(256) char scratch[KV800_SCRATCH_BYTES];

namespace {
constexpr int KV800_MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[KV800_MAX_DEVICES];   // device address of `scratch` on each device, resolved on its first call
}  // namespace

extern "C" int kv800_hip_decode_noalloc(const kv800_paged_t* P, const uint16_t* q, int64_t B, const uint16_t* cos_t,
                                        const uint16_t* sin_t, int64_t rope_rows, const uint32_t* cs2,
                                        int64_t qpool_bytes, int64_t epool_elems, int64_t sink_elems, uint16_t* out,
                                        int64_t spb, void* stream) {
  KV800_REQUIRE(P && B >= 0, "decode_noalloc: bad arguments");
  if (B == 0) return KV800_OK;
  // bytes this call's schedule needs (the same carving as kv800_hip_decode's workspace)
  const int64_t nqmax = P->win ? 0 : P->nqmax;
  KV800_REQUIRE(nqmax >= 0, "decode_noalloc: nqmax < 0");
  int64_t need;
  if (!nqmax) {
    need = kv800_hip_decode_workspace(B, 0, 0);
  } else if (spb > 0) {
    need = kv800_hip_decode_workspace(B, (nqmax + spb - 1) / spb, cs2 ? 0 : nqmax * BLK);
  } else {
    int64_t G = -spb;
    int rc;
    if (!G && (rc = kv800_hip_plan_balanced(B, nqmax, &G)) != KV800_OK) return rc;
    need = kv800_hip_decode_workspace_balanced(B, G, cs2 ? 0 : nqmax * BLK);
  }
  KV800_REQUIRE(need <= KV800_SCRATCH_BYTES,
                "decode_noalloc: this call needs %lld bytes of scratch, the per-device scratch holds %lld (pass a "
                "prebuilt cs2 table, or decode fewer rows / groups per call)",
                (long long)need, (long long)KV800_SCRATCH_BYTES);
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= KV800_MAX_DEVICES) {
    kv800::set_error("decode_noalloc: hipGetDevice: %s (device %d)", hipGetErrorString(e), dev);
    return KV800_EHIP;
  }
  if (stream) {   // the scratch address is the current device's: the stream must run there
    int sdev = -1;
    e = hipStreamGetDevice((hipStream_t)stream, &sdev);
    KV800_REQUIRE(e == hipSuccess && sdev == dev, "decode_noalloc: the stream is not on the current device (%d vs %d)",
                  sdev, dev);
  }
  void* ws = nullptr;
  {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
      void* p = nullptr;
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess || !p) {
        kv800::set_error("decode_noalloc: hipGetSymbolAddress of the scratch on device %d: %s", dev,
                         hipGetErrorString(e));
        return KV800_EHIP;
      }
      g_scratch_ptr[dev] = p;
    }
    ws = g_scratch_ptr[dev];
  }
  return kv800_hip_decode_sized(P, q, B, cos_t, sin_t, rope_rows, cs2, qpool_bytes, epool_elems, sink_elems, out, ws,
                                KV800_SCRATCH_BYTES, spb, stream);
}
