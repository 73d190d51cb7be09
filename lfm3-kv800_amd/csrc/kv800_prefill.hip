// kv800_prefill.hip -- prefill / extend attention of the 800h layers on gfx950 (the attention of vllm_attn.py:168-211
// and 351-402 for rows that bring more than one new token).
//
//   rope_rows_kernel  keys (S, 4, 128) bf16 rotated at their positions with the (P, 32) bf16 tables of the 32 rotating
//                     frequencies, as vllm_attn.py:160-163 does over its 128-wide tables (cos32 | 1 | cos32 | 1,
//                     sin32 | 0 | sin32 | 0): every element is k * c + rot(k) * s in fp32 (both products exact), then
//                     rounded to bf16 -- the same value, bit for bit, dims without a frequency included.
//   prefill_kernel    flash attention of R ragged rows. Row i has queries q[qsl[i], qsl[i+1]) (T, 16 heads, 128) at the
//                     consecutive positions qpos0[i], qpos0[i] + 1, ... and keys / values K, V[ksl[i], ksl[i+1])
//                     (S, 4 KV heads, 128) at the ascending positions kp (kp = null: key j of a row at position
//                     j, as quantized layers assemble them); query head h reads KV head h / 4. A key is
//                     kept when kp <= query position and, with window > 0, kp > query position - window or kp < nsink
//                     (the quantized, window + sinks and sliding masks of vllm_attn.py:168-184). fp32 scores and
//                     online softmax, bf16 probabilities for the P.V product, fp32 accumulation, bf16 out.
//
// prefill_kernel, one workgroup = 32 consecutive queries of one row and one KV head g; wave w computes query head
// 4 g + w for its 32 queries as two 16-query blocks, so the 4 waves share each 64-key tile staged in LDS. Per wave and
// tile, with v_mfma_f32_16x16x32_bf16 (lane l: D column l % 16, D rows 4 (l / 16) + 0..3; A row l % 16 and B column
// l % 16 over k = 8 (l / 16) + 0..7):
//   S^T = K . Q^T   (keys x queries): A = K rows from LDS, B = the wave's queries held in registers;
//   O^T += V^T . P^T (dims x queries): A = V^T read from the V rows by ds_read_b64_tr_b16, B = the lane's own
//                    probabilities;
// each A operand feeds both query blocks. Both results keep one query per lane column (l % 16), so the softmax
// statistics of a query live in the four lanes l % 16 and are combined with two cross-lane steps, and the O rescale
// (lazy: only when a query's running max grows by more than PLAZY) needs no data movement. P^T's B operand is the
// lane's 8 probabilities of keys 4 G + i and 16 + 4 G + i (G = l / 16) of each 32-key half, the key order in which
// the transposed reads deliver V^T. The tiles are double-buffered in LDS and loaded straight into it (buffer loads
// with the lds modifier, through a buffer resource whose reads past the row's keys return zeros; the next tile's
// loads are in flight while the current one is multiplied, one barrier per tile), and a tile whose keys are all in
// range and precede the workgroup's first query is not masked.
// Key tiles outside [first key a query of the workgroup can see, last key not in its future] are skipped: for window
// layers only the sink keys and the keys of the window are read.
// The grid is one workgroup per (KV head, 32-query tile), numbered so that each XCD runs whole (KV head, row) runs of
// tiles: the 64 workgroups of a 2048-query chunk walk the same key tiles together through one L2.
#include "kv800_common.h"
#include "../../include/kv800_hip.h"

namespace kv800 {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef short b8 __attribute__((ext_vector_type(8)));
typedef uint32_t u4v __attribute__((ext_vector_type(4)));
typedef uint32_t u2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
typedef short s4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s4 lds_s4;

__device__ __forceinline__ f4 mfma_bf(u4v a, u4v b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(b8, a), __builtin_bit_cast(b8, b), c, 0, 0, 0);
}

// ---------------------------------------------------------------- RoPE of key rows
// one thread per (row, head, d < 64): the pair (d, d + 64)
__global__ void __launch_bounds__(256)
rope_rows_kernel(const uint16_t* __restrict__ k, const int64_t* __restrict__ pos, int64_t S,
                 const uint16_t* __restrict__ cos_t, const uint16_t* __restrict__ sin_t, int64_t P,
                 uint16_t* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= S * 256) return;
  const int64_t row = i >> 8;
  const int hd = (int)(i & 255), h = hd >> 6, d = hd & 63;
  int64_t p = pos[row];
  p = p < 0 ? 0 : (p >= P ? P - 1 : p);            // positions past the table are a caller error; stay in bounds
  const float c = d < 32 ? bf2f(cos_t[p * 32 + d]) : 1.0f;
  const float s = d < 32 ? bf2f(sin_t[p * 32 + d]) : 0.0f;
  const int64_t base = (row * 4 + h) * 128;
  const float lo = bf2f(k[base + d]), hi = bf2f(k[base + d + 64]);
  out[base + d] = (uint16_t)f2bf(lo * c + (-hi) * s);
  out[base + d + 64] = (uint16_t)f2bf(hi * c + lo * s);
}

// two floats -> packed bf16, round to nearest even (one v_cvt_pk_bf16_f32; equal to f2bf for finite values)
__device__ __forceinline__ uint32_t bfpk(float a, float b) {
  const bf2 v = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, v);
}

// ---------------------------------------------------------------- flash attention of ragged rows
// A workgroup of 4 waves takes PQ = 32 consecutive queries of one row (one interface tile) and one KV head g; wave w
// computes query head 4 g + w for its 32 queries as two column blocks of 16. Every workgroup of the grid has work (a
// grid whose idle workgroups sat at every other index put all the work on half the XCDs under round-robin dispatch),
// and the workgroups of one (KV head, row) run on one XCD, in order, so the row's key tiles are read once into that
// XCD's L2 for its 64 query tiles. Keys come in tiles of 64, loaded into LDS as K and V rows by LDS-direct loads (no
// register staging) and double-buffered: the next tile's loads are in flight while the current one is multiplied, one
// barrier per tile. Per
// wave and tile on f32_16x16x32_bf16: S^T = K . Q^T (keys x queries: 4 key blocks x 2 query blocks x 4 k-steps, every
// K operand read once for both query blocks) and O^T += V^T . P^T (8 dim blocks x 2 query blocks x 2 k-steps; the
// V^T operand is read from the V rows by two ds_read_b64_tr_b16, in the key order of the lane's own probabilities,
// once for both query blocks), so both results keep one query per lane column: a query's softmax statistics live in
// four lanes (two cross-lane steps) and the O rescale moves no data. A tile whose keys all precede the workgroup's
// first query (and are all in range) needs no mask: in a chunk over a long history, nearly every tile.
constexpr int PQ = 32;      // queries per workgroup = per interface tile (tile_off counts these)
constexpr int PPART = 132;  // floats per key-split partial of (query, head): 128 dims of o, m, l, 2 of padding
constexpr int PMAXSPLIT = 256;
constexpr int PK = 64;      // keys per LDS tile

// a tile as staged by LDS-direct loads: K and V rows of 256 bytes, unpadded, their 16-byte pieces permuted within
// each row so that the operand reads spread over the banks: piece p of key row j at piece p ^ (j & 15) (K: 16 rows
// read at one piece per instruction) and p ^ 2 (j & 7) (V: 32-byte pairs of pieces, 4 rows per 16 lanes)
struct alignas(16) PTile {
  uint16_t k[PK * 128];
  uint16_t v[PK * 128];
  int32_t kp[PK];
};
__device__ __forceinline__ int kswz(int j, int p) { return p ^ (j & 15); }
__device__ __forceinline__ int vswz(int j, int p) { return p ^ (2 * (j & 7)); }
constexpr float PLAZY = 8.f;   // log2 units a query's running max may lag its scores (p <= 2^8 in bf16)
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr int RSRC_WORD3 = 0x00020000;   // raw (untyped, unswizzled) buffer access on gfx9-family parts

// first index in [0, n) with a[index] > x (a ascending; a = null: a[i] = i), n if none: a 64-way search by the whole
// wave (lane l probes lo + l step; the count of probes <= x, from a ballot, narrows [lo, hi) 64-fold), so n = 16K
// entries take three dependent loads instead of fourteen. All 64 lanes must be active; the result is the same in every lane.
__device__ __forceinline__ int64_t upper(const int32_t* a, int64_t n, int64_t x) {
  if (!a) return x < 0 ? 0 : (x + 1 < n ? x + 1 : n);   // positions = indices 0 .. n - 1
  const int lane = threadIdx.x & 63;
  int64_t lo = 0, hi = n;   // the answer lies in [lo, hi]
  while (hi > lo) {
    const int64_t step = (hi - lo + 63) / 64;
    const int64_t idx = lo + lane * step;
    const bool le = idx < hi && (int64_t)a[idx < hi ? idx : lo] <= x;
    const int c = __popcll(__ballot(le));   // probes 0 .. c - 1 are <= x (a ascending)
    if (c == 0) return lo;
    const int64_t last = lo + (int64_t)(c - 1) * step;   // a[last] <= x
    const int64_t next = lo + (int64_t)c * step;          // the first probe > x, or past hi
    lo = last + 1;
    hi = next < hi ? next : hi;
    if (step == 1) return lo;
  }
  return lo;
}

// max / sum over the lanes l, l ^ 16, l ^ 32, l ^ 48 without an LDS round trip: v_permlane16_swap and
// v_permlane32_swap on two copies of x leave both 16-lane (32-lane) halves in every lane of a pair. All 64 lanes must
// be active.
__device__ __forceinline__ float max4rows(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum4rows(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__global__ void __launch_bounds__(256, 2)
prefill_kernel(const uint16_t* __restrict__ q, const int64_t* __restrict__ qsl, const int64_t* __restrict__ qpos0,
               const uint16_t* __restrict__ K, const uint16_t* __restrict__ V, const int32_t* __restrict__ kp,
               const int64_t* __restrict__ ksl, const int64_t* __restrict__ tile_off, int64_t R, int64_t window,
               int64_t nsink, float scale_log2, uint16_t* __restrict__ out, int splits, float* __restrict__ part) {
  __shared__ PTile tA, tB;   // two buffers as two objects: a read of one is not held for the other's loads
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  // workgroup b runs on XCD b % 8 (round-robin dispatch): XCD x takes the contiguous run L = [x per + min(x, rem),
  // ...) of the (g, t, split) order (split fastest, then t), so the workgroups sharing a row's keys of one KV head
  // share that XCD's L2
  const int nb = (int)gridDim.x, xcd = (int)blockIdx.x & 7, per = nb >> 3, rem = nb & 7;
  const int L = xcd * per + min(xcd, rem) + ((int)blockIdx.x >> 3);
  const int ntl = nb / (4 * splits);
  const int g = L / (ntl * splits), h = 4 * g + w;
  const int lr = L - g * ntl * splits, sp = lr % splits;
  const int col = lane & 15, G = lane >> 4;
  // ---- row of this tile: last i with tile_off[i] <= t
  const int64_t t = lr / splits;
  int64_t lo = 0, hi = R;
  while (hi - lo > 1) {
    const int64_t mid = (lo + hi) >> 1;
    if (tile_off[mid] <= t) lo = mid; else hi = mid;
  }
  const int64_t row = lo, lt = t - tile_off[row];
  const int64_t q0 = qsl[row] + lt * PQ;
  const int nq = (int)min((int64_t)PQ, qsl[row + 1] - q0);
  const int64_t p0 = qpos0[row] + (q0 - qsl[row]);
  const int64_t ks = ksl[row], S = ksl[row + 1] - ks;
  const int32_t* kpr = kp ? kp + ks : nullptr;   // null: key j of the row at position j

  // ---- key ranges: [0, sink_end) and [kbeg, kend)
  const int64_t kend = upper(kpr, S, p0 + nq - 1);
  int64_t kbeg = 0, sink_end = 0;
  if (window > 0) {
    kbeg = upper(kpr, S, p0 - window);
    sink_end = min(upper(kpr, S, nsink - 1), kbeg);
    if (kbeg <= sink_end) { kbeg = 0; sink_end = 0; }
  }
  const int n0 = (int)((sink_end + PK - 1) / PK), nt = n0 + (int)((kend - kbeg + PK - 1) / PK);
  // key split sp of `splits` takes tiles [i0, i1) of the nt (all of them without a split)
  const int per_sp = (nt + splits - 1) / splits, i0 = min(nt, sp * per_sp), i1 = min(nt, i0 + per_sp);
  // ---- the wave's queries as the B operands of S^T = K . Q^T (query block cq, 4 k-steps of 32 dims)
  bool qok[2];
  int qpos[2];
  u4v qb[2][4];
#pragma unroll
  for (int cq = 0; cq < 2; ++cq) {
    qok[cq] = 16 * cq + col < nq;
    qpos[cq] = (int)(p0 + 16 * cq + col);
#pragma unroll
    for (int s = 0; s < 4; ++s)
      qb[cq][s] = qok[cq] ? *reinterpret_cast<const u4v*>(q + ((q0 + 16 * cq + col) * 16 + h) * 128 + 32 * s + 8 * G)
                          : u4v{0, 0, 0, 0};
  }
  f4 o[2][8];
#pragma unroll
  for (int cq = 0; cq < 2; ++cq)
#pragma unroll
    for (int j = 0; j < 8; ++j) o[cq][j] = f4{0.f, 0.f, 0.f, 0.f};
  float m[2] = {-1e30f, -1e30f}, lsum[2] = {0.f, 0.f};

  // ---- tile i's keys [k0, k0 + 64) clipped to r1: from the sink range, then from the main range
  auto range_of = [&](int i, int64_t& k0, int64_t& r1) {
    if (i < n0) { k0 = (int64_t)i * PK; r1 = sink_end; }
    else { k0 = kbeg + (int64_t)(i - n0) * PK; r1 = kend; }
  };
  int32_t skp = 0;             // the next tile's key positions (lanes < 64), stored with the tile's last reads done
  auto fetch = [&](int i, PTile& T) {
    int64_t k0, r1;
    range_of(i, k0, r1);
    // the tile's K and V rows as buffers (base and size in SGPRs): a read past the row's S keys returns zeros, so every
    // staging load is issued unconditionally (keys past a range's end carry the position 0x7FFFFFFF and are masked)
    const int nbytes = (int)(min(S - k0, (int64_t)PK) * 1024);
    const rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(K + (ks + k0) * 512), (short)0, nbytes,
                                                        RSRC_WORD3);
    const rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(V + (ks + k0) * 512), (short)0, nbytes,
                                                        RSRC_WORD3);
    // LDS-direct: instruction r of wave w fills key rows 16 r + 4 w .. + 3 (1 KB, lane l at byte 16 l); lane l
    // fetches the global piece that belongs in its slot
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int j = 16 * r + 4 * w + (lane >> 4), qs = lane & 15;
      const int base = j * 1024 + g * 256;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (__attribute__((address_space(3))) void*)&T.k[(16 * r + 4 * w) * 128],
                                               16, base + 16 * kswz(j, qs), 0, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (__attribute__((address_space(3))) void*)&T.v[(16 * r + 4 * w) * 128],
                                               16, base + 16 * vswz(j, qs), 0, 0, 0);
    }
    if (tid < PK) skp = (k0 + tid < r1) ? (kpr ? kpr[k0 + tid] : (int32_t)(k0 + tid)) : 0x7FFFFFFF;
    // the loads write T behind the compiler's view of the buffer: its address escapes here
    asm volatile("" ::"s"((uint32_t)(uintptr_t)&T) : "memory");
  };

  if (i0 < i1) {
    fetch(i0, tA);
    if (tid < PK) tA.kp[tid] = skp;
  }
  __syncthreads();
  auto step = [&](int i, const PTile& T, PTile& Nx) {
    if (i + 1 < i1) fetch(i + 1, Nx);
    // ---- S^T = K . Q^T: 4 blocks of 16 keys x 2 blocks of 16 queries
    f4 sc[2][4];
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      f4 a0 = {0.f, 0.f, 0.f, 0.f}, a1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const u4v a = *reinterpret_cast<const u4v*>(&T.k[(nb * 16 + col) * 128 + 8 * kswz(col, 4 * s + G)]);
        a0 = mfma_bf(a, qb[0][s], a0);
        a1 = mfma_bf(a, qb[1][s], a1);
      }
      sc[0][nb] = a0;
      sc[1][nb] = a1;
    }
    // ---- mask, scale, online softmax per query block (the lane's 16 keys: nb * 16 + 4 G + i). No mask when every key
    // of the tile is in range and precedes the workgroup's first query (quantized layers: no window).
    int64_t tk0, tr1;
    range_of(i, tk0, tr1);
    const bool full = window <= 0 && tk0 + PK <= tr1 && (int64_t)T.kp[PK - 1] <= p0;
    uint32_t pb[2][4][2];   // bf16 probabilities, packed in key pairs
#pragma unroll
    for (int cq = 0; cq < 2; ++cq) {
      if (!full) {
        const int wlo = window > 0 ? (int)max((int64_t)qpos[cq] - window, (int64_t)INT32_MIN) : INT32_MIN;
        const int ns = window > 0 ? (int)nsink : 0;
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) {
#pragma unroll
          for (int i2 = 0; i2 < 4; ++i2) {
            const int kpos = T.kp[nb * 16 + 4 * G + i2];
            const bool keep = qok[cq] & (kpos <= qpos[cq]) & ((kpos > wlo) | (kpos < ns));
            sc[cq][nb][i2] = keep ? sc[cq][nb][i2] : -INFINITY;
          }
        }
      }
      float tmax = -INFINITY;
#pragma unroll
      for (int nb = 0; nb < 4; ++nb)
        tmax = fmaxf(tmax, fmaxf(fmaxf(sc[cq][nb][0], sc[cq][nb][1]), fmaxf(sc[cq][nb][2], sc[cq][nb][3])));
      tmax = max4rows(tmax) * scale_log2;   // scale > 0: the max of the scaled scores
      if (__any(tmax > m[cq] + PLAZY)) {   // rescale only when a query's max outgrows its state (wave-uniform)
        const float mnew = fmaxf(m[cq], tmax);
        const float alpha = __builtin_amdgcn_exp2f(m[cq] - mnew);
        m[cq] = mnew;
        lsum[cq] *= alpha;
#pragma unroll
        for (int j = 0; j < 8; ++j) o[cq][j] *= alpha;
      }
      const float mnew = m[cq];
      float psum = 0.f;
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) {
        float p[4];
#pragma unroll
        for (int i2 = 0; i2 < 4; ++i2) {
          p[i2] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[cq][nb][i2], scale_log2, -mnew));   // masked: -inf -> 0
          psum += p[i2];
        }
        pb[cq][nb][0] = bfpk(p[0], p[1]);
        pb[cq][nb][1] = bfpk(p[2], p[3]);
      }
      lsum[cq] += psum;
    }
    // ---- O^T += V^T . P^T: 2 halves of 32 keys x 8 blocks of 16 dims x 2 query blocks. A = V^T (row = dim; K = the
    // half's keys 4 G .. 4 G + 3 and 16 + 4 G .. + 3, whose probabilities the lane holds) by two transposed reads
    const int vrow = 4 * G + (col >> 2);
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const u4v b0 = {pb[0][2 * hh][0], pb[0][2 * hh][1], pb[0][2 * hh + 1][0], pb[0][2 * hh + 1][1]};
      const u4v b1 = {pb[1][2 * hh][0], pb[1][2 * hh][1], pb[1][2 * hh + 1][0], pb[1][2 * hh + 1][1]};
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int vo = 8 * vswz(vrow, 2 * j + ((col >> 1) & 1)) + 4 * (col & 1);   // rows vrow and vrow + 16 alike
        const s4 t0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_s4*)const_cast<uint16_t*>(&T.v[(32 * hh + vrow) * 128 + vo]));
        const s4 t1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_s4*)const_cast<uint16_t*>(&T.v[(32 * hh + vrow + 16) * 128 + vo]));
        const u4v a = {__builtin_bit_cast(uint32_t, __builtin_shufflevector(t0, t0, 0, 1)),
                       __builtin_bit_cast(uint32_t, __builtin_shufflevector(t0, t0, 2, 3)),
                       __builtin_bit_cast(uint32_t, __builtin_shufflevector(t1, t1, 0, 1)),
                       __builtin_bit_cast(uint32_t, __builtin_shufflevector(t1, t1, 2, 3))};
        o[0][j] = mfma_bf(a, b0, o[0][j]);
        o[1][j] = mfma_bf(a, b1, o[1][j]);
      }
    }
    // the next tile's positions into its buffer, whose last reads (tile i - 1) ended at the previous barrier; the
    // barrier waits for the tile's LDS-direct loads
    if (i + 1 < i1 && tid < PK) Nx.kp[tid] = skp;
    __syncthreads();
  };
  for (int i = i0; i < i1; i += 2) {
    step(i, tA, tB);
    if (i + 1 < i1) step(i + 1, tB, tA);
  }
  // ---- normalise and write: lane holds dims 16 j + 4 G + 0..3 of query 16 cq + col. With a key split, the
  // unnormalised partial (o, m, l) of (query, head, split) instead: PPART floats, o relative to 2^m
#pragma unroll
  for (int cq = 0; cq < 2; ++cq) {
    const float l = sum4rows(lsum[cq]);
    if (!qok[cq]) continue;
    if (part) {
      float* pp = part + (((q0 + 16 * cq + col) * 16 + h) * splits + sp) * PPART;
#pragma unroll
      for (int j = 0; j < 8; ++j) *reinterpret_cast<f4*>(pp + 16 * j + 4 * G) = o[cq][j];
      if (G == 0) { pp[128] = m[cq]; pp[129] = l; }
      continue;
    }
    const float inv = l > 0.f ? 1.0f / l : 0.f;
    uint16_t* dst = out + ((q0 + 16 * cq + col) * 16 + h) * 128 + 4 * G;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const u2v v2 = {bfpk(o[cq][j][0] * inv, o[cq][j][1] * inv), bfpk(o[cq][j][2] * inv, o[cq][j][3] * inv)};
      *reinterpret_cast<u2v*>(dst + 16 * j) = v2;
    }
  }
}

// ---------------------------------------------------------------- key-split merge
// One wave per (query, head). Lanes read the splits' (m, l) in parallel: M = max m_s and L = sum l_s 2^(m_s - M) by
// wave reductions; then lane holds dims 2 lane, 2 lane + 1 and sums o_s 2^(m_s - M) over the splits, eight loads in
// flight; out = bf16(O / L) (a split without keys has l = 0 and o = 0).
__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int k = 1; k < 64; k <<= 1) x = fmaxf(x, __shfl_xor(x, k, 64));
  return x;
}
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int k = 1; k < 64; k <<= 1) x += __shfl_xor(x, k, 64);
  return x;
}
__global__ void __launch_bounds__(256)
prefill_merge_kernel(const float* __restrict__ part, int64_t pairs, int splits, uint16_t* __restrict__ out) {
  const int64_t pr = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (pr >= pairs) return;   // uniform over the wave
  const int lane = threadIdx.x & 63;
  const float* pp = part + pr * splits * PPART;
  float M = -INFINITY;
  for (int s = lane; s < splits; s += 64) M = fmaxf(M, pp[s * PPART + 128]);
  M = wave_max(M);
  float Ls = 0.f;
  for (int s = lane; s < splits; s += 64) Ls += __builtin_amdgcn_exp2f(pp[s * PPART + 128] - M) * pp[s * PPART + 129];
  Ls = wave_sum(Ls);
  float o0 = 0.f, o1 = 0.f;
  for (int s0 = 0; s0 < splits; s0 += 8) {
    float mv[8];
    float2 av[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int sk = s0 + k < splits ? s0 + k : s0;   // past the last split: a repeat, weighted 0 below
      mv[k] = s0 + k < splits ? pp[sk * PPART + 128] : -INFINITY;
      av[k] = *reinterpret_cast<const float2*>(pp + sk * PPART + 2 * lane);
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float wgt = __builtin_amdgcn_exp2f(mv[k] - M);
      o0 += wgt * av[k].x;
      o1 += wgt * av[k].y;
    }
  }
  const float inv = Ls > 0.f ? 1.0f / Ls : 0.f;
  *reinterpret_cast<uint32_t*>(out + pr * 128 + 2 * lane) = bfpk(o0 * inv, o1 * inv);
}

}  // namespace
}  // namespace kv800

using namespace kv800;

extern "C" {

int kv800_hip_rope_rows(const uint16_t* k, const int64_t* pos, int64_t S, const uint16_t* cos_t,
                        const uint16_t* sin_t, int64_t rope_rows, uint16_t* out, void* stream) {
  KV800_REQUIRE(S >= 0, "rope_rows: S < 0");
  if (S == 0) return KV800_OK;
  KV800_REQUIRE(k && pos && cos_t && sin_t && out, "rope_rows: null pointer");
  KV800_REQUIRE(rope_rows > 0, "rope_rows: empty RoPE tables");
  const int64_t n = S * 256;
  hipLaunchKernelGGL(rope_rows_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, k, pos, S,
                     cos_t, sin_t, rope_rows, out);
  return check_launch("rope_rows");
}

int kv800_hip_prefill_split(const uint16_t* q, const int64_t* qsl, const int64_t* qpos0, const uint16_t* K,
                            const uint16_t* V, const int32_t* kp, const int64_t* ksl, const int64_t* tile_off,
                            int64_t R, int64_t ntiles, int64_t T, int64_t window, int64_t nsink, int64_t splits,
                            float* part, int64_t part_floats, uint16_t* out, void* stream) {
  KV800_REQUIRE(R >= 0 && ntiles >= 0 && T >= 0, "prefill: negative R, tile count or query count");
  if (R == 0 || ntiles == 0) return KV800_OK;
  KV800_REQUIRE(q && qsl && qpos0 && K && V && ksl && tile_off && out, "prefill: null pointer");
  KV800_REQUIRE(((uintptr_t)q % 16) == 0 && ((uintptr_t)K % 16) == 0 && ((uintptr_t)V % 16) == 0 &&
                ((uintptr_t)out % 8) == 0, "prefill: q, K, V need 16-byte and out 8-byte alignment");
  KV800_REQUIRE(window >= 0 && nsink >= 0, "prefill: negative window or sink count");
  KV800_REQUIRE(splits >= 1 && splits <= PMAXSPLIT, "prefill: splits must be in [1, %d]", PMAXSPLIT);
  KV800_REQUIRE(ntiles * 4 * splits < (1ll << 31), "prefill: too many query tiles x splits");
  KV800_REQUIRE(ntiles <= (T + PQ - 1) / PQ + R, "prefill: more query tiles than T queries can hold");
  if (splits > 1) {
    KV800_REQUIRE(part && ((uintptr_t)part % 16) == 0, "prefill: a key split needs a 16-byte aligned part buffer");
    KV800_REQUIRE(part_floats >= T * 16 * splits * PPART, "prefill: part holds %lld floats, the split needs %lld",
                  (long long)part_floats, (long long)(T * 16 * splits * PPART));
  }
  const float scale_log2 = 0.088388347648318440f * 1.4426950408889634f;   // 128^-0.5 * log2(e)
  hipLaunchKernelGGL(prefill_kernel, dim3((unsigned)(ntiles * 4 * splits)), dim3(256), 0, (hipStream_t)stream, q, qsl,
                     qpos0, K, V, kp, ksl, tile_off, R, window, nsink, scale_log2, out, (int)splits,
                     splits > 1 ? part : (float*)nullptr);
  int rc = check_launch("prefill");
  if (rc != KV800_OK || splits == 1 || T == 0) return rc;
  const int64_t pairs = T * 16;
  hipLaunchKernelGGL(prefill_merge_kernel, dim3((unsigned)((pairs + 3) / 4)), dim3(256), 0, (hipStream_t)stream, part,
                     pairs, (int)splits, out);
  return check_launch("prefill_merge");
}

int kv800_hip_prefill(const uint16_t* q, const int64_t* qsl, const int64_t* qpos0, const uint16_t* K,
                      const uint16_t* V, const int32_t* kp, const int64_t* ksl, const int64_t* tile_off, int64_t R,
                      int64_t ntiles, int64_t window, int64_t nsink, uint16_t* out, void* stream) {
  KV800_REQUIRE(ntiles < (1ll << 29), "prefill: too many query tiles");
  return kv800_hip_prefill_split(q, qsl, qpos0, K, V, kp, ksl, tile_off, R, ntiles, ntiles * PQ, window, nsink, 1,
                                 nullptr, 0, out, stream);
}

}  // extern "C"
