// kv800_prefill.hip -- prefill / extend attention of the 800h layers on gfx950 (the attention of vllm_attn.py:168-211
// and 351-402 for rows that bring more than one new token).
//
//   rope_rows_kernel  keys (S, 4, 128) bf16 rotated at their positions with the (P, 32) bf16 tables of the 32 rotating
//                     frequencies, as vllm_attn.py:160-163 does over its 128-wide tables (cos32 | 1 | cos32 | 1,
//                     sin32 | 0 | sin32 | 0): every element is k * c + rot(k) * s in fp32 (both products exact), then
//                     rounded to bf16 -- the same value, bit for bit, dims without a frequency included.
//   prefill_kernel    flash attention of R ragged rows. Row i has queries q[qsl[i], qsl[i+1]) (T, 16 heads, 128) at the
//                     consecutive positions qpos0[i], qpos0[i] + 1, ... and keys / values K, V[ksl[i], ksl[i+1])
//                     (S, 4 KV heads, 128) at the ascending positions kp; query head h reads KV head h / 4. A key is
//                     kept when kp <= query position and, with window > 0, kp > query position - window or kp < nsink
//                     (the quantized, window + sinks and sliding masks of vllm_attn.py:168-184). fp32 scores and
//                     online softmax, bf16 probabilities for the P.V product, fp32 accumulation, bf16 out.
//
// prefill_kernel, one workgroup = 16 consecutive queries of one row and one KV head g; wave w computes query head
// 4 g + w, so the 4 waves share each 64-key tile staged in LDS. Per wave and tile, with v_mfma_f32_16x16x32_bf16
// (lane l: D column l % 16, D rows 4 (l / 16) + 0..3; A row l % 16 and B column l % 16 over k = 8 (l / 16) + 0..7):
//   S^T = K . Q^T   (keys x queries): A = K rows from LDS, B = the wave's 16 queries held in registers,
//   O^T += V^T . P^T (dims x queries): A = V^T rows from LDS, B = the lane's own probabilities.
// Both results keep one query per lane column (l % 16), so the softmax statistics of a query live in the four lanes
// l % 16 and are combined with two cross-lane steps, and the O rescale needs no data movement. P^T's B operand is the
// lane's 8 probabilities of keys 4 G + i and 16 + 4 G + i (G = l / 16) of each 32-key half; V^T is written to LDS with
// its keys in that order (position 8 G + i and 8 G + 4 + i) so that its A operand is one 16-byte read.
// Key tiles outside [first key a query of the tile can see, last key not in its future] are skipped: for window
// layers only the sink keys and the keys of the window are read.
#include "kv800_common.h"
#include "../../include/kv800_hip.h"

namespace kv800 {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef short b8 __attribute__((ext_vector_type(8)));
typedef uint32_t u4v __attribute__((ext_vector_type(4)));
typedef uint32_t u2v __attribute__((ext_vector_type(2)));

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

// ---------------------------------------------------------------- flash attention of ragged rows
constexpr int PQ = 16;      // queries per workgroup
constexpr int PK = 64;      // keys per LDS tile
constexpr int KROW = 136;   // K tile row stride (elements): 272 B, rows 4 banks apart for the 16-byte A reads
constexpr int VROW = 72;    // V^T tile row stride (elements): 144 B, likewise

struct PLds {
  uint16_t k[PK * KROW];
  uint16_t vt[128 * VROW];
  int32_t kp[PK];
};

// first index in [0, n) with a[index] > x (a ascending)
__device__ __forceinline__ int64_t upper(const int32_t* a, int64_t n, int64_t x) {
  int64_t lo = 0, hi = n;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if ((int64_t)a[mid] <= x) lo = mid + 1; else hi = mid;
  }
  return lo;
}

// LDS position of key k (0..63) in the V^T tile: within each 32-key half, keys 4 G + i -> 8 G + i, 16 + 4 G + i ->
// 8 G + 4 + i
__device__ __forceinline__ int vt_pos(int k) {
  const int h = k & 31;
  return (k & 32) + 8 * ((h & 15) >> 2) + 4 * (h >> 4) + (h & 3);
}

__device__ __forceinline__ float xmax(float v, int mask) {
  return fmaxf(v, __shfl_xor(v, mask, 64));
}

__global__ void __launch_bounds__(256)
prefill_kernel(const uint16_t* __restrict__ q, const int64_t* __restrict__ qsl, const int64_t* __restrict__ qpos0,
               const uint16_t* __restrict__ K, const uint16_t* __restrict__ V, const int32_t* __restrict__ kp,
               const int64_t* __restrict__ ksl, const int64_t* __restrict__ tile_off, int64_t R, int64_t window,
               int64_t nsink, float scale_log2, uint16_t* __restrict__ out) {
  __shared__ PLds lds;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = blockIdx.y, h = 4 * g + w;
  const int col = lane & 15, G = lane >> 4;
  // ---- row of this tile: last i with tile_off[i] <= t
  const int64_t t = blockIdx.x;
  int64_t lo = 0, hi = R;
  while (hi - lo > 1) {
    const int64_t mid = (lo + hi) >> 1;
    if (tile_off[mid] <= t) lo = mid; else hi = mid;
  }
  const int64_t row = lo;
  const int64_t q0 = qsl[row] + (t - tile_off[row]) * PQ;
  const int nq = (int)min((int64_t)PQ, qsl[row + 1] - q0);
  const int64_t p0 = qpos0[row] + (q0 - qsl[row]);
  const int64_t ks = ksl[row], S = ksl[row + 1] - ks;
  const int32_t* kpr = kp + ks;
  // ---- key ranges: [0, sink_end) and [kbeg, kend)
  const int64_t kend = upper(kpr, S, p0 + nq - 1);
  int64_t kbeg = 0, sink_end = 0;
  if (window > 0) {
    kbeg = upper(kpr, S, p0 - window);
    sink_end = min(upper(kpr, S, nsink - 1), kbeg);
    if (kbeg <= sink_end) { kbeg = 0; sink_end = 0; }
  }
  // ---- the wave's queries as the B operand of S^T = K . Q^T (4 k-steps of 32 dims)
  const bool qok = col < nq;
  const int64_t qpos = p0 + col;
  u4v qb[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    qb[s] = qok ? *reinterpret_cast<const u4v*>(q + ((q0 + col) * 16 + h) * 128 + 32 * s + 8 * G) : u4v{0, 0, 0, 0};
  }
  f4 o[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) o[j] = f4{0.f, 0.f, 0.f, 0.f};
  float m = -1e30f, lsum = 0.f;

  for (int range = 0; range < 2; ++range) {
    const int64_t r0 = range ? kbeg : 0, r1 = range ? kend : sink_end;
    for (int64_t k0 = r0; k0 < r1; k0 += PK) {
      __syncthreads();                               // the previous tile has been read by every wave
      // ---- stage K rows, V^T and positions of keys [k0, k0 + 64) clipped to r1
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int c = tid + 256 * r, j = c >> 4, part = c & 15;
        u4v x = {0, 0, 0, 0};
        if (k0 + j < r1) x = *reinterpret_cast<const u4v*>(K + ((ks + k0 + j) * 4 + g) * 128 + 8 * part);
        *reinterpret_cast<u4v*>(&lds.k[j * KROW + 8 * part]) = x;
      }
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int u = tid + 256 * r, jp = u >> 4, part = u & 15, j = 2 * jp;
        u4v a = {0, 0, 0, 0}, b = {0, 0, 0, 0};
        if (k0 + j < r1) a = *reinterpret_cast<const u4v*>(V + ((ks + k0 + j) * 4 + g) * 128 + 8 * part);
        if (k0 + j + 1 < r1) b = *reinterpret_cast<const u4v*>(V + ((ks + k0 + j + 1) * 4 + g) * 128 + 8 * part);
        const int pcol = vt_pos(j);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t lo2 = (a[e] & 0xFFFFu) | (b[e] << 16), hi2 = (a[e] >> 16) | (b[e] & 0xFFFF0000u);
          *reinterpret_cast<uint32_t*>(&lds.vt[(8 * part + 2 * e) * VROW + pcol]) = lo2;
          *reinterpret_cast<uint32_t*>(&lds.vt[(8 * part + 2 * e + 1) * VROW + pcol]) = hi2;
        }
      }
      if (tid < PK) lds.kp[tid] = (k0 + tid < r1) ? kpr[k0 + tid] : 0x7FFFFFFF;
      __syncthreads();
      // ---- S^T = K . Q^T: 4 blocks of 16 keys
      f4 sc[4];
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) {
        f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const u4v a = *reinterpret_cast<const u4v*>(&lds.k[(nb * 16 + col) * KROW + 32 * s + 8 * G]);
          acc = mfma_bf(a, qb[s], acc);
        }
        sc[nb] = acc;
      }
      // ---- mask, scale, online softmax (the lane's 16 keys: nb * 16 + 4 G + i)
      float tmax = -INFINITY;
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int64_t kpos = lds.kp[nb * 16 + 4 * G + i];
          const bool keep = qok && kpos <= qpos && (window <= 0 || kpos > qpos - window || kpos < nsink);
          const float x = keep ? sc[nb][i] * scale_log2 : -INFINITY;
          sc[nb][i] = x;
          tmax = fmaxf(tmax, x);
        }
      }
      tmax = xmax(xmax(tmax, 16), 32);
      const float mnew = fmaxf(m, tmax);
      const float alpha = exp2f(m - mnew);
      m = mnew;
      float psum = 0.f;
      uint32_t pb[4][2];                             // bf16 probabilities, packed in key pairs
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) {
        float p[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          p[i] = exp2f(sc[nb][i] - mnew);
          psum += p[i];
        }
        pb[nb][0] = f2bf(p[0]) | (f2bf(p[1]) << 16);
        pb[nb][1] = f2bf(p[2]) | (f2bf(p[3]) << 16);
      }
      lsum = lsum * alpha + psum;
#pragma unroll
      for (int j = 0; j < 8; ++j) o[j] *= alpha;
      // ---- O^T += V^T . P^T: 2 halves of 32 keys x 8 blocks of 16 dims
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const u4v b = {pb[2 * hh][0], pb[2 * hh][1], pb[2 * hh + 1][0], pb[2 * hh + 1][1]};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const u4v a = *reinterpret_cast<const u4v*>(&lds.vt[(16 * j + col) * VROW + 32 * hh + 8 * G]);
          o[j] = mfma_bf(a, b, o[j]);
        }
      }
    }
  }
  // ---- normalise and write: lane holds dims 16 j + 4 G + 0..3 of query col
  lsum += __shfl_xor(lsum, 16, 64);
  lsum += __shfl_xor(lsum, 32, 64);
  if (!qok) return;
  const float inv = lsum > 0.f ? 1.0f / lsum : 0.f;
  uint16_t* dst = out + ((q0 + col) * 16 + h) * 128 + 4 * G;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const u2v v2 = {f2bf(o[j][0] * inv) | (f2bf(o[j][1] * inv) << 16), f2bf(o[j][2] * inv) | (f2bf(o[j][3] * inv) << 16)};
    *reinterpret_cast<u2v*>(dst + 16 * j) = v2;
  }
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

int kv800_hip_prefill(const uint16_t* q, const int64_t* qsl, const int64_t* qpos0, const uint16_t* K,
                      const uint16_t* V, const int32_t* kp, const int64_t* ksl, const int64_t* tile_off, int64_t R,
                      int64_t ntiles, int64_t window, int64_t nsink, uint16_t* out, void* stream) {
  KV800_REQUIRE(R >= 0 && ntiles >= 0, "prefill: negative R or tile count");
  if (R == 0 || ntiles == 0) return KV800_OK;
  KV800_REQUIRE(q && qsl && qpos0 && K && V && kp && ksl && tile_off && out, "prefill: null pointer");
  KV800_REQUIRE(((uintptr_t)q % 16) == 0 && ((uintptr_t)K % 16) == 0 && ((uintptr_t)V % 16) == 0 &&
                ((uintptr_t)out % 8) == 0, "prefill: q, K, V need 16-byte and out 8-byte alignment");
  KV800_REQUIRE(window >= 0 && nsink >= 0, "prefill: negative window or sink count");
  KV800_REQUIRE(ntiles < (1ll << 31), "prefill: too many query tiles");
  const float scale_log2 = 0.088388347648318440f * 1.4426950408889634f;   // 128^-0.5 * log2(e)
  hipLaunchKernelGGL(prefill_kernel, dim3((unsigned)ntiles, 4), dim3(256), 0, (hipStream_t)stream, q, qsl, qpos0, K, V,
                     kp, ksl, tile_off, R, window, nsink, scale_log2, out);
  return check_launch("prefill");
}

}  // extern "C"
