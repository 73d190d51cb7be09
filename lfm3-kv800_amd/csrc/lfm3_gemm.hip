// lfm3_gemm.hip -- the dense products of the LFM3-shaped engine loop (lfm3-kv800_amd/model.py) for gfx950:
// y (R, N) bf16 = x (R, K) bf16 . W^T with W (N, K) bf16, fp32 accumulation, for the decode batch sizes of the loop
// (R of a few hundred rows, N up to 65,536, K 2,048 or 8,192).
//
// At R = 256 the products are as much weight streaming as MFMA work (w13: 67 MB of weights, 17 GFLOP), and a
// 128 x 128 output tile per workgroup is the largest that still gives every CU of the chip a tile. The kernel is
// built around what one CU can feed its matrix cores with:
//   * W is stored once, at model setup, in the B-operand order of v_mfma_f32_32x32x16_bf16 (lfm3_hip_shuffle_weight):
//     a 1 KB block per (32 columns, 16 k), lane l's 16 bytes = W[32 nt + l % 32][16 ks + 8 (l / 32) .. + 8]. A wave
//     reads its blocks with one coalesced 16-byte load per lane straight into MFMA registers, no LDS.
//   * x is staged through LDS per 64-wide k slab (rows padded by 16 bytes so the A-operand reads of 8 consecutive rows
//     fall on distinct banks) and shared by the workgroup's 8 waves.
//   * Each wave owns 32 columns of the tile for all 128 rows (4 accumulators of 32 x 32) and half of each slab's
//     k-steps; x and the weights of a slab are requested two slabs before it is multiplied.
// With glu the weight's rows come in 128-row groups [64 rows of the gate half | the matching 64 rows of the up half]
// (lfm3_model.py's w13 = [g | u]) and the epilogue writes bf16(bf16(silu(g)) u) of the rounded products, the FFN's
// gated activation, so the (R, 2F) product never reaches memory.
// With split > 1 the K range is cut into `split` equal parts, one per grid z, and the fp32 partials go to a
// workspace; a second kernel sums them in a fixed order and rounds to bf16 (deterministic, no atomics).
#include "kv800_common.h"
#include "../../include/kv800_hip.h"
#include "../../include/lfm3_model.h"

namespace lfm3 {
namespace {

typedef __bf16 gbf8 __attribute__((ext_vector_type(8)));
typedef float gf16 __attribute__((ext_vector_type(16)));
typedef uint32_t gu4 __attribute__((ext_vector_type(4)));

constexpr int GT = 128;          // output tile rows and columns per workgroup
constexpr int GK = 64;           // k per LDS slab
constexpr int XROW = GK + 8;     // bf16 per staged x row (+16 bytes)

__device__ __forceinline__ gf16 mfma32(gu4 a, gu4 b, gf16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(gbf8, a), __builtin_bit_cast(gbf8, b), c, 0, 0, 0);
}

// Shuffled block (nt, ks): 64 lanes x 8 bf16; rows n >= N (up to the padded width) are zeros.
__global__ void __launch_bounds__(256) shuffle_kernel(const uint16_t* __restrict__ w, int64_t N, int64_t K,
                                                      int64_t Npad, uint16_t* __restrict__ wsh) {
  const int64_t nks = K / 16;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;   // (block, lane)
  if (i >= Npad / 32 * nks * 64) return;
  const int64_t blk = i >> 6, l = i & 63, nt = blk / nks, ks = blk % nks;
  const int64_t n = 32 * nt + (l & 31), k = 16 * ks + 8 * (l >> 5);
  gu4 v = {0u, 0u, 0u, 0u};
  if (n < N) v = *reinterpret_cast<const gu4*>(w + n * K + k);
  *reinterpret_cast<gu4*>(wsh + i * 8) = v;
}

// One workgroup (8 waves) = a 128 x 128 output tile over the k range [kb, kb + kpart). Wave w owns columns
// 32 (w & 3) .. + 32 for all 128 rows (4 accumulators of 32 x 32) and the k-steps 2 (w >> 2), 2 (w >> 2) + 1 of
// every 64-wide slab, so two waves share each column strip; 126 VGPRs and 66 KB of LDS let two workgroups share a CU
// (four waves per SIMD): one waits on LDS or memory while another multiplies. x and the weights of slab s + 2 are
// requested together while slab s is multiplied, into a ring of two register sets; x of slab s + 1 is staged into LDS
// (double buffer, one barrier per slab). The memory counter retires loads in issue order, so every wait is for loads
// issued a slab earlier. Loads past the last slab re-read the last one (in bounds, unused), so the steady-state loop
// has no branches and the counters stay exact across it.
// At the end the upper k-half waves hand their accumulators to the lower ones through LDS (a fixed-order sum) and the
// tile leaves through LDS as row-contiguous 16-byte stores.
constexpr int WD = 2;   // slabs in flight per wave
constexpr int TROW = GT + 4;                   // floats per row of the output tile in LDS (rows on different banks)
constexpr int LIN_LDS = GT * TROW * 4;         // 66 KB: the output tile; holds the x slabs and the hand-over before
static_assert(2 * GT * XROW * 2 <= LIN_LDS && 4 * 4 * 16 * 64 * 4 <= LIN_LDS, "LDS regions must fit");

template <bool GLU>
__global__ void __launch_bounds__(512, 2) linear_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                        const uint16_t* __restrict__ wsh, int64_t R, int64_t K,
                                                        int64_t kpart, uint16_t* __restrict__ y, int64_t ldy,
                                                        float* __restrict__ part, int64_t Npad) {
  __shared__ __align__(16) char lds[LIN_LDS];
  uint16_t (*xs)[GT * XROW] = reinterpret_cast<uint16_t (*)[GT * XROW]>(lds);
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int wc = w & 3, kh = w >> 2;
  const int64_t r0 = (int64_t)blockIdx.y * GT, n0 = (int64_t)blockIdx.x * GT;
  const int64_t kb = (int64_t)blockIdx.z * kpart, nks = K / 16;
  const int nslab = (int)(kpart / GK), last = nslab - 1;

  // x loader: thread -> row tid / 4 of the tile, 16 k from 16 (tid & 3); rows past R read row R - 1 (not stored)
  const int xr = tid >> 2, xq4 = tid & 3;
  const int64_t grow = r0 + xr < R ? r0 + xr : R - 1;
  const uint16_t* xsrc = x + grow * ldx + kb + 16 * xq4;
  const int xoff = xr * XROW + 16 * xq4;
  // this wave's weight blocks (n-tile n0 / 32 + wc, k-steps 2 kh, 2 kh + 1 of each slab)
  const uint16_t* wsrc = wsh + ((n0 / 32 + wc) * nks + kb / 16 + 2 * kh) * 512 + 8 * lane;
  const int aoff = (lane & 31) * XROW + 8 * (lane >> 5) + 32 * kh;   // A operand: row lane % 32, k 8 (lane / 32) ..

  gu4 xq[WD][2], wr[WD][2];
  auto load = [&](int s, int slot) {   // x, then the weights, of slab s
#pragma unroll
    for (int j = 0; j < 2; ++j) xq[slot][j] = *reinterpret_cast<const gu4*>(xsrc + (int64_t)s * GK + 8 * j);
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) wr[slot][kk] = *reinterpret_cast<const gu4*>(wsrc + ((int64_t)s * 4 + kk) * 512);
    asm volatile("" ::: "memory");   // the next slab's loads stay behind these
  };
  auto stage = [&](int slot, int buf) {
#pragma unroll
    for (int j = 0; j < 2; ++j) *reinterpret_cast<gu4*>(&xs[buf][xoff + 8 * j]) = xq[slot][j];
  };

  gf16 acc[4];
#pragma unroll
  for (int ms = 0; ms < 4; ++ms)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[ms][v] = 0.f;

#pragma unroll
  for (int j = 0; j < WD; ++j) load(min(j, last), j);
  stage(0, 0);
  __syncthreads();

  // slab s from ring slot j = s % 4 (compile-time) and LDS buffer s & 1
  auto step = [&](int s, int j) {
    const int b = j & 1;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      gu4 a[4];
#pragma unroll
      for (int ms = 0; ms < 4; ++ms) a[ms] = *reinterpret_cast<const gu4*>(&xs[b][aoff + 32 * ms * XROW + 16 * kk]);
#pragma unroll
      for (int ms = 0; ms < 4; ++ms) acc[ms] = mfma32(a[ms], wr[j][kk], acc[ms]);
    }
    stage((j + 1) % WD, b ^ 1);      // x of slab s + 1 into the buffer read a slab ago
    load(min(s + WD, last), j);      // slot j is free once slab s's MFMAs are issued
    __syncthreads();
  };
  int s0 = 0;
  for (; s0 + WD <= nslab; s0 += WD) {
#pragma unroll
    for (int j = 0; j < WD; ++j) step(s0 + j, j);
  }
#pragma unroll
  for (int j = 0; j < WD - 1; ++j)
    if (s0 + j < nslab) step(s0 + j, j);   // uniform

  // Epilogue through LDS (the loop's last barrier ended every read of the x slabs). The upper k-half waves hand their
  // accumulators over as [wc][ms][v / 4][lane] float4s; the lower ones add them (a fixed-order sum) and write the
  // tile row-major (rows padded to TROW floats); then every thread stores 32 consecutive columns of one row with
  // 16-byte stores (bf16, or the fp32 partial of a K part).
  float* tl = reinterpret_cast<float*>(lds);
  float4* ho = reinterpret_cast<float4*>(lds) + wc * (4 * 4 * 64) + lane;
  if (kh == 1) {
#pragma unroll
    for (int ms = 0; ms < 4; ++ms)
#pragma unroll
      for (int vq = 0; vq < 4; ++vq)
        ho[(ms * 4 + vq) * 64] = make_float4(acc[ms][4 * vq], acc[ms][4 * vq + 1], acc[ms][4 * vq + 2], acc[ms][4 * vq + 3]);
  }
  __syncthreads();
  if (kh == 0) {
#pragma unroll
    for (int ms = 0; ms < 4; ++ms)
#pragma unroll
      for (int vq = 0; vq < 4; ++vq) {
        const float4 h = ho[(ms * 4 + vq) * 64];
        acc[ms][4 * vq] += h.x; acc[ms][4 * vq + 1] += h.y; acc[ms][4 * vq + 2] += h.z; acc[ms][4 * vq + 3] += h.w;
      }
  }
  __syncthreads();
  if (kh == 0) {   // C layout of the 32 x 32 MFMA: lane l holds column l % 32, rows 8 (v / 4) + 4 (l / 32) + v % 4
    const int c = 32 * wc + (lane & 31), rr = 4 * (lane >> 5);
#pragma unroll
    for (int ms = 0; ms < 4; ++ms)
#pragma unroll
      for (int v = 0; v < 16; ++v) tl[(32 * ms + 8 * (v >> 2) + rr + (v & 3)) * TROW + c] = acc[ms][v];
  }
  __syncthreads();
  if (GLU) {   // thread -> row tid / 4, output columns 16 (tid & 3) .. + 16 of the tile's 64
    const int orow = tid >> 2, oc = 16 * (tid & 3);
    const int64_t row = r0 + orow;
    if (row < R) {
      const float4* g4 = reinterpret_cast<const float4*>(tl + orow * TROW + oc);
      const float4* u4 = reinterpret_cast<const float4*>(tl + orow * TROW + 64 + oc);
      uint4* dst = reinterpret_cast<uint4*>(y + row * ldy + n0 / 2 + oc);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        uint32_t o[4];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const float4 g = g4[2 * i + h], u = u4[2 * i + h];
          const float gv[4] = {g.x, g.y, g.z, g.w}, uv[4] = {u.x, u.y, u.z, u.w};
          uint32_t b[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float gg = kv800::bfround(gv[e]);
            b[e] = kv800::f2bf(kv800::bfround(gg / (1.0f + __expf(-gg))) * kv800::bfround(uv[e]));
          }
          o[2 * h] = b[0] | (b[1] << 16);
          o[2 * h + 1] = b[2] | (b[3] << 16);
        }
        dst[i] = make_uint4(o[0], o[1], o[2], o[3]);
      }
    }
    return;
  }
  const int orow = tid >> 2, oc = 32 * (tid & 3);
  const int64_t row = r0 + orow;
  if (row < R) {
    const float4* src = reinterpret_cast<const float4*>(tl + orow * TROW + oc);
    if (part) {
      float4* dst = reinterpret_cast<float4*>(part + ((int64_t)blockIdx.z * R + row) * Npad + n0 + oc);
#pragma unroll
      for (int i = 0; i < 8; ++i) dst[i] = src[i];
    } else {
      uint4* dst = reinterpret_cast<uint4*>(y + row * ldy + n0 + oc);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float4 p0 = src[2 * i], p1 = src[2 * i + 1];
        dst[i] = make_uint4(kv800::f2bf(p0.x) | (kv800::f2bf(p0.y) << 16), kv800::f2bf(p0.z) | (kv800::f2bf(p0.w) << 16),
                            kv800::f2bf(p1.x) | (kv800::f2bf(p1.y) << 16), kv800::f2bf(p1.z) | (kv800::f2bf(p1.w) << 16));
      }
    }
  }
}

// y = bf16(sum over z of part[z]) in z order
__global__ void __launch_bounds__(256) reduce_kernel(const float* __restrict__ part, int split, int64_t R, int64_t Npad,
                                                     uint16_t* __restrict__ y, int64_t ldy) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i >= R * Npad) return;
  const int64_t row = i / Npad, col = i % Npad;
  float4 s = *reinterpret_cast<const float4*>(part + i);
  for (int z = 1; z < split; ++z) {
    const float4 p = *reinterpret_cast<const float4*>(part + (int64_t)z * R * Npad + i);
    s.x += p.x; s.y += p.y; s.z += p.z; s.w += p.w;
  }
  const uint32_t lo = kv800::f2bf(s.x) | (kv800::f2bf(s.y) << 16), hi = kv800::f2bf(s.z) | (kv800::f2bf(s.w) << 16);
  *reinterpret_cast<uint2*>(y + row * ldy + col) = make_uint2(lo, hi);
}

}  // namespace
}  // namespace lfm3

extern "C" {

int lfm3_hip_shuffle_weight(const uint16_t* w, int64_t N, int64_t K, int64_t Npad, uint16_t* wsh, void* stream) {
  KV800_REQUIRE(N > 0 && K > 0 && K % 64 == 0 && Npad >= N && Npad % 128 == 0,
                "shuffle_weight: K must be a multiple of 64 and Npad a multiple of 128 covering N");
  KV800_REQUIRE(w && wsh, "shuffle_weight: null pointer");
  const int64_t n = Npad / 32 * (K / 16) * 64;
  hipLaunchKernelGGL(lfm3::shuffle_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, w, N,
                     K, Npad, wsh);
  return kv800::check_launch("shuffle_weight");
}

int lfm3_hip_linear(const uint16_t* x, int64_t ldx, const uint16_t* wsh, int64_t R, int64_t Npad, int64_t K,
                    uint16_t* y, int64_t ldy, int split, float* work, int glu, void* stream) {
  KV800_REQUIRE(R > 0 && K > 0 && K % 64 == 0 && Npad > 0 && Npad % 128 == 0 && ldx >= K && ldx % 8 == 0 &&
                    ldy >= (glu ? Npad / 2 : Npad) && ldy % 8 == 0,
                "linear: K must be a multiple of 64, Npad of 128, ldx >= K and ldy >= the output width (multiples of 8)");
  KV800_REQUIRE(glu == 0 || (glu == 1 && split == 1), "linear: glu is 0 or 1, and 1 takes no K split");
  KV800_REQUIRE(split >= 1 && split <= 64 && K % (64 * split) == 0, "linear: split must divide K into 64-multiples");
  KV800_REQUIRE(x && wsh && y && (split == 1 || work), "linear: null pointer");
  const dim3 grid((unsigned)(Npad / lfm3::GT), (unsigned)((R + lfm3::GT - 1) / lfm3::GT), (unsigned)split);
  float* part = split > 1 ? work : nullptr;
  if (glu)
    hipLaunchKernelGGL(lfm3::linear_kernel<true>, grid, dim3(512), 0, (hipStream_t)stream, x, ldx, wsh, R, K, K, y, ldy,
                       nullptr, Npad);
  else
    hipLaunchKernelGGL(lfm3::linear_kernel<false>, grid, dim3(512), 0, (hipStream_t)stream, x, ldx, wsh, R, K,
                       K / split, y, ldy, part, Npad);
  int rc = kv800::check_launch("linear");
  if (rc != KV800_OK || split == 1) return rc;
  const int64_t n4 = R * Npad / 4;
  hipLaunchKernelGGL(lfm3::reduce_kernel, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, (hipStream_t)stream, work,
                     split, R, Npad, y, ldy);
  return kv800::check_launch("linear_reduce");
}

}  // extern "C"
