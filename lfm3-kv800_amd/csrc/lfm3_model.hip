// lfm3_model.hip -- fused elementwise kernels of the LFM3-shaped engine loop (lfm3-kv800_amd/model.py) for gfx950.
//
// The engine loop that drives the 800h attention path runs a 24-layer LFM3-shaped model whose dense products are
// library GEMMs; these kernels replace the chains of small torch ops between them, one launch each, with the same
// roundings as those ops (every torch op on bf16 tensors computes in fp32 and rounds its result to bf16):
//   add_rmsnorm   x' = x + bf16(rms(h) w_post), n = bf16(rms(x') w_next)   (sandwich norms, vllm_model.py:446-471)
//   rmsnorm       n = bf16(rms(x) w)
//   silu_mul      bf16(bf16(silu(g)) u) of the [g | u] halves of a row      (the FFN's gated activation)
//   qkv_post      per-head RMS norm of q and k, neox RoPE of q and k from bf16 cos / sin tables, v copied out
//                 (vllm_model.py:195-304)
//   conv_step     y = sum_k bf16(win_k w_k) over the 7-wide window [state | B x], state shifted, out = bf16(C y)
//                 (the short-conv decode step, vllm_model.py:327-431)
//   gate_mul      o bf16(sigmoid(g)) per head (the attention output gate)
//   argmax        index of the largest bf16 logit of a row (the greedy token; torch.argmax's choice among equals)
// rms(x) = x rsqrt(mean(x^2) + eps) in fp32. Sums run in a fixed tree order, so results equal torch's up to the
// order of fp32 additions inside a mean or a 7-term sum.
#include <mutex>

#include "kv800_common.h"
#include "../../include/kv800_hip.h"
#include "../../include/lfm3_model.h"

namespace lfm3 {
namespace {

using kv800::bf2f;
using kv800::f2bf;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// sum over the 256 threads of a workgroup (4 waves)
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

__device__ __forceinline__ void load8(const uint16_t* p, float (&f)[8]) {
  const uint4 u = *reinterpret_cast<const uint4*>(p);
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) { f[2 * i] = bf2f(w[i] & 0xFFFFu); f[2 * i + 1] = bf2f(w[i] >> 16); }
}
__device__ __forceinline__ void store8(uint16_t* p, const float (&f)[8]) {
  uint4 u;
  u.x = f2bf(f[0]) | (f2bf(f[1]) << 16); u.y = f2bf(f[2]) | (f2bf(f[3]) << 16);
  u.z = f2bf(f[4]) | (f2bf(f[5]) << 16); u.w = f2bf(f[6]) | (f2bf(f[7]) << 16);
  *reinterpret_cast<uint4*>(p) = u;
}
__device__ __forceinline__ float bfr(float x) { return bf2f(f2bf(x)); }   // round to bf16, back to float

// ---------------------------------------------------------------- norms (one workgroup of 256 threads per row)
// H = 2048: 8 elements per thread
__global__ void __launch_bounds__(256)
add_rmsnorm_kernel(const uint16_t* __restrict__ h, const uint16_t* __restrict__ x, const uint16_t* __restrict__ wp,
                   const uint16_t* __restrict__ wn, float eps, int64_t H, uint16_t* __restrict__ xo,
                   uint16_t* __restrict__ no) {
  __shared__ float red[4];
  const int64_t r = blockIdx.x;
  const int64_t c0 = 8 * (int64_t)threadIdx.x;
  float a[8], b[8], w[8];
  float ss = 0.f;
  if (h) {
    load8(h + r * H + c0, a);
#pragma unroll
    for (int i = 0; i < 8; ++i) ss += a[i] * a[i];
    const float inv = rsqrtf(block_sum(ss, red) / (float)H + eps);
    load8(wp + c0, w);
    load8(x + r * H + c0, b);
#pragma unroll
    for (int i = 0; i < 8; ++i) b[i] = bfr(b[i] + bfr(a[i] * inv * w[i]));   // x + bf16(rms(h) w_post)
    store8(xo + r * H + c0, b);
  } else {
    load8(x + r * H + c0, b);
  }
  if (!no) return;
  ss = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) ss += b[i] * b[i];
  const float inv2 = rsqrtf(block_sum(ss, red) / (float)H + eps);
  load8(wn + c0, w);
#pragma unroll
  for (int i = 0; i < 8; ++i) a[i] = b[i] * inv2 * w[i];
  store8(no + r * H + c0, a);
}

// ---------------------------------------------------------------- gated activation
__global__ void __launch_bounds__(256)
silu_mul_kernel(const uint16_t* __restrict__ gu, int64_t R, int64_t F, uint16_t* __restrict__ out) {
  const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;   // element of the (R, F) output
  if (i >= R * F) return;
  const int64_t r = i / F, c = i % F;
  float g[8], u[8];
  load8(gu + r * 2 * F + c, g);
  load8(gu + r * 2 * F + F + c, u);
#pragma unroll
  for (int k = 0; k < 8; ++k) g[k] = bfr(g[k] / (1.0f + __expf(-g[k]))) * u[k];
  store8(out + i, g);
}

// ---------------------------------------------------------------- q / k norm + RoPE, v copy
// grid (R, 24): head-rows 0..15 q, 16..19 k, 20..23 v; one wave per head-row, lane = dims lane, lane + 64.
// cos_t / sin_t: (P, 64) bf16 per frequency f (dims f and f + 64 share frequency f).
__global__ void __launch_bounds__(64)
qkv_post_kernel(const uint16_t* __restrict__ qkv, int64_t stride, const uint16_t* __restrict__ qw,
                const uint16_t* __restrict__ kw, const uint16_t* __restrict__ cos_t, const uint16_t* __restrict__ sin_t,
                int64_t P, const int64_t* __restrict__ pos, float eps, uint16_t* __restrict__ qo,
                uint16_t* __restrict__ kpre, uint16_t* __restrict__ krot, uint16_t* __restrict__ vo) {
  const int64_t r = blockIdx.x;
  const int hr = blockIdx.y, lane = threadIdx.x;
  const uint16_t* src = qkv + r * stride + hr * 128;
  float lo = bf2f(src[lane]), hi = bf2f(src[lane + 64]);
  if (hr >= 20) {   // v: copied as it is
    uint16_t* dst = vo + (r * 4 + (hr - 20)) * 128;
    dst[lane] = src[lane];
    dst[lane + 64] = src[lane + 64];
    return;
  }
  const bool isq = hr < 16;
  const uint16_t* w = isq ? qw : kw;
  const float inv = rsqrtf(wave_sum(lo * lo + hi * hi) / 128.0f + eps);
  lo = bfr(lo * inv * bf2f(w[lane]));
  hi = bfr(hi * inv * bf2f(w[lane + 64]));
  if (!isq) {
    uint16_t* dst = kpre + (r * 4 + (hr - 16)) * 128;
    dst[lane] = (uint16_t)f2bf(lo);
    dst[lane + 64] = (uint16_t)f2bf(hi);
  }
  int64_t p = pos[r];
  p = p < 0 ? 0 : (p >= P ? P - 1 : p);
  const float c = bf2f(cos_t[p * 64 + lane]), s = bf2f(sin_t[p * 64 + lane]);
  const float rlo = lo * c + (-hi) * s, rhi = hi * c + lo * s;   // x c + rotate_half(x) s
  uint16_t* dst = isq ? qo + (r * 16 + hr) * 128 : krot + (r * 4 + (hr - 16)) * 128;
  dst[lane] = (uint16_t)f2bf(rlo);
  dst[lane + 64] = (uint16_t)f2bf(rhi);
}

// ---------------------------------------------------------------- short conv decode step
// one thread per (row, channel); bcx (R, 3H) = [B | C | x]; conv_w (H, 7); state (R, H, 6) updated in place
__global__ void __launch_bounds__(256)
conv_step_kernel(const uint16_t* __restrict__ bcx, int64_t stride, const uint16_t* __restrict__ cw,
                 uint16_t* __restrict__ state, int64_t R, int64_t H, uint16_t* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= R * H) return;
  const int64_t r = i / H, c = i % H;
  const uint16_t* row = bcx + r * stride;
  const float bx = bfr(bf2f(row[c]) * bf2f(row[2 * H + c]));
  uint16_t* st = state + i * 6;
  float win[7];
#pragma unroll
  for (int k = 0; k < 6; ++k) win[k] = bf2f(st[k]);
  win[6] = bx;
  float y = 0.f;
#pragma unroll
  for (int k = 0; k < 7; ++k) y += bfr(win[k] * bf2f(cw[c * 7 + k]));
#pragma unroll
  for (int k = 0; k < 6; ++k) st[k] = (uint16_t)f2bf(win[k + 1]);
  out[i] = (uint16_t)f2bf(bf2f(row[H + c]) * bfr(y));
}

// ---------------------------------------------------------------- attention output gate
// o (R, 16, 128); g: row r's 16 gate logits at g + r * gstride
__global__ void __launch_bounds__(256)
gate_mul_kernel(const uint16_t* __restrict__ o, const uint16_t* __restrict__ g, int64_t gstride, int64_t R,
                uint16_t* __restrict__ out) {
  const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
  if (i >= R * 2048) return;
  const int64_t r = i / 2048, head = (i % 2048) / 128;
  const float gl = bf2f(g[r * gstride + head]);
  const float sg = bfr(1.0f / (1.0f + __expf(-gl)));
  float v[8];
  load8(o + i, v);
#pragma unroll
  for (int k = 0; k < 8; ++k) v[k] *= sg;
  store8(out + i, v);
}

// ---------------------------------------------------------------- greedy token (one workgroup per row)
// (a, ia) ranks before (b, ib): the larger value, the smaller index among equals; NaN ranks above every number, the
// first NaN first (torch.argmax)
__device__ __forceinline__ bool ranks_before(float a, int ia, float b, int ib) {
  const bool na = a != a, nb = b != b;
  if (na || nb) return na && (!nb || ia < ib);
  return a > b || (a == b && ia < ib);
}
// thread t scans the 8-element pieces t, t + AT, ... of the row, eight loads at a time (a 65,536-wide row is one
// round of loads for 1,024 threads, two for 512); the workgroup then reduces the AT bests (the order of the compares
// does not matter: ranks_before breaks ties by index). 1,024 threads a row while every row has a CU of its own (one
// workgroup per CU at 98 VGPRs); 512 beyond that, so that two rows share a CU in one round.
template <int AT>
__global__ void __launch_bounds__(AT)
argmax_kernel(const uint16_t* __restrict__ x, int64_t V, int64_t stride, int64_t* __restrict__ out) {
  __shared__ float rv[AT / 64];
  __shared__ int ri[AT / 64];
  const uint16_t* row = x + (int64_t)blockIdx.x * stride;
  float cv[8];
  int ci[8];   // eight independent running bests, one per in-flight piece
#pragma unroll
  for (int u = 0; u < 8; ++u) { cv[u] = -INFINITY; ci[u] = (int)V; }   // index V ranks after every element
  for (int64_t p0 = threadIdx.x; p0 * 8 < V; p0 += AT * 8) {   // 8 pieces' loads in flight, then their compares
    float f[8][8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int64_t p = p0 + AT * u;
      if (p * 8 < V) load8(row + 8 * p, f[u]);
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int64_t p = p0 + AT * u;
      if (p * 8 < V) {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (ranks_before(f[u][e], (int)(8 * p) + e, cv[u], ci[u])) { cv[u] = f[u][e]; ci[u] = (int)(8 * p) + e; }
      }
    }
  }
  float bv = cv[0];
  int bi = ci[0];
#pragma unroll
  for (int u = 1; u < 8; ++u)
    if (ranks_before(cv[u], ci[u], bv, bi)) { bv = cv[u]; bi = ci[u]; }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float v2 = __shfl_xor(bv, o, 64);
    const int i2 = __shfl_xor(bi, o, 64);
    if (ranks_before(v2, i2, bv, bi)) { bv = v2; bi = i2; }
  }
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) { rv[w] = bv; ri[w] = bi; }
  __syncthreads();
  if (threadIdx.x == 0) {
#pragma unroll
    for (int k = 1; k < AT / 64; ++k)
      if (ranks_before(rv[k], ri[k], bv, bi)) { bv = rv[k]; bi = ri[k]; }
    out[blockIdx.x] = bi;
  }
}

}  // namespace
}  // namespace lfm3

using namespace lfm3;

// CUs of the current device (cached per device; 256 if the query fails)
static int64_t device_cus() {
  static std::mutex mu;
  static int64_t cache[64] = {0};
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    (void)hipGetLastError();
    return 256;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (cache[dev] == 0) {
    int cu = 0;
    if (hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cu <= 0) {
      (void)hipGetLastError();
      cu = 256;
    }
    cache[dev] = cu;
  }
  return cache[dev];
}

extern "C" {

int lfm3_hip_add_rmsnorm(const uint16_t* h, const uint16_t* x, const uint16_t* w_post, const uint16_t* w_next,
                         float eps, int64_t R, int64_t H, uint16_t* x_out, uint16_t* n_out, void* stream) {
  KV800_REQUIRE(R >= 0 && H == 2048, "add_rmsnorm: rows must be 2048 wide");
  if (R == 0) return KV800_OK;
  KV800_REQUIRE(x && (!h || (w_post && x_out)) && (!n_out || w_next) && (h || n_out), "add_rmsnorm: null pointer");
  hipLaunchKernelGGL(add_rmsnorm_kernel, dim3((unsigned)R), dim3(256), 0, (hipStream_t)stream, h, x, w_post, w_next,
                     eps, H, x_out, n_out);
  return kv800::check_launch("add_rmsnorm");
}

int lfm3_hip_silu_mul(const uint16_t* gu, int64_t R, int64_t F, uint16_t* out, void* stream) {
  KV800_REQUIRE(R >= 0 && F > 0 && F % 8 == 0, "silu_mul: F must be a positive multiple of 8");
  if (R == 0) return KV800_OK;
  KV800_REQUIRE(gu && out, "silu_mul: null pointer");
  const int64_t n = R * F / 8;
  hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, gu, R, F,
                     out);
  return kv800::check_launch("silu_mul");
}

int lfm3_hip_qkv_post(const uint16_t* qkv, int64_t stride, const uint16_t* q_w, const uint16_t* k_w,
                      const uint16_t* cos_t, const uint16_t* sin_t, int64_t P, const int64_t* pos, float eps,
                      int64_t R, uint16_t* q_out, uint16_t* k_pre, uint16_t* k_rot, uint16_t* v_out, void* stream) {
  KV800_REQUIRE(R >= 0 && stride >= 3072 && P > 0, "qkv_post: bad shape");
  if (R == 0) return KV800_OK;
  KV800_REQUIRE(qkv && q_w && k_w && cos_t && sin_t && pos && q_out && k_pre && k_rot && v_out,
                "qkv_post: null pointer");
  hipLaunchKernelGGL(qkv_post_kernel, dim3((unsigned)R, 24), dim3(64), 0, (hipStream_t)stream, qkv, stride, q_w, k_w,
                     cos_t, sin_t, P, pos, eps, q_out, k_pre, k_rot, v_out);
  return kv800::check_launch("qkv_post");
}

int lfm3_hip_conv_step(const uint16_t* bcx, int64_t stride, const uint16_t* conv_w, uint16_t* state, int64_t R,
                       int64_t H, uint16_t* out, void* stream) {
  KV800_REQUIRE(R >= 0 && H > 0 && stride >= 3 * H, "conv_step: bad shape");
  if (R == 0) return KV800_OK;
  KV800_REQUIRE(bcx && conv_w && state && out, "conv_step: null pointer");
  const int64_t n = R * H;
  hipLaunchKernelGGL(conv_step_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, bcx,
                     stride, conv_w, state, R, H, out);
  return kv800::check_launch("conv_step");
}

int lfm3_hip_gate_mul(const uint16_t* o, const uint16_t* g, int64_t gstride, int64_t R, uint16_t* out,
                      void* stream) {
  KV800_REQUIRE(R >= 0 && gstride >= 16, "gate_mul: bad shape");
  if (R == 0) return KV800_OK;
  KV800_REQUIRE(o && g && out, "gate_mul: null pointer");
  const int64_t n = R * 2048 / 8;
  hipLaunchKernelGGL(gate_mul_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, o, g,
                     gstride, R, out);
  return kv800::check_launch("gate_mul");
}

int lfm3_hip_argmax(const uint16_t* x, int64_t R, int64_t V, int64_t stride, int64_t* out, void* stream) {
  KV800_REQUIRE(R >= 0 && V > 0 && V % 8 == 0 && V < (1LL << 31) && stride >= V && stride % 8 == 0,
                "argmax: needs 0 < V < 2^31, V and the row stride multiples of 8");
  if (R == 0) return KV800_OK;
  KV800_REQUIRE(x && out && ((uintptr_t)x % 16) == 0, "argmax: null or misaligned pointer");
  if (R <= device_cus())
    hipLaunchKernelGGL(argmax_kernel<1024>, dim3((unsigned)R), dim3(1024), 0, (hipStream_t)stream, x, V, stride, out);
  else
    hipLaunchKernelGGL(argmax_kernel<512>, dim3((unsigned)R), dim3(512), 0, (hipStream_t)stream, x, V, stride, out);
  return kv800::check_launch("argmax");
}

}  // extern "C"
