// kv800_common.h -- constants, bit-exact scalar helpers and host-side error plumbing shared by the gfx950 kernels
// of the 800h path. Layout constants follow kv800.py:32-34; the fp8 / bf16 helpers follow the semantics the
// reference gets from torch (fp8 e4m3fn encode: round to nearest even, |x| > 464 -> 0x7F NaN; bf16: round to nearest
// even) and its kernels (fp8 decode without NaN handling, kv800_sycl.sycl:41-45).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kv800 {

constexpr int BLK = 256;      // tokens per quantized sub-block
constexpr int LAG = 128;      // newest tokens that always stay exact
constexpr int NSINK = 4;
constexpr int SUB = 51200;    // bytes per sub-block
constexpr int KC_O = 0, VB_O = 32768, VLO_O = 49152, VSC_O = 49664, KLO_O = 50176, KSC_O = 50688;

// ---------------------------------------------------------------- device scalar helpers
__device__ __forceinline__ float bf2f(uint32_t b16) { return __uint_as_float(b16 << 16); }
__device__ __forceinline__ float bf2f_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }
__device__ __forceinline__ float bf2f_lo(uint32_t w) { return __uint_as_float(w << 16); }

// float -> bf16 bits, round to nearest even (finite values)
__device__ __forceinline__ uint32_t f2bf(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}
__device__ __forceinline__ float bfround(float f) { return __uint_as_float(f2bf(f) << 16); }

// fp8 e4m3fn byte -> float, exact; no NaN handling (the scales the quantizer writes are finite for finite input)
__device__ __forceinline__ float f8d(uint32_t b) {
  const uint32_t e = (b >> 3) & 15u, m = b & 7u;
  const uint32_t nrm = ((e + 120u) << 23) | (m << 20);
  const uint32_t sub = __float_as_uint((float)m * 0.001953125f);
  return __uint_as_float((e ? nrm : sub) | ((b & 0x80u) << 24));   // selects, no control flow
}

// float -> fp8 e4m3fn byte with torch's .to(float8_e4m3fn) semantics (round to nearest even on the e4m3 grid,
// results past 448 and inf / NaN -> 0x7F with the sign bit)
__device__ __forceinline__ uint32_t f8e(float f) {
  const uint32_t x = __float_as_uint(f);
  const uint32_t sign = (x >> 24) & 0x80u;
  const uint32_t a = x & 0x7FFFFFFFu;
  if (a >= 0x7F800000u) return sign | 0x7Fu;
  const float v = __uint_as_float(a);
  if (v < 0.015625f) return sign | (uint32_t)__builtin_rintf(v * 512.0f);   // subnormal grid, step 2^-9
  uint32_t keep = (a >> 20) & 7u, rest = a & 0xFFFFFu, e8 = ((a >> 23) & 0xFFu) - 120u;
  if (rest > 0x80000u || (rest == 0x80000u && (keep & 1u))) {
    keep += 1u;
    if (keep == 8u) { keep = 0u; e8 += 1u; }
  }
  if (e8 > 15u || (e8 == 15u && keep == 7u)) return sign | 0x7Fu;
  return sign | (e8 << 3) | keep;
}

__device__ __forceinline__ float clamp_min_1e8(float a) { return a < 1e-8f ? 1e-8f : a; }

// v_min_f32 / v_max_f32 / v_max3_f32 as the bare instructions. fminf and fmaxf first quiet signalling NaNs of operands
// whose origin the compiler cannot see (cross-lane moves, selects, inline assembly); arithmetic never produces a
// signalling NaN, so for arithmetic results and copies of them the quieting is dead work. The operands must be written
// by ordinary VALU or memory instructions, not straight by an MFMA (no hazard wait states are inserted for inline
// assembly reading an MFMA result).
__device__ __forceinline__ float vmin(float a, float b) {
  float r;
  asm("v_min_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
__device__ __forceinline__ float vmax(float a, float b) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
__device__ __forceinline__ float vmax3(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

}  // namespace kv800

// ---------------------------------------------------------------- host error plumbing
namespace kv800 {
void set_error(const char* fmt, ...);
int check_launch(const char* what);
}  // namespace kv800

#define KV800_REQUIRE(cond, ...)                 \
  do {                                           \
    if (!(cond)) {                               \
      ::kv800::set_error(__VA_ARGS__);           \
      return KV800_EINVAL;                       \
    }                                            \
  } while (0)
