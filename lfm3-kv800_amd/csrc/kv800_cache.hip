// kv800_cache.hip -- per-step cache bookkeeping of the 800h path in vLLM's page geometry, for gfx950.
//
//   write_exact_kernel   the step's K / V rows into the exact pages through the slot mapping (vllm_attn.py:263-272),
//                        and, for tokens at positions < 4 of a window layer, into the sink aux area of the host
//                        layers' first quant page (vllm_attn.py:276-291).
//   step_tables_kernel   per row of the quant KV group: NQ = max(N - 128, 0) / 256 flushed sub-blocks and the byte
//                        offsets of its first nqmax sub-blocks in the quant pool, qbt[r, 256 j / bsq] * qs0 +
//                        (256 j % bsq) / 256 * 51200 (vllm_attn.py:332-340); optionally the sub-blocks flushed before
//                        the step's nnew tokens (the flush range's start, vllm_attn.py:297-317), the block table as
//                        int64 and the offsets of the sink aux areas (vllm_attn.py:276-291).
//   step_meta_kernel     per row of a decode step: the new token's slot, its position and the int32 length
//   page_offsets_kernel  off[r, p] = bt[r, p] * scale + add: an exact group's block table as element offsets of its
//                        pages (the eoff table of the decode and flush kernels).
// All are plain data movement: one thread per 16-byte piece or per table entry, coalesced along the row.
#include "kv800_common.h"
#include "../../include/kv800_hip.h"

namespace kv800 {
namespace {

// thread -> (row r, piece): 4 heads x 128 dims = 64 pieces of 8 bf16 per K row and as many per V row
__global__ void __launch_bounds__(256)
write_exact_kernel(uint16_t* __restrict__ ep, int64_t s0, int64_t s1, int64_t s2, int64_t e_v, int64_t ebs,
                   const int64_t* __restrict__ slot, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
                   int64_t R, const int64_t* __restrict__ pos, uint16_t* __restrict__ skp, uint16_t* __restrict__ svp,
                   const int64_t* __restrict__ skoff, const int64_t* __restrict__ svoff, int nsink) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= R * 128) return;
  const int64_t r = i >> 7;
  const int piece = (int)(i & 127), isv = piece >> 6, h = (piece >> 4) & 3, d0 = 8 * (piece & 15);
  const uint4 x = *reinterpret_cast<const uint4*>((isv ? v : k) + (r * 4 + h) * 128 + d0);
  const int64_t sl = slot[r];
  if (sl >= 0) {   // slot < 0: padding token, not written (vllm_attn.py:265)
    const int64_t o = (sl / ebs) * s0 + h * s1 + (sl % ebs) * s2 + (isv ? e_v : 0) + d0;
    *reinterpret_cast<uint4*>(ep + o) = x;
  }
  if (nsink > 0 && pos[r] >= 0 && pos[r] < nsink) {   // sink rows of a window layer
    uint16_t* dst = isv ? svp : skp;
    const int64_t base = isv ? svoff[r] : skoff[r];
    *reinterpret_cast<uint4*>(dst + base + (pos[r] * 4 + h) * 128 + d0) = x;
  }
}

__global__ void __launch_bounds__(256)
step_tables_kernel(const int32_t* __restrict__ qbt, int64_t qbt_stride, int64_t bsq, int64_t qs0,
                   const int32_t* __restrict__ N, int64_t R, int64_t nqmax, int64_t nnew,
                   const int32_t* __restrict__ nnew_rows, int64_t* __restrict__ boff,
                   int32_t* __restrict__ NQ, int32_t* __restrict__ NP, int64_t* __restrict__ qbt64,
                   int64_t* __restrict__ aux, int64_t aux_scale, int64_t aux_add) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t w = max(max(nqmax, (int64_t)1), qbt64 ? qbt_stride : (int64_t)1);   // entries per row
  if (i >= R * w) return;
  const int64_t r = i / w, j = i % w;
  if (j == 0) {
    NQ[r] = max(N[r] - LAG, 0) / BLK;
    if (NP) NP[r] = max(N[r] - (nnew_rows ? max(nnew_rows[r], 0) : (int)nnew) - LAG, 0) / BLK;
    if (aux) aux[r] = (int64_t)qbt[r * qbt_stride] * aux_scale + aux_add;
  }
  if (j < nqmax) {
    const int64_t tok0 = j * BLK;
    boff[r * nqmax + j] = (int64_t)qbt[r * qbt_stride + tok0 / bsq] * qs0 + ((tok0 % bsq) / BLK) * SUB;
  }
  if (qbt64 && j < qbt_stride) qbt64[r * qbt_stride + j] = qbt[r * qbt_stride + j];
}

__global__ void __launch_bounds__(256)
page_offsets_kernel(const int32_t* __restrict__ bt, int64_t bt_stride, int64_t R, int64_t npages, int64_t scale,
                    int64_t add, int64_t* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= R * npages) return;
  const int64_t r = i / npages, p = i % npages;
  out[i] = (int64_t)bt[r * bt_stride + p] * scale + add;
}

// One decode step's slot, position and int32 length of row r (every row appends one token at position len - 1): the
// slot is the token's page bt[r, pos / ebs] times ebs plus pos % ebs; a row of length 0 gets slot and position -1
// (a padding token, which write_exact skips); a position past the row's npages pages gets slot -1 as well.
__global__ void __launch_bounds__(256)
step_meta_kernel(const int32_t* __restrict__ bt, int64_t bt_stride, int64_t npages, const int64_t* __restrict__ lens,
                 int64_t R, int64_t ebs, int64_t* __restrict__ slot, int64_t* __restrict__ pos,
                 int32_t* __restrict__ lens32) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= R) return;
  const int64_t n = lens[r], p = n - 1, pg = p >= 0 ? p / ebs : -1;
  slot[r] = (pg >= 0 && pg < npages) ? (int64_t)bt[r * bt_stride + pg] * ebs + p % ebs : -1;
  pos[r] = p >= 0 ? p : -1;
  lens32[r] = (int32_t)n;
}

// Streaming-read probe (a measurement aid of bench.py, not part of the cache path): workgroup g reads the 16-byte
// units g * 2048 + tid + 256 k (k < 8) of the buffer and every gridDim.x * 2048 units after, xor-folds them and writes
// one word; with 8 loads in flight per lane and two workgroups per CU it reads at what the part sustains for
// plain (cached) loads.
typedef uint32_t pv4 __attribute__((ext_vector_type(4)));
__global__ void __launch_bounds__(256) read_probe_kernel(const pv4* __restrict__ p, int64_t n16,
                                                         uint32_t* __restrict__ out) {
  constexpr int U = 8;
  const int64_t stride = (int64_t)gridDim.x * 256 * U;
  pv4 acc = {0u, 0u, 0u, 0u};
  for (int64_t i = (int64_t)blockIdx.x * 256 * U + threadIdx.x; i < n16; i += stride) {
    pv4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = (i + 256 * u < n16) ? p[i + 256 * u] : pv4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u];
  }
  __shared__ uint32_t red[256];
  red[threadIdx.x] = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t x = 0;
    for (int k = 0; k < 256; ++k) x ^= red[k];
    out[blockIdx.x] = x;
  }
}

}  // namespace
}  // namespace kv800

using namespace kv800;

extern "C" {

int kv800_hip_write_exact(uint16_t* epool, int64_t s0, int64_t s1, int64_t s2, int64_t e_v, int64_t ebs,
                          const int64_t* slot, const uint16_t* k, const uint16_t* v, int64_t R, const int64_t* pos,
                          uint16_t* sk, uint16_t* sv, const int64_t* skoff, const int64_t* svoff, void* stream) {
  KV800_REQUIRE(R >= 0, "write_exact: R < 0");
  if (R == 0) return KV800_OK;
  KV800_REQUIRE(epool && slot && k && v, "write_exact: null pointer");
  KV800_REQUIRE(ebs > 0 && s0 % 8 == 0 && s1 % 8 == 0 && s2 % 8 == 0 && e_v % 8 == 0,
                "write_exact: strides must be multiples of 8 elements and ebs > 0");
  KV800_REQUIRE(((uintptr_t)epool % 16) == 0 && ((uintptr_t)k % 16) == 0 && ((uintptr_t)v % 16) == 0,
                "write_exact: epool, k and v must be 16-byte aligned");
  const int nsink = sk ? NSINK : 0;
  KV800_REQUIRE(!nsink || (sv && pos && skoff && svoff && ((uintptr_t)sk % 16) == 0 && ((uintptr_t)sv % 16) == 0),
                "write_exact: sinks need sv, pos, skoff, svoff and 16-byte aligned sink buffers");
  KV800_REQUIRE(R * 128 <= 0x7FFFFFFFLL * 256, "write_exact: R too large");
  hipLaunchKernelGGL(write_exact_kernel, dim3((unsigned)((R * 128 + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     epool, s0, s1, s2, e_v, ebs, slot, k, v, R, pos, sk, sv, skoff, svoff, nsink);
  return check_launch("write_exact");
}

int kv800_hip_step_tables(const int32_t* qbt, int64_t qbt_stride, int64_t bsq, int64_t qs0, const int32_t* N,
                          int64_t R, int64_t nqmax, int64_t nnew, const int32_t* nnew_rows, int64_t* boff,
                          int32_t* NQ, int32_t* NP, int64_t* qbt64, int64_t* aux, int64_t aux_scale, int64_t aux_add,
                          void* stream) {
  KV800_REQUIRE(R >= 0 && nqmax >= 0 && nnew >= 0, "step_tables: R, nqmax and nnew must be >= 0");
  if (R == 0) return KV800_OK;
  KV800_REQUIRE(N && NQ && (!nqmax || boff) && ((!nqmax && !qbt64 && !aux) || (qbt && qbt_stride > 0)),
                "step_tables: null pointer");
  KV800_REQUIRE(bsq > 0 && bsq % BLK == 0, "step_tables: bsq must be a positive multiple of 256");
  KV800_REQUIRE(!nqmax || (nqmax - 1) * BLK / bsq < qbt_stride, "step_tables: nqmax exceeds the quant block table");
  KV800_REQUIRE(nnew <= 0x7FFFFFFF, "step_tables: nnew too large");
  int64_t w = nqmax > 0 ? nqmax : 1;
  if (qbt64 && qbt_stride > w) w = qbt_stride;
  const int64_t n = R * w;
  KV800_REQUIRE(n <= 0x7FFFFFFFLL * 256, "step_tables: table too large");
  hipLaunchKernelGGL(step_tables_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, qbt,
                     qbt_stride, bsq, qs0, N, R, nqmax, nnew, nnew_rows, boff, NQ, NP, qbt64, aux, aux_scale,
                     aux_add);
  return check_launch("step_tables");
}

int kv800_hip_decode_tables(const int32_t* qbt, int64_t qbt_stride, int64_t bsq, int64_t qs0, const int32_t* N,
                            int64_t R, int64_t nqmax, int64_t* boff, int32_t* NQ, void* stream) {
  return kv800_hip_step_tables(qbt, qbt_stride, bsq, qs0, N, R, nqmax, 0, nullptr, boff, NQ, nullptr, nullptr, nullptr,
                               0, 0, stream);
}

int kv800_hip_page_offsets(const int32_t* bt, int64_t bt_stride, int64_t R, int64_t npages, int64_t scale, int64_t add,
                           int64_t* out, void* stream) {
  KV800_REQUIRE(R >= 0 && npages >= 0 && bt_stride >= npages, "page_offsets: need R, npages >= 0, bt_stride >= npages");
  if (R == 0 || npages == 0) return KV800_OK;
  KV800_REQUIRE(bt && out, "page_offsets: null pointer");
  const int64_t n = R * npages;
  KV800_REQUIRE(n <= 0x7FFFFFFFLL * 256, "page_offsets: table too large");
  hipLaunchKernelGGL(page_offsets_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, bt,
                     bt_stride, R, npages, scale, add, out);
  return check_launch("page_offsets");
}

int kv800_hip_step_meta(const int32_t* bt, int64_t bt_stride, int64_t npages, const int64_t* lens, int64_t R,
                        int64_t ebs, int64_t* slot, int64_t* pos, int32_t* lens32, void* stream) {
  KV800_REQUIRE(R >= 0 && ebs > 0 && npages >= 0 && bt_stride >= npages, "step_meta: need R >= 0, ebs > 0, "
                "bt_stride >= npages >= 0");
  if (R == 0) return KV800_OK;
  KV800_REQUIRE((bt || npages == 0) && lens && slot && pos && lens32, "step_meta: null pointer");
  hipLaunchKernelGGL(step_meta_kernel, dim3((unsigned)((R + 255) / 256)), dim3(256), 0, (hipStream_t)stream, bt,
                     bt_stride, npages, lens, R, ebs, slot, pos, lens32);
  return check_launch("step_meta");
}

int kv800_hip_read_probe(const void* buf, int64_t bytes, uint32_t* out, int64_t groups, void* stream) {
  KV800_REQUIRE(buf && out, "read_probe: null pointer");
  KV800_REQUIRE(bytes >= 16 && bytes % 16 == 0 && ((uintptr_t)buf % 16) == 0,
                "read_probe: bytes must be a positive multiple of 16 and buf 16-byte aligned");
  KV800_REQUIRE(groups >= 1 && groups <= 65536, "read_probe: groups must be in [1, 65536]");
  hipLaunchKernelGGL(read_probe_kernel, dim3((unsigned)groups), dim3(256), 0, (hipStream_t)stream,
                     reinterpret_cast<const pv4*>(buf), bytes / 16, out);
  return check_launch("read_probe");
}

}  // extern "C"
