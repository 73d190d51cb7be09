/* kv800_hip.h -- C ABI of the MI355X (gfx950) backend of the lfm3-kv800 800h compressed KV-cache path.
 *
 * Conventions (all entry points):
 *   - Pointers are device pointers (HIP), except `kv800_paged_t` itself, which lives on the host and is read
 *     before launch. Offsets and strides are int64; byte offsets into the quant pool, element offsets (bf16) into
 *     the exact pool and the sink buffers, as in the reference's Paged descriptor (kv800.py:239-248).
 *   - `stream` is a hipStream_t passed as void* (torch.cuda.current_stream().cuda_stream); NULL = default stream.
 *     Launches are asynchronous: no entry point synchronizes, allocates or frees device memory.
 *   - Return 0 on success, otherwise a negative status; kv800_hip_last_error() returns a message for the calling
 *     thread's most recent failure. Invalid arguments are rejected on the host before any launch.
 *   - Layouts: quantized sub-block = 51,200 bytes (kv800.py:3-10): kc [256,4,32] | vb [256,4,16] | vlo [256,2] |
 *     vsc [256,2] | klo [4,128] | ksc [4,128]; exact token rows bf16 pre-RoPE K | unrotated V (V at +e_v elements).
 *   - Head shape is fixed by the format: 16 query heads over 4 KV heads, head_dim 128.
 */
#ifndef KV800_HIP_H
#define KV800_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KV800_OK 0
#define KV800_EINVAL (-1)   /* bad argument (checked on the host) */
#define KV800_EHIP (-2)     /* HIP runtime error at launch */

/* Paged descriptor of one layer; field for field kv800.Paged (kv800.py:239-248). */
typedef struct kv800_paged {
  const uint8_t* qpool;        /* quant pool base (bytes) */
  const int64_t* boff;         /* (B, boff_stride) byte offsets of sub-block j of row b */
  int64_t boff_stride;
  const uint16_t* epool;       /* exact pool base (bf16 elements) */
  const int64_t* eoff;         /* (B, eoff_stride) element offsets of the exact page holding position p (p / ebs) */
  int64_t eoff_stride;
  int64_t ebs, e_hs, e_ts, e_v;/* tokens per exact page; element strides of head, token; V offset from K */
  const uint16_t* sk;          /* sink K base (bf16) or NULL: no sinks (kv800.py:378-382) */
  const uint16_t* sv;          /* sink V base (bf16) */
  const int64_t* skoff;        /* (B,) element offsets of the [4 sinks, 4 heads, 128] K block of row b */
  const int64_t* svoff;        /* (B,) same for V */
  const int32_t* N;            /* (B,) sequence length including the current token */
  const int32_t* NQ;           /* (B,) flushed sub-blocks */
  int64_t nqmax;               /* host bound >= max(NQ) (0 on window layers) */
  int64_t win;                 /* 0: quantized layer; 256: window + sinks layer */
} kv800_paged_t;

/* Version of this ABI (major * 100 + minor). */
int kv800_hip_version(void);

/* Message of the calling thread's last failure ("" if none). */
const char* kv800_hip_last_error(void);

/* Quantize M dense sub-blocks. Replaces kv800.quantize_blocks (kv800.py:56-76).
 * k, v: (M, 256, 4, 128) bf16 (pre-RoPE K, unrotated V), contiguous. out: (M, 51200) bytes.
 * Bit-identical to the reference on CPU torch (fp8 e4m3fn RNE encode, IEEE division, v @ H as the sequential
 * fused multiply-add chain torch-CPU evaluates). */
int kv800_hip_quantize_blocks(const uint16_t* k, const uint16_t* v, int64_t M, uint8_t* out, void* stream);

/* Paged flush of the sub-blocks that became eligible. Replaces the flush plan + quantize of vllm_attn.py:297-317
 * (and the PagedStore flush loop, kv800.py:433-440) with one launch and no host loop:
 *   for every row r < R and sub-block j in [nq_prev[r], nq_new[r]) (at most max_new per row):
 *     gather tokens [256 j, 256 j + 256) of row r from the exact pool (K at eoff[r, p / ebs] + h e_hs + (p % ebs) e_ts,
 *     V at + e_v), quantize, and write the 51,200-byte sub-block to
 *     qpool + qbt[r, (256 j) / bsq] * qs0 + ((256 j) % bsq) / 256 * 51200.
 * vLLM geometry: qbt = the quant layer's block table, bsq = 1280 tokens per quant page, qs0 = 262144 bytes.
 * PagedStore geometry: qbt = boff (byte offsets), bsq = 256, qs0 = 1. */
int kv800_hip_flush(const uint16_t* epool, const int64_t* eoff, int64_t eoff_stride, int64_t ebs, int64_t e_hs,
                    int64_t e_ts, int64_t e_v, uint8_t* qpool, const int64_t* qbt, int64_t qbt_stride, int64_t bsq,
                    int64_t qs0, const int32_t* nq_prev, const int32_t* nq_new, int64_t R, int64_t max_new,
                    void* stream);

/* kv800_hip_flush with the same arguments and bytes, organised for the latency of a flush of few sub-blocks (a decode
 * step flushes at most one per row, usually one or two per layer): one token per V wave, each K row read once. Use
 * kv800_hip_flush when many sub-blocks are flushed at once (prefill chunks). */
int kv800_hip_flush_latency(const uint16_t* epool, const int64_t* eoff, int64_t eoff_stride, int64_t ebs, int64_t e_hs,
                            int64_t e_ts, int64_t e_v, uint8_t* qpool, const int64_t* qbt, int64_t qbt_stride,
                            int64_t bsq, int64_t qs0, const int32_t* nq_prev, const int32_t* nq_new, int64_t R,
                            int64_t max_new, void* stream);

/* Dequantize M sub-blocks. Replaces kv800.dequantize_blocks (kv800.py:79-92).
 * k_out: (M, 256, 4, 128) bf16 = bf16(code * ksc + klo); v_out: (M, 256, 4, 128) f32 = (bit * vsc + vlo) @ H. */
int kv800_hip_dequantize_blocks(const uint8_t* sb, int64_t M, uint16_t* k_out, float* v_out, void* stream);

/* bf16 (cos, sin) pair table used by the quantized-decode kernel: cs2[p * 32 + j] = cos[p, j] | sin[p, j] << 16 (bf16
 * bits) for p < P. cos_t, sin_t: (>= P, 32) bf16. No reference counterpart (it reads the two bf16 tables per token,
 * kv800.py:146-147); the interleave lets one 16-byte load give a lane both values of 4 channels. */
int kv800_hip_rope_table(const uint16_t* cos_t, const uint16_t* sin_t, int64_t P, uint32_t* cs2, void* stream);

/* Split-K partial attention over the flushed sub-blocks. Replaces torch.ops.kv800.qdecode (kv800_sycl.sycl:510-526,
 * Triton _qdec kv800.py:120-170). For each row b and split s < ns: sub-blocks [s spb, min((s+1) spb, nq[b])) ->
 * mo, lo (B, ns+1, 16) and ao (B, ns+1, 16, 128) at slot s, V in the Hadamard domain (acc + sum p vlo).
 * q: (B, 16, 128) bf16 post-RoPE; cs2: kv800_hip_rope_table of rows >= max(nq) * 256 (the reference op takes the two
 * bf16 tables instead); scale = log2(e)/sqrt(128). Keys as torch_decode forms them: bf16(code * ksc + klo), rotated in
 * fp32 and rounded to bf16 (torch_decode.py:16-24). */
int kv800_hip_decode_quant(const uint16_t* q, const uint8_t* qpool, const int64_t* boff, int64_t boff_stride,
                           const int32_t* nq, const uint32_t* cs2, float* mo, float* lo, float* ao, int64_t B,
                           int64_t ns, int64_t spb, float scale, void* stream);

/* Sinks + exact tail. Replaces torch.ops.kv800.xdecode (kv800_sycl.sycl:528-542, Triton _xdec kv800.py:197-228):
 * positions [lo_e, N[b]) with lo_e = NQ[b] * 256 (window layers: max(lo_e, N - win)) and, when P->sk != NULL,
 * sinks at positions < min(4, lo_e, N) -> slot ns of mo / lo / ao. cos_t, sin_t: (>= max(N), 32) bf16.
 * The exact pool must hold at least one 128-element row (masked lanes read row 0 and discard it). */
int kv800_hip_decode_exact(const kv800_paged_t* P, const uint16_t* q, const uint16_t* cos_t, const uint16_t* sin_t,
                           float* mo, float* lo, float* ao, int64_t B, int64_t ns, float scale, void* stream);

/* LSE merge of the ns + 1 slots. Replaces torch.ops.kv800.combine (kv800_sycl.sycl:544-551, kv800.combine
 * kv800.py:231-236): H (FWHT) on the quantized slots, exact slot as is, bf16 (B, 16, 128) out. */
int kv800_hip_decode_merge(const float* mo, const float* lo, const float* ao, int64_t B, int64_t ns, uint16_t* out,
                           void* stream);

/* Fixed-grid split plan, (ns, spb) with about two workgroups per CU, for the staged entry points above
 * (kv800.py:366-367 plans for the reference kernels). */
int kv800_hip_plan(int64_t B, int64_t nqmax, int64_t* ns, int64_t* spb);

/* Workspace bytes kv800_hip_decode needs for B rows, ns splits (spb > 0) and rope rows (0 if cs2 is passed in). */
int64_t kv800_hip_decode_workspace(int64_t B, int64_t ns, int64_t rope_rows);

/* Balanced schedule of kv800_hip_decode (spb <= 0): the batch's sub-blocks laid end to end and cut into `groups`
 * equal ranges, one workgroup each, so ragged batches keep every CU busy to the end. No reference counterpart (the
 * reference splits every row into ns fixed splits). plan_balanced: the group count used for spb == 0;
 * workspace_balanced: the workspace bytes for `groups` groups. */
int kv800_hip_plan_balanced(int64_t B, int64_t nqmax, int64_t* groups);
int64_t kv800_hip_decode_workspace_balanced(int64_t B, int64_t groups, int64_t rope_rows);

/* Fused decode of one layer. Replaces kv800.decode's backend body (kv800.py:352-383): [rope table], the quantized
 * work and the exact tail in one grid, then the merge, all on `stream` (window layers: one launch, the exact tail
 * fused with the merge). cs2 may be NULL (then it is built in the workspace from cos_t / sin_t for the nqmax * 256
 * rows the quantized kernel reads). spb > 0: fixed grid of ceil(nqmax / spb) splits per row; spb == 0: balanced
 * schedule with kv800_hip_plan_balanced's groups; spb < 0: balanced schedule with -spb groups. */
int kv800_hip_decode(const kv800_paged_t* P, const uint16_t* q, int64_t B, const uint16_t* cos_t,
                     const uint16_t* sin_t, const uint32_t* cs2, uint16_t* out, void* workspace,
                     int64_t workspace_bytes, int64_t spb, void* stream);

/* Training fake quantization, the forward value of train.py's straight-through 800h K / V (train.py:82-100), on the
 * device: fake_quant_k replaces fake_quant_k (x (G, 256, C) fp32 -> c * sc8 + lo8 per (group, channel), bit-identical
 * to the quantizer's K path); fake_quant_v replaces fake_quant_v (v (N, 4, 128) fp32 -> the V of a quantize ->
 * dequantize round trip, Hadamard in the quantizer's / dequantizer's fp32 chain). out may not alias the input. */
int kv800_hip_fake_quant_k(const float* x, int64_t G, int64_t C, float* out, void* stream);
int kv800_hip_fake_quant_v(const float* v, int64_t N, float* out, void* stream);

/* Prefill over compressed history (vllm_attn.py:351-380): row r's positions [0, P->N[r]) written as contiguous bf16
 * K and V at rows out_off[r] + p of k_out / v_out ((S, 4, 128) each). Positions below 256 * P->NQ[r] are dequantized
 * from their sub-block (dequantize_blocks, kv800.py:79-92; V cast to bf16), the others read from the exact pages.
 * With cos_t / sin_t ((rope_rows, 32) bf16) the keys are rotated as the reference's _rope (vllm_attn.py:160-163) does
 * over its 128-wide tables; NULL leaves them unrotated (sliding layers). P's sink and window fields are ignored.
 * max_n >= every P->N[r]; rows, sub-blocks or positions outside their pools / tables are written as zeros. */
int kv800_hip_history(const kv800_paged_t* P, int64_t R, int64_t max_n, const uint16_t* cos_t, const uint16_t* sin_t,
                      int64_t rope_rows, int64_t qpool_bytes, int64_t epool_elems, const int64_t* out_off,
                      uint16_t* k_out, uint16_t* v_out, void* stream);

/* Keys (S, 4, 128) bf16 rotated at positions pos (S,) int64 with the (rope_rows, 32) bf16 tables of the 32 rotating
 * frequencies, replacing the reference's _rope over its 128-wide tables (vllm_attn.py:160-163): per element
 * k * c + rot(k) * s in fp32 with c = 1, s = 0 on dims without a frequency, rounded to bf16 -- bit-identical. out may
 * not alias k. Positions outside the table are clamped into it (a caller error that stays in bounds). */
int kv800_hip_rope_rows(const uint16_t* k, const int64_t* pos, int64_t S, const uint16_t* cos_t,
                        const uint16_t* sin_t, int64_t rope_rows, uint16_t* out, void* stream);

/* Prefill / extend attention of R ragged rows, replacing the reference's prefill attention (vllm_attn.py:168-211 with
 * the masks of 176-184): row r has queries q[qsl[r], qsl[r+1]) ((T, 16, 128) bf16, post-RoPE) at positions
 * qpos0[r] + 0, 1, ... and keys / values K, V[ksl[r], ksl[r+1]) ((S, 4, 128) bf16, rotated as the layer stores them for
 * attention) at positions kp (int32, ascending within a row; kp = NULL: key j of a row is at position j, the order in
 * which quantized layers assemble history and new rows); query head h reads KV head h / 4. A key is kept when
 * kp <= the query's position and, with window > 0, kp > position - window or kp < nsink (nsink 4 for window + sinks
 * layers, 0 for sliding layers; window 0 for quantized layers). Scale 128^-0.5, fp32 scores and softmax, bf16
 * probabilities times bf16 V with fp32 accumulation, bf16 out (T, 16, 128). tile_off (R + 1, int64) is the prefix sum of
 * ceil((qsl[r+1] - qsl[r]) / 32) (the rows' 32-query tiles), ntiles = tile_off[R] < 2^29. */
int kv800_hip_prefill(const uint16_t* q, const int64_t* qsl, const int64_t* qpos0, const uint16_t* K,
                      const uint16_t* V, const int32_t* kp, const int64_t* ksl, const int64_t* tile_off, int64_t R,
                      int64_t ntiles, int64_t window, int64_t nsink, uint16_t* out, void* stream);

/* kv800_hip_prefill with each (query tile, KV head) split over `splits` (1 .. 256) ranges of its key tiles, for
 * batches of few query tiles over long histories (a short extend chunk, a decode-like row): each split writes the
 * unnormalised partial (o, m, l) of its queries to part (T x 16 heads x splits x 132 floats, T = qsl[R] the total
 * query count, part_floats its size), and a second launch merges the splits (log-sum-exp) into out. splits = 1 is
 * kv800_hip_prefill (part unused). Same arguments and masks otherwise; the same reference attention
 * (vllm_attn.py:168-211), summed in a different order across the splits. */
int kv800_hip_prefill_split(const uint16_t* q, const int64_t* qsl, const int64_t* qpos0, const uint16_t* K,
                            const uint16_t* V, const int32_t* kp, const int64_t* ksl, const int64_t* tile_off,
                            int64_t R, int64_t ntiles, int64_t T, int64_t window, int64_t nsink, int64_t splits,
                            float* part, int64_t part_floats, uint16_t* out, void* stream);

/* Step bookkeeping in vLLM's page geometry (exact page [4 heads, ebs, K128 | V128] bf16 with element strides s0 (page),
 * s1 (head), s2 (token); quant page = 5 x 51,200-byte sub-blocks per 1280 tokens, qs0 bytes apart). */

/* Write the step's pre-RoPE K and unrotated V rows, k / v (R, 4, 128) bf16, to slot[r] (page slot / ebs, offset
 * slot % ebs; slot < 0 = padding, skipped). Replaces the index_put of vllm_attn.py:263-272. With sk != NULL (window
 * layers) rows at pos[r] < 4 are also written to the sink blocks [4 sinks, 4, 128] at sk + skoff[r] / sv + svoff[r]
 * (the aux area of the host layers' first quant page), replacing vllm_attn.py:276-291. */
int kv800_hip_write_exact(uint16_t* epool, int64_t s0, int64_t s1, int64_t s2, int64_t e_v, int64_t ebs,
                          const int64_t* slot, const uint16_t* k, const uint16_t* v, int64_t R, const int64_t* pos,
                          uint16_t* sk, uint16_t* sv, const int64_t* skoff, const int64_t* svoff, void* stream);

/* Decode tables of a quantized layer, replacing vllm_attn.py:332-340: NQ[r] = max(N[r] - 128, 0) / 256 and, for
 * j < nqmax, boff[r, j] = qbt[r, 256 j / bsq] * qs0 + (256 j % bsq) / 256 * 51200 (boff row stride nqmax). qbt: the
 * quant group's (R, qbt_stride) int32 block table. */
int kv800_hip_decode_tables(const int32_t* qbt, int64_t qbt_stride, int64_t bsq, int64_t qs0, const int32_t* N,
                            int64_t R, int64_t nqmax, int64_t* boff, int32_t* NQ, void* stream);

/* All per-step tables of the quant KV group in one launch: decode_tables' NQ / boff plus, where non-NULL,
 * NP[r] = max(N[r] - m_r - 128, 0) / 256 with m_r = nnew_rows[r] if nnew_rows is non-NULL, else nnew (the sub-blocks
 * flushed before the step's m_r tokens of row r, i.e. nq(seq_len - query_len): the flush range is [NP, NQ),
 * vllm_attn.py:270-277, 297-317; a mixed step's decode rows have m_r = 1, its extend rows their chunk length),
 * qbt64 = qbt as int64 (R, qbt_stride) for kv800_hip_flush, and aux[r] = qbt[r, 0] * aux_scale + aux_add (the sink
 * aux area of each row's first quant page, vllm_attn.py:276-291). */
int kv800_hip_step_tables(const int32_t* qbt, int64_t qbt_stride, int64_t bsq, int64_t qs0, const int32_t* N,
                          int64_t R, int64_t nqmax, int64_t nnew, const int32_t* nnew_rows, int64_t* boff,
                          int32_t* NQ, int32_t* NP, int64_t* qbt64, int64_t* aux, int64_t aux_scale, int64_t aux_add,
                          void* stream);

/* One decode step's metadata of a KV group (every row appends one token): for r < R with lens[r] = n (int64, the
 * length including the new token), pos[r] = n - 1, slot[r] = bt[r, pos / ebs] * ebs + pos % ebs (int64; -1 for n = 0
 * or a page index >= npages, a padding token) and lens32[r] = n. bt: (R, bt_stride) int32 block table. The
 * reference's vLLM scheduler hands these to the backend (slot_mapping, seq_lens, vllm_attn.py:255-270); here one
 * launch replaces the per-step torch ops that derive them. */
int kv800_hip_step_meta(const int32_t* bt, int64_t bt_stride, int64_t npages, const int64_t* lens, int64_t R,
                        int64_t ebs, int64_t* slot, int64_t* pos, int32_t* lens32, void* stream);

/* off[r, p] = bt[r, p] * scale + add for p < npages (off row stride npages): an exact group's (R, bt_stride) int32
 * block table as element offsets of its pages, the eoff table the decode and flush read (the reference forms it with
 * torch ops per step, vllm_attn.py:320-323). */
int kv800_hip_page_offsets(const int32_t* bt, int64_t bt_stride, int64_t R, int64_t npages, int64_t scale, int64_t add,
                           int64_t* out, void* stream);

/* Bounds-checked forms used by the Python layer. They take the extent of every pool the kernels read, measured from
 * the pointer passed in: qpool_bytes (bytes), epool_elems / sink_elems (bf16 elements), rope_rows (rows of cos_t /
 * sin_t and of cs2). A sub-block, page or row whose offset falls outside its pool is skipped instead of read, so a
 * malformed table yields a wrong (finite) result rather than a memory fault. The unsized forms above pass
 * INT64_MAX / 2 for every extent. No reference counterpart: the reference's kernels read unchecked. */
int kv800_hip_decode_quant_sized(const uint16_t* q, const uint8_t* qpool, int64_t qpool_bytes, const int64_t* boff,
                                 int64_t boff_stride, const int32_t* nq, const uint32_t* cs2, int64_t rope_rows,
                                 float* mo, float* lo, float* ao, int64_t B, int64_t ns, int64_t spb, float scale,
                                 void* stream);
int kv800_hip_decode_exact_sized(const kv800_paged_t* P, const uint16_t* q, const uint16_t* cos_t,
                                 const uint16_t* sin_t, int64_t rope_rows, int64_t epool_elems, int64_t sink_elems,
                                 float* mo, float* lo, float* ao, int64_t B, int64_t ns, float scale, void* stream);
int kv800_hip_decode_sized(const kv800_paged_t* P, const uint16_t* q, int64_t B, const uint16_t* cos_t,
                           const uint16_t* sin_t, int64_t rope_rows, const uint32_t* cs2, int64_t qpool_bytes,
                           int64_t epool_elems, int64_t sink_elems, uint16_t* out, void* workspace,
                           int64_t workspace_bytes, int64_t spb, void* stream);

/* kv800_hip_decode_sized without a workspace argument and without any allocation: the partials (and the rope pair table
 * when cs2 is NULL) go to a static per-device scratch of 32 MiB inside the library, resolved with hipGetSymbolAddress on
 * the first call on each device. No counterpart in the reference: it is for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). Limit: a call whose schedule
 * needs more than 32 MiB (kv800_hip_decode_workspace / _balanced) is rejected with KV800_EINVAL. Every call on one device
 * shares that device's scratch: calls that overlap on one device (concurrent streams or threads) race. The stream must
 * belong to the current device. Nothing in the scratch has to start at zero (every slot a kernel reads is written by
 * the same call). */
int kv800_hip_decode_noalloc(const kv800_paged_t* P, const uint16_t* q, int64_t B, const uint16_t* cos_t,
                             const uint16_t* sin_t, int64_t rope_rows, const uint32_t* cs2, int64_t qpool_bytes,
                             int64_t epool_elems, int64_t sink_elems, uint16_t* out, int64_t spb, void* stream);

/* Streaming read of bytes (a positive multiple of 16) from buf with `groups` workgroups (8 plain 16-byte loads in
 * flight per lane), writing one xor word per workgroup to out[0 .. groups). No counterpart in the reference: a
 * measurement aid, the read bandwidth the part sustains for plain loads, against which bench.py sets the kernels'
 * achieved bandwidth. */
int kv800_hip_read_probe(const void* buf, int64_t bytes, uint32_t* out, int64_t groups, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* KV800_HIP_H */
