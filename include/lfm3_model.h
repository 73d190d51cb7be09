/* lfm3_model.h -- C ABI of the fused elementwise kernels of the LFM3-shaped engine loop (lfm3-kv800_amd/model.py),
 * in the same library as the 800h path (lfm3-kv800_amd/_lib/libkv800_hip.so).
 *
 * No counterpart in the reference's own code: its model (vllm_model.py:195-471) runs these steps through vLLM's fused
 * RMSNorm / rotary / activation ops and its linear layers. Conventions as include/kv800_hip.h: device pointers to bf16 (uint16_t) data,
 * `stream` a hipStream_t as void*, asynchronous launches, 0 on success or a negative status with
 * kv800_hip_last_error(). Every result is rounded to bf16 where the corresponding torch op on bf16 tensors rounds;
 * rms(x) = x rsqrt(mean(x^2) + eps) in fp32.
 */
#ifndef LFM3_MODEL_H
#define LFM3_MODEL_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Sandwich-norm step on (R, H) rows, H = 2048: with h != NULL, x_out = x + bf16(rms(h) w_post) (the residual after a
 * sub-layer, vllm_model.py:446-471); then, with n_out != NULL, n_out = bf16(rms(x') w_next), x' = x_out (or x when h
 * is NULL: a plain RMS norm). x_out may alias x. */
int lfm3_hip_add_rmsnorm(const uint16_t* h, const uint16_t* x, const uint16_t* w_post, const uint16_t* w_next,
                         float eps, int64_t R, int64_t H, uint16_t* x_out, uint16_t* n_out, void* stream);

/* Gated activation: row r of gu (R, 2F) is [g | u]; out (R, F) = bf16(bf16(silu(g)) u). */
int lfm3_hip_silu_mul(const uint16_t* gu, int64_t R, int64_t F, uint16_t* out, void* stream);

/* Attention input of one layer: row r of qkv (row stride `stride` >= 3072) holds q (16 heads x 128), k (4 x 128),
 * v (4 x 128). q and k get a per-head RMS norm (weights q_w, k_w of 128), then the neox RoPE at position pos[r] from
 * the (P, 64) bf16 tables cos_t / sin_t of the 64 frequencies (dims f and f + 64 share frequency f; a zero frequency
 * has cos 1, sin 0): q_out (R, 16, 128) rotated, k_pre (R, 4, 128) normalized and unrotated, k_rot rotated, v_out
 * (R, 4, 128) the v rows. Positions outside the tables are clamped into them. */
int lfm3_hip_qkv_post(const uint16_t* qkv, int64_t stride, const uint16_t* q_w, const uint16_t* k_w,
                      const uint16_t* cos_t, const uint16_t* sin_t, int64_t P, const int64_t* pos, float eps,
                      int64_t R, uint16_t* q_out, uint16_t* k_pre, uint16_t* k_rot, uint16_t* v_out, void* stream);

/* Short-conv decode step: row r of bcx (row stride >= 3H) is [B | C | x]; with window = [state (6 taps) | bf16(B x)]
 * per channel, y = bf16(sum_k bf16(window_k conv_w[c, k])), state <- window[1:] (in place), out = bf16(C y).
 * conv_w (H, 7), state (R, H, 6), out (R, H). */
int lfm3_hip_conv_step(const uint16_t* bcx, int64_t stride, const uint16_t* conv_w, uint16_t* state, int64_t R,
                       int64_t H, uint16_t* out, void* stream);

/* Attention output gate: out (R, 16, 128) = o bf16(sigmoid(g)) per head; row r's 16 gate logits at g + r gstride. */
int lfm3_hip_gate_mul(const uint16_t* o, const uint16_t* g, int64_t gstride, int64_t R, uint16_t* out, void* stream);

/* Greedy token: out[r] (int64) = index of the largest of the V bf16 values of row r (row stride `stride` elements):
 * among equal values the first, and a NaN ranks above every number (the first NaN wins), as torch.argmax over the
 * same values. V and stride multiples of 8, x 16-byte aligned. */
int lfm3_hip_argmax(const uint16_t* x, int64_t R, int64_t V, int64_t stride, int64_t* out, void* stream);

/* Dense products y = x W^T of the decode batch (lfm3-kv800_amd/csrc/lfm3_gemm.hip). W (N, K) bf16 is stored once in
 * the B-operand order of the 32 x 32 x 16 bf16 MFMA: wsh holds Npad / 32 x K / 16 blocks of 512 bf16, block
 * (nt, ks) lane l = W[32 nt + l % 32][16 ks + 8 (l / 32) .. + 8], rows n >= N zero. K a multiple of 64, Npad of 128. */
int lfm3_hip_shuffle_weight(const uint16_t* w, int64_t N, int64_t K, int64_t Npad, uint16_t* wsh, void* stream);

/* y (R, Npad; row stride ldy) = bf16(x (R, K; row stride ldx) . W^T) with fp32 accumulation, W as shuffled above;
 * ldx and ldy multiples of 8, x and y 16-byte aligned.
 * split > 1 cuts K into `split` equal parts (multiples of 64) whose fp32 partials go to work (split x R x Npad floats)
 * and are summed in part order before the rounding (split 1: work unused). glu = 1 (split 1): W's rows come in 128-row
 * groups [64 gate rows | the matching 64 up rows] and y (R, Npad / 2) = bf16(bf16(silu(g)) u) of the bf16 products,
 * the gated activation of lfm3_hip_silu_mul on a [g | u] product. */
int lfm3_hip_linear(const uint16_t* x, int64_t ldx, const uint16_t* wsh, int64_t R, int64_t Npad, int64_t K,
                    uint16_t* y, int64_t ldy, int split, float* work, int glu, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LFM3_MODEL_H */
