/*
 * mq4.h -- C ABI of the MI355X (gfx950) MLX-affine Q4 matrix-product library.
 *
 * Data formats are MLX's affine 4-bit layout, byte for byte, so tensors
 * produced by mx::quantize load unchanged:
 *   w      bf16 [N, K] row-major (uint16_t bit patterns)
 *   wq     uint32 [N, K/8]; nibble p (bits 4p..4p+3) of word j holds element
 *          8j+p of the row (low nibble first)
 *   scales bf16 [N, K/64], biases bf16 [N, K/64]; element k of row n
 *          dequantizes to scales[n, k/64] * q + biases[n, k/64]
 *   x      bf16 [M, K] row-major; y bf16 [M, N] row-major
 * Only group_size 64 and bits 4 are implemented; other values return
 * MQ4_ERR_UNSUPPORTED.  K must be a positive multiple of 64, at most 32768
 * for the matrix products (larger K returns MQ4_ERR_UNSUPPORTED).
 *
 * All pointers are device pointers (hipMalloc'd or equivalent) and `stream`
 * is a hipStream_t (NULL = the default stream).  Every call is asynchronous
 * and stream-ordered: it validates its arguments on the host, enqueues its
 * kernels and returns; no call synchronizes the device.  Errors are returned
 * as negative status codes with a message in mq4_last_error() (per host
 * thread); no C++ exception crosses this boundary.
 *
 * Reference seams replaced (paths relative to the marlin-mlx repository):
 *   mq4_quantize         mx::quantize(w, 64, 4) in quantize_weight
 *                        (src/model/weights.cpp:45-56) and the lm_head load
 *                        (src/model/weights.cpp:180-194)
 *   mq4_quantize_batch   the loader's loop of those quantizes over every
 *                        layer (src/model/weights.cpp:97-104, 147-160, 180-194)
 *   mq4_qmm              mx::quantized_matmul(x, w, s, b, true, 64, 4) in
 *                        qmatmul (src/model/marlin.cpp:18-25) and
 *                        MarlinModel::lm_head (src/model/marlin.cpp:161-169)
 *   mq4_mlp_gate_up_silu swiglu(qmatmul(x, gate), qmatmul(x, up))
 *                        (src/model/marlin.cpp:27-33)
 *   mq4_rmsnorm_gate_up_silu  the same after rms_norm (src/model/marlin.cpp:141)
 *   mq4_swiglu_bf16      swiglu(gate, up) (src/model/marlin.cpp:27-29)
 *   mq4_qmm_residual     hidden + qmatmul(h, down)
 *   mq4_mlp_residual     hidden + mlp_forward(rms_norm(hidden)) in one call
 *                        (src/model/marlin.cpp:141-142, 31-35)
 *                        (src/model/marlin.cpp:34, 142)
 *   mq4_lm_head_argmax   sample_token(lm_head(h)) with temperature <= 0
 *                        (src/model/marlin.cpp:161-169,
 *                        src/sampling/sampler.cpp:9-16)
 *   mq4_rmsnorm_lm_head_argmax  the same after the final rms_norm
 *                        (src/model/marlin.cpp:145)
 *   mq4_argmax_bf16      mx::argmax(last_logits, -1)
 *                        (src/sampling/sampler.cpp:15)
 *   mq4_sample_bf16      sample_token (src/sampling/sampler.cpp:9-39):
 *                        temperature, top-k, top-p and the categorical draw
 *   mq4_rms_norm         rms_norm (src/model/marlin.cpp:12-16)
 *   mq4_decode_step      the per-token MLP + lm_head + greedy token loop body
 *                        (src/model/marlin.cpp:110-145, 161-169;
 *                        src/sampling/sampler.cpp:14-16) in one launch
 */
#ifndef MQ4_H
#define MQ4_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum mq4_status {
    MQ4_OK = 0,
    MQ4_ERR_INVALID_ARG = -1,   /* null pointer, non-positive or inconsistent shape */
    MQ4_ERR_UNSUPPORTED = -2,   /* group_size != 64, bits != 4, transpose == 0, K too large */
    MQ4_ERR_ALIGNMENT = -3,     /* pointer not aligned as the call requires */
    MQ4_ERR_HIP = -4,           /* a HIP runtime call or kernel launch failed */
    MQ4_ERR_WORKSPACE = -5      /* workspace missing or too small */
};

/* Message for the last failing call on this host thread ("" if none). */
const char* mq4_last_error(void);

/* Library version, major*10000 + minor*100 + patch. */
int mq4_version(void);

/* ---------------------------------------------------------------------- */
/* Quantize / pack.  Replaces mx::quantize(w, group_size=64, bits=4)
 * (src/model/weights.cpp:46 and :183).  Bit-exact MLX affine quantization
 * computed in float32: per group of 64, scale = +-max((max-min)/15, 1e-7)
 * (negative unless |min| > |max|), edge = the larger-magnitude extreme,
 * q0 = rint(edge/scale), scale = edge/q0 and bias = edge when q0 != 0 (else
 * bias = 0), q = clip(rint((w - bias)/scale), 0, 15) with round-half-even.
 * w must be 16-byte aligned, wq 4-byte, scales/biases 2-byte. */
int mq4_quantize(const uint16_t* w, int64_t N, int64_t K, int group_size, int bits,
                 uint32_t* wq, uint16_t* scales, uint16_t* biases, void* stream);

/* One matrix of a batched quantize: w bf16 [N, K] in, wq/scales/biases out,
 * the same layout and alignment as mq4_quantize. */
typedef struct mq4_quantize_job {
    const uint16_t* w;
    int64_t N, K;
    uint32_t* wq;
    uint16_t* scales;
    uint16_t* biases;
} mq4_quantize_job;

/* Quantize every job of a weight set in as few launches as possible (one per
 * 32 jobs), with the same bits as n_jobs separate mq4_quantize calls.
 * Replaces the loader's loop of quantizes: quantize_weight for gate, up and
 * down of every layer (load_mlp, src/model/weights.cpp:97-104, called per
 * layer at :147-160) and the lm_head's mx::quantize (:180-194).  The job
 * table is read on the host during the call; every job is validated before
 * anything is enqueued (on an error nothing runs and the message names the
 * job).  Jobs must not overlap in their outputs. */
int mq4_quantize_batch(const mq4_quantize_job* jobs, int64_t n_jobs, int group_size, int bits,
                       void* stream);

/* Dequantize: out = scales*q + biases, rounded once (round-to-nearest-even)
 * to bf16 (out_f32 == 0, out is uint16_t*) or stored exactly as float
 * (out_f32 != 0, out is float*).  Test and inspection helper. */
int mq4_dequantize(const uint32_t* wq, const uint16_t* scales, const uint16_t* biases,
                   int64_t N, int64_t K, int group_size, int bits, void* out, int out_f32,
                   void* stream);

/* ---------------------------------------------------------------------- */
/* y[M, N] = x[M, K] @ dequant(wq, scales, biases)^T, fp32 accumulation,
 * one bf16 rounding of each output.  Replaces
 * mx::quantized_matmul(x, w, scales, biases, transpose=true, 64, 4)
 * (src/model/marlin.cpp:20-22 and :164-166).  transpose must be 1 (the only
 * form the reference uses).  x and wq must be 16-byte aligned. */
int mq4_qmm(const uint16_t* x, int64_t M, int64_t K,
            const uint32_t* wq, const uint16_t* scales, const uint16_t* biases, int64_t N,
            int transpose, int group_size, int bits, uint16_t* y, void* stream);

/* Same product as mq4_qmm with the fp32 accumulator stored unrounded in
 * y (float [M, N]): for accuracy checks against an fp64 reference and for
 * callers that keep fp32 outputs.  y must be 4-byte aligned. */
int mq4_qmm_f32(const uint16_t* x, int64_t M, int64_t K,
                const uint32_t* wq, const uint16_t* scales, const uint16_t* biases, int64_t N,
                float* y, void* stream);

/* y = bf16(residual + bf16(x @ W^T)): the down projection with the residual
 * add that follows it (src/model/marlin.cpp:34 and :142).  residual [M, N]
 * may alias y (in-place update of the hidden state). */
int mq4_qmm_residual(const uint16_t* x, int64_t M, int64_t K,
                     const uint32_t* wq, const uint16_t* scales, const uint16_t* biases,
                     int64_t N, const uint16_t* residual, uint16_t* y, void* stream);

/* h[M, N] = swiglu(x @ Wg^T, x @ Wu^T) with MLX's bf16 op order
 * (src/model/marlin.cpp:27-33): g = bf16(x@Wg^T), u = bf16(x@Wu^T),
 * h = bf16(bf16(bf16(sigmoid(g)) * g) * u).  gate and up are both [N, K]. */
int mq4_mlp_gate_up_silu(const uint16_t* x, int64_t M, int64_t K,
                         const uint32_t* gate_wq, const uint16_t* gate_scales,
                         const uint16_t* gate_biases,
                         const uint32_t* up_wq, const uint16_t* up_scales,
                         const uint16_t* up_biases,
                         int64_t N, uint16_t* h, void* stream);

/* The same with the (1 + w) RMSNorm that precedes the MLP fused in front:
 * xn = bf16(x * rsqrt(mean(x^2) + eps) * (1 + norm_weight)) per row (fp32
 * math, one rounding), h = swiglu(xn @ Wg^T, xn @ Wu^T).  Replaces
 * rms_norm(hidden, post_attn_norm) + mlp_forward's gate/up/swiglu
 * (src/model/marlin.cpp:141, 12-16, 27-33).  norm_weight is bf16 [K],
 * 16-byte aligned.  From M = 33 rows on, mq4_rms_norm into a [M, K] buffer
 * followed by mq4_mlp_gate_up_silu gives the same normalized operand and
 * takes about half the time (this fused form normalizes every activation
 * tile in registers before staging it). */
int mq4_rmsnorm_gate_up_silu(const uint16_t* x, int64_t M, int64_t K,
                             const uint16_t* norm_weight, float eps,
                             const uint32_t* gate_wq, const uint16_t* gate_scales,
                             const uint16_t* gate_biases,
                             const uint32_t* up_wq, const uint16_t* up_scales,
                             const uint16_t* up_biases,
                             int64_t N, uint16_t* h, void* stream);

/* One transformer block's MLP half: y = x + down(swiglu(gate(n), up(n))),
 * n = rms_norm(x) with the (1 + w) multiplier, i.e. rms_norm (marlin.cpp:141,
 * 12-16), mlp_forward (:31-35) and the residual add (:142) of
 * text_forward_embeddings, for M rows.  gate and up are [N, K], down [K, N];
 * norm_weight is bf16 [K], 16-byte aligned.  The result is within the GEMM
 * bar of the chain mq4_rmsnorm_gate_up_silu + mq4_qmm_residual (the same
 * normalized operand and bf16 h; fp32 sums in another order, so not always
 * bit for bit).  From M = 33 rows on (K and N multiples of 512, scale and
 * bias rows 4-byte aligned) it runs the MFMA GEMM on activations stored in
 * the matrix cores' operand order: a pre-pass writes the normalized x so, the
 * SwiGLU epilogue writes h so.  With every scale and bias row 16-byte
 * aligned the products use fp16 weights (fp16(s q + b), about 2e-6 of the
 * output rms from the exact product) on an fp16 copy of the operands, and
 * the down product runs in 1, 2 or 4 K parts whose fp32 sums go to the
 * workspace and are added in order with the residual; otherwise the exact
 * bf16 operands with their group sums.  From 5 to 32 rows
 * (with 64 < N / 64 <= 96) the down product runs as two halves of K per
 * 16-row tile on different workgroups.  Their fp32 sums go to the workspace
 * and a combine pass adds them with the residual, bit for bit what
 * mq4_qmm_residual gives.  workspace: at least mq4_mlp_workspace_size(M, K,
 * N) bytes, 256-byte aligned, no initialisation; calls that overlap in time
 * need separate workspaces.  y may equal x (in place).
 * mq4_mlp_workspace_size(M, K, N) is enough for every call of at most M rows
 * with the same K and N: it never shrinks as M grows. */
size_t mq4_mlp_workspace_size(int64_t M, int64_t K, int64_t N);
int mq4_mlp_residual(const uint16_t* x, int64_t M, int64_t K,
                     const uint16_t* norm_weight, float eps,
                     const uint32_t* gate_wq, const uint16_t* gate_scales,
                     const uint16_t* gate_biases,
                     const uint32_t* up_wq, const uint16_t* up_scales,
                     const uint16_t* up_biases,
                     const uint32_t* down_wq, const uint16_t* down_scales,
                     const uint16_t* down_biases,
                     int64_t N, void* workspace, size_t workspace_bytes,
                     uint16_t* y, void* stream);

/* out[i] = bf16(bf16(bf16(sigmoid(gate[i])) * gate[i]) * up[i]): the
 * unfused swiglu (src/model/marlin.cpp:27-29) over n bf16 elements. */
int mq4_swiglu_bf16(const uint16_t* gate, const uint16_t* up, int64_t n, uint16_t* out,
                    void* stream);

/* out[m, :] = bf16(x[m, :] * rsqrt(mean(x[m, :]^2) + eps) * (1 + weight)),
 * computed in fp32 with one rounding: rms_norm with the (1 + w) multiplier
 * (src/model/marlin.cpp:12-16), the step before the lm_head
 * (src/model/marlin.cpp:145).  Not a quantized op; provided so a decode step
 * runs entirely in this library. */
int mq4_rms_norm(const uint16_t* x, int64_t M, int64_t K, const uint16_t* weight, float eps,
                 uint16_t* out, void* stream);

/* ---------------------------------------------------------------------- */
/* Greedy lm_head: logits = bf16(h @ W^T) for each of the M rows and
 * idx[m] = argmax over the N bf16 logits of row m, the lowest index winning
 * ties (mx::argmax semantics; src/sampling/sampler.cpp:15).  logits (may be
 * NULL) receives the [M, N] bf16 logits.  workspace is device memory of at
 * least mq4_lm_head_argmax_workspace_size(M, N) bytes, 8-byte aligned, that
 * holds per-block partial results (no initialisation needed); it may be
 * reused by later calls on the same stream, and calls that overlap in time
 * must use different workspaces. */
size_t mq4_lm_head_argmax_workspace_size(int64_t M, int64_t N);
int mq4_lm_head_argmax(const uint16_t* h, int64_t M, int64_t K,
                       const uint32_t* wq, const uint16_t* scales, const uint16_t* biases,
                       int64_t N, uint32_t* idx, uint16_t* logits,
                       void* workspace, size_t workspace_bytes, void* stream);

/* mq4_lm_head_argmax without a workspace: no counterpart in the reference.
 * For callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  The
 * per-block partial results live in a static 1 MiB device array inside the
 * library, one per GPU, held until the process ends; so M <= 32
 * (MQ4_ERR_UNSUPPORTED above), and calls that overlap in time on one GPU race
 * (they share that GPU's array).  stream must belong to the current device;
 * the first call on a device looks the array's address up (no allocation).
 * Results are identical to mq4_lm_head_argmax's. */
int mq4_lm_head_argmax_noalloc(const uint16_t* h, int64_t M, int64_t K,
                               const uint32_t* wq, const uint16_t* scales, const uint16_t* biases,
                               int64_t N, uint32_t* idx, uint16_t* logits, void* stream);

/* The same with the final (1 + w) RMSNorm fused in front
 * (src/model/marlin.cpp:145, 12-16): logits = bf16(rms_norm(h) @ W^T). */
int mq4_rmsnorm_lm_head_argmax(const uint16_t* h, int64_t M, int64_t K,
                               const uint16_t* norm_weight, float eps,
                               const uint32_t* wq, const uint16_t* scales,
                               const uint16_t* biases, int64_t N, uint32_t* idx,
                               uint16_t* logits, void* workspace, size_t workspace_bytes,
                               void* stream);

/* idx[m] = argmax of row m of bf16 logits [M, N] (lowest index wins ties,
 * NaN never wins over a number).  Same workspace rule as above with
 * mq4_argmax_workspace_size. */
size_t mq4_argmax_workspace_size(int64_t M, int64_t N);
int mq4_argmax_bf16(const uint16_t* logits, int64_t M, int64_t N, uint32_t* idx,
                    void* workspace, size_t workspace_bytes, void* stream);

/* sample_token over each row of bf16 logits [M, N] (src/sampling/sampler.cpp:
 * 9-39), one token per row into idx[m]:
 *   temperature <= 0: the greedy argmax (lowest index among equal maxima).
 *   otherwise scaled = float(logit) / temperature, then
 *     top_k > 0 (and < N): elements below the k-th largest scaled value are
 *       masked (ties at the k-th value kept; top_k >= N masks nothing);
 *     0 < top_p < 1: with the kept elements' probabilities sorted ascending
 *       (equal probabilities in index order), an element is masked when the
 *       probability mass before it exceeds top_p -- the reference's mask,
 *       which drops the largest probabilities;
 *   and the token is drawn from softmax(scaled) over the kept elements by
 *   Gumbel-max with this library's counter-based generator: a pure function
 *   of (logits, parameters, seed, m), so equal seeds give equal tokens.  The
 *   reference draws from MLX's global key instead (its seed field is unused),
 *   so tokens agree with it in distribution, not draw by draw.
 * The top-p mass is summed exactly (64-bit fixed point), where the reference
 * sums in float32; masks agree except where a cumulative sum lies within
 * float32 rounding of top_p.  NaN logits are never drawn.  keep (may be NULL,
 * uint8 [M, N]) receives 1 for each element left unmasked (not written when
 * temperature <= 0).  M <= 65535 and N <= 2^23 (MQ4_ERR_UNSUPPORTED above);
 * top_k < 0 or a NaN temperature or top_p is MQ4_ERR_INVALID_ARG.
 * workspace (may be NULL) is device memory of mq4_sample_workspace_size(M, N)
 * bytes, 256-byte aligned, no initialisation needed: with it, a few long
 * rows (M <= 128, N >= 8192, N % 8 == 0, 16-byte aligned logits) are split
 * over many workgroups; without it, or for other shapes (size 0), one
 * workgroup handles each row.  Both give identical results.  Calls that
 * overlap in time must use different workspaces. */
size_t mq4_sample_workspace_size(int64_t M, int64_t N);
int mq4_sample_bf16(const uint16_t* logits, int64_t M, int64_t N, float temperature, int top_k,
                    float top_p, uint64_t seed, uint32_t* idx, uint8_t* keep,
                    void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------- */
/* One whole decode step for one token (M = 1) in a single persistent launch:
 *   for each layer:  x = x + down(swiglu(gate n, up n)),  n = rms_norm(x, norm)
 *   idx = argmax(lm_head(rms_norm(x, final_norm)))
 * i.e. the MLP half of the per-token layer loop (src/model/marlin.cpp:141-142,
 * 31-35), the final norm (:145), lm_head (:161-169) and greedy sample_token
 * (src/sampling/sampler.cpp:14-16), with the arithmetic of the separate entry
 * points above.  Built for hidden = 2048 and intermediate = 6144 (other
 * shapes return MQ4_ERR_UNSUPPORTED; use the separate entry points), up to
 * 32 layers, any vocab.  x_out (may be NULL) receives the hidden state after
 * the last layer.  The launch needs 256 co-resident workgroups, so it must
 * not overlap other work on the device.  workspace: at least
 * mq4_decode_workspace_size() bytes, 256-byte aligned, zero-filled once
 * before first use and then reused by every call on the same stream (calls
 * that overlap in time need separate workspaces).  If a call ever times out
 * internally (it cannot when the device runs nothing else), idx receives
 * 0xFFFFFFFF and every later call with that workspace does the same until
 * it is zero-filled again. */
typedef struct mq4_mlp_layer {
    const uint16_t* norm_weight;                 /* bf16 [hidden] (1 + w) RMSNorm */
    const uint32_t* gate_wq; const uint16_t* gate_scales; const uint16_t* gate_biases;
    const uint32_t* up_wq;   const uint16_t* up_scales;   const uint16_t* up_biases;
    const uint32_t* down_wq; const uint16_t* down_scales; const uint16_t* down_biases;
} mq4_mlp_layer;

/* Bytes of workspace mq4_decode_step needs (0 for unsupported sizes). */
size_t mq4_decode_workspace_size(int64_t hidden, int64_t intermediate, int64_t vocab);
int mq4_decode_step(const uint16_t* x_in, int64_t hidden, int64_t intermediate, int64_t n_layers,
                    const mq4_mlp_layer* layers, const uint16_t* final_norm, float eps,
                    const uint32_t* lm_wq, const uint16_t* lm_scales, const uint16_t* lm_biases,
                    int64_t vocab, uint32_t* idx, uint16_t* x_out,
                    void* workspace, size_t workspace_bytes, void* stream);

/* The MLP half of n_layers decoder layers for M token rows (1 <= M <= 32),
 * one launch per layer: x <- x + down(swiglu(gate n, up n)),
 * n = rms_norm(x, norm_weight), applied layer after layer to the bf16 hidden
 * states x_in [M, hidden]; the result lands in x_out [M, hidden].  Replaces,
 * for M concurrent decode streams (src/core/engine.cpp:79-94), the per-layer
 * MLP residual of src/model/marlin.cpp:141-142 (rms_norm :12-16,
 * mlp_forward :31-35) that mq4_mlp_forward_residual computes in separate
 * launches; same per-element arithmetic (exact (128 + q) bf16 products,
 * fp32 sums, bf16 SwiGLU and residual), sums grouped differently.  Built for
 * hidden = 2048 and intermediate = 6144 (other shapes return
 * MQ4_ERR_UNSUPPORTED).  x_out must overlap neither x_in nor the workspace.
 * Every pointer (x_in, x_out, and each layer's norm weight, packed weights,
 * scales and biases) must be 16-byte aligned.
 * Each launch needs 256 co-resident workgroups, so it must not overlap
 * other work on the device.  workspace: at least
 * mq4_mlp_layers_workspace_size(M, ...) bytes, 256-byte aligned,
 * zero-filled once before first use and then reused by every call on the
 * same stream (calls that overlap in time need separate workspaces; a
 * workspace sized for M serves every smaller M).  If a launch ever times out
 * internally (it cannot when the device runs nothing else), x_out is NaN and
 * every later call with that workspace does the same until it is
 * zero-filled again. */
size_t mq4_mlp_layers_workspace_size(int64_t M, int64_t hidden, int64_t intermediate);
int mq4_mlp_layers(const uint16_t* x_in, int64_t M, int64_t hidden, int64_t intermediate, int64_t n_layers,
                   const mq4_mlp_layer* layers, float eps, uint16_t* x_out,
                   void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------- */
/* Synthetic-input generator (bench and test inputs, not a reference seam):
 * out[i] = bf16(mu + sigma * z_{offset+i}) where z is the standard-normal
 * stream (SplitMix64 counter stream with state seed ^ stream_id, Box-Muller
 * in fp64, one round-to-nearest-even step from fp64 to bf16). */
int mq4_fill_normal_bf16(uint16_t* out, int64_t n, uint64_t seed, uint64_t stream_id,
                         double mu, double sigma, int64_t offset, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MQ4_H */
