/*
 * nvjsel -- decode-step token selection for MI355X (gfx950).
 *
 * C ABI of libnvjsel.so: the fused LM-head projection with greedy top-1, the
 * fused LM-head + Gumbel-max temperature sampler, and the full-vocab
 * temperature / top-k / top-p sampler over logits.  Plain pointers and sizes
 * only; every device pointer is HIP device memory; `stream` is a hipStream_t
 * (NULL = the default stream).  Launches are asynchronous on `stream`; no entry
 * point synchronises and none allocates device memory: callers pass a
 * workspace sized by the matching *_workspace_size() query.
 *
 * Workspace contract: zero-fill a workspace once when it is allocated.  Every
 * call that returns NVJSEL_OK leaves it zero-filled again (its accumulators are
 * reset by the call's last kernel), so it can be reused by the next call in
 * stream order without a memset.  Calls that overlap in time must not share a
 * workspace.
 *
 * Errors: entry points return NVJSEL_OK (0) or a negative nvjsel_status and
 * record a message readable with nvjsel_last_error() (thread-local).  Argument
 * validation mirrors the reference Triton wrapper
 * (nanovllm_jax/kernels/lm_head_triton.py:128-143): non-empty dimensions,
 * matching hidden sizes, dtypes in {f32, bf16, f16}.
 */
#ifndef NVJSEL_H
#define NVJSEL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NVJSEL_ABI_VERSION 2

typedef enum {
  NVJSEL_F32 = 0,
  NVJSEL_BF16 = 1,
  NVJSEL_F16 = 2
} nvjsel_dtype;

/* Storage of the LM-head weight.  VH is the tied embedding table [V, H]
 * (row-major, one token per row); HV is the reference's `lm_head` / `E.T`
 * operand [H, V] (nanovllm_jax/model.py:759; lm_head_triton.py:51-55). */
typedef enum {
  NVJSEL_W_VH = 0,
  NVJSEL_W_HV = 1
} nvjsel_layout;

typedef enum {
  NVJSEL_OK = 0,
  NVJSEL_EINVAL = -1,       /* bad shape, dtype, layout or null pointer      */
  NVJSEL_EUNSUPPORTED = -2, /* valid request this build does not serve       */
  NVJSEL_EWORKSPACE = -3,   /* workspace null or smaller than the query says */
  NVJSEL_EHIP = -4          /* a HIP runtime call failed                     */
} nvjsel_status;

/* ABI version of the loaded library (NVJSEL_ABI_VERSION at build time). */
int nvjsel_abi_version(void);

/* Message of the last failing call on this thread ("" if none). */
const char* nvjsel_last_error(void);

/* Workspace bytes for nvjsel_lm_head_top1 / nvjsel_lm_head_sample at `batch`
 * (per-row keys and a ticket line). */
size_t nvjsel_lm_head_workspace_size(int batch);

/*
 * Greedy LM-head top-1: out_ids[b] = argmax_v sum_k hidden[b,k] * W(v,k).
 *
 * Replaces lm_head_greedy_top1_triton(hidden_norm[B,1,H], output_weight[H,V])
 * -> int32[B,1] (nanovllm_jax/kernels/lm_head_triton.py:114-186) and the jax
 * route jnp.argmax(jnp.dot(hidden_norm, W)) (nanovllm_jax/model.py:815-819).
 *
 * hidden [batch, hidden_dim] of hidden_dtype; weight per weight_layout of
 * weight_dtype.  Accumulation is fp32.  reduce_cast: 0 = compare fp32 logits,
 * 1 = round logits to bf16 first, 2 = round to f16 first (the reference's
 * REDUCE_CAST, set when both operands are bf16 / f16, lm_head_triton.py:146-150).
 * Ties resolve to the lowest vocabulary index; a NaN logit wins (first NaN).
 * out_best (nullable) receives the winning (rounded) logit.
 */
int nvjsel_lm_head_top1(const void* hidden, int hidden_dtype,
                        const void* weight, int weight_dtype, int weight_layout,
                        int batch, int hidden_dim, int vocab, int reduce_cast,
                        int32_t* out_ids, float* out_best,
                        void* workspace, size_t workspace_bytes, void* stream);

/*
 * The same greedy LM-head top-1 for callers that cannot allocate (no
 * counterpart in the reference): code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc.  It takes no workspace; the
 * library keeps the per-row keys and ticket in a fixed device array of its
 * own (one per GPU, held until the process ends) and calls no allocating
 * routine.  batch <= 4096 (NVJSEL_EUNSUPPORTED above).  Every call on a GPU
 * shares that GPU's array, so calls that overlap in time on one GPU (other
 * streams, other threads) race; calls ordered on a stream do not.  The array
 * starts zeroed (static device storage without an initializer, zero-filled
 * when the code object is loaded) and every call leaves it zeroed; the first
 * call on a device only looks up its address, so it may itself be captured
 * into a graph.
 */
int nvjsel_lm_head_top1_noalloc(const void* hidden, int hidden_dtype,
                                const void* weight, int weight_dtype, int weight_layout,
                                int batch, int hidden_dim, int vocab, int reduce_cast,
                                int32_t* out_ids, float* out_best, void* stream);

/*
 * Fused LM-head + temperature sampling without writing logits.
 *
 * Replaces lm_head_sample_token_ids (nanovllm_jax/model.py:901-938): per row,
 * temperature[b] <= 0 -> argmax of the logits; otherwise
 * jax.random.categorical(key_b, logits / max(T, 1e-6)), i.e. the argmax of
 * logits/T' + gumbel(key_b)[v] with JAX's Threefry-2x32 noise at flat index v.
 * keys [batch, 2] uint32 (see nvjsel_derive_keys).  reduce_cast as above
 * (logits are rounded before the division, as the reference's bf16 dot).
 */
int nvjsel_lm_head_sample(const void* hidden, int hidden_dtype,
                          const void* weight, int weight_dtype, int weight_layout,
                          int batch, int hidden_dim, int vocab, int reduce_cast,
                          const float* temperature, const uint32_t* keys,
                          int32_t* out_ids,
                          void* workspace, size_t workspace_bytes, void* stream);

/*
 * Dense LM-head logits, for the routes that need them: the top-k verifier
 * route of lm_head_token_ids_and_topk(top_k > 0) (nanovllm_jax/model.py:
 * 866-898: jnp.dot(hidden_norm, W) then lax.top_k / radix_topk) and sampling
 * with top-k / top-p from the hidden state.  out_logits[b, v] (rows
 * out_row_stride elements apart, out_dtype f32, bf16 or f16) = sum_k
 * hidden[b,k] * W(v,k) accumulated in fp32 and rounded per reduce_cast (the
 * reference's dot output: bf16 for bf16 x bf16, f16 for f16 x f16), then
 * stored as out_dtype (bf16 / f16: round to nearest even).  Same kernels as nvjsel_lm_head_top1, with a store epilogue;
 * no workspace.
 */
int nvjsel_lm_head_logits(const void* hidden, int hidden_dtype,
                          const void* weight, int weight_dtype, int weight_layout,
                          int batch, int hidden_dim, int vocab, int reduce_cast,
                          void* out_logits, int out_dtype, int64_t out_row_stride, void* stream);

/*
 * Final-RMSNorm prologue variants: the same as nvjsel_lm_head_top1 /
 * nvjsel_lm_head_sample, but `hidden` is the pre-norm hidden state and the
 * library first forms, per row, the LM-head input of
 * _lm_head_normed_hidden_and_weight(hidden_is_normed=False)
 * (nanovllm_jax/model.py:734-762) with rms_norm (nanovllm_jax/layers.py:11-29):
 *   y = x * (1 / sqrt(mean(x^2) + eps)) * (1 + norm_weight)   in fp32,
 * rounded to hidden_dtype (rms_norm's astype(input_dtype)) and then to
 * act_dtype (lm_head_decode_act_dtype: f32 by default, bf16 when promoted).
 * reduce_cast applies to the act_dtype x weight_dtype dot as above.  On the
 * streaming and bf16 tile paths the prologue runs inside the LM-head launch;
 * otherwise a prologue kernel writes the normalised rows into the workspace.
 * norm_weight [hidden_dim] of norm_dtype.
 */
size_t nvjsel_lm_head_prenorm_workspace_size(int batch, int hidden_dim);

/* The prologue alone: out [batch, hidden_dim] of act_dtype receives the
 * LM-head input described above (for callers that form dense logits). */
int nvjsel_rms_norm(const void* hidden, int hidden_dtype, const void* norm_weight, int norm_dtype,
                    float eps, int act_dtype, int batch, int hidden_dim, void* out, void* stream);

int nvjsel_lm_head_top1_prenorm(const void* hidden, int hidden_dtype,
                                const void* norm_weight, int norm_dtype, float eps, int act_dtype,
                                const void* weight, int weight_dtype, int weight_layout,
                                int batch, int hidden_dim, int vocab, int reduce_cast,
                                int32_t* out_ids, float* out_best,
                                void* workspace, size_t workspace_bytes, void* stream);

int nvjsel_lm_head_sample_prenorm(const void* hidden, int hidden_dtype,
                                  const void* norm_weight, int norm_dtype, float eps, int act_dtype,
                                  const void* weight, int weight_dtype, int weight_layout,
                                  int batch, int hidden_dim, int vocab, int reduce_cast,
                                  const float* temperature, const uint32_t* keys,
                                  int32_t* out_ids, void* workspace, size_t workspace_bytes,
                                  void* stream);


/* Workspace bytes for nvjsel_sample at (batch, vocab). */
size_t nvjsel_sample_workspace_size(int batch, int vocab);

/*
 * Temperature / top-k / top-p sampler over logits [batch, vocab] (row stride
 * `row_stride` elements) of dtype f32, bf16 or f16.
 *
 * Replaces the per-row sampler of lm_head_sample_token_ids
 * (nanovllm_jax/model.py:923-938) and the planned
 * sample_topk_topp(logits, temperature, top_k, top_p, rng_state) -> token_ids
 * (docs/kernel_roadmap.md:436-439).  Per row b:
 *   T <= 0                      -> argmax(logits)                 (greedy)
 *   else x = logits / max(T, 1e-6) (fp32, correctly rounded);
 *   top_k in (0, vocab)         -> keep x >= k-th largest x (ties kept)
 *   top_p < 1                   -> over the survivors keep the smallest
 *                                  top-probability prefix whose softmax mass
 *                                  exceeds top_p, ties at the threshold kept
 *                                  (nanovllm_jax/spec_decode.py:72-76)
 *   token = argmax over kept v of x[v] + gumbel(key_b)[v]  (lowest index on ties)
 * top_k (nullable = all disabled) <= 0 or >= vocab disables top-k; top_p
 * (nullable = all 1.0) >= 1 disables top-p.  A filtered row holding a NaN
 * returns its first NaN, else one holding +inf its first +inf, else one that is
 * all -inf returns 0.
 * noise (nullable): fp32 [batch, vocab] (stride vocab) Gumbel values used in
 * place of the Threefry draws -- the "identical uniform draws" test mode.
 */
int nvjsel_sample(const void* logits, int dtype, int batch, int vocab, int64_t row_stride,
                  const float* temperature, const int32_t* top_k, const float* top_p,
                  const uint32_t* keys, const float* noise,
                  int32_t* out_ids,
                  void* workspace, size_t workspace_bytes, void* stream);

/*
 * Top-k values and indices of logits, for the verifier / diagnostic route of
 * lm_head_token_ids_and_topk(top_k > 0) (nanovllm_jax/model.py:893-898:
 * jax.lax.top_k(logits.astype(float32), k); the FlashInfer radix_topk route,
 * model.py:874-892, returns the same set).
 *
 * logits [batch, vocab] of dtype, rows row_stride elements apart.  For each
 * row: out_values[b, j] (f32, the row's own elements, bitwise) and
 * out_indices[b, j], j < k, sorted by value descending and, among equal
 * values, by index ascending; NaN orders above every number (the first NaN
 * first) and -0.0 equals +0.0, the argmax conventions of this library.
 * out_indices[b, 0] is the greedy token.  1 <= k <= min(256, vocab).
 * Workspace: nvjsel_topk_workspace_size(batch, vocab) bytes of scratch; any
 * contents on entry.  It writes none of the zero-at-rest accumulators of
 * nvjsel_sample, so a sampler workspace at least this large can be shared.
 */
size_t nvjsel_topk_workspace_size(int batch, int vocab);

int nvjsel_topk(const void* logits, int dtype, int batch, int vocab, int64_t row_stride, int k,
                float* out_values, int32_t* out_indices,
                void* workspace, size_t workspace_bytes, void* stream);

/*
 * Per-row sampling keys of the executor's sampled route:
 * keys[b] = fold_in(fold_in(PRNGKey(0), uint32(slots[b])), uint32(counters[b]))
 * (nanovllm_jax/engine/model_executor.py:2131, 2214-2219), and
 * counters_out[b] = counters[b] + 1 (model_executor.py:2231; nullable).
 * Negative slots are clamped to 0 (model_runner.py:4785).
 */
int nvjsel_derive_keys(const int32_t* slots, const int32_t* counters, int batch,
                       uint32_t* keys, int32_t* counters_out, void* stream);

/*
 * The same keys from a device-resident counter table, with the table bumped
 * in the same launch (nanovllm_jax/engine/model_executor.py:3593-3619:
 * counters = table[slot_ids]; keys = fold_in(fold_in(PRNGKey(0), slot),
 * counter); table.at[slot_ids].set(counters + 1)).  Negative slots read slot 0
 * (model_runner.py:4785); slots >= num_slots read the last entry and are not
 * written (jnp gather clamps, scatter drops).  Rows sharing a slot read the
 * same counter: every row's counter is read before any is written, for any
 * batch.  counter_table [num_slots] int32, updated in place.  batch <= 8192
 * (NVJSEL_EUNSUPPORTED above).
 */
int nvjsel_derive_keys_table(const int32_t* slots, int batch, int32_t* counter_table, int num_slots,
                             uint32_t* keys, void* stream);

/*
 * Diagnostic (no counterpart in the reference): the Gumbel draw of every
 * 23-bit uniform mantissa m in [first, first + n), i.e. random bits
 * (m << 9), two ways -- fast[i] with the hardware fp32 log the kernels use to
 * pre-select candidates, exact[i] with the correctly rounded log every
 * returned token is decided on.  first + n <= 2^23.  Lets a test bound the
 * fast draw's error over its whole domain.
 */
int nvjsel_debug_gumbel_draws(uint32_t first, int n, float* fast, float* exact, void* stream);

/*
 * Diagnostic (no counterpart in the reference): nvjsel_sample (no noise
 * override) that also reports, per row, the top-p / top-k threshold the
 * kernels settled on and the softmax mass of the kept set.  out_tau[b] is the
 * threshold in x = logit / max(T, 1e-6) space (kept = {x >= tau}); out_mass[b]
 * is mass(kept) / mass(top-k survivors) as the kernels' own fixed-point and
 * grid-bin weights give it -- the intermediate that decides the threshold
 * (nanovllm_jax/spec_decode.py:69-83).  Rows without a threshold (greedy,
 * unfiltered, non-finite) get NaN in both.  out_ids as nvjsel_sample.
 */
int nvjsel_debug_sample_topp(const void* logits, int dtype, int batch, int vocab, int64_t row_stride,
                             const float* temperature, const int32_t* top_k, const float* top_p,
                             const uint32_t* keys, int32_t* out_ids, float* out_tau, double* out_mass,
                             void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NVJSEL_H */
