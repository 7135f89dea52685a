/*
 * mlcvla.h -- C ABI of the MI355X (gfx950) pi0.5 M1 denoise library.
 *
 * Drop-in for the TVM Relax VM entry points of mlc-vla's M1 path.  In the
 * reference every entry point is a PackedFunc called as
 *     vm["<fn>"](*tensors, params)
 * (python/mlc_vla/sample.py:128,158-160,184-186), with signatures fixed by
 * Pi0Model.get_default_spec (python/mlc_vla/model/pi0/pi0_model.py:197-255).
 * Here the parameters are bound once to a context and the tensors are passed
 * as plain device pointers; outputs are caller-allocated.
 *
 * Conventions
 *  - Every function returns 0 on success, a negative code on failure
 *    (-1 HIP runtime error, -2 invalid argument, -3 not bound / unsupported,
 *    -4 a bounded device-side wait gave up -- a phase of the persistent step or a
 *    split-K meeting of the tile GEMM -- reported by mlcv_sync or the synchronous call);
 *    mlcv_last_error() returns the message of the last failure on this thread.
 *  - All tensor pointers are device pointers (HBM), row-major, no padding.
 *    "f16" is IEEE binary16, "f32" IEEE binary32.
 *  - `stream` is a hipStream_t (0 = the null stream).  Work is asynchronous
 *    with respect to the host; order with the stream.
 *  - One context is not thread-safe; use it from one thread / one stream.
 *  - Kernels and their workspaces are sized at mlcv_create from the config.
 */
#ifndef MLCVLA_H_
#define MLCVLA_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MLCV_DTYPE_F16 1
/* float32 models (Pi0Config(dtype="float32"), pi0_config.py:97): prefill, denoise_step_kv,
 * denoise_loop_kv and mlcv_chunk in float32 throughout (values, prefix_embs, x_t and time
 * embeddings are then float32 too), on generic kernels meant for the small shapes the
 * reference runs in float32; the other entry points and options of the step forms report that
 * they are not built for them. */
#define MLCV_DTYPE_F32 2
#define MLCV_QUANT_NONE 0
#define MLCV_QUANT_Q4F16_1 1

/* Model dimensions: Pi0Config + GemmaExpertConfig
 * (python/mlc_vla/model/pi0/pi0_config.py:15-170). */
typedef struct mlcv_config {
  int32_t vlm_width;     /* expert-0 width (gemma_2b: 2048)              */
  int32_t vlm_mlp;       /* expert-0 mlp_dim (16384)                     */
  int32_t ae_width;      /* expert-1 width (gemma_300m: 1024)            */
  int32_t ae_mlp;        /* expert-1 mlp_dim (4096)                      */
  int32_t depth;         /* shared depth (18)                            */
  int32_t num_heads;     /* shared query heads (8)                       */
  int32_t num_kv_heads;  /* shared kv heads (1)                          */
  int32_t head_dim;      /* shared head_dim (256)                        */
  int32_t prefix_len;    /* Pi0Config.prefix_len (968)                   */
  int32_t suffix_len;    /* Pi0Config.suffix_len = action_horizon        */
  int32_t action_dim;    /* 32                                           */
  int32_t num_steps;     /* num_denoise_steps (10)                       */
  float rms_norm_eps;    /* 1e-6                                         */
  float rope_theta;      /* 10000                                        */
  int32_t dtype;         /* MLCV_DTYPE_F16 or MLCV_DTYPE_F32             */
  int32_t quant;         /* MLCV_QUANT_NONE or MLCV_QUANT_Q4F16_1        */
} mlcv_config;

typedef struct mlcv_ctx mlcv_ctx;

/* Message of the last failure on the calling thread ("" if none). */
const char* mlcv_last_error(void);

/* Number of parameter pointers mlcv_bind_params expects for `cfg`:
 * 18*depth + 11 for fp16 weights (the named_params of the reference's
 * backbone + action head, pi0_model.py:81-88), one extra pointer per Linear
 * weight for q4f16_1 (q_weight + q_scale, quant.py:269-288). */
int mlcv_param_count(const mlcv_config* cfg, int32_t* count);

/* Create / destroy a context (allocates activations and workspaces). */
int mlcv_create(const mlcv_config* cfg, mlcv_ctx** out);
int mlcv_destroy(mlcv_ctx* ctx);

/* Bind the parameters, in named_params order, as device pointers.  Replaces the
 * `params` argument the reference passes on every VM call.  Pointers are
 * borrowed: the caller keeps the tensors alive and unchanged.  Rebinding
 * invalidates captured graphs. */
int mlcv_bind_params(mlcv_ctx* ctx, const void* const* ptrs, int32_t count, void* stream);

/* Options: MLCV_OPT_USE_GRAPH (default 1): capture step / loop / chunk as hipGraphs.
 * MLCV_OPT_HOIST_MODULATION (default 1): denoise_loop_kv / chunk compute the time
 * MLP and all adaRMS modulations of all steps as one M=num_steps GEMM. */
#define MLCV_OPT_USE_GRAPH 1
#define MLCV_OPT_HOIST_MODULATION 2
/* MLCV_OPT_PERSIST (default 0; env MLCV_PERSIST=1): run each step after its modulations as
 * one persistent kernel (one workgroup per CU) instead of one launch per operation. Built
 * only for fragment-major shapes; setting it elsewhere returns an error.
 * MLCV_OPT_PERSIST_SPIN: polls before a wait between the persistent step's phases gives up
 * (the launch then ends early and mlcv_sync reports it). */
#define MLCV_OPT_PERSIST 3
#define MLCV_OPT_PERSIST_SPIN 4
/* MLCV_OPT_MEET_POLLS (default 2^22): polls of a split-K meeting of the prefill's tile GEMMs
 * before a waiting workgroup gives up; the outputs of that call are then invalid and the next
 * mlcv_sync on the context returns -4. */
#define MLCV_OPT_MEET_POLLS 5
/* MLCV_OPT_XTP (default 1 where it applies; env MLCV_XTP=0 turns it off): run the decoder
 * layers of each step tensor-parallel over the GPU's 8 XCDs, two launches per layer (built for
 * width 1024, MLP 4096, 8 query heads / 1 kv head of 256, T < 64, prefix + T <= 1024, fp16, on
 * a part of 8 XCDs x 32 CUs; setting it elsewhere returns an error).  Its barrier waits are
 * bounded by MLCV_OPT_PERSIST_SPIN polls; a wait that gives up makes the next mlcv_sync
 * return -4.  MLCV_OPT_PERSIST = 1 turns it off, MLCV_OPT_XTP = 1 turns the persistent step off.
 * Value 2 runs it without skipping the key chunks whose keys are all masked (testing: the skip
 * is exact, the results are bit-identical). */
#define MLCV_OPT_XTP 6
/* MLCV_OPT_XTP_KEEP (default 0): the XCD step keeps every layer's intermediates for
 * mlcv_step_probe (1) or reuses one set of buffers for all layers (0, faster; probes then
 * return an error). */
#define MLCV_OPT_XTP_KEEP 7
/* MLCV_OPT_SYNC_WORDS (testing): set every progress word of the persistent step and every
 * barrier word of the XCD step to `value` mod 2^32 (no step may be in flight).  The words only
 * grow, wrapping at 2^32, and each launch compares them with wrapping arithmetic against its
 * own start value; a value just below 2^32 makes the next launches wrap. */
#define MLCV_OPT_SYNC_WORDS 8
/* MLCV_OPT_MASK_SKIP (default 1): the attentions of prefill and of every step form skip the
 * 32-key chunks whose mask values are all <= -1e9.  For a row with at least one valid key their
 * probabilities underflow to 0 in fp32, so the results are bit-identical; 0 computes them
 * (testing). */
#define MLCV_OPT_MASK_SKIP 9
/* MLCV_OPT_STEP_GRAPH (default 0): denoise_step_kv replays a captured hipGraph (1) or launches
 * its kernels directly (0).  A graph launch ends with about 8 us before the stream's next work
 * starts, more than the graph saves on a step of about 45 launches while the host stays ahead of
 * the GPU; denoise_loop_kv and the chunk (MLCV_OPT_USE_GRAPH) keep their graphs. */
#define MLCV_OPT_STEP_GRAPH 10
int mlcv_set_option(mlcv_ctx* ctx, int32_t key, int64_t value);

/* Synchronize `stream` and report a persistent step that ended early (a wait between its
 * phases gave up, e.g. when its workgroups could not all be resident): returns -4 with a
 * message and resets the context's step state; the affected outputs are invalid.  No
 * counterpart in the reference (whose VM raises at .numpy()); the Python VM calls it where
 * the reference would synchronize. */
int mlcv_sync(mlcv_ctx* ctx, void* stream);

/* Copy one intermediate of the last step on this context to host memory `out` (testing
 * only; no counterpart in the reference): synchronizes `stream` first.  The persistent step
 * keeps every layer's intermediates; the launch chain (fragment-major form, T < 64) reuses
 * one set of buffers, which hold the outputs of the last operation run (mlcv_bench_op): there
 * `layer` must be 0.
 *   MLCV_PROBE_X      residual stream entering layer `layer` (layer == depth: after the last) [T][W1] f16
 *   MLCV_PROBE_Q      q roped and scaled by 1/sqrt(hd) [T][H*hd] f32 (the attention's operand)
 *   MLCV_PROBE_K      suffix k roped [T][KV*hd] f32;  MLCV_PROBE_V  suffix v [T][KV*hd] f16
 *   MLCV_PROBE_ATTN   joint attention output [T][H*hd] f16
 *   MLCV_PROBE_X_MID  residual stream after the attention's gated residual [T][W1] f16
 *   MLCV_PROBE_H      GeGLU output [T][ae_mlp] f16
 *   MLCV_PROBE_MOD    adaRMS modulations [2 depth + 1][3 W1] f16 (layer 0)
 *   MLCV_PROBE_VOUT   the velocity of the last head [T][A] f32 (layer 0)
 *   MLCV_PROBE_XCD_X  the XCD step's copy of the residual stream on XCD `layer % 8` entering
 *                     layer `layer / 8` [T][W1] f16 (every XCD keeps its own copy)
 * The XCD step keeps every layer's intermediates too (XCD 0's copy of the residual stream). */
#define MLCV_PROBE_X 0
#define MLCV_PROBE_Q 1
#define MLCV_PROBE_K 2
#define MLCV_PROBE_V 3
#define MLCV_PROBE_ATTN 4
#define MLCV_PROBE_X_MID 5
#define MLCV_PROBE_H 6
#define MLCV_PROBE_MOD 7
#define MLCV_PROBE_VOUT 8
#define MLCV_PROBE_XCD_X 9
int mlcv_step_probe(mlcv_ctx* ctx, int32_t what, int32_t layer, void* out, size_t bytes, void* stream);

/* prefill -- Pi0Model.prefill (pi0_model.py:128-140).
 *   prefix_embs [1, P, vlm_width] f16, prefix_mask [1,1,1,P] f32 (0 / -1e9)
 *   -> keys [depth, 1, kv, P, head_dim] f32 (post-RoPE), values [..] f16 */
int mlcv_prefill(mlcv_ctx* ctx, const void* prefix_embs, const float* prefix_mask, float* keys, void* values,
                 void* stream);

/* embed_image -- Pi0Model.embed_image (pi0_model.py:97-99): the SigLIP tower and the
 * PaliGemma projector (siglip.py:20-120) over one channels-last image [S,S,C] f16
 * -> out [num_patches, projection_dim] f16.  `params` are the vision tower's parameters in
 * named_params order (mlcv_vision_param_count of them: 3 + 16 per layer + 4), device
 * pointers to f16.  `workspace` is caller-owned device memory of
 * mlcv_embed_image_workspace bytes; the image is copied into it, the tower runs as a hipGraph
 * kept per device (captured again when the parameters, workspace or config change), and the
 * result is copied to `out`.  The split-K scratch of its GEMMs is kept per device
 * and shared with mlcv_tile_linear: calls that run concurrently on different streams of
 * one device race on it, so issue them on one stream. */
typedef struct mlcv_vision_config {
  int32_t image_size, patch_size, num_channels, hidden_size, intermediate_size, num_hidden_layers,
      num_attention_heads, projection_dim;
  float layer_norm_eps;
} mlcv_vision_config;
int mlcv_vision_param_count(const mlcv_vision_config* cfg, int32_t* count);
int mlcv_embed_image_workspace(const mlcv_vision_config* cfg, size_t* bytes);
int mlcv_embed_image(const mlcv_vision_config* cfg, const void* const* params, int32_t count, const void* image,
                     void* out, void* workspace, size_t workspace_bytes, void* stream);

/* embed_language -- Pi0Model.embed_language (pi0_model.py:101-104), exported as
 * "embed_language" (pi0_model.py:217-220): input_ids [n] int32 (device), the embedding table
 * embed_tokens.weight [vocab, width] f16 -> out [n, width] f16 with
 * out[t] = fp16(table[ids[t]] * fp16(sqrt(width))).  Ids outside [0, vocab) are clamped. */
int mlcv_embed_language(const int32_t* input_ids, int32_t n, const void* table, int32_t vocab, int32_t width,
                        void* out, void* stream);

/* denoise_step -- Pi0Model.denoise_step (pi0_model.py:111-125), the joint prefix + suffix
 * ("M0") velocity that get_default_spec exports as "denoise_step" (pi0_model.py:221-225):
 *   prefix_embs [1,P,vlm_width] f16, x_t [1,T,A] f16, time_emb [1, ae_width] f16
 *   ->  v_out [1,T,A] f32.
 * Every prefix token is valid, and the RoPE positions run over 0..P+T-1
 * (pi0_model.py:113-115).  The prefix rows attend the prefix only and the suffix rows
 * attend all (the mask of _build_additive_mask, pi0_model.py:29-41). So the forward is
 * the prefix expert over the prefix, whose per-layer K/V go to the context's cache, then the
 * suffix path over that cache, in one graph.  Overwrites the context's prefill cache. */
int mlcv_denoise_step(mlcv_ctx* ctx, const void* prefix_embs, const void* x_t, const void* time_emb, float* v_out,
                      void* stream);

/* denoise_step_kv -- Pi0Model.denoise_step_kv (pi0_model.py:142-163).
 *   keys f32 / values f16 as produced by prefill, x_t [1,T,A] f16,
 *   time_emb [1, ae_width] f16, suffix_cos / suffix_sin [1,T,1,hd/2] f32,
 *   prefix_mask [1,1,1,P] f32  ->  v_out [1,T,A] f32 */
int mlcv_denoise_step_kv(mlcv_ctx* ctx, const float* keys, const void* values, const void* x_t, const void* time_emb,
                         const float* suffix_cos, const float* suffix_sin, const float* prefix_mask, float* v_out,
                         void* stream);

/* denoise_loop_kv -- Pi0Model.denoise_loop_kv (pi0_model.py:165-194).
 *   x0 [1,T,A] f32, time_embs [num_steps, ae_width] f16 -> x_out [1,T,A] f32 */
int mlcv_denoise_loop_kv(mlcv_ctx* ctx, const float* keys, const void* values, const float* x0,
                         const void* time_embs, const float* suffix_cos, const float* suffix_sin,
                         const float* prefix_mask, float* x_out, void* stream);

/* One action chunk: prefill followed by denoise_loop_kv, as one graph
 * (PiZeroRunner.sample_graph, sample.py:165-187, without the host helpers).
 * keys/values are kept in the context. */
int mlcv_chunk(mlcv_ctx* ctx, const void* prefix_embs, const float* prefix_mask, const float* x0,
               const void* time_embs, const float* suffix_cos, const float* suffix_sin, float* x_out, void* stream);

/* ---- kernel-level entry points (used by tests and the benchmark) ---------- */

/* Isolated joint attention (gemma_dual.py:97-122 as called from
 * attn_decode_e1 :255-275): q [Tq, H*hd] f16 already roped and scaled,
 * prefix K [KV, Sp, hd] (f32 if k_f32 else f16) / V [KV, Sp, hd] f16,
 * mask [Sp] f32 or NULL, suffix k/v [Ts, KV*hd] f16 already roped
 * -> out [Tq, H*hd] f16. */
int mlcv_joint_attention(const void* q, int32_t Tq, int32_t H, int32_t KV, int32_t hd, const void* kp,
                         int32_t k_f32, const void* vp, int32_t Sp, const float* mask, const void* ks,
                         const void* vs, int32_t Ts, void* out, void* stream);

/* The prefill's attention as prefill runs it (attn_prefill_e0, gemma_dual.py:236-253,
 * 334-341; testing): q [P][q_ld] f16 as the q/k/v projection leaves it (heads of hd columns
 * from column 0, not yet roped), roped with cos / sin [P][hd/2] f32 and scaled by 1/sqrt(hd)
 * (hd a multiple of 64: by a kernel that writes q split hi/lo in the attention's fragment
 * order, then the 8-wave attention; otherwise in the attention's loader); keys [KV][P][hd]
 * f32 roped and values [KV][P][hd] f16 (one layer of the cache), mask [P] f32 additive ->
 * out [P][H*hd] f16.  The same split plan and launches as prefill. */
int mlcv_prefill_attention(const void* q, int32_t q_ld, const float* cos, const float* sin, int32_t P, int32_t H,
                           int32_t KV, int32_t hd, const float* keys, const void* values, const float* mask, void* out,
                           void* stream);

/* Group quantization q4f16_1 (quant.py:217-266 + pack_weight :65-86):
 * w [N,K] f16 -> q_weight [N, K/8] u32, q_scale [N, K/32] f16. */
int mlcv_q4_quantize(const void* w, uint32_t* q_weight, void* q_scale, int32_t N, int32_t K, void* stream);

/* Dequantization (quant.py:176-193): -> w [N,K] f16. */
int mlcv_q4_dequantize(const uint32_t* q_weight, const void* q_scale, void* w, int32_t N, int32_t K, void* stream);

/* Linear y[M,N] = x[M,K] . W[N,K]^T (+ bias) in f16 with f32 accumulation, W
 * either f16 (w) or q4f16_1 (q_weight, q_scale) -- nn.Linear / GroupQuantizeLinear
 * (quant.py:301-325).  Runs the skinny MFMA GEMM of the denoise step. */
int mlcv_linear(const void* x, int32_t M, int32_t K, const void* w, const uint32_t* q_weight, const void* q_scale,
                const void* bias, void* y, int32_t N, void* stream);

/* mlcv_linear without any allocation (no counterpart in the reference): for callers that
 * cannot allocate device memory -- code under hipGraph capture, tight serving loops, hosts
 * that forbid it.  Same arguments, kernels and results as mlcv_linear, but asynchronous on
 * `stream`; its split-K partials, arrival counters and zero page live in one static device
 * array of about 8.3 MiB per GPU (held until the process ends), so it accepts at most 65536
 * output tiles of 64 x 64 (returns -2 beyond).  Calls that overlap on one GPU race on that
 * array: order them on one stream. */
int mlcv_linear_noalloc(const void* x, int32_t M, int32_t K, const void* w, const uint32_t* q_weight,
                        const void* q_scale, const void* bias, void* y, int32_t N, void* stream);

/* Prefill linear on the long-M tile GEMM (testing / benchmarking; no counterpart in the
 * reference): x [M,K] f16, w [N,K] f16 (MLCV_TILE_GEGLU: [2N,K], gate rows then up rows),
 * y [M,N] f16 with f32 accumulation:
 *   MLCV_TILE_STORE     y = x . w^T
 *   MLCV_TILE_RESIDUAL  y = fp16(y + fp16(x . w^T))
 *   MLCV_TILE_GEGLU     y = fp16(fp16(gelu_tanh(fp16(x . wg^T))) * fp16(x . wu^T))
 * small_tiles = 1 runs the 128 x 128 tile kernel instead of the 256-row one.  Synchronous.
 * meet_polls: polls of a split-K meeting before a waiting workgroup gives up (negative: the
 * default, 2^22); a meeting that gives up makes the call return -4.  The split-K scratch is
 * per device and shared with mlcv_embed_image: a meeting of an earlier mlcv_embed_image that
 * gave up is reported by the next call of either. */
#define MLCV_TILE_STORE 0
#define MLCV_TILE_RESIDUAL 1
#define MLCV_TILE_GEGLU 2
int mlcv_tile_linear(const void* x, int32_t M, int32_t K, const void* w, int32_t N, void* y, int32_t epi,
                     int32_t small_tiles, int32_t meet_polls, void* stream);

/* Enqueue `iters` launches of one operation of denoise_step_kv on `stream`, on the
 * context's current buffers (benchmarking / profiling only; no counterpart in the
 * reference).  `layer` selects the decoder layer; `keys` / `values` are needed for
 * MLCV_OP_ATTENTION.  The results are the op's normal outputs. */
#define MLCV_OP_TIME_MOD 0   /* time MLP (2 GEMVs) + all 2*depth+1 adaRMS modulations */
#define MLCV_OP_MODULATION 1 /* the modulation GEMV alone (3*ae_width x (2*depth+1) rows) */
#define MLCV_OP_QKV 2        /* adaRMS + q/k/v projections */
#define MLCV_OP_ATTENTION 3  /* joint attention (+ split combine) */
#define MLCV_OP_OPROJ 4      /* o_proj + gated residual */
#define MLCV_OP_GATEUP 5     /* adaRMS + gate_up + GeGLU */
#define MLCV_OP_DOWN 6       /* down + gated residual */
#define MLCV_OP_HEAD 7       /* final adaRMS + action_out_proj */
#define MLCV_OP_ATTENTION_ONLY 8 /* MLCV_OP_ATTENTION without the workgroups that prefetch the next ops' weights */
#define MLCV_OP_ACTION_IN 9  /* action_in_proj: the residual stream entering layer 0 */
/* The XCD step's two launches of `layer` (MLCV_OPT_XTP on; they read the context's copies of the
 * last denoise_step_kv call's inputs and the given keys / values): the attention launch (residual stream in,
 * adaRMS, q/k/v, attention, combine, o_proj partials) and the MLP launch (residual stream,
 * adaRMS, gate_up + GeGLU, down partials). */
#define MLCV_OP_XT_ATTN 10
#define MLCV_OP_XT_MLP 11
int mlcv_bench_op(mlcv_ctx* ctx, int32_t op, int32_t layer, int32_t iters, const float* keys, const void* values,
                  void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MLCVLA_H_ */
