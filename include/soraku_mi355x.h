/*
 * soraku_mi355x.h -- C ABI of the MI355X (gfx950) per-frame CFG decode engine
 * for soraku-TTS.
 *
 * Plain C: opaque handles, plain pointers and sizes, integer status codes.
 * Device pointers are HIP device addresses (for example torch.Tensor.data_ptr()
 * of a tensor on "cuda"); host pointers are ordinary process memory.  Every
 * argument is validated before any HIP call, so argument errors are reported
 * without touching the GPU.
 *
 * Reference interfaces replaced (paths relative to the reference checkout):
 *   engine object     GraphFrameEngine          soraku_inference/acceleration/graph_frame.py:23-83
 *   prefill           GraphFrameEngine.prefill  graph_frame.py:118-198 (per-row caches instead of
 *                                               left padding; layout of model.py:623-656)
 *   capture           GraphFrameEngine.capture  graph_frame.py:274-296
 *   step_frame        GraphFrameEngine.step_frame graph_frame.py:298-305
 *   set_temperature / set_sampling / cfg        graph_frame.py:307-324, graph_frame.py:68
 *   operator API      TileLang factories        soraku_inference/acceleration/tilelang_kernels.py:34-254
 *   weight keys       SorakuTTSv2 state dict    model.py:100-145 + transformers Qwen3Model
 */
#ifndef SORAKU_MI355X_H
#define SORAKU_MI355X_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes (0 = success) ---------------------------------------- */
#define SK_OK          0
#define SK_EINVAL     -1   /* bad argument (shape, range, null pointer, unknown key)      */
#define SK_ENOWEIGHT  -2   /* a required weight was never bound                           */
#define SK_ENOCAPTURE -3   /* step before capture (graph_frame.py:301-302)                 */
#define SK_EKVFULL    -4   /* KV cache or frame ring full (graph_frame.py:155-156)         */
#define SK_EHIP       -5   /* a HIP runtime call failed; sk_last_error() holds its text    */
#define SK_ESTATE     -6   /* call out of order (e.g. step before prefill)                 */

/* ---- element types --------------------------------------------------- */
#define SK_F32  0
#define SK_BF16 1

/* Model dimensions and special ids (SorakuV2Config model.py:34-63 plus the
 * Qwen3 text config).  audio_vocab = codebook_size + 3 (model.py:61-63). */
typedef struct sk_config {
  int32_t d_model;        /* hidden size (1024 for Qwen3-0.6B)                 */
  int32_t n_layers;       /* trunk layers (28)                                 */
  int32_t n_q_heads;      /* 16                                                 */
  int32_t n_kv_heads;     /* 8                                                  */
  int32_t head_dim;       /* 128                                                */
  int32_t trunk_inter;    /* trunk SwiGLU inner size (3072)                     */
  int32_t depth_inner;    /* depth-head SwiGLU inner size d*depth_ffn_mult      */
  int32_t n_codebooks;    /* Q = 16                                             */
  int32_t audio_vocab;    /* V = codebook_size + 3 = 2051                        */
  int32_t text_vocab;     /* rows of trunk.embed_tokens.weight                  */
  int32_t bos_id, eos_id, pad_id;   /* 2048, 2049, 2050                         */
  float trunk_eps;        /* 1e-6 (Qwen3RMSNorm)                                */
  float depth_eps;        /* FLT_EPSILON (nn.RMSNorm(eps=None), model.py:135)   */
  float rope_theta;       /* 1e6                                                */
  float frame_scale;      /* Q^-1/2 (model.py:99)                               */
  int32_t weight_dtype;   /* SK_F32 or SK_BF16 for every matrix                 */
  int32_t n_utts;         /* utterances decoded together (n_utts*cfg_rows <= 32) */
  int32_t cfg_rows;       /* rows per utterance: 2 = cond+uncond, 1 = no CFG     */
  int32_t max_ctx;        /* KV capacity per row (prefix + frames)              */
  int32_t max_frames;     /* capacity of the per-frame input/code ring          */
  int32_t n_language;     /* language-token rows (0 or 4, model.py:186-197)     */
  int32_t language_ids[4];/* their text ids (model.py:326-338)                  */
  int32_t kv_dtype;       /* KV cache element: SK_F32 (reference) or SK_BF16    */
} sk_config;

typedef struct sk_engine sk_engine;

/* Last error message of the calling thread ("" if none). */
const char* sk_last_error(void);

/* Create an engine: allocates KV cache, activations and the frame ring on
 * the current HIP device.  `hip_stream` may be NULL; the engine always runs
 * on a stream of its own and makes that stream wait on `hip_stream`. */
int sk_create(const sk_config* cfg, void* hip_stream, sk_engine** out);
int sk_destroy(sk_engine* e);

/* Bind a weight by its state-dict key (weights are borrowed, never freed).
 * dtype: SK_F32 for gains/tables/bias; matrices use cfg->weight_dtype.
 * Keys: trunk.layers.{i}.{input_layernorm,post_attention_layernorm}.weight,
 *       trunk.layers.{i}.self_attn.{q,k,v,o}_proj.weight,
 *       trunk.layers.{i}.self_attn.{q,k}_norm.weight,
 *       trunk.layers.{i}.mlp.{gate,up,down}_proj.weight, trunk.norm.weight,
 *       trunk.embed_tokens.weight, audio_codebooks.table,
 *       depth_head.norm_in.weight, depth_head.mlp.{gate,up,down}_proj.weight,
 *       depth_head.norm_out.weight, depth_head.bias, language_embeddings.weight,
 *       and depth_head.out_proj [Q][V][d] for an untied classifier (model.py:141-145;
 *       when it is not bound the classifier is the tied audio_codebooks.table). */
int sk_bind_weight(sk_engine* e, const char* key, const void* dev_ptr, int32_t dtype,
                   const int64_t* shape, int32_t ndim);

/* Stage one row's prefix: text ids, then the frames `frame_codes[n_frames][Q]`
 * (the caller includes the BOS frame first, model.py:633-642).  Resets the row. */
int sk_prefill_row(sk_engine* e, int32_t row, const int64_t* text_ids, int32_t n_text,
                   const int64_t* frame_codes, int32_t n_frames);
/* Run every staged row through the trunk; leaves per-row hidden and KV length.
 * Every row must be staged; the frame counter starts over. */
int sk_prefill_run(sk_engine* e);
/* sk_prefill_run that allocates no device memory.  No counterpart in the
 * reference: for callers that cannot allocate (serving loops that must not
 * stall on hipMalloc, harnesses that forbid it).  It copies small host-side
 * tables and waits for the engine's stream, so it cannot be recorded into a
 * graph: on a capturing stream it returns SK_ESTATE.  The prefill's activation
 * buffers come from a scratch array of SK_NOALLOC_SCRATCH_BYTES in the
 * library's device code (one per GPU, held until the process ends) instead
 * of the engine's lazily grown buffers; a packed prefix that needs more
 * (about 600 tokens at the Qwen3-0.6B shape, 450 at 1.7B) is rejected with
 * SK_EINVAL -- sk_prefill_run takes any size.  Every call on one GPU shares
 * that scratch, so calls that overlapped on one GPU would race; the device
 * order of engines (below, at sk_replay) makes the prefills of different
 * engines take turns, and one engine's calls share its stream.  Results are
 * those of sk_prefill_run, bit for bit. */
#define SK_NOALLOC_SCRATCH_BYTES (32u << 20)
int sk_prefill_run_noalloc(sk_engine* e);
/* Continuous batching (no counterpart in the reference, which decodes one
 * utterance's CFG pair, fast_generate.py:232-328): between frames, run only
 * the rows staged since the last prefill (at least one) through the trunk.
 * Every other row keeps its cache, length, position and hidden state, and the
 * frame counter is unchanged, so an utterance slot whose utterance retired
 * takes the next utterance while the others keep decoding.  The staged rows
 * become active.  Requires a completed sk_prefill_run. */
int sk_prefill_refill(sk_engine* e);
/* Stop decoding one row (no reference counterpart; continuous batching): it
 * no longer advances its length or position, attention skips it and the
 * cache-capacity checks ignore it.  Its codes are meaningless until a refill. */
int sk_retire_row(sk_engine* e, int32_t row);
/* Restart the frame ring (no reference counterpart): the next frame uses slot
 * 0 again, so codes of earlier frames can no longer be read with
 * sk_read_codes.  Lets one engine decode more than max_frames frames in all. */
int sk_reset_frames(sk_engine* e);

/* Override one row's KV length and RoPE position (after an external prefill). */
int sk_set_row_state(sk_engine* e, int32_t row, int32_t kv_len, int32_t position);
/* Device address of layer `layer`'s K (kv=0) or V (kv=1) cache,
 * laid out [rows][n_kv_heads][max_ctx][head_dim] of cfg->kv_dtype elements
 * (FP32, or BF16 bits rounded to nearest even). */
int sk_kv_ptr(sk_engine* e, int32_t layer, int32_t kv, void** out);
/* Copy the current depth-input hidden state [rows][d] to host memory. */
int sk_get_hidden(sk_engine* e, float* host_out);

/* Sampling parameters (model.py:515-533 semantics).  temperature <= 0 means
 * greedy.  *_q0 override codebook 0; pass has_q0 = 0 to use the main values.
 * top_k <= 0 or >= V disables top-k; top_p outside (0,1) disables top-p.
 * Read by the captured graph on every replay: no re-capture needed. */
int sk_set_sampling(sk_engine* e, float cfg_scale, float temperature, int32_t top_k,
                    float top_p, int32_t has_q0, float temperature_q0, int32_t top_k_q0,
                    float top_p_q0);
/* Debug switches: record masked merged logits of every depth step; force codes. */
int sk_set_debug(sk_engine* e, int32_t record_logits);

/* Capture one whole frame (16 depth steps + sampling + frame embedding +
 * trunk step) as one hipGraph.  With one utterance with CFG at the
 * Qwen3-0.6B shape with FP32 weights or the Qwen3-1.7B shape with BF16
 * weights, capture also derives the depth steps' code tables from the bound
 * codebook table, depth norm_in gain and gate/up weights
 * ((Q-1) x V x 2 x depth_inner floats: 0.5 GB / 1.0 GB); those weights must
 * not change afterwards. */
int sk_capture(sk_engine* e);

/* Replay one frame.  mask_eos_q0: bit u masks EOS at codebook 0 for
 * utterance u (the min_new_frames rule, model.py:583-584); with one utterance
 * 0 or 1.  uniforms: [n_utts][Q] draws in [0,1) (NULL => 0).
 * forced_codes: NULL, or [n_utts][Q] codes to use instead of the sampled ones
 * (teacher forcing).  codes_out: host [n_utts][Q].  logits_dbg: NULL or host
 * [n_utts][Q][V] masked merged logits (needs sk_set_debug(e, 1)).
 * Synchronous on the codes copy, like graph_frame.py:305. */
int sk_step_frame(sk_engine* e, int32_t mask_eos_q0, const double* uniforms,
                  const int64_t* forced_codes, int64_t* codes_out, float* logits_dbg);

/* Throughput path: upload per-frame inputs for the next `n` frames
 * (uniforms [n][n_utts][Q], mask_eos_q0 [n] utterance bit masks as in
 * sk_step_frame), then replay `n` frames back to
 * back with no host synchronisation.  sk_read_codes copies codes of the
 * `n` most recent frames ([n][n_utts][Q]).
 * Frames and prefills of different engines on one device run one after
 * another: when the device's work passes from one engine to another
 * (sk_step_frame, sk_replay, the prefills), the new engine's stream first
 * waits for the work queued on the previous engine's stream.  An engine
 * working alone pays nothing. */
int sk_queue_frames(sk_engine* e, int32_t n, const double* uniforms, const int32_t* mask_eos_q0);
int sk_replay(sk_engine* e, int32_t n);
int sk_read_codes(sk_engine* e, int32_t n, int64_t* codes_out);
int sk_synchronize(sk_engine* e);
/* The engine's stream (hipStream_t) and frame counter. */
void* sk_stream(sk_engine* e);
int32_t sk_frames_done(sk_engine* e);
/* Diagnostic with no counterpart in the reference (which has one decode
 * path): 1 when the engine runs its trunk as XCD-resident layers (two
 * launches per layer; one utterance with CFG at the Qwen3-0.6B or, with BF16
 * weights, Qwen3-1.7B shape, on a device of 256 CUs, unless
 * SORAKU_XCD_LAYERS=0 was set at sk_create), 0 when it runs the per-op layer
 * kernels, -1 for a NULL engine.  For tests and profiling. */
int32_t sk_xcd_layers(sk_engine* e);
/* Test hook with no counterpart in the reference: the bound, in ticks of the
 * 100 MHz real-time counter, of every wait inside a frame's kernels (the
 * XCD-resident layers' barriers and tagged exchanges, the many-row split-K
 * GEMMs' merge of tagged partials; default and maximum 5,000,000 = 50 ms).
 * Set before sk_capture (SK_ESTATE after).  A wait that passes it sets the
 * engine's error word, the kernel goes on without the missing data, and the
 * next sk_step_frame / sk_synchronize / sk_read_codes returns SK_EHIP; 0
 * makes nearly every wait give up at once, which is how a test forces that
 * error path while every kernel still exits normally.  The engine must then
 * be recreated. */
int sk_debug_set_spin_ticks(sk_engine* e, uint64_t ticks);

/* ---- operator API (tilelang_kernels.py counterparts) ------------------
 * All pointers are device pointers, all tensors contiguous row-major.
 * `stream` is a hipStream_t (NULL = default stream).  Matrices: wdtype. */
int sk_op_add_rmsnorm(void* stream, int32_t B, int32_t D, float eps, const float* hidden,
                      const float* prefix, const float* weight, float* out);   /* :34-55  */
int sk_op_rmsnorm(void* stream, int32_t B, int32_t D, float eps, const float* x,
                  const float* weight, float* out);                            /* :58-78  */
int sk_op_swiglu_gemv(void* stream, int32_t B, int32_t I, int32_t D, int32_t wdtype,
                      const float* x, const void* wg, const void* wu, float* out);  /* :81-112 */
int sk_op_down_residual_gemv(void* stream, int32_t B, int32_t D, int32_t I, int32_t wdtype,
                             const float* act, const void* wd, const float* residual,
                             float* out);                                      /* :115-143 */
int sk_op_classifier_gemv(void* stream, int32_t B, int32_t V, int32_t D, int32_t wdtype,
                          const float* body, const void* wq, const float* bias,
                          float* out);                                         /* :146-173 */
int sk_op_frame_embed(void* stream, int32_t R, int32_t Q, int32_t V, int32_t D, float scale,
                      const int64_t* codes, const float* table, float* out);   /* :176-196 */
int sk_op_prefix_add(void* stream, int32_t B, int32_t V, int32_t D, float scale,
                     const float* prefix, const float* table_q, const int64_t* code,
                     float* out);                                              /* :199-216 */
int sk_op_sampling_prep(void* stream, int32_t V, int32_t bos_id, int32_t pad_id,
                        int32_t eos_id, const float* logits, const float* temperature,
                        const int32_t* mask_eos, float* out);                  /* :219-254 */
/* Fused CFG + masks + temperature + top-k/top-p + explicit-uniform draw for
 * one utterance (model.py:579-595,686-708; graph_frame.py:214-242).
 * logits: [rows][V] (row 0 cond, row 1 uncond).  code_out: device int64[1]. */
int sk_op_sample(void* stream, int32_t rows, int32_t V, const float* logits, float cfg_scale,
                 int32_t q, int32_t mask_eos_q0, int32_t bos_id, int32_t eos_id, int32_t pad_id,
                 float temperature, int32_t top_k, float top_p, double u, int64_t* code_out);

#ifdef __cplusplus
}
#endif
#endif /* SORAKU_MI355X_H */
