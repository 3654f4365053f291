/*
 * dflash_hip.h -- C ABI of libdflash_hip.so, the MI355X (gfx950) implementation of the
 * DFlash block-diffusion draft forward (W8A16) of 0xClandestine/mirror-sd.
 *
 * The library replaces the reference's native draft back-end, the PyO3 module
 * `mirror_sd_ane` (ane/src/lib.rs:6-16, ane/src/wrapper.rs) and the MLX draft
 * (mirror_sd/dflash.py), behind the same Python draft-model interface.  Every entry
 * point below names the reference interface it stands in for.
 *
 * Conventions
 *  - All tensor pointers are DEVICE pointers (hipMalloc / torch CUDA tensors).
 *    fp16 tensors are passed as uint16_t*.  Shapes are row-major.
 *  - `stream` is a hipStream_t (NULL = default stream).  Every call only enqueues
 *    work on `stream`; results are valid after the stream is synchronised.
 *  - Return value: DFL_OK (0) or an error code; dfl_last_error() returns the message
 *    of the last failed call on the calling thread (wrapper.rs:204-209, 334-339 raise
 *    RuntimeError / ValueError with the kernel name; the Python layer does the same).
 *  - Threading: a context is used from one host thread / one stream at a time; calls
 *    on different contexts are independent.  Weights are copied into context-owned
 *    device memory at load (wrapper.rs:88-92, 451-465 copy into Rust-owned memory).
 */
#ifndef DFLASH_HIP_H
#define DFLASH_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DFL_OK 0
#define DFL_EINVAL 1   /* bad argument / shape (reference: ValueError) */
#define DFL_ERANGE 2   /* capacity exceeded (ane_model.py:389-393, 620-624) */
#define DFL_EHIP 3     /* HIP runtime error */
#define DFL_ESTATE 4   /* weights not loaded / wrong call order */

typedef struct dfl_ctx dfl_ctx;

/* Model dimensions; field meaning follows DFlashConfig (mirror_sd/dflash.py:34-50). */
typedef struct dfl_config {
  int32_t hidden;          /* hidden_size (multiple of 128, <= 8192)       */
  int32_t n_heads;         /* num_attention_heads                          */
  int32_t n_kv_heads;      /* num_key_value_heads (n_heads % n_kv_heads == 0) */
  int32_t head_dim;        /* head_dim; must be 128                        */
  int32_t intermediate;    /* intermediate_size (multiple of 128)          */
  int32_t n_layers;        /* num_hidden_layers (draft layers)             */
  int32_t n_target_feat;   /* len(target_layer_ids); fc input = n_target_feat*hidden; 0 = no fc */
  int32_t vocab;           /* vocab_size of embedding / lm_head; 0 = none  */
  int32_t max_block;       /* largest block (query rows) per draft call    */
  int32_t max_ctx;         /* KV-cache capacity in context rows            */
  float rms_eps;           /* rms_norm_eps                                 */
  double rope_theta;       /* rope_theta (neox / split-half RoPE)          */
  int32_t max_seqs;        /* independent sequences (each its own KV cache) for
                              dfl_draft_batch; 0 or 1 = single sequence      */
} dfl_config;

/* Create / destroy a draft context (replaces ANEDraftModel.__init__ kernel compile
 * + buffer allocation, ane_model.py:47-150; compile_dflash_kernels*, wrapper.rs:308-361). */
int dfl_create(const dfl_config* cfg, dfl_ctx** out);
int dfl_destroy(dfl_ctx* ctx);
const char* dfl_last_error(void);

/* W8A16 quantiser on device (ane_model.py:265-279 `_quantize_weight_q8`):
 * w fp32 [oc][ic] -> q int8 [oc][ic], scale fp16 [oc]; scale = max|w_row|/127 (0 -> 1/127),
 * q = clamp(round_half_even(w/scale), -127, 127).  Bit-identical to the numpy quantiser. */
int dfl_quantize_w8(const float* w, int64_t oc, int64_t ic, int8_t* q, uint16_t* scale,
                    void* stream);

/* Load one layer (replaces Q8LayerWeights, wrapper.rs:363-428, + _load_layer_norm_weights,
 * ane_model.py:281-292).  q[i]/scale[i] in the order q,k,v,o,gate,up,down, reference byte
 * layout: int8 [oc][ic] row-major + fp16 [oc].  Norm gains fp16: input_layernorm [H],
 * post_attention_layernorm [H], q_norm [128], k_norm [128].  Data are copied. */
int dfl_load_layer_w8(dfl_ctx* ctx, int layer, const int8_t* const q[7],
                      const uint16_t* const scale[7], const uint16_t* in_norm,
                      const uint16_t* post_norm, const uint16_t* q_norm, const uint16_t* k_norm,
                      void* stream);

/* fc [H][n_target_feat*H] fp16 and hidden_norm [H] fp16 (dflash.py:373-378; the
 * reference never quantises fc, ane_model.py:319-322).  Copied. */
int dfl_load_fc(dfl_ctx* ctx, const uint16_t* fc_weight, const uint16_t* hidden_norm,
                void* stream);

/* Final norm [H] (dflash.py:379), the target's embedding table [V][H] (kept as a
 * caller-owned pointer; must outlive the context) and lm_head [V][H] (copied into the
 * context's layout) -- target.py:188-197; compile_lm_head_kernel, wrapper.rs:507-523.
 * embed / lm_head may be NULL. */
int dfl_load_head(dfl_ctx* ctx, const uint16_t* final_norm, const uint16_t* embed,
                  const uint16_t* lm_head, void* stream);

/* Context ingest (dflash.py:392 `hidden_norm(fc(target_hidden))` then, per layer,
 * k_norm(k_proj(ctx)) + RoPE and v_proj(ctx), appended to the KV cache at positions
 * offset .. offset+C-1 -- the context half of Qwen3DFlashAttention, dflash.py:287-308;
 * `_compute_context`, ane_model.py:632-637).  target_hidden [C][n_target_feat*H] fp16. */
int dfl_ingest_context(dfl_ctx* ctx, const uint16_t* target_hidden, int32_t C, void* stream);
/* Same for context rows that are already fused ([C][H] fp16): skips fc + hidden_norm. */
int dfl_ingest_fused(dfl_ctx* ctx, const uint16_t* ctx_hidden, int32_t C, void* stream);

/* Context capture fused with the ingest: the n_feats tapped target-layer outputs
 * (forward_with_hidden_states, target.py:258-278, in target_layer_ids order) are read
 * where they lie -- feats[j] -> [C][ld] fp16 device rows, first H columns used, 16-byte
 * aligned, ld >= H and ld % 8 == 0 -- as if concatenated along the hidden axis
 * (extract_context_feature, dflash.py:122-130) and passed to dfl_ingest_context.
 * n_feats must equal n_target_feat. */
int dfl_ingest_features(dfl_ctx* ctx, const uint16_t* const* feats, int32_t n_feats,
                        int64_t ld, int32_t C, void* stream);
/* extract_context_feature materialised: out [C][n_feats * H] fp16 (16-byte aligned) =
 * the feature rows concatenated along the hidden axis; same feats / ld rules. */
int dfl_concat_features(const uint16_t* const* feats, int32_t n_feats, int64_t ld, int32_t C,
                        int32_t H, uint16_t* out, void* stream);

/* Draft one block (DFlashDraftModel.__call__, dflash.py:384-403, with the block K/V
 * appended and trimmed again as generate.py:599-609 does; ANEDraftModel.run_kernels +
 * read_output + read_draft_tokens, ane_model.py:564-604; read_argmax, wrapper.rs:108-140).
 * Input: exactly one of noise_emb [B][H] fp16 or ids [B] int32 (rows of the loaded
 * embedding).  Outputs (each may be NULL): out_hidden [B][H] fp16 (final-normed),
 * out_prenorm [B][H] fp16 (residual stream before the final norm), out_logits [B][V]
 * fp32, out_ids [B] int32 (argmax, lowest index on ties).  Block rows use positions
 * offset .. offset+B-1 and attend to all cached context rows plus the block. */
int dfl_draft_block(dfl_ctx* ctx, const uint16_t* noise_emb, const int32_t* ids, int32_t B,
                    uint16_t* out_hidden, uint16_t* out_prenorm, float* out_logits,
                    int32_t* out_ids, void* stream);

/* Batched drafting (no counterpart in the single-sequence reference; it stacks what the
 * serial caller does per sequence, generate.py:591-609, for sequences 0 .. n_seq-1):
 * one block of B rows for each sequence, rows stacked sequence-major (row = s*B + b) in
 * every input and output buffer, same meaning as dfl_draft_block per row.  Each sequence
 * attends to its own cached context (ragged lengths allowed) plus its own block, at its
 * own positions.  The projections run once over all n_seq*B rows. */
int dfl_draft_batch(dfl_ctx* ctx, int32_t n_seq, const uint16_t* noise_emb, const int32_t* ids,
                    int32_t B, uint16_t* out_hidden, uint16_t* out_prenorm, float* out_logits,
                    int32_t* out_ids, void* stream);
/* Select the sequence (0 <= seq < max_seqs) that dfl_ingest_*, dfl_draft_block and the
 * dfl_cache_* calls address.  A context starts with sequence 0 selected. */
int dfl_select_seq(dfl_ctx* ctx, int32_t seq);

/* Run only the first n draft layers (DFlashDraftModel.num_draft_layers, dflash.py:382,
 * 394, lowered by generate.py:423-426); 1 <= n <= n_layers.  Ingest then fills only
 * those layers' caches. */
int dfl_set_num_layers(dfl_ctx* ctx, int32_t n);

/* KV-cache bookkeeping (DFlashKVCache, dflash.py:139-212). */
/* Drop the last n cached context rows; offset -= n (trim, dflash.py:195-207). */
int dfl_cache_trim(dfl_ctx* ctx, int32_t n);
/* Keep the first n block rows of the last dfl_draft_block as cached context
 * (what update_and_fetch did before the caller's trim). */
int dfl_cache_commit(dfl_ctx* ctx, int32_t n);
int dfl_cache_reset(dfl_ctx* ctx);
/* Sink + sliding-window eviction (DFlashKVCache(sink_size, window_size) and
 * _apply_window, dflash.py:160-193): clears the cache, then keeps the first `sink` rows and
 * the newest `window` rows once more than sink + window are cached.  Both 0 (or either 0,
 * as in the reference) = no eviction.  sink + window within the cache capacity; a drafted
 * block must fit in the window.  dfl_cache_reset keeps the setting. */
int dfl_cache_set_window(dfl_ctx* ctx, int32_t sink, int32_t window);
/* Set the absolute position of the next context row without touching cached rows
 * (the ANE caller assigns cache.offset directly, generate.py:1409-1417). */
int dfl_cache_set_offset(dfl_ctx* ctx, int64_t offset);
/* Assign one layer's cache (c_new.keys = c_old.keys / .values in generate.py:917-941;
 * DFlashKVCache.keys / .values, dflash.py:161-162): keys and values are [NKV][L][128] fp16
 * device rows in the reference's order (post-RoPE keys, values), either may be NULL (then
 * that half is left as it is).  The sequence's cache then holds these L rows -- with a sink +
 * window, L > sink + window keeps the first sink and the newest window rows, as the
 * reference's next update_and_fetch does.  The offset is not changed (set it with
 * dfl_cache_set_offset).  The cached row count is shared by all layers of the sequence:
 * assign every layer with the same L. */
int dfl_cache_assign(dfl_ctx* ctx, int32_t layer, const uint16_t* keys, const uint16_t* values,
                     int32_t L, void* stream);
/* Current cached rows and absolute position offset. */
int dfl_cache_state(const dfl_ctx* ctx, int32_t* len, int64_t* offset);
/* Device pointers of layer `layer`'s cache: K [NKV][cap][128], Vt [NKV][128][cap]. */
int dfl_cache_kv(const dfl_ctx* ctx, int32_t layer, uint16_t** k, uint16_t** vt, int32_t* cap);
/* The cache row holding each cached row in the reference's order (sink rows, then the
 * window oldest first) -- the order of DFlashKVCache.keys (dflash.py:170-193).  Writes
 * *n = cached rows and, if rows != NULL, rows[0 .. *n). */
int dfl_cache_rows(const dfl_ctx* ctx, int32_t* rows, int32_t max_rows, int32_t* n);

/* Kernel timing with HIP events (the reference times phases and kernels with
 * time.perf_counter wrappers: bench_ane_profile.py:41-245, ANEKernel.run_timed
 * wrapper.rs:284-301).  on = 1: each kernel group launched by dfl_draft_block /
 * dfl_ingest_* is timed -- stream-K GEMM launches (projections, lm_head) by their own
 * dispatch timestamps, other groups by events recorded around them on the stream.
 * on = 2: only the stream-K GEMM launches, by dispatch timestamps, which adds no packets
 * to the stream (usable inside a timed run).  on = 0: off.  dfl_profile_read synchronises,
 * returns per-category totals (name <= 31 chars each, in names[i*32]), launch counts
 * and algorithmic bytes (weights + scales for GEMMs, K/V read for attention), then
 * clears the records. */
int dfl_profile_enable(dfl_ctx* ctx, int32_t on);
int dfl_profile_read(dfl_ctx* ctx, int32_t max_cat, char* names, double* total_ms,
                     int64_t* launches, int64_t* bytes, int32_t* n_cat);

/* Block noise embedding (generate.py:594-597 builds embed([anchor, mask x (B-1)])), with the
 * soft anchor of the parallel caller (generate.py:1419-1437): out_noise [B][H] fp16 rows
 * embed[ids[b]] of the loaded embedding; when correction_logits ([V] verify logits at the
 * correction position, logits_dtype 0 fp32 / 1 fp16 / 2 bf16) is not NULL, row 0 is instead
 * sum_r softmax(l)_r * embed[i_r] over the top_k (1..8, the reference uses 8) largest
 * logits l at ids i_r -- fp32 softmax and sum, cast to fp16; lower index first on equal
 * logits, NaN after every number.  V <= vocab. */
int dfl_embed_block(dfl_ctx* ctx, const int32_t* ids, int32_t B, const void* correction_logits,
                    int32_t logits_dtype, int32_t V, int32_t top_k, uint16_t* out_noise,
                    void* stream);

/* No counterpart in the reference: the block noise embedding of dfl_embed_block for callers
 * that cannot allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No context is needed: the caller passes the embedding
 * table embed [Vemb][H] fp16 (16-byte aligned rows, H % 8 == 0) and a device word err_flags
 * that receives the same error bits as dfl_device_errors (OR'ed in; bit 0 a token id outside
 * [0, Vemb), bit 1 soft-anchor logits without a single number).  Other arguments, checks and
 * results as dfl_embed_block.  The soft anchor's top-k candidates go to a fixed 4 KiB device
 * array of the library (64 scan workgroups x 8 keys, one copy per GPU, held until the process
 * ends), so the call allocates nothing; concurrent calls on one GPU share that array and
 * race, so a caller serialises them (one stream, or events between streams). */
int dfl_embed_block_noalloc(const int32_t* ids, int32_t B, const uint16_t* embed, int32_t Vemb,
                            int32_t H, const void* correction_logits, int32_t logits_dtype,
                            int32_t V, int32_t top_k, uint16_t* out_noise, int32_t* err_flags,
                            void* stream);

/* Scaled RoPE (the scaling_config of mlx_lm's initialize_rope, called by
 * Qwen3DFlashAttention, dflash.py:254-261): type DFL_ROPE_DEFAULT (unscaled, the state after
 * dfl_create), DFL_ROPE_LINEAR (positions divided by factor) or DFL_ROPE_LLAMA3 (Llama 3.1:
 * frequencies of wavelength above original_max_position_embeddings / low_freq_factor divided
 * by factor, below original / high_freq_factor kept, smooth in between).  The other
 * arguments are unused for the default type. */
#define DFL_ROPE_DEFAULT 0
#define DFL_ROPE_LINEAR 1
#define DFL_ROPE_LLAMA3 2
int dfl_set_rope_scaling(dfl_ctx* ctx, int32_t type, double factor, double low_freq_factor,
                         double high_freq_factor, int32_t original_max_position_embeddings);

/* Draft tokens as samples (sample(logits, temperature), dflash.py:133-136, called at
 * generate.py:605): with temperature >= 1e-5 the out_ids of later dfl_draft_block /
 * dfl_draft_batch calls are categorical draws from softmax(logits / temperature) per row,
 * taken by the Gumbel-max rule inside the lm_head (argmax of logits / T + Gumbel noise; the
 * optional fp32 logits stay the plain logits); below 1e-5 (the state after dfl_create) they
 * are the argmax.  The noise of each call is a function of seed and the number of sampling
 * calls since this one (deterministic for a given seed; the reference draws from MLX's
 * global generator, so individual draws cannot match it). */
int dfl_set_sampling(dfl_ctx* ctx, float temperature, uint64_t seed);

/* Test hook, no counterpart in the reference: on != 0 makes every work-queue wait of the
 * balanced lm_head give up after a few hundred rounds (its bounded-wait path: every wave
 * still ends, the ids of those calls are invalid and device error bit 2 is set); 0 restores
 * normal operation.  Off when a context is created. */
int dfl_test_queue_timeout(dfl_ctx* ctx, int32_t on);

/* Sticky device-side error flags (bit 0: a token id outside [0, vocab); bit 1: soft-anchor
 * logits without a single number; bit 2: a work-queue wait of the lm_head gave up, its
 * results are invalid); reading clears. */
int dfl_device_errors(dfl_ctx* ctx, int32_t* flags, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DFLASH_HIP_H */
