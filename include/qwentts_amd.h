/*
 * qwentts_amd.h -- C ABI of the MI355X (gfx950) decode kernels for Qwen3-TTS.
 *
 * Two persistent HIP kernels each run a full per-token transformer pass in one launch of
 * 256 co-resident workgroups (one per CU):
 *   - backbone ("talker") kernel: N layers of RMSNorm -> QKV -> interleaved 3D mRoPE -> GQA
 *     attention over a bf16 KV cache -> SwiGLU MLP, final RMSNorm, optional codec-head logits
 *     and on-device token selection;
 *   - code-predictor kernel: N layers with 1D RoPE and an f32 KV cache, stepped once
 *     (reference entry point) or 16 positions per launch with the 15 lm-heads, on-device
 *     token selection, embedding gathers and the codebook-embedding combine (frame entry).
 *
 * All pointers are device pointers unless stated otherwise. Every entry point returns a
 * hipError_t (the reference's launchers return void). Errors detected on the device (a wait
 * that timed out, i.e. a grid that cannot be co-resident or a corrupted workspace) are
 * latched in the workspace and reported by qtts_workspace_check().
 *
 * Dimensions are fixed by the model (reference config.cuh:33-40): hidden 1024, 16 query
 * heads, 8 KV heads, head_dim 128, intermediate 3072. Layer counts, positions and cache
 * lengths are runtime arguments.
 */
#ifndef QWENTTS_AMD_H
#define QWENTTS_AMD_H

#include <hip/hip_runtime_api.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Per-layer weight pointers, in the reference's struct order: bf16 tensors, row-major
 * [out, in] as nn.Linear stores them.
 * Replaces: TTSLayerWeights   (/root/reference/qwentts_turbo/csrc/fused_decode_tts.cu:22-34)
 *           CPLayerWeights    (/root/reference/qwentts_turbo/csrc/fused_decode_code_predictor.cu:30-42)
 * Host mirrors: megakernel_backbone.py:43-55, megakernel_code_predictor.py:47-59. */
typedef struct TTSLayerWeights {
    const void* input_layernorm_weight;     /* [1024]        */
    const void* q_proj_weight;              /* [2048, 1024]  */
    const void* k_proj_weight;              /* [1024, 1024]  */
    const void* v_proj_weight;              /* [1024, 1024]  */
    const void* q_norm_weight;              /* [128]         */
    const void* k_norm_weight;              /* [128]         */
    const void* o_proj_weight;              /* [1024, 2048]  */
    const void* post_attn_layernorm_weight; /* [1024]        */
    const void* gate_proj_weight;           /* [3072, 1024]  */
    const void* up_proj_weight;             /* [3072, 1024]  */
    const void* down_proj_weight;           /* [1024, 3072]  */
} TTSLayerWeights;
typedef TTSLayerWeights CPLayerWeights;

/* ---------------------------------------------------------------------------------------
 * Reference-compatible launchers (same argument lists; hipStream_t; return hipError_t).
 *
 * The scratch arguments (hidden_buffer .. g_mlp_intermediate) keep the reference's sizes and
 * meaning at the boundary: on return hidden_buffer holds the last layer's residual stream
 * (bf16 [1024] for the backbone, f32 [1024] for the code predictor) and g_normalized the
 * final-RMSNorm hidden (f32 [1024]). The inter-workgroup exchange buffers these kernels need
 * live in a library-owned workspace per (device, stream), allocated with hipMalloc on the
 * first call on that stream and freed by qtts_shutdown(): calls on one stream are ordered, and
 * calls on different streams use different workspaces, so concurrent callers on separate
 * streams (e.g. a backbone and a code-predictor decoder) do not share exchange slots.
 *
 * k_cache / v_cache: [num_layers, 8, max_seq_len, 128], bf16 (backbone) or f32 (CP).
 * cache_len must equal position + 1 (the reference passes it that way) and position must be
 * < max_seq_len; attn_scale is 1/sqrt(128). cos_table / sin_table: bf16 [>= max_seq_len, 128].
 * ------------------------------------------------------------------------------------- */

/* Replaces: launch_tts_decode (/root/reference/qwentts_turbo/csrc/fused_decode_tts.cu:664-722) */
hipError_t launch_tts_decode(
    int input_token_id, const void* embed_weight, const TTSLayerWeights* layer_weights,
    const void* final_norm_weight, const void* cos_table, const void* sin_table,
    void* k_cache, void* v_cache, void* hidden_buffer, void* g_activations, void* g_residual,
    void* g_q, void* g_k, void* g_v, void* g_attn_out, void* g_mlp_intermediate,
    void* g_normalized, int num_layers, int position, int cache_len, int max_seq_len,
    float attn_scale, hipStream_t stream);

/* Replaces: launch_tts_decode_with_embedding (/root/reference/qwentts_turbo/csrc/fused_decode_tts.cu:834-890) */
hipError_t launch_tts_decode_with_embedding(
    const void* input_embedding, const TTSLayerWeights* layer_weights,
    const void* final_norm_weight, const void* cos_table, const void* sin_table,
    void* k_cache, void* v_cache, void* hidden_buffer, void* g_activations, void* g_residual,
    void* g_q, void* g_k, void* g_v, void* g_attn_out, void* g_mlp_intermediate,
    void* g_normalized, int num_layers, int position, int cache_len, int max_seq_len,
    float attn_scale, hipStream_t stream);

/* No counterpart in the reference. For callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc): the same step as
 * launch_tts_decode_with_embedding, but the exchange workspace is a static device array of
 * QTTS_STATIC_SCRATCH_BYTES per GPU (one qtts_workspace_bytes() workspace), held until the
 * process ends; no hipMalloc / hipFree / allocating routine is called (the first call on a
 * device runs the one-time device set-up: property queries, a probe launch, an event).
 * num_layers must be in [1, 440] (the launch tags of one workspace cover 440 layers); larger
 * values return hipErrorInvalidValue. Every call on a GPU uses that GPU's one array, which
 * keeps the last call's contents (the library zero-fills it before its first use and tags
 * every later exchange, so nothing needs clearing between calls). The library orders its own
 * launches on a device, but calls that are made to overlap on one GPU (other processes,
 * graphs replayed concurrently on several streams) race on the array. */
#define QTTS_STATIC_SCRATCH_BYTES 1261824u
hipError_t launch_tts_decode_with_embedding_static(
    const void* input_embedding, const TTSLayerWeights* layer_weights,
    const void* final_norm_weight, const void* cos_table, const void* sin_table,
    void* k_cache, void* v_cache, void* hidden_buffer, void* g_activations, void* g_residual,
    void* g_q, void* g_k, void* g_v, void* g_attn_out, void* g_mlp_intermediate,
    void* g_normalized, int num_layers, int position, int cache_len, int max_seq_len,
    float attn_scale, hipStream_t stream);

/* Replaces: launch_cp_decode_with_embedding (/root/reference/qwentts_turbo/csrc/fused_decode_code_predictor.cu:674-730) */
hipError_t launch_cp_decode_with_embedding(
    const void* input_embedding, const CPLayerWeights* layer_weights,
    const void* final_norm_weight, const void* cos_table, const void* sin_table,
    void* k_cache, void* v_cache, void* hidden_buffer, void* g_activations, void* g_residual,
    void* g_q, void* g_k, void* g_v, void* g_attn_out, void* g_mlp_intermediate,
    void* g_normalized, int num_layers, int position, int cache_len, int max_seq_len,
    float attn_scale, hipStream_t stream);

/* ---------------------------------------------------------------------------------------
 * Extended API: explicit workspace, 3D rotary positions, fused heads and token selection.
 * Used by the PyTorch extension (MegakernelTTSDecoder / MegakernelCodePredictorDecoder).
 * ------------------------------------------------------------------------------------- */

typedef struct QttsWorkspace QttsWorkspace; /* opaque, device-resident */

/* Bytes of device memory a workspace needs. */
size_t qtts_workspace_bytes(void);

/* Validates the device (gfx950, 256 CUs in 8 XCDs, one workgroup of each kernel per CU) once
 * per device and binds a caller-allocated workspace of qtts_workspace_bytes() bytes (256-byte
 * aligned): the first launch that uses it zero-fills it on the launch stream.
 * Returns hipErrorInvalidDevice when the device cannot run these kernels. */
hipError_t qtts_workspace_init(void* workspace, int device);

/* Forgets the launch sequence of `count` consecutive workspaces at `workspace`; call before
 * their memory is freed or reused (the next launch on that memory zero-fills it first). */
hipError_t qtts_workspace_release(void* workspace, int count);

/* Frees the library-owned workspaces of the reference-compatible launchers (after
 * synchronising their devices) and forgets every workspace's launch sequence. Call when no
 * launch is in flight, e.g. at process teardown while the HIP runtime is still up; the
 * library stays usable afterwards (workspaces are re-created on demand). */
hipError_t qtts_shutdown(void);

/* Test hook: sets the launch sequence of one workspace (1 .. 2^20 - 1) so that a test can
 * cross the point where the sequence space is used up and the workspace is zero-filled. */
hipError_t qtts_debug_set_sequence(void* workspace, unsigned int sequence);

/* Reads and clears the device-side error word of a workspace (synchronises the stream).
 * *error_code = 0 when every wait completed; bit 0 = a wait timed out. */
hipError_t qtts_workspace_check(void* workspace, unsigned int* error_code, hipStream_t stream);

/* Launch residency. The launches are plain (not cooperative): all 256 workgroups are resident
 * at once only when no other kernel holds CUs. The waits of a launch's first layer pass can
 * complete only once every workgroup has started, so they run under a short cap (about 30 ms of
 * polling, against about 4 s for later waits): a launch that does not find the whole GPU sets
 * the error word within milliseconds, every later wait gives up at its next check, and every
 * workgroup runs to its end; qtts_workspace_check (the extension's check_error) reports it.
 * No counterpart in the reference, whose cooperative launch would fail at launch instead. */

/* Test hook: pre-sets the error word of a workspace that has been launched on at least once
 * (its first launch zero-fills it) to `code` (nonzero), so that every wait of the next launch
 * gives up at its first check, as after a timed-out wait. Synchronises the stream. */
hipError_t qtts_debug_set_error(void* workspace, unsigned int code, hipStream_t stream);

/* Test hook: the poll cap of the first layer pass of every later persistent launch (0 restores
 * the default of 2^15 poll rounds). */
hipError_t qtts_debug_entry_spin_cap(unsigned int cap);

/* Diagnostics: when device_buffer is non-NULL (>= 256 * 1024 * 2 * 8 bytes), every later launch
 * records, per workgroup and step, the s_memrealtime stamp (100 MHz) at which its poller wave
 * (slot 1) and math waves (slot 0) finished the step: buffer[(wg * 1024 + step) * 2 + slot].
 * NULL switches recording off. Not thread-safe against concurrent launches. */
hipError_t qtts_debug_trace(void* device_buffer, size_t bytes);

/* Token selection for one head (backbone g0 or a code-predictor group).
 * Mirrors generator.py:178-207: optional EOS suppression, greedy argmax (lowest index on
 * ties) or temperature -> top-k (ties with the k-th value kept) -> top-p (a value is kept
 * when the probability mass of strictly larger values is <= top_p) -> Gumbel-max draw with
 * Philox-4x64-10 noise keyed by (seed, frame_step, group, vocab id). */
typedef struct QttsSampling {
    int do_sample;
    float temperature;
    int top_k;
    float top_p;
    unsigned long long seed;
} QttsSampling;

/* One backbone decode step.
 *   input_embedding: bf16 [1024] (or NULL to gather row input_token_id of embed_weight)
 *   pos3: rotary positions (t, h, w) for interleaved mRoPE; all equal = 1D RoPE
 *   position: cache slot written (attends to slots [0, position])
 *   out_hidden: f32 [1024] final-norm hidden; out_residual: bf16 [1024] (may be NULL)
 *   codec_head: bf16 [vocab, 1024] or NULL (no logits); out_logits: f32 [vocab] or NULL
 *   When codec_head != NULL and out_token != NULL the step also selects a token:
 *     if mask_tail != 0 the ids [vocab-1024, vocab) except eos_id are masked (the
 *     generator's suppress mask, generator.py:71-75), the repetition penalty is
 *     applied to the ids in history[0..n_history) (device int array), eos_id is additionally
 *     masked when suppress_eos != 0, then QttsSampling picks *out_token (device int).
 *   skip_if: device int or NULL; when it holds a nonzero value the launch does nothing (used
 *     to stop a queued frame loop after EOS without a host round trip). */
hipError_t qtts_backbone_step(
    void* workspace, const TTSLayerWeights* layer_weights, int num_layers,
    const void* final_norm_weight, const void* cos_table, const void* sin_table,
    void* k_cache, void* v_cache, int max_seq_len, int position, const int pos3[3],
    const void* input_embedding, const void* embed_weight, int input_token_id,
    float* out_hidden, void* out_residual,
    const void* codec_head, int vocab, float* out_logits,
    int* out_token, int mask_tail, const int* history, int n_history, float repetition_penalty,
    int eos_id, int suppress_eos, const QttsSampling* sampling, int frame_step,
    const int* skip_if, hipStream_t stream);

/* One code-predictor step (no head): the reference's CP decode with a workspace. */
hipError_t qtts_cp_step(
    void* workspace, const CPLayerWeights* layer_weights, int num_layers,
    const void* final_norm_weight, const void* cos_table, const void* sin_table,
    void* k_cache, void* v_cache, int max_seq_len, int position,
    const void* input_embedding, float* out_hidden, float* out_residual, hipStream_t stream);

/* Whole code-predictor frame in one launch (generator.py:309-362 moved on-device):
 *   position 0 input = bf16(bb_hidden) (f32 [1024]), position 1 input = bb_embedding[*g0],
 *   then for g = 0..n_groups-1: logits_g = lm_heads[g] . bf16(h), token g+1 selected with
 *   `sampling` (group g+1), next input = cp_embeddings[g][token];
 *   writes out_tokens[0] = *g0, out_tokens[1..n_groups] = the selected ids, and
 *   out_combined (bf16 [1024]) = bf16 running sum of bb_embedding[g0] and the n_groups
 *   code-predictor embeddings, plus text_row (bf16 [1024], may be NULL).
 *   lm_heads / cp_embeddings: device arrays of n_groups pointers to bf16 [cp_vocab, 1024].
 *   g0_history_slot: device int or NULL; receives *g0 (the repetition-penalty history).
 *   If *g0 == eos_id (eos_id >= 0) nothing is computed and *done is set to 1.
 *   k_cache / v_cache: f32 [num_layers, 8, >= n_groups + 1, 128]. */
hipError_t qtts_cp_frame(
    void* workspace, const CPLayerWeights* layer_weights, int num_layers,
    const void* final_norm_weight, const void* cos_table, const void* sin_table,
    void* k_cache, void* v_cache, int max_seq_len,
    const float* bb_hidden, const int* g0, const void* bb_embedding,
    const void* const* lm_heads, const void* const* cp_embeddings, int n_groups, int cp_vocab,
    const void* text_row, int* out_tokens, void* out_combined, int* g0_history_slot,
    int eos_id, int* done, const QttsSampling* sampling, int frame_step, hipStream_t stream);

/* One stream of qtts_backbone_step_streams (host memory; device pointers inside). */
typedef struct QttsBackboneStream {
    void* k_cache;                /* bf16 [num_layers, 8, max_seq_len, 128] of this stream */
    void* v_cache;
    int position;                 /* cache slot written; attention covers slots 0..position */
    int pos3[3];                  /* rotary (t, h, w) */
    const void* input_embedding;  /* bf16 [1024] */
    float* out_hidden;            /* f32 [1024] final-norm hidden, or NULL */
    void* out_residual;           /* bf16 [1024] pre-norm residual, or NULL */
    float* out_logits;            /* f32 [vocab], or NULL */
    int* out_token;               /* int32 [1] selected group-0 token, or NULL */
    const int* history;           /* int32 [n_history] previously generated group-0 tokens */
    int n_history;
    unsigned long long seed;      /* sampler key */
    const int* skip_if;           /* device int or NULL: nonzero = this stream computes nothing
                                     (its XCD idles; used for streams that reached EOS) */
} QttsBackboneStream;

/* Backbone steps (codec head + selection as in qtts_backbone_step) of n_streams (1..8) independent
 * streams in one launch; no counterpart in the reference, whose decode is batch 1
 * (fused_decode_tts.cu:728-831). Stream s runs on XCD s alone (its 32 workgroups, every exchange in
 * that XCD's L2) with its own KV cache, position and length, and computes exactly what
 * qtts_backbone_step computes for it. workspaces: n_streams x qtts_workspace_bytes(), 256-byte
 * aligned, zero-filled before first use. */
hipError_t qtts_backbone_step_streams(
    int n_streams, void* workspaces, const TTSLayerWeights* layer_weights, int num_layers,
    const void* final_norm_weight, const void* cos_table, const void* sin_table, int max_seq_len,
    const QttsBackboneStream* streams, const void* codec_head, int vocab, int mask_tail,
    float repetition_penalty, int eos_id, int suppress_eos, const QttsSampling* sampling,
    int frame_step, hipStream_t stream);

/* Backbone prefill: n_tokens prompt embeddings (bf16 [n_tokens, 1024], device) through all
 * layers at once, replacing the reference's PyTorch talker prefill and KV handoff
 * (generator.py:209-225, :245-257; megakernel_backbone.py:285-294). K/V of cache positions
 * position .. position + n_tokens - 1 are written into k_cache / v_cache (bf16
 * [num_layers, 8, max_seq_len, 128], the decode layout); attention covers cache positions
 * 0 .. position + n_tokens - 1 (causal), so a prefix already in the cache is attended.
 * Arithmetic follows the transformers bf16 forward (bf16 storage after every op, f32 sums on
 * bf16 MFMA). pos3: NULL (t = h = w = position of the token) or device int32 [3][n_tokens]
 * rotary (t, h, w) rows of the bf16 tables (clamped to [0, max_seq_len)). out_hidden: f32 [1024],
 * the final-norm hidden of the last token (bf16 values). When codec_head is not NULL the first
 * group-0 token is selected from bf16(codec_head . hidden) as in generator.py:113-119 (suppress
 * mask when mask_tail, EOS removed when suppress_eos, greedy or sampled) into out_token; the
 * logits go to out_logits when not NULL. workspace: >= qtts_prefill_workspace_bytes(n_tokens,
 * vocab) bytes, 256-byte aligned (contents need no initialisation). */
size_t qtts_prefill_workspace_bytes(int n_tokens, int vocab);
hipError_t qtts_backbone_prefill(
    void* workspace, size_t workspace_bytes, const TTSLayerWeights* layer_weights, int num_layers,
    const void* final_norm_weight, const void* cos_table, const void* sin_table, void* k_cache,
    void* v_cache, int max_seq_len, int position, int n_tokens, const int* pos3,
    const void* input_embeddings, float* out_hidden, const void* codec_head, int vocab,
    float* out_logits, int* out_token, int mask_tail, int eos_id, int suppress_eos,
    const QttsSampling* sampling, int frame_step, hipStream_t stream);

/* Code-predictor frames of n_streams (1..8) independent streams in one launch; no counterpart in the
 * reference, whose decode is batch 1 (fused_decode_code_predictor.cu:565-668 runs one stream). Stream s
 * runs on XCD s alone (its 32 workgroups, every exchange in that XCD's L2) and computes exactly what
 * qtts_cp_frame computes for it. Per-stream data is contiguous with fixed strides:
 *   workspaces: n_streams x qtts_workspace_bytes(), 256-byte aligned, zero-filled before first use;
 *   k_caches / v_caches: n_streams x (num_layers x 8 x max_seq_len x 128) f32;
 *   bb_hidden [n, 1024] f32; g0 [n] int32; text_rows [n, 1024] bf16 or NULL;
 *   out_tokens [n, n_groups + 1] int32; out_combined [n, 1024] bf16; done [n] int32.
 * Stream s draws with key sampling->seed + s. n_groups + 1 <= 16 (one attention pass). */
hipError_t qtts_cp_frame_streams(
    int n_streams, void* workspaces, const CPLayerWeights* layer_weights, int num_layers,
    const void* final_norm_weight, const void* cos_table, const void* sin_table,
    void* k_caches, void* v_caches, int max_seq_len,
    const float* bb_hidden, const int* g0, const void* bb_embedding,
    const void* const* lm_heads, const void* const* cp_embeddings, int n_groups, int cp_vocab,
    const void* text_rows, int* out_tokens, void* out_combined,
    int eos_id, int* done, const QttsSampling* sampling, int frame_step, hipStream_t stream);

/* Weight-shared decode of several streams (config 4); no counterpart in the reference, whose
 * decode is batch 1 (fused_decode_tts.cu:728-831, fused_decode_code_predictor.cu:565-668).
 * Same arguments as qtts_backbone_step_streams / qtts_cp_frame_streams, but the n_streams (1..8)
 * streams share every weight read: each workgroup applies its weight tile to all streams at once
 * on bf16 MFMA, with each stream's f32 input split exactly into three bf16 pieces and f32 sums
 * (the reference's f32 GEMV accuracy; results agree with the batch-1 kernels to rounding, not bit
 * for bit). One workspace of qtts_shared_workspace_bytes() serves all streams of a launch
 * (256-byte aligned; zero-filled by its first launch, or after qtts_workspace_release(ws, 1)).
 * Backbone: each stream at its own position and length; codec_head rows vocab / 256 <= 16.
 * Code predictor: n_groups + 1 <= 16, cp_vocab / 256 <= 16. qtts_shared_workspace_check reads
 * and clears the workspace's wait-timeout error word (synchronises the stream). */
size_t qtts_shared_workspace_bytes(void);
hipError_t qtts_shared_workspace_check(void* workspace, unsigned int* error_code, hipStream_t stream);
hipError_t qtts_backbone_step_shared(
    int n_streams, void* workspace, const TTSLayerWeights* layer_weights, int num_layers,
    const void* final_norm_weight, const void* cos_table, const void* sin_table, int max_seq_len,
    const QttsBackboneStream* streams, const void* codec_head, int vocab, int mask_tail,
    float repetition_penalty, int eos_id, int suppress_eos, const QttsSampling* sampling,
    int frame_step, hipStream_t stream);
hipError_t qtts_cp_frame_shared(
    int n_streams, void* workspace, const CPLayerWeights* layer_weights, int num_layers,
    const void* final_norm_weight, const void* cos_table, const void* sin_table,
    void* k_caches, void* v_caches, int max_seq_len,
    const float* bb_hidden, const int* g0, const void* bb_embedding,
    const void* const* lm_heads, const void* const* cp_embeddings, int n_groups, int cp_vocab,
    const void* text_rows, int* out_tokens, void* out_combined,
    int eos_id, int* done, const QttsSampling* sampling, int frame_step, hipStream_t stream);

/* Debugging aid (no reference counterpart): record the weight-shared kernels' step timeline
 * (s_memrealtime stamps, [256 workgroups][1024 steps][16]: after the entry barrier, after the
 * partials barrier, the end of each of the 8 waves' vector work, 6 points inside a step) into
 * device_buffer (>= 33,554,432 bytes); NULL turns it off. */
hipError_t qtts_debug_trace_shared(void* device_buffer, size_t bytes);

#ifdef __cplusplus
}
#endif

#endif /* QWENTTS_AMD_H */
