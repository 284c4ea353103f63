/*
 * tokhip.h - C ABI of the MI355X (gfx950) session attention library.
 *
 * Drop-in device replacement for toklet's session attention path: the
 * scalar operators in src/cpu/{attention,window_attention,span_attention,
 * softcap}.rs and the KV owners in src/model/{cache,window_cache}.rs.
 * Plain pointers and sizes only; no C++ or torch types cross this boundary.
 *
 * Conventions
 *  - Every entry point returns a tkh_status code and, when `err` is not NULL,
 *    fills it with the same code plus the payload of the matching toklet
 *    error (tensor name, index, expected/actual length, message).
 *  - Codes 1..7 mirror toklet::cpu::Error (src/cpu/mod.rs:47-68) in order;
 *    the remaining codes mirror model::Error::Capacity/InvalidConfig and the
 *    device runtime.  The message rule follows toklet's C ABI
 *    (apple/include/toklet.h:9-35): a NULL `err` suppresses the payload.
 *  - Element lengths (`*_len`) are checked on the host against the shape
 *    before any launch, as the reference checks slice lengths before writes.
 *  - Finiteness of Q/K/V is checked inside the kernels through a device
 *    status word (the Metal precedent's status atomic,
 *    src/metal/kernels.metal:31-35).  A synchronous context reports
 *    TKH_NON_FINITE after the call; the context contents are then
 *    unspecified and must be discarded, as the reference discards partial
 *    output after an arithmetic failure (src/cpu/mod.rs:5-7).  Shape and
 *    length errors are reported before any launch and leave every output
 *    untouched.  Every finite input is computed, at every dtype and by every
 *    kernel (the chunk kernel forms rows whose bf16 V exceeds f16's range
 *    again in FP32).
 *  - Tensors passed to operators are device pointers (HBM).  Q/context use
 *    [tokens, query_heads, head_dim]; K/V use the reference's head-major
 *    [kv_heads, capacity, head_dim] layout (strides [capacity*D, D, 1]).
 *  - Q is stored in the same dtype as K/V (the Metal precedent in
 *    src/metal/kernels.metal:104-107 and :136-139 also consumes half Q and
 *    half K/V); context is always FP32.
 *  - A tkh_context owns one HIP stream, a device workspace and the status
 *    word.  It is not thread-safe; separate contexts are independent.
 *  - No operator allocates.  Device memory is allocated only by
 *    tkh_context_create and tkh_kv_create.
 */
#ifndef TOKHIP_H
#define TOKHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* 2: tkh_producer_shape and tkh_session_options end with the Llama 3 rotary
 * parameters (low/high frequency factors, original context length), and
 * tkh_session_options with shared_layers. */
#define TKH_ABI_VERSION 2u

typedef enum tkh_status {
    TKH_OK = 0,
    TKH_ZERO_DIMENSION = 1,    /* cpu::Error::ZeroDimension */
    TKH_SIZE_OVERFLOW = 2,     /* cpu::Error::SizeOverflow */
    TKH_LENGTH = 3,            /* cpu::Error::Length */
    TKH_TOKEN = 4,             /* cpu::Error::Token */
    TKH_NON_FINITE = 5,        /* cpu::Error::NonFinite */
    TKH_INVALID_PARAMETER = 6, /* cpu::Error::InvalidParameter */
    TKH_FULLY_MASKED = 7,      /* cpu::Error::FullyMasked */
    TKH_CAPACITY = 8,          /* model::Error::Capacity (src/model/window_cache.rs:214-228) */
    TKH_INVALID_CONFIG = 9,    /* model::Error::InvalidConfig (stale/foreign KV frame, geometry) */
    TKH_DEVICE = 10,           /* HIP runtime failure */
    TKH_UNSUPPORTED = 11,      /* a shape/dtype this build does not run */
} tkh_status;

typedef struct tkh_error {
    uint32_t code;
    uint64_t index;    /* NonFinite index / FullyMasked row */
    uint64_t expected; /* Length */
    uint64_t actual;   /* Length */
    char tensor[64];
    char message[256];
} tkh_error;

typedef enum tkh_dtype { TKH_F32 = 0, TKH_F16 = 1, TKH_BF16 = 2 } tkh_dtype;

typedef struct tkh_context tkh_context;
typedef struct tkh_kv tkh_kv;

/* ---------------- library / context ---------------- */

uint32_t tkh_abi_version(void);

/* Create a context on `device`.  `stream` is the hipStream_t every call of
 * this context is queued on (NULL: the null stream).  `workspace_bytes` bounds the
 * split-K partial buffers (0: 256 MiB).  `synchronous` != 0 makes every
 * operator wait for completion and report the device status; otherwise
 * status accumulates until tkh_context_synchronize. */
uint32_t tkh_context_create(int device, void *stream, size_t workspace_bytes, int synchronous,
                            tkh_context **out, tkh_error *err);
void tkh_context_destroy(tkh_context *ctx);
/* Wait for queued work, report and clear the accumulated device status. */
uint32_t tkh_context_synchronize(tkh_context *ctx, tkh_error *err);
void *tkh_context_stream(tkh_context *ctx);

/* Kernel timing with HIP events on the context's stream (the role of the
 * reference's Metal encoder timestamps, src/metal/profile.rs:1-3).  Enabling
 * resets the totals; reading waits for the stream.  Times are milliseconds
 * summed over launches: `attention` is the attention kernel alone, `combine`
 * the split-K combine/publish kernel. */
typedef struct tkh_profile {
    uint64_t launches;
    double attention_ms;
    double combine_ms;
} tkh_profile;
uint32_t tkh_context_profile(tkh_context *ctx, int enable, tkh_error *err);
uint32_t tkh_context_profile_read(tkh_context *ctx, tkh_profile *out, tkh_error *err);

/* ---------------- operators ---------------- */

/* Shape of toklet::cpu::CachedAttentionShape (src/cpu/attention.rs:180-189). */
typedef struct tkh_cached_shape {
    uint64_t tokens, query_heads, kv_heads, head_dim, capacity, offset;
} tkh_cached_shape;

/* Replaces cpu::attention_cached (src/cpu/attention.rs:201-296).
 * q/context: [tokens, Hq, D]; k/v: [Hkv, capacity, D] in `dtype`.
 * scores/probabilities: optional (NULL) [capacity] FP32 rows; when given they
 * receive the row the reference leaves behind (last query head, last query). */
uint32_t tkh_attention_cached(tkh_context *ctx, const tkh_cached_shape *shape, tkh_dtype dtype,
                              const void *q, uint64_t q_len, const void *k, uint64_t k_len,
                              const void *v, uint64_t v_len, float *context,
                              uint64_t context_len, float *scores, uint64_t scores_len,
                              float *probabilities, uint64_t probabilities_len, tkh_error *err);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): tkh_attention_cached without a context and without the
 * score/probability rows.  Its split-K partials, decode completion flags and
 * (with status == NULL) its status word live in a fixed device array of
 * TKH_STATIC_SCRATCH_BYTES per GPU, set up by the first call on each device
 * and held until the process ends; no call allocates or frees memory.  A
 * shape whose partials cannot fit the array returns TKH_UNSUPPORTED and
 * computes nothing.  `stream` is the hipStream_t the work is queued on (NULL:
 * the null stream).
 *  - status != NULL: a device word owned by the caller; the kernels OR their
 *    status bits into it and the call returns once the work is queued.  The
 *    word is never cleared here.  Nonzero means the results are invalid:
 *    bit 3 (8) a decode merge timed out (TKH_DEVICE), any other bit a
 *    non-finite input or result (TKH_NON_FINITE).
 *  - status == NULL: the call waits for the stream and reports as a
 *    synchronous context does.
 * Every call on one GPU shares that GPU's array and keeps its last contents:
 * calls that overlap on a GPU (from other streams or threads) race. */
#define TKH_STATIC_SCRATCH_BYTES (16u << 20)
uint32_t tkh_attention_cached_static(int device, void *stream, const tkh_cached_shape *shape,
                                     tkh_dtype dtype, const void *q, uint64_t q_len, const void *k,
                                     uint64_t k_len, const void *v, uint64_t v_len, float *context,
                                     uint64_t context_len, uint32_t *status, tkh_error *err);

/* Shape of toklet::cpu::AttentionShape (src/cpu/attention.rs:67-72). */
typedef struct tkh_attention_shape {
    uint64_t tokens, query_heads, kv_heads, head_dim;
} tkh_attention_shape;

/* Replaces cpu::attention (src/cpu/attention.rs:85-178): full-prefix causal
 * GQA with token-major K/V [tokens, Hkv, D].  scores/probabilities: optional
 * [Hq, tokens, tokens] FP32 with masked probabilities exactly +0. */
uint32_t tkh_attention(tkh_context *ctx, const tkh_attention_shape *shape, tkh_dtype dtype,
                       const void *q, uint64_t q_len, const void *k, uint64_t k_len,
                       const void *v, uint64_t v_len, float *context, uint64_t context_len,
                       float *scores, uint64_t scores_len, float *probabilities,
                       uint64_t probabilities_len, tkh_error *err);

/* Shape of toklet::cpu::WindowAttentionShape (src/cpu/window_attention.rs:6-17)
 * with Option<usize> window as (has_window, window).  `softcap` (> 0) applies
 * cap*tanh(score/cap) to every score after scaling (0: disabled). */
typedef struct tkh_window_shape {
    uint64_t queries, keys, capacity, query_heads, kv_heads, head_dim;
    uint64_t query_start, key_start;
    uint32_t has_window;
    uint64_t window;
    float scale;
    float softcap;
} tkh_window_shape;

/* Replaces cpu::window_attention (src/cpu/window_attention.rs:36-168).
 * scores/probabilities: optional [Hq, queries, keys]. */
uint32_t tkh_window_attention(tkh_context *ctx, const tkh_window_shape *shape, tkh_dtype dtype,
                              const void *q, uint64_t q_len, const void *k, uint64_t k_len,
                              const void *v, uint64_t v_len, float *context,
                              uint64_t context_len, float *scores, uint64_t scores_len,
                              float *probabilities, uint64_t probabilities_len, tkh_error *err);

/* toklet::cpu::AttentionKvSegment (src/cpu/span_attention.rs:9-16): rows of
 * KV head h start at h*head_stride elements; an empty segment has keys = 0. */
typedef struct tkh_segment {
    const void *k;
    uint64_t k_len;
    const void *v;
    uint64_t v_len;
    uint64_t keys, head_stride, key_start;
} tkh_segment;

/* toklet::cpu::SpanAttentionShape (src/cpu/span_attention.rs:18-28) + softcap. */
typedef struct tkh_span_shape {
    uint64_t queries, keys, query_heads, kv_heads, head_dim;
    uint64_t query_start, key_start;
    uint32_t has_window;
    uint64_t window;
    float scale;
    float softcap;
} tkh_span_shape;

/* Replaces cpu::span_attention (src/cpu/span_attention.rs:42-220): attention
 * over <=2 old ring spans plus the staged chunk, without linearising the ring. */
uint32_t tkh_span_attention(tkh_context *ctx, const tkh_span_shape *shape, tkh_dtype dtype,
                            const void *q, uint64_t q_len, const tkh_segment segments[3],
                            float *context, uint64_t context_len, float *scores,
                            uint64_t scores_len, float *probabilities, uint64_t probabilities_len,
                            tkh_error *err);

/* The step after attention, for token identity without host logits: the
 * FP32 o-projection of cpu::matmul (src/cpu/mod.rs:140-247, no bias) followed
 * by sampling::greedy (src/sampling.rs:5-18) on every row, in one call (no
 * single reference call does both).  logits[r, v] = sum_d context[r, d] *
 * weights[v, d], each product and each addition rounded in feature order as
 * the reference's loop rounds them, so the logits are the reference's bit for
 * bit; tokens[r] is the lowest id of row r's largest logit (+0 and -0 tie).
 * context: [rows, hidden], weights: [vocab, hidden], logits: optional (NULL)
 * [rows, vocab], all FP32; tokens: [rows] uint32; device pointers.  The
 * checks follow matmul's order, then greedy's vocabulary bound; a non-finite
 * logit (from any non-finite input) is TKH_NON_FINITE. */
uint32_t tkh_project_greedy(tkh_context *ctx, uint64_t rows, uint64_t hidden, uint64_t vocab,
                            const float *context, uint64_t context_len, const float *weights,
                            uint64_t weights_len, float *logits, uint64_t logits_len,
                            uint32_t *tokens, uint64_t tokens_len, tkh_error *err);

/* Replaces cpu::logit_softcap (src/cpu/softcap.rs:16-29) on a device buffer. */
uint32_t tkh_logit_softcap(tkh_context *ctx, float *logits, uint64_t len, float cap,
                           tkh_error *err);

/* Batched single-token decode over independent sessions (no reference
 * counterpart; the batched form of attention_cached with tokens = 1 that a
 * multi-session host loop would otherwise issue per session).
 * q: [batch, Hq, D] in `dtype`; context: [batch, Hq, D] FP32.
 * Session b reads K/V rows [0, lengths[b]) of head-major caches whose first
 * element is k_base/v_base + offsets[b] (elements) with per-head stride
 * head_strides[b].  lengths/offsets/head_strides are host arrays. */
uint32_t tkh_decode_batch(tkh_context *ctx, uint64_t batch, uint64_t query_heads,
                          uint64_t kv_heads, uint64_t head_dim, tkh_dtype dtype, const void *q,
                          const void *k_base, const void *v_base, const uint64_t *offsets,
                          const uint64_t *head_strides, const uint64_t *lengths, float scale,
                          float *context, tkh_error *err);

/* Batched chunk prefill: `batch` sessions, each with `tokens` new queries at
 * cache offset offsets_pos[b] (keys [0, offsets_pos[b] + tokens) visible
 * causally), K/V addressed as in tkh_decode_batch.  q: [batch, tokens, Hq, D]. */
uint32_t tkh_prefill_batch(tkh_context *ctx, uint64_t batch, uint64_t tokens,
                           uint64_t query_heads, uint64_t kv_heads, uint64_t head_dim,
                           tkh_dtype dtype, const void *q, const void *k_base,
                           const void *v_base, const uint64_t *offsets,
                           const uint64_t *head_strides, const uint64_t *positions, float scale,
                           float *context, tkh_error *err);

/* ---------------- KV owners ---------------- */

/* Byte accounting of capacity::KvOwner::at_capacity (src/capacity.rs:49-80)
 * for one K/V pair with `storage` element size (bf16 is this build's
 * addition to KvStorage).  has_window selects Retention::Sliding. */
uint32_t tkh_kv_planned_bytes(uint64_t heads, uint64_t head_dim, uint64_t capacity,
                              uint32_t has_window, uint64_t window, tkh_dtype storage,
                              uint64_t copies, uint64_t *total_bytes, tkh_error *err);

/* Device-resident owner of separate head-major K/V [heads, capacity, dims].
 * Full retention mirrors model::KvCache's LayerKv (src/model/cache.rs:1-97);
 * sliding retention mirrors WindowKvCache (src/model/window_cache.rs:21-464)
 * with slot = position mod capacity and capacity == window. */
uint32_t tkh_kv_create(tkh_context *ctx, uint64_t heads, uint64_t dims, uint64_t capacity,
                       uint64_t max_positions, uint32_t has_window, uint64_t window,
                       tkh_dtype storage, tkh_kv **out, tkh_error *err);
/* Safe in any order with tkh_context_destroy of the owning context. */
void tkh_kv_destroy(tkh_kv *kv);

typedef struct tkh_kv_info {
    uint64_t heads, dims, capacity, max_positions, window, offset, generation, owner;
    uint32_t has_window;
    tkh_dtype storage;
    void *k; /* device base of K [heads, capacity, dims] */
    void *v;
    uint64_t allocated_bytes;
} tkh_kv_info;
uint32_t tkh_kv_info_get(const tkh_kv *kv, tkh_kv_info *info);

/* LayerKv::append (src/model/cache.rs:64-85): convert token-major new rows
 * [tokens, heads, dims] (device, `src_dtype`) into head-major rows
 * [offset, offset+tokens) of a full-retention cache, rounding to the storage
 * dtype.  Non-finite inputs set the device status (TKH_NON_FINITE). */
uint32_t tkh_kv_append(tkh_kv *kv, uint64_t offset, uint64_t tokens, tkh_dtype src_dtype,
                       const void *k, const void *v, tkh_error *err);

/* WindowKvCache::prepare (src/model/window_cache.rs:193-212).  k/v are the
 * caller's staged new rows [heads, tokens, dims] in the storage dtype on the
 * device; they must stay unchanged until the frame is committed or dropped. */
typedef struct tkh_kv_frame {
    const void *k;
    const void *v;
    uint64_t owner, generation, offset, tokens;
} tkh_kv_frame;
uint32_t tkh_kv_prepare(const tkh_kv *kv, const void *k, uint64_t k_len, const void *v,
                        uint64_t v_len, uint64_t tokens, tkh_kv_frame *frame, tkh_error *err);

/* WindowKvCache::view + KvView::segments/attention_shape
 * (src/model/window_cache.rs:256-267, 355-406): the three segments (<=2 old
 * spans in the ring, then the staged chunk) and the matching span shape. */
uint32_t tkh_kv_view(const tkh_kv *kv, const tkh_kv_frame *frame, uint64_t query_heads,
                     float scale, tkh_segment segments[3], tkh_span_shape *shape,
                     tkh_error *err);

/* commit_batch (src/model/window_cache.rs:328-337): validate every frame,
 * then copy only window_rows::copy_runs rows of each into its ring. */
uint32_t tkh_kv_commit_batch(tkh_kv *const *kvs, const tkh_kv_frame *frames, uint64_t count,
                             tkh_error *err);

/* reset_batch (src/model/window_cache.rs:342-350): offset 0, new generation. */
uint32_t tkh_kv_reset_batch(tkh_kv *const *kvs, uint64_t count, tkh_error *err);

/* ---------------- producer (the step before attention) ---------------- */

/* Rotary variants: none, Qwen split-half (src/cpu/attention.rs:10-64),
 * proportional (src/cpu/proportional_rotary.rs:32-91) and Llama 3
 * wavelength-band scaling (src/cpu/llama3_rotary.rs:13-146, selected by
 * PositionPlan::Llama3, src/model/position.rs:7-45). */
typedef enum tkh_rotary {
    TKH_ROTARY_NONE = 0,
    TKH_ROTARY_SPLIT_HALF = 1,
    TKH_ROTARY_PROPORTIONAL = 2,
    TKH_ROTARY_LLAMA3 = 3
} tkh_rotary;

/* Per-layer producer of Model::run (src/model/mod.rs:611-662): optional
 * per-head RMSNorm of Q and K (cpu::rmsnorm, src/cpu/reductions.rs:8-49,
 * FP64), then rotary at absolute positions position..position+tokens-1. */
typedef struct tkh_producer_shape {
    uint64_t tokens, query_heads, kv_heads, head_dim;
    uint64_t position;
    float norm_epsilon;  /* used when norm weights are given */
    uint32_t rotary;     /* tkh_rotary */
    float theta;         /* split-half / Llama 3 theta, or proportional base */
    uint64_t rotated_dims; /* proportional only */
    float factor;          /* proportional and Llama 3 (Llama3Scaling::new: >= 1) */
    float low_freq_factor;           /* Llama 3 only: > 0 */
    float high_freq_factor;          /* Llama 3 only: > low_freq_factor */
    uint64_t original_max_positions; /* Llama 3 only: 1..2^53 */
} tkh_producer_shape;

/* Replaces the rmsnorm -> rotary -> LayerKv::append sequence of Model::run
 * for one layer and chunk, fused into one launch (no reference counterpart
 * as a single call).  q/k/v_proj: device FP32 token-major [tokens, H, D].
 * q_norm/k_norm: device FP32 [D] or NULL (no norm).  q_out: [tokens, Hq, D]
 * in `dtype`; k_out/v_out: element (h, t, d) at h*out_head_stride + t*D + d
 * in `dtype` (a cache's rows at an offset: base + offset*D, stride
 * capacity*D).  Non-finite inputs or results: TKH_NON_FINITE at the next
 * status check (synchronous contexts: on return). */
uint32_t tkh_produce_qkv(tkh_context *ctx, const tkh_producer_shape *shape, tkh_dtype dtype,
                         const float *q_proj, const float *k_proj, const float *v_proj,
                         const float *q_norm, const float *k_norm, void *q_out, void *k_out,
                         void *v_out, uint64_t out_head_stride, tkh_error *err);

/* ---------------- session (src/session.rs) ---------------- */

typedef struct tkh_session tkh_session;

/* Options of session::Options (src/session.rs:38-62) plus the attention
 * geometry the session's KV owners need.  layer_windows (per layer, 0 = full
 * retention) select ring caches for sliding layers (WindowKvCache).
 * score_scale 0 selects attention_cached semantics (dot / sqrt(D), no
 * softcap) for full layers, and a nonzero softcap with it is rejected
 * (TKH_INVALID_CONFIG); otherwise every layer uses window/span semantics
 * with this scale and the optional score softcap.
 * shared_layers: the last shared_layers layers own no KV cache; each attends
 * over the current-step view of the last earlier owning layer of its kind
 * (sliding: nonzero window, which must be equal; full: 0), as
 * SharedKvPlan::new routes them (src/model/shared_kv.rs:50-120).  Their K/V
 * projections and k_norm are not read (they may be NULL); only Q is
 * normalised and rotated.  At least one layer must own a cache
 * (TKH_INVALID_CONFIG otherwise, as for a shared layer without a producer of
 * its kind or with a different window). */
typedef struct tkh_session_options {
    uint64_t capacity;
    uint64_t prefill_chunk_size;
    uint64_t position_offset;
    uint64_t vocab_size;      /* token admission (Session::validate) */
    uint64_t layers, query_heads, kv_heads, head_dim;
    tkh_dtype storage;
    float score_scale;
    float softcap;
    float norm_epsilon;
    uint32_t rotary;          /* tkh_rotary */
    float theta;
    uint64_t rotated_dims;
    float factor;
    float low_freq_factor;    /* Llama 3 parameters, as in tkh_producer_shape */
    float high_freq_factor;
    uint64_t original_max_positions;
    uint64_t shared_layers;   /* trailing layers that borrow an earlier layer's KV */
} tkh_session_options;

/* Session::new (src/session.rs:205-245): validates, then allocates every
 * device buffer the session will use (KV owners, Q scratch, ring staging).
 * ctx may be NULL: a host-only session that runs the token state machine
 * alone (evaluation commits state and computes nothing), for planning and
 * for testing transitions without a device. */
uint32_t tkh_session_create(tkh_context *ctx, const tkh_session_options *options,
                            const uint64_t *layer_windows, tkh_session **out, tkh_error *err);
/* Safe in any order with tkh_context_destroy of the owning context. */
void tkh_session_destroy(tkh_session *s);

/* Session::append / set_tokens (src/session.rs:320-356). */
uint32_t tkh_session_append(tkh_session *s, const uint32_t *tokens, uint64_t count,
                            tkh_error *err);
uint32_t tkh_session_set_tokens(tkh_session *s, const uint32_t *tokens, uint64_t count,
                                tkh_error *err);
/* Session::discard_pending / reset (src/session.rs:428-446). */
void tkh_session_discard_pending(tkh_session *s);
void tkh_session_reset(tkh_session *s);

typedef struct tkh_session_state {
    uint64_t history_len, evaluated_len, pending_len, capacity;
    uint32_t distribution_valid; /* Session::logits().is_some() */
    uint64_t kv_bytes, scratch_bytes;
} tkh_session_state;
uint32_t tkh_session_state_get(const tkh_session *s, tkh_session_state *out);
/* SharedKvPlan::producer_for (src/model/shared_kv.rs:141-146): the layer
 * whose KV cache `layer` attends over (itself for an owning layer). */
uint32_t tkh_session_kv_producer(const tkh_session *s, uint64_t layer, uint64_t *producer);
/* Copies min(capacity_tokens, history_len) tokens of Session::history(). */
uint64_t tkh_session_history(const tkh_session *s, uint32_t *tokens, uint64_t capacity_tokens);

/* Tokens the next chunk evaluates: positions [start, start + count) of the
 * history, count = min(pending, prefill_chunk_size) (src/session.rs:384). */
uint32_t tkh_session_next_chunk(const tkh_session *s, uint64_t *start, uint64_t *count);

/* One layer's inputs for a chunk.  Projections are device FP32 token-major
 * [rows, H, D]; context receives [rows, Hq, D] FP32.  `rows` start at the
 * chunk's first token (chunk-relative) in tkh_session_evaluate_next_chunk and
 * at session position 0 in tkh_session_evaluate. */
typedef struct tkh_layer_io {
    const float *q_proj, *k_proj, *v_proj;
    const float *q_norm, *k_norm; /* [D] or NULL */
    float *context;
} tkh_layer_io;

/* Session::evaluate_next_chunk (src/session.rs:364-418) for the attention
 * path: per layer, produce Q/K/V, stage or append K/V, attend; then commit
 * every layer (ring frames and evaluated_len) together.  With a synchronous
 * context the status word is checked before the commit and a failure leaves
 * the committed prefix and the pending history as they were.  With a queued
 * context the commit is provisional until tkh_session_synchronize.
 * *count receives the evaluated token count (0 when nothing is pending). */
uint32_t tkh_session_evaluate_next_chunk(tkh_session *s, const tkh_layer_io *layers,
                                         uint64_t *count, tkh_error *err);

/* Session::evaluate (src/session.rs:420-423) with a per-call chunk limit
 * (<= prefill_chunk_size; 1 evaluates pending tokens one decode step at a
 * time): every pending token, with position-indexed layer inputs. */
uint32_t tkh_session_evaluate(tkh_session *s, const tkh_layer_io *layers, uint64_t chunk_limit,
                              uint64_t *evaluated, tkh_error *err);

/* Session::evaluate_chunk (src/session.rs:364-418) for a host whose model
 * runs between the layers: Model::run (src/model/mod.rs:530-755) computes
 * layer l + 1's projections from layer l's context, so the layers of a chunk
 * are evaluated one call at a time.  chunk_begin fixes the chunk: the next
 * min(pending, chunk_limit, prefill_chunk_size) tokens from *start
 * (*count 0: nothing pending, no chunk).  chunk_layer runs layer `layer`
 * (0, 1, .. in order; inputs chunk-relative, as in evaluate_next_chunk): its
 * producer and attention, ring layers staging their rows.  chunk_commit,
 * after the last layer, checks the status word (synchronous contexts) and
 * commits every ring and evaluated_len together, as the whole-chunk calls do
 * (*count: the tokens committed).  Nothing is committed before it: a failing
 * layer, a commit before the last layer (TKH_INVALID_CONFIG), chunk_abort,
 * and every state edit, evaluate call or synchronize drop the chunk and leave
 * the session as it was.  Layers out of order, or chunk_layer without a
 * chunk, return TKH_INVALID_CONFIG without dropping it.  With a queued
 * context, the kernels of a dropped chunk's layers still run: a non-finite
 * value they meet is reported by the next synchronize, which then also
 * returns the session to its last checked prefix, dropping chunks committed
 * since; a caller that may drop a chunk keeps earlier chunks by calling
 * tkh_session_synchronize before beginning it. */
uint32_t tkh_session_chunk_begin(tkh_session *s, uint64_t chunk_limit, uint64_t *start,
                                 uint64_t *count, tkh_error *err);
uint32_t tkh_session_chunk_layer(tkh_session *s, uint64_t layer, const tkh_layer_io *io,
                                 tkh_error *err);
uint32_t tkh_session_chunk_commit(tkh_session *s, uint64_t *count, tkh_error *err);
void tkh_session_chunk_abort(tkh_session *s);

/* Waits for queued chunks and checks the status word.  On failure the
 * provisional chunks are dropped: the session returns to the last checked
 * prefix, or, with sliding layers, to the end of the last chunk whose ring
 * commit ran before the failure (ring commits of a queued context run on the
 * device only while the status word is clean).  set_tokens,
 * discard_pending and reset settle provisional chunks first. */
uint32_t tkh_session_synchronize(tkh_session *s, tkh_error *err);

#ifdef __cplusplus
}
#endif
#endif
