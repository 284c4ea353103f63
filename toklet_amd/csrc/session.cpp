// session.cpp - the session state machine of the attention path and the
// fused Q/K/V producer entry point (include/tokhip.h, "producer" and
// "session").
//
// tkh_session mirrors toklet's Session (src/session.rs:192-446) for what the
// attention path needs: token history with longest-prefix reuse, one pending
// chunk evaluated per call, every layer committed together, discard and
// reset.  The model around attention (embeddings, projections, MLP, logits)
// stays with the caller: a chunk's evaluation takes each layer's Q/K/V
// projections and returns its attention context.  Per layer it runs the
// producer (RMSNorm, rotary, cache rounding), appends or stages K/V, and
// attends; ring caches of sliding layers commit after every layer succeeded,
// as the reference commits a Gemma step's frames in one batch
// (src/model/gemma3/forward.rs:401).
#include <algorithm>
#include <cmath>

#include "host.hpp"

extern "C" hipError_t tkh_launch_produce(const tkh::ProduceParams *p, int dtype, hipStream_t stream);
extern "C" hipError_t tkh_launch_fill_u64(uint64_t *p, uint64_t v, hipStream_t stream);
extern "C" int tkh_rotary_pairs(int rotary, int head_dim, int rotated_dims);
extern "C" hipError_t tkh_launch_rotary_table(float *out, int64_t pos0, int64_t rows,
                                              const tkh::RotarySpec *rot, int head_dim,
                                              hipStream_t stream);

using namespace tkh_host;

namespace {

uint32_t check_producer(const tkh_producer_shape *sh, tkh_error *err) {
    if (!sh) return invalid("producer shape", err);
    TRY(nonzero(sh->tokens, "tokens", err));
    TRY(nonzero(sh->query_heads, "query_heads", err));
    TRY(nonzero(sh->kv_heads, "kv_heads", err));
    TRY(nonzero(sh->head_dim, "head_dim", err));
    if (sh->query_heads % sh->kv_heads != 0)
        return invalid("query heads must be a multiple of KV heads", err);
    if (sh->head_dim % 2 != 0) return invalid("rotary head_dim must be even", err);
    if (sh->head_dim > 512) return fail(err, TKH_UNSUPPORTED, "head_dim", 0, 512, sh->head_dim,
                                        "head_dim above 512 is not supported");
    if (sh->rotary > TKH_ROTARY_LLAMA3) return invalid("rotary kind", err);
    if (sh->rotary != TKH_ROTARY_NONE && (!std::isfinite(sh->theta) || sh->theta <= 0.0f))
        return invalid("theta must be finite and positive", err);
    if (sh->rotary == TKH_ROTARY_PROPORTIONAL) {
        if (sh->rotated_dims % 2 != 0 || sh->rotated_dims > sh->head_dim)
            return invalid("proportional rotary dimensions", err);
        if (!std::isfinite(sh->factor) || sh->factor <= 0.0f)
            return invalid("proportional rotary base/factor", err);
    }
    if (sh->rotary == TKH_ROTARY_LLAMA3) {
        // Llama3Scaling::new (src/cpu/llama3_rotary.rs:14-37).
        const float f = sh->factor, lo = sh->low_freq_factor, hi = sh->high_freq_factor;
        if (!std::isfinite(f) || f < 1.0f || !std::isfinite(lo) || lo <= 0.0f ||
            !std::isfinite(hi) || hi <= lo || sh->original_max_positions == 0 ||
            sh->original_max_positions > (uint64_t{1} << 53))
            return invalid("Llama3 rotary scaling", err);
        // The scaled frequency of every pair must stay finite and positive
        // (src/cpu/llama3_rotary.rs:57-59); the kernels evaluate the same band
        // formula.
        const double orig = (double)sh->original_max_positions;
        for (uint64_t j = 0; j < sh->head_dim / 2; ++j) {
            const double ordinary =
                std::pow((double)sh->theta, -(2.0 * (double)j) / (double)sh->head_dim);
            const double wavelength = 6.283185307179586 / ordinary;
            double inv = ordinary;
            if (f != 1.0f && !(wavelength < orig / hi)) {
                if (wavelength > orig / lo) {
                    inv = ordinary / f;
                } else {
                    const double smooth = (orig / wavelength - lo) / ((double)hi - lo);
                    inv = (1.0 - smooth) * ordinary / f + smooth * ordinary;
                }
            }
            if (!std::isfinite(ordinary) || ordinary <= 0.0 || !std::isfinite(inv) || inv <= 0.0)
                return invalid("Llama3 scaled frequency underflow", err);
        }
    }
    uint64_t last;
    TRY(add(sh->position, sh->tokens - 1, &last, err));
    if (last > (uint64_t{1} << 53)) return invalid("rotary positions must be at most 2^53", err);
    return TKH_OK;
}

tkh::RotarySpec rotary_spec(const tkh_producer_shape *sh) {
    tkh::RotarySpec r{};
    r.kind = (int32_t)sh->rotary;
    r.rotated_dims = (int32_t)sh->rotated_dims;
    r.theta = sh->theta;
    r.factor = sh->factor;
    r.low = sh->low_freq_factor;
    r.high = sh->high_freq_factor;
    r.original = (double)sh->original_max_positions;
    return r;
}

uint32_t launch_producer(tkh_context *ctx, const tkh_producer_shape *sh, tkh_dtype dtype,
                         const float *q, const float *k, const float *v, const float *qn,
                         const float *kn, void *q_out, void *k_out, void *v_out,
                         uint64_t head_stride, tkh_error *err, const float *rope = nullptr,
                         uint64_t rope_pos0 = 0) {
    tkh::ProduceParams p{};
    p.rope = rope;
    p.rope_pos0 = (int64_t)rope_pos0;
    p.q = q;
    p.k = k;
    p.v = v;
    p.q_norm = qn;
    p.k_norm = kn;
    p.q_out = q_out;
    p.k_out = k_out;
    p.v_out = v_out;
    p.out_head_stride = (int64_t)head_stride;
    p.tokens = (int64_t)sh->tokens;
    p.position = (int64_t)sh->position;
    p.hq = (int32_t)sh->query_heads;
    p.hkv = (int32_t)sh->kv_heads;
    p.d = (int32_t)sh->head_dim;
    p.rot = rotary_spec(sh);
    p.eps = sh->norm_epsilon;
    p.status = ctx->status_dev;
    HIP_TRY(hipSetDevice(ctx->device), "hipSetDevice");
    HIP_TRY(tkh_launch_produce(&p, (int)dtype, ctx->stream), "producer launch");
    return TKH_OK;
}

}  // namespace

extern "C" uint32_t tkh_produce_qkv(tkh_context *ctx, const tkh_producer_shape *shape,
                                    tkh_dtype dtype, const float *q_proj, const float *k_proj,
                                    const float *v_proj, const float *q_norm, const float *k_norm,
                                    void *q_out, void *k_out, void *v_out,
                                    uint64_t out_head_stride, tkh_error *err) {
    if (!ctx) return invalid("context", err);
    if (!valid_dtype(dtype)) return invalid("dtype", err);
    TRY(check_producer(shape, err));
    if ((q_norm || k_norm) && (!std::isfinite(shape->norm_epsilon) || shape->norm_epsilon <= 0.0f))
        return invalid("epsilon must be finite and positive", err);
    if (!q_proj || !k_proj || !v_proj || !q_out || !k_out || !v_out)
        return invalid("producer buffers", err);
    uint64_t rows;
    TRY(product(shape->tokens, shape->head_dim, &rows, err));
    if (out_head_stride < rows) return invalid("output head stride below tokens * head_dim", err);
    TRY(launch_producer(ctx, shape, dtype, q_proj, k_proj, v_proj, q_norm, k_norm, q_out, k_out,
                        v_out, out_head_stride, err));
    if (ctx->synchronous) return tkh_context_synchronize(ctx, err);
    return ok(err);
}

// ---------------------------------------------------------------- session

struct tkh_session {
    tkh_context *ctx = nullptr;
    int device = 0;
    tkh_session_options opt{};
    std::vector<uint64_t> windows;  // per layer, 0 = full retention
    std::vector<uint64_t> route;    // per layer: the owning layer whose KV it attends over
    uint64_t producers = 0;         // layers [0, producers) own a KV cache
    std::vector<tkh_kv *> kv;       // per owning layer
    std::vector<uint32_t> history;
    uint64_t evaluated = 0;
    bool dist_valid = false, dist_replay = false;
    // Queued contexts: the prefix (and distribution validity) confirmed by the
    // last status check.
    uint64_t checked = 0;
    bool checked_valid = false;
    bool rings = false;                        // some layer keeps a ring cache
    // Queued ring sessions: the end of the last chunk whose ring commit ran
    // with a clean status word (written by the gated commit on the device).
    uint64_t *committed_dev = nullptr;
    void *q_scratch = nullptr;                 // [chunk, Hq, D] cache dtype
    float *rope = nullptr;                     // (cos, sin) per (position, pair), or null
    bool fused_decode = false;                 // decode steps fold the producer into attention
    std::vector<void *> stage_k, stage_v;      // sliding layers: [Hkv, chunk, D]
    uint64_t scratch_bytes = 0, kv_bytes = 0;
    // The chunk being evaluated (layer by layer through tkh_session_chunk_*,
    // or every layer at once), until its commit or abort.
    struct Chunk {
        bool active = false;
        uint64_t start = 0, count = 0, next_layer = 0;
        bool position_indexed = false;
        uint64_t checked = 0;  // the checked prefix when the chunk began
        bool checked_valid = false;
        // Sized at tkh_session_create (one entry per owning layer) and only
        // cleared afterwards, so evaluating allocates nothing.
        std::vector<tkh_kv *> ring_kv;  // ring owners staged by this chunk
        std::vector<tkh_kv_frame> frames, owner_frame;
        // Drops the chunk, keeping the vectors' storage.
        void clear() {
            active = false;
            start = count = next_layer = 0;
            position_indexed = false;
            checked = 0;
            checked_valid = false;
            ring_kv.clear();
            frames.clear();
            owner_frame.clear();
        }
    } chunk;
    std::vector<tkh_kv *> ring_owners;  // the ring caches, for reset_batch
};

namespace {

void free_session(tkh_session *s) {
    if (!s) return;
    // Like tkh_kv_destroy, the context is not touched (it may be gone first).
    if (s->ctx) hipSetDevice(s->device);
    for (auto *k : s->kv) tkh_kv_destroy(k);
    if (s->q_scratch) hipFree(s->q_scratch);
    if (s->committed_dev) hipFree(s->committed_dev);
    if (s->rope) hipFree(s->rope);
    for (auto *p : s->stage_k)
        if (p) hipFree(p);
    for (auto *p : s->stage_v)
        if (p) hipFree(p);
    delete s;
}

// Session::validate (src/session.rs:292-318): capacity, then every token id.
uint32_t validate_tokens(const tkh_session *s, const uint32_t *tokens, uint64_t count,
                         uint64_t base, tkh_error *err) {
    uint64_t end;
    TRY(add(base, count, &end, err));
    if (end > s->opt.capacity)
        return fail(err, TKH_CAPACITY, "session", base, s->opt.capacity, end,
                    "offset %llu plus %llu tokens exceeds capacity %llu", (unsigned long long)base,
                    (unsigned long long)count, (unsigned long long)s->opt.capacity);
    if (count && !tokens) return invalid("tokens", err);
    for (uint64_t i = 0; i < count; ++i)
        if (tokens[i] >= s->opt.vocab_size)
            return fail(err, TKH_TOKEN, "token", base + i, s->opt.vocab_size, tokens[i],
                        "token %u at position %llu is outside vocabulary %llu", tokens[i],
                        (unsigned long long)(base + i), (unsigned long long)s->opt.vocab_size);
    return TKH_OK;
}

// session::reusable_prefix (src/session.rs:17-36).
void reusable_prefix(const std::vector<uint32_t> &history, uint64_t evaluated,
                     const uint32_t *tokens, uint64_t count, bool distribution_valid,
                     uint64_t *keep, bool *recover) {
    uint64_t shared = 0;
    while (shared < evaluated && shared < count && history[shared] == tokens[shared]) ++shared;
    if (shared == count && (shared < evaluated || !distribution_valid)) {
        *keep = shared > 0 ? shared - 1 : 0;
        *recover = shared > 0;
    } else {
        *keep = shared;
        *recover = false;
    }
}

// The committed prefix moves back to `keep`.  Linear caches need nothing
// (only the evaluated length defines validity, src/model/cache.rs:9-10).  A
// ring of window W at committed length E holds positions [E - W, E); a chunk
// starting at `keep` needs [keep - W + 1, keep), present only for keep >= E - 1.
// Deeper rewinds restart every ring (and the prefix) from position 0.
uint64_t rewind(tkh_session *s, uint64_t keep) {
    if (!s->rings) return keep;
    bool restart = false;
    for (auto *kv : s->kv)
        if (kv->has_window && keep + 1 < kv->offset) restart = true;
    const uint64_t kept = restart ? 0 : keep;
    for (auto *kv : s->kv) {
        if (!kv->has_window) continue;
        kv->offset = std::min(kv->offset, kept);
        kv->generation += 1;  // frames prepared before the rewind are stale
    }
    if (s->committed_dev) tkh_launch_fill_u64(s->committed_dev, kept, s->ctx->stream);
    return kept;
}

uint32_t synchronize(tkh_session *s, tkh_error *err);

// Queued contexts: state edits first settle the provisional chunks, so that
// a late failure cannot land on an edited history.
void settle(tkh_session *s) {
    s->chunk.clear();  // a chunk in progress is dropped
    if (s->ctx && !s->ctx->synchronous && s->checked != s->evaluated) synchronize(s, nullptr);
}

// Waits for queued work and checks the status word.  On failure the
// provisional chunks are dropped: linear-cache sessions return to the last
// checked prefix; ring sessions to the last chunk whose gated ring commit ran
// (read back from the device), which is where their rings stand.  The status
// word belongs to the context, and whoever reads it first clears it (another
// session, tkh_context_synchronize): a ring session therefore also reads back
// its committed length when the status is clean, and a commit that was
// skipped for a failure reported elsewhere is a failure here too.
uint32_t synchronize(tkh_session *s, tkh_error *err) {
    if (!s->ctx) return ok(err);
    uint32_t rc = tkh_context_synchronize(s->ctx, err);
    uint64_t back = s->checked;
    bool valid = s->checked_valid;
    const bool provisional = s->checked != s->evaluated;
    if (s->rings && provisional) {
        uint64_t c = s->checked;
        const hipError_t e = hipMemcpy(&c, s->committed_dev, sizeof c, hipMemcpyDeviceToHost);
        if (e == hipSuccess && c >= s->checked && c <= s->evaluated) {
            valid = c > s->checked ? true : s->checked_valid;
            back = c;
        }
        if (rc == TKH_OK && e != hipSuccess) rc = device_error(e, "session ring commit", err);
        else if (rc == TKH_OK && back != s->evaluated)
            rc = fail(err, TKH_DEVICE, "session ring commit", back, s->evaluated, back,
                      "ring commits of queued chunks stopped at %llu of %llu: a failure on this "
                      "context was reported to another caller",
                      (unsigned long long)back, (unsigned long long)s->evaluated);
    }
    if (rc == TKH_OK) {
        s->checked = s->evaluated;
        s->checked_valid = s->dist_valid;
        return rc;
    }
    if (!provisional) return rc;
    if (s->rings) {
        for (auto *kv : s->kv) {
            if (!kv->has_window) continue;
            kv->offset = back;
            kv->generation += 1;
        }
    }
    s->evaluated = back;
    s->checked = back;
    s->dist_valid = valid && back > 0;
    s->checked_valid = s->dist_valid;
    s->dist_replay = false;
    return rc;
}

}  // namespace

extern "C" uint32_t tkh_session_create(tkh_context *ctx, const tkh_session_options *o,
                                       const uint64_t *layer_windows, tkh_session **out,
                                       tkh_error *err) {
    if (!out || !o) return invalid("session options", err);
    *out = nullptr;
    TRY(nonzero(o->capacity, "capacity", err));
    TRY(nonzero(o->prefill_chunk_size, "prefill_chunk_size", err));
    TRY(nonzero(o->vocab_size, "vocab_size", err));
    TRY(nonzero(o->layers, "layers", err));
    if (!valid_dtype(o->storage)) return invalid("dtype", err);
    tkh_producer_shape sh{};
    sh.tokens = 1;
    sh.query_heads = o->query_heads;
    sh.kv_heads = o->kv_heads;
    sh.head_dim = o->head_dim;
    sh.rotary = o->rotary;
    sh.theta = o->theta;
    sh.rotated_dims = o->rotated_dims;
    sh.factor = o->factor;
    sh.low_freq_factor = o->low_freq_factor;
    sh.high_freq_factor = o->high_freq_factor;
    sh.original_max_positions = o->original_max_positions;
    TRY(check_producer(&sh, err));
    uint64_t last;
    TRY(add(o->position_offset, o->capacity, &last, err));
    if (last > (uint64_t{1} << 53)) return invalid("rotary positions must be at most 2^53", err);
    if (o->score_scale != 0.0f && !(std::isfinite(o->score_scale) && o->score_scale > 0.0f))
        return invalid("score scale must be finite and positive", err);
    if (!(o->softcap == 0.0f || (std::isfinite(o->softcap) && o->softcap > 0.0f)))
        return invalid("softcap must be finite and positive (0 disables)", err);
    auto *s = new tkh_session();
    s->ctx = ctx;
    s->device = ctx ? ctx->device : 0;
    s->opt = *o;
    s->opt.prefill_chunk_size = std::min(o->prefill_chunk_size, o->capacity);
    // windows: the attention mask of each layer.  A window shorter than the
    // capacity also selects a ring cache of that many rows.
    s->windows.assign(o->layers, 0);
    if (layer_windows)
        for (uint64_t l = 0; l < o->layers; ++l) s->windows[l] = layer_windows[l];
    bool windowed = false;
    for (uint64_t w : s->windows) windowed |= w != 0;
    if (windowed && o->score_scale == 0.0f) {
        free_session(s);
        return invalid("windowed layers need an explicit score scale", err);
    }
    // score_scale 0 selects attention_cached semantics, which have no softcap:
    // a softcap there would be silently ignored.
    if (o->softcap != 0.0f && o->score_scale == 0.0f) {
        free_session(s);
        return fail(err, TKH_INVALID_CONFIG, "session options", 0, 0, 0,
                    "a score softcap needs an explicit score scale (window/span semantics)");
    }
    // SharedKvPlan::new (src/model/shared_kv.rs:50-120): the first
    // layers - shared_layers layers own caches; a shared layer borrows the
    // last owning layer of its kind (sliding or full), whose geometry (here:
    // the window) must be its own.
    if (o->shared_layers >= o->layers) {
        free_session(s);
        return fail(err, TKH_INVALID_CONFIG, "KV routing", 0, o->layers, o->shared_layers,
                    "KV routing needs a producer");
    }
    s->producers = o->layers - o->shared_layers;
    s->route.resize(o->layers);
    for (uint64_t l = 0; l < o->layers; ++l) {
        if (l < s->producers) {
            s->route[l] = l;
            continue;
        }
        const bool sliding = s->windows[l] != 0;
        uint64_t p = s->producers;
        for (uint64_t c = s->producers; c-- > 0;)
            if ((s->windows[c] != 0) == sliding) {
                p = c;
                break;
            }
        if (p == s->producers) {
            free_session(s);
            return fail(err, TKH_INVALID_CONFIG, "KV routing", l, 0, 0,
                        "missing shared KV producer kind for layer %llu", (unsigned long long)l);
        }
        if (s->windows[p] != s->windows[l]) {
            free_session(s);
            return fail(err, TKH_INVALID_CONFIG, "KV routing", l, s->windows[p], s->windows[l],
                        "shared KV producer geometry differs for layer %llu",
                        (unsigned long long)l);
        }
        s->route[l] = p;
    }
    s->history.reserve(o->capacity);
    // Decode steps with the producer inside the decode kernel (one launch per
    // step and layer instead of two; TKH_FUSED_DECODE=0 turns it off): the
    // kernel's bf16/f16 builds of head_dim 64, 128 and 256 (256: with or
    // without the score softcap; 64 and 128: without), GQA groups of at most
    // 1 KiB of cache-dtype rows.
    {
        const uint64_t G = o->query_heads / o->kv_heads;
        const uint64_t rowb = o->head_dim * (uint64_t)esize(o->storage);
        const uint64_t limit = rowb <= 256 ? 8 : (rowb <= 512 ? 4 : 2);
        const bool dims = o->head_dim == 64 || o->head_dim == 128 || o->head_dim == 256;
        s->fused_decode = dims && o->storage != TKH_F32 && G <= limit && G * rowb <= 1024 &&
                          (o->softcap == 0.0f || o->head_dim == 256) &&
                          env_int("TKH_FUSED_DECODE", 1) != 0;
    }
    if (ctx) {
        const uint64_t D = o->head_dim, es = (uint64_t)esize(o->storage);
        const uint64_t chunk = s->opt.prefill_chunk_size;
        s->kv.assign(s->producers, nullptr);
        s->stage_k.assign(s->producers, nullptr);
        s->stage_v.assign(s->producers, nullptr);
        for (uint64_t l = 0; l < s->producers; ++l) {
            const uint64_t w = s->windows[l];
            const bool ring = w != 0 && w < o->capacity;
            uint32_t rc = tkh_kv_create(ctx, o->kv_heads, D, ring ? w : o->capacity, o->capacity,
                                        ring ? 1u : 0u, ring ? w : 0, o->storage, &s->kv[l], err);
            if (rc != TKH_OK) {
                free_session(s);
                return rc;
            }
            s->kv_bytes += s->kv[l]->allocated_bytes;
            s->rings |= ring;
            if (ring) s->ring_owners.push_back(s->kv[l]);
        }
        s->chunk.ring_kv.reserve(s->producers);
        s->chunk.frames.reserve(s->producers);
        s->chunk.owner_frame.reserve(s->producers);
        s->scratch_bytes = chunk * o->query_heads * D * es;
        hipError_t e = hipMalloc(&s->q_scratch, chunk * o->query_heads * D * es);
        if (e == hipSuccess) e = hipMalloc(&s->committed_dev, sizeof(uint64_t));
        if (e == hipSuccess) e = tkh_launch_fill_u64(s->committed_dev, 0, ctx->stream);
        // The rotary (cos, sin) of every session position, once.
        const int pairs = tkh_rotary_pairs((int)o->rotary, (int)D, (int)o->rotated_dims);
        if (e == hipSuccess && pairs > 0) {
            const size_t bytes = (size_t)o->capacity * pairs * 2 * sizeof(float);
            e = hipMalloc(&s->rope, bytes);
            const tkh::RotarySpec rot = rotary_spec(&sh);
            if (e == hipSuccess)
                e = tkh_launch_rotary_table(s->rope, (int64_t)o->position_offset,
                                            (int64_t)o->capacity, &rot, (int)D, ctx->stream);
            if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
            s->scratch_bytes += bytes;
        }
        for (uint64_t l = 0; e == hipSuccess && l < s->producers; ++l) {
            if (!s->kv[l]->has_window) continue;
            const size_t bytes = chunk * o->kv_heads * D * es;
            e = hipMalloc(&s->stage_k[l], bytes);
            if (e == hipSuccess) e = hipMalloc(&s->stage_v[l], bytes);
            s->scratch_bytes += 2 * bytes;
        }
        if (e != hipSuccess) {
            free_session(s);
            return device_error(e, "session allocation", err);
        }
    }
    *out = s;
    return ok(err);
}

extern "C" void tkh_session_destroy(tkh_session *s) { free_session(s); }

extern "C" uint32_t tkh_session_append(tkh_session *s, const uint32_t *tokens, uint64_t count,
                                       tkh_error *err) {
    if (!s) return invalid("session", err);
    TRY(validate_tokens(s, tokens, count, s->history.size(), err));
    s->history.insert(s->history.end(), tokens, tokens + count);
    return ok(err);
}

extern "C" uint32_t tkh_session_set_tokens(tkh_session *s, const uint32_t *tokens, uint64_t count,
                                           tkh_error *err) {
    if (!s) return invalid("session", err);
    TRY(validate_tokens(s, tokens, count, 0, err));
    settle(s);
    uint64_t keep;
    bool recover;
    reusable_prefix(s->history, s->evaluated, tokens, count, s->dist_valid, &keep, &recover);
    // Option<&u32> equality of tokens.get(keep) and history.get(keep): two
    // absent values compare equal.
    const bool t_has = keep < count, h_has = keep < s->history.size();
    const bool same_next = t_has == h_has && (!t_has || tokens[keep] == s->history[keep]);
    recover = recover || (s->dist_replay && keep == s->evaluated && same_next);
    if (keep < s->evaluated) s->dist_valid = false;
    const uint64_t kept = rewind(s, keep);
    if (kept != keep) recover = false;  // every token is pending again
    s->evaluated = kept;
    s->checked = std::min(s->checked, kept);
    s->dist_replay = recover;
    s->history.assign(tokens, tokens + count);
    return ok(err);
}

extern "C" void tkh_session_discard_pending(tkh_session *s) {
    if (!s) return;
    settle(s);
    s->history.resize(std::min<uint64_t>(s->history.size(), s->evaluated + (s->dist_replay ? 1 : 0)));
    if (s->dist_replay) return;
    if (!s->dist_valid && s->evaluated > 0) {
        // A one-position rewind, which every ring can take.
        s->evaluated = rewind(s, s->evaluated - 1);
        s->checked = std::min(s->checked, s->evaluated);
        s->dist_replay = true;
    }
}

extern "C" void tkh_session_reset(tkh_session *s) {
    if (!s) return;
    settle(s);
    s->history.clear();
    s->evaluated = 0;
    s->checked = 0;
    s->checked_valid = false;
    s->dist_valid = false;
    s->dist_replay = false;
    if (!s->ring_owners.empty())
        tkh_kv_reset_batch(s->ring_owners.data(), s->ring_owners.size(), nullptr);
    if (s->committed_dev) tkh_launch_fill_u64(s->committed_dev, 0, s->ctx->stream);
}

extern "C" uint32_t tkh_session_state_get(const tkh_session *s, tkh_session_state *out) {
    if (!s || !out) return TKH_INVALID_PARAMETER;
    out->history_len = s->history.size();
    out->evaluated_len = s->evaluated;
    out->pending_len = s->history.size() - s->evaluated;
    out->capacity = s->opt.capacity;
    out->distribution_valid = s->dist_valid && s->evaluated > 0 && out->pending_len == 0;
    out->kv_bytes = s->kv_bytes;
    out->scratch_bytes = s->scratch_bytes;
    return TKH_OK;
}

extern "C" uint32_t tkh_session_kv_producer(const tkh_session *s, uint64_t layer,
                                            uint64_t *producer) {
    if (!s || !producer || layer >= s->route.size()) return TKH_INVALID_PARAMETER;
    *producer = s->route[layer];
    return TKH_OK;
}

extern "C" uint64_t tkh_session_history(const tkh_session *s, uint32_t *tokens,
                                        uint64_t capacity_tokens) {
    if (!s) return 0;
    const uint64_t n = std::min<uint64_t>(capacity_tokens, s->history.size());
    if (tokens && n) std::memcpy(tokens, s->history.data(), n * sizeof(uint32_t));
    return s->history.size();
}

extern "C" uint32_t tkh_session_next_chunk(const tkh_session *s, uint64_t *start, uint64_t *count) {
    if (!s || !start || !count) return TKH_INVALID_PARAMETER;
    *start = s->evaluated;
    *count = std::min<uint64_t>(s->history.size() - s->evaluated, s->opt.prefill_chunk_size);
    return TKH_OK;
}

namespace {

// The commit of Session::evaluate_chunk (src/session.rs:413-417).
void commit_state(tkh_session *s, uint64_t count) {
    s->evaluated += count;
    s->dist_valid = true;
    s->dist_replay = false;
    s->checked = s->evaluated;
    s->checked_valid = true;
}

// A chunk of `count` tokens at session position `start`, evaluated layer by
// layer: begin fixes it, eval_layer runs layers 0.. in order (the producer,
// then attention; ring layers stage their rows), commit_chunk checks the
// status (synchronous contexts) and commits every ring and evaluated_len
// together.  Nothing is committed before commit_chunk, so dropping the chunk
// (abort_chunk) leaves the session as it was: rows a layer wrote past
// evaluated_len in a linear cache are not part of any prefix.
void begin_chunk(tkh_session *s, uint64_t start, uint64_t count, bool position_indexed) {
    tkh_session::Chunk &c = s->chunk;
    c.clear();
    c.active = true;
    c.start = start;
    c.count = count;
    c.position_indexed = position_indexed;
    c.checked = s->checked;
    c.checked_valid = s->checked_valid;
    c.owner_frame.assign(s->kv.size(), tkh_kv_frame{});
}

void abort_chunk(tkh_session *s) { s->chunk.clear(); }

uint32_t eval_layer(tkh_session *s, uint64_t l, const tkh_layer_io &io, tkh_error *err) {
    tkh_session::Chunk &c = s->chunk;
    const uint64_t start = c.start, count = c.count;
    const bool position_indexed = c.position_indexed;
    std::vector<tkh_kv *> &ring_kv = c.ring_kv;
    std::vector<tkh_kv_frame> &frames = c.frames;
    std::vector<tkh_kv_frame> &owner_frame = c.owner_frame;
    tkh_context *ctx = s->ctx;
    const tkh_session_options &o = s->opt;
    const uint64_t Hq = o.query_heads, Hkv = o.kv_heads, D = o.head_dim;
    const uint64_t es = (uint64_t)esize(o.storage);
    const uint64_t row0 = position_indexed ? start : 0;
    tkh_producer_shape sh{};
    sh.tokens = count;
    sh.query_heads = Hq;
    sh.kv_heads = Hkv;
    sh.head_dim = D;
    sh.position = o.position_offset + start;
    sh.norm_epsilon = o.norm_epsilon;
    sh.rotary = o.rotary;
    sh.theta = o.theta;
    sh.rotated_dims = o.rotated_dims;
    sh.factor = o.factor;
    sh.low_freq_factor = o.low_freq_factor;
    sh.high_freq_factor = o.high_freq_factor;
    sh.original_max_positions = o.original_max_positions;
    // Attention of the chunk's Q (in the Q scratch) over a linear cache's keys
    // [0, start + count): Model::run -> LayerKv::attend -> attention_cached
    // (src/model/mod.rs:645-662), or the window form with a score scale.
    auto attend_linear = [&](tkh_kv *kv, uint64_t window, float *context) -> uint32_t {
        if (o.score_scale == 0.0f) {
            tkh_cached_shape cs{count, Hq, Hkv, D, kv->capacity, start};
            return tkh_attention_cached(ctx, &cs, o.storage, s->q_scratch, count * Hq * D, kv->k,
                                        Hkv * kv->capacity * D, kv->v, Hkv * kv->capacity * D,
                                        context, count * Hq * D, nullptr, 0, nullptr, 0, err);
        }
        tkh_window_shape ws{};
        ws.queries = count;
        ws.keys = start + count;
        ws.capacity = kv->capacity;
        ws.query_heads = Hq;
        ws.kv_heads = Hkv;
        ws.head_dim = D;
        ws.query_start = start;
        ws.key_start = 0;
        ws.has_window = window != 0;
        ws.window = window;
        ws.scale = o.score_scale;
        ws.softcap = o.softcap;
        return tkh_window_attention(ctx, &ws, o.storage, s->q_scratch, count * Hq * D, kv->k,
                                    Hkv * kv->capacity * D, kv->v, Hkv * kv->capacity * D, context,
                                    count * Hq * D, nullptr, 0, nullptr, 0, err);
    };
    const uint64_t owner = s->route[l];
    const bool shared = l >= s->producers;
    if (!io.q_proj || !io.context || (!shared && (!io.k_proj || !io.v_proj)))
        return invalid("layer inputs", err);
    if ((io.q_norm || (!shared && io.k_norm)) &&
        (!std::isfinite(o.norm_epsilon) || o.norm_epsilon <= 0.0f))
        return invalid("epsilon must be finite and positive", err);
    const float *q = io.q_proj + row0 * Hq * D;
    const float *k = shared ? nullptr : io.k_proj + row0 * Hkv * D;
    const float *v = shared ? nullptr : io.v_proj + row0 * Hkv * D;
    float *context = io.context + row0 * Hq * D;
    tkh_kv *kv = s->kv[owner];
    const bool ring = kv->has_window;
    const uint64_t window = s->windows[l];
    // A decode step folds the producer into the decode kernel: its Q/K/V
    // projections are normalised, rotated and rounded there, and the new
    // K/V row goes to the cache (linear) or the staging rows (ring).
    auto fused_desc = [&](void *kc, void *vc, int64_t head_stride, int64_t new_key,
                          int64_t new_row) {
        tkh::FusedDecode f{};
        f.q_proj = q;
        f.k_proj = k;
        f.v_proj = v;
        f.q_norm = io.q_norm;
        f.k_norm = io.k_norm;
        f.pairs = tkh_rotary_pairs((int)o.rotary, (int)D, (int)o.rotated_dims);
        f.rope = f.pairs > 0 ? s->rope + 2 * start * (uint64_t)f.pairs : nullptr;
        f.eps = o.norm_epsilon;
        f.k_cache = kc;
        f.v_cache = vc;
        f.head_stride = head_stride;
        f.new_key = new_key;
        f.new_row = new_row;
        return f;
    };
    const bool fused_step = count == 1 && s->fused_decode;
    // The span form of a decode step over a linear cache: keys [first
    // visible, start] (window/score-scale layers).
    auto linear_span = [&](tkh_span_shape &span, tkh_segment (&segs)[3]) {
        span = tkh_span_shape{};
        const uint64_t first = window != 0 && start + 1 > window ? start + 1 - window : 0;
        span.queries = 1;
        span.keys = start + 1 - first;
        span.query_heads = Hq;
        span.kv_heads = Hkv;
        span.head_dim = D;
        span.query_start = start;
        span.key_start = first;
        span.has_window = window != 0;
        span.window = window;
        span.scale = o.score_scale;
        span.softcap = o.softcap;
        const uint64_t stride = kv->capacity * D;
        segs[0] = tkh_segment{(const uint8_t *)kv->k + first * D * es, (Hkv - 1) * stride + span.keys * D,
                              (const uint8_t *)kv->v + first * D * es, (Hkv - 1) * stride + span.keys * D,
                              span.keys, stride, first};
        segs[1] = segs[2] = tkh_segment{};
        segs[1].key_start = segs[2].key_start = start + 1;
    };
    if (shared) {
        // A shared layer (SharedKvPlan::view, src/model/shared_kv.rs:333-343):
        // its own Q, normalised and rotated, over the owner's current-step
        // view; no K/V is produced or appended.  A decode step makes the Q
        // rows inside the decode kernel, with no new row to make (new_key -1:
        // the owner's step has written it, to the cache or its staging row).
        if (fused_step) {
            tkh::FusedDecode f = fused_desc(nullptr, nullptr, 0, -1, 0);
            f.k_norm = nullptr;
            tkh_segment segs[3]{};
            tkh_span_shape span{};
            if (!ring && o.score_scale != 0.0f) {
                linear_span(span, segs);
                TRY(span_attention_fused(ctx, &span, o.storage, segs, context, f, err));
            } else if (!ring) {
                tkh_cached_shape cs{1, Hq, Hkv, D, kv->capacity, start};
                TRY(attention_cached_fused(ctx, &cs, o.storage, kv->k, kv->v, context, f, err));
            } else {
                TRY(tkh_kv_view(kv, &owner_frame[owner], Hq, o.score_scale, segs, &span, err));
                span.softcap = o.softcap;
                TRY(span_attention_fused(ctx, &span, o.storage, segs, context, f, err));
            }
            return ok(err);
        }
        tkh_producer_shape qs = sh;
        qs.kv_heads = 0;
        TRY(launch_producer(ctx, &qs, o.storage, q, nullptr, nullptr, io.q_norm, nullptr,
                            s->q_scratch, nullptr, nullptr, 0, err, s->rope, o.position_offset));
        if (!ring) {
            TRY(attend_linear(kv, window, context));
        } else {
            tkh_segment segs[3];
            tkh_span_shape span{};
            TRY(tkh_kv_view(kv, &owner_frame[owner], Hq, o.score_scale, segs, &span, err));
            span.softcap = o.softcap;
            TRY(tkh_span_attention(ctx, &span, o.storage, s->q_scratch, count * Hq * D, segs,
                                   context, count * Hq * D, nullptr, 0, nullptr, 0, err));
        }
        return ok(err);
    }
    if (!ring && fused_step && o.score_scale != 0.0f) {
        tkh_span_shape span{};
        tkh_segment segs[3]{};
        linear_span(span, segs);
        const tkh::FusedDecode f = fused_desc(kv->k, kv->v, (int64_t)(kv->capacity * D),
                                              (int64_t)(span.keys - 1), (int64_t)start);
        TRY(span_attention_fused(ctx, &span, o.storage, segs, context, f, err));
    } else if (!ring && fused_step) {
        // attention_cached form: every key up to the new one.
        const tkh::FusedDecode f = fused_desc(kv->k, kv->v, (int64_t)(kv->capacity * D),
                                              (int64_t)start, (int64_t)start);
        tkh_cached_shape cs{1, Hq, Hkv, D, kv->capacity, start};
        TRY(attention_cached_fused(ctx, &cs, o.storage, kv->k, kv->v, context, f, err));
    } else if (!ring) {
        uint8_t *kb = (uint8_t *)kv->k + start * D * es, *vb = (uint8_t *)kv->v + start * D * es;
        TRY(launch_producer(ctx, &sh, o.storage, q, k, v, io.q_norm, io.k_norm, s->q_scratch,
                            kb, vb, kv->capacity * D, err, s->rope, o.position_offset));
        TRY(attend_linear(kv, window, context));
    } else {
        // Sliding layer: stage the chunk, attend over the ring's old spans
        // plus the staged rows (WindowKvCache::view), commit later.
        if (kv->offset != start)
            return fail(err, TKH_INVALID_CONFIG, "KV frame", l, start, kv->offset,
                        "ring cache of layer %llu is at %llu, chunk starts at %llu",
                        (unsigned long long)l, (unsigned long long)kv->offset,
                        (unsigned long long)start);
        if (!fused_step)
            TRY(launch_producer(ctx, &sh, o.storage, q, k, v, io.q_norm, io.k_norm, s->q_scratch,
                                s->stage_k[owner], s->stage_v[owner], count * D, err, s->rope,
                                o.position_offset));
        tkh_kv_frame f{};
        f.k = s->stage_k[owner];
        f.v = s->stage_v[owner];
        f.owner = kv->owner;
        f.generation = kv->generation;
        f.offset = kv->offset;
        f.tokens = count;
        tkh_segment segs[3];
        tkh_span_shape span{};
        TRY(tkh_kv_view(kv, &f, Hq, o.score_scale, segs, &span, err));
        span.softcap = o.softcap;
        if (fused_step) {
            // The new row is the view's last key; its K/V go to staging row 0.
            const tkh::FusedDecode fd = fused_desc(s->stage_k[owner], s->stage_v[owner],
                                                   (int64_t)D, (int64_t)(span.keys - 1), 0);
            TRY(span_attention_fused(ctx, &span, o.storage, segs, context, fd, err));
        } else {
            TRY(tkh_span_attention(ctx, &span, o.storage, s->q_scratch, count * Hq * D, segs,
                                   context, count * Hq * D, nullptr, 0, nullptr, 0, err));
        }
        ring_kv.push_back(kv);
        frames.push_back(f);
        owner_frame[owner] = f;
    }
    return ok(err);
}

uint32_t commit_chunk(tkh_session *s, tkh_error *err) {
    tkh_context *ctx = s->ctx;
    tkh_session::Chunk &c = s->chunk;
    // The chunk is dropped on every way out (its vectors keep their storage).
    struct Drop {
        tkh_session *s;
        ~Drop() { abort_chunk(s); }
    } drop{s};
    // Commit only after every layer of the chunk succeeded.
    if (ctx->synchronous) TRY(tkh_context_synchronize(ctx, err));
    if (!c.ring_kv.empty()) {
        // Queued: the ring copies run on the device only while the status word
        // is clean, and record how far the rings got.
        const bool gated = !ctx->synchronous;
        TRY(commit_frames(c.ring_kv.data(), c.frames.data(), c.ring_kv.size(),
                          gated ? ctx->status_dev : nullptr, gated ? s->committed_dev : nullptr,
                          c.start + c.count, err));
    }
    commit_state(s, c.count);
    if (!ctx->synchronous) {
        // Provisional until tkh_session_synchronize confirms the status word.
        s->checked = c.checked;
        s->checked_valid = c.checked_valid;
    }
    return ok(err);
}

// One chunk, every layer at once (the inputs of all layers given together).
uint32_t evaluate_chunk(tkh_session *s, const tkh_layer_io *layers, uint64_t start,
                        uint64_t count, bool position_indexed, tkh_error *err) {
    begin_chunk(s, start, count, position_indexed);
    for (uint64_t l = 0; l < s->opt.layers; ++l) {
        const uint32_t rc = eval_layer(s, l, layers[l], err);
        if (rc != TKH_OK) {
            abort_chunk(s);
            return rc;
        }
    }
    return commit_chunk(s, err);
}

}  // namespace

extern "C" uint32_t tkh_session_chunk_begin(tkh_session *s, uint64_t chunk_limit, uint64_t *start,
                                            uint64_t *count, tkh_error *err) {
    if (!s || !start || !count) return invalid("session", err);
    abort_chunk(s);
    *start = s->evaluated;
    *count = 0;
    TRY(nonzero(chunk_limit, "chunk limit", err));
    const uint64_t n = std::min<uint64_t>(s->history.size() - s->evaluated,
                                          std::min<uint64_t>(chunk_limit, s->opt.prefill_chunk_size));
    if (n == 0) return ok(err);
    begin_chunk(s, s->evaluated, n, false);
    *count = n;
    return ok(err);
}

extern "C" uint32_t tkh_session_chunk_layer(tkh_session *s, uint64_t layer, const tkh_layer_io *io,
                                            tkh_error *err) {
    if (!s) return invalid("session", err);
    tkh_session::Chunk &c = s->chunk;
    if (!c.active)
        return fail(err, TKH_INVALID_CONFIG, "chunk", layer, 0, 0,
                    "no chunk in progress (tkh_session_chunk_begin)");
    if (layer != c.next_layer)
        return fail(err, TKH_INVALID_CONFIG, "chunk layer", layer, c.next_layer, layer,
                    "layers are evaluated in order: layer %llu expected, %llu given",
                    (unsigned long long)c.next_layer, (unsigned long long)layer);
    if (!io) return invalid("layer inputs", err);
    if (s->ctx) {
        const uint32_t rc = eval_layer(s, layer, *io, err);
        if (rc != TKH_OK) {
            abort_chunk(s);
            return rc;
        }
    }
    ++c.next_layer;
    return ok(err);
}

extern "C" uint32_t tkh_session_chunk_commit(tkh_session *s, uint64_t *count, tkh_error *err) {
    if (!s) return invalid("session", err);
    if (count) *count = 0;
    tkh_session::Chunk &c = s->chunk;
    if (!c.active)
        return fail(err, TKH_INVALID_CONFIG, "chunk", 0, 0, 0,
                    "no chunk in progress (tkh_session_chunk_begin)");
    if (c.next_layer != s->opt.layers) {
        const uint64_t done = c.next_layer;
        abort_chunk(s);
        return fail(err, TKH_INVALID_CONFIG, "chunk", done, s->opt.layers, done,
                    "chunk committed after %llu of %llu layers", (unsigned long long)done,
                    (unsigned long long)s->opt.layers);
    }
    const uint64_t n = c.count;
    if (!s->ctx) {
        abort_chunk(s);
        commit_state(s, n);
    } else {
        TRY(commit_chunk(s, err));
    }
    if (count) *count = n;
    return ok(err);
}

extern "C" void tkh_session_chunk_abort(tkh_session *s) {
    if (s) abort_chunk(s);
}

extern "C" uint32_t tkh_session_evaluate_next_chunk(tkh_session *s, const tkh_layer_io *layers,
                                                    uint64_t *count, tkh_error *err) {
    if (!s) return invalid("session", err);
    abort_chunk(s);
    if (count) *count = 0;
    const uint64_t n = std::min<uint64_t>(s->history.size() - s->evaluated, s->opt.prefill_chunk_size);
    if (n == 0) return ok(err);
    if (!s->ctx) {
        commit_state(s, n);
    } else {
        if (!layers) return invalid("layer inputs", err);
        TRY(evaluate_chunk(s, layers, s->evaluated, n, false, err));
    }
    if (count) *count = n;
    return ok(err);
}

extern "C" uint32_t tkh_session_evaluate(tkh_session *s, const tkh_layer_io *layers,
                                         uint64_t chunk_limit, uint64_t *evaluated, tkh_error *err) {
    if (!s) return invalid("session", err);
    abort_chunk(s);
    if (evaluated) *evaluated = 0;
    TRY(nonzero(chunk_limit, "chunk limit", err));
    const uint64_t limit = std::min<uint64_t>(chunk_limit, s->opt.prefill_chunk_size);
    uint64_t done = 0;
    while (s->history.size() > s->evaluated) {
        const uint64_t n = std::min<uint64_t>(s->history.size() - s->evaluated, limit);
        if (!s->ctx) {
            commit_state(s, n);
        } else {
            if (!layers) return invalid("layer inputs", err);
            TRY(evaluate_chunk(s, layers, s->evaluated, n, true, err));
        }
        done += n;
        if (evaluated) *evaluated = done;
    }
    return ok(err);
}

extern "C" uint32_t tkh_session_synchronize(tkh_session *s, tkh_error *err) {
    if (!s) return invalid("session", err);
    abort_chunk(s);
    return synchronize(s, err);
}
