// api.cpp - host side of the tokhip C ABI (include/tokhip.h).
//
// Validation mirrors the reference operators' check order (dimensions,
// divisibility, size arithmetic, lengths) so error codes agree with
// toklet::cpu::Error before anything is launched.  A call then becomes a
// list of device "problems" (device.hpp), a flat tile space split along the
// key axis when the grid would otherwise be too small for 256 CUs, one
// attention launch and one combine launch that publishes the context.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <new>
#include <vector>

#include "../../include/tokhip.h"
#include "device.hpp"
#include "host.hpp"

extern "C" hipError_t tkh_launch_generic(const tkh::Params *p, int dtype, hipStream_t stream,
                                         hipEvent_t start, hipEvent_t stop);
extern "C" hipError_t tkh_launch_combine(const tkh::Params *p, int64_t total_rows,
                                         hipStream_t stream, hipEvent_t start, hipEvent_t stop);
extern "C" hipError_t tkh_launch_kv_append(int src, int dst, const void *k, const void *v,
                                           void *kc, void *vc, int64_t tokens, int heads,
                                           int dims, int64_t capacity, int64_t offset,
                                           uint32_t *status, hipStream_t stream);
extern "C" hipError_t tkh_launch_check_finite(int dtype, const void *a, const void *b, int64_t n,
                                              uint32_t *status, hipStream_t stream);
extern "C" hipError_t tkh_launch_softcap(float *x, int64_t n, float cap, uint32_t *status,
                                         hipStream_t stream);
extern "C" hipError_t tkh_launch_fill_u32(uint32_t *p, uint32_t v, hipStream_t stream);
extern "C" hipError_t tkh_launch_zero_u64(uint64_t *p, int64_t words, hipStream_t stream);
extern "C" int tkh_decode_max_rows(int dtype, int head_dim);
extern "C" int tkh_prefill_waves(int head_dim, int wide);
extern "C" hipError_t tkh_launch_decode_merge(const tkh::Params *p, int head_dim, int rows, int kv_heads,
                                              hipStream_t stream, hipEvent_t start, hipEvent_t stop);
extern "C" hipError_t tkh_launch_decode_merge_batch(const tkh::DecodeArgs *a, int head_dim, int rows,
                                                    hipStream_t stream, hipEvent_t start, hipEvent_t stop);
extern "C" hipError_t tkh_launch_copy_batch(const tkh::CopyBatch *b, hipStream_t stream);
extern "C" int tkh_prefill_max_splits(void);
extern "C" int tkh_prefill_merge_blocks_per_row_block(int head_dim, int rows);
extern "C" hipError_t tkh_launch_prefill_merge(const tkh::Params *p, int head_dim, int rows,
                                               int64_t blocks, hipStream_t stream,
                                               hipEvent_t start, hipEvent_t stop);
extern "C" hipError_t tkh_launch_prefill16(const tkh::PrefillArgs *p, int dtype, int head_dim, int waves,
                                           int64_t groups, hipStream_t stream, hipEvent_t start,
                                           hipEvent_t stop);
extern "C" hipError_t tkh_launch_prefill(const tkh::PrefillArgs *p, int dtype, int head_dim, int waves,
                                         int64_t groups, hipStream_t stream, hipEvent_t start,
                                         hipEvent_t stop);
extern "C" int tkh_decode_keys_per_lane(int dtype, int head_dim, int rows, int want);
extern "C" int tkh_decode_max_waves(int dtype, int head_dim, int rows);
extern "C" int tkh_decode_max_splits(void);
extern "C" int tkh_project_vocab_per_block(void);
extern "C" hipError_t tkh_launch_project(const tkh::ProjectParams *p, hipStream_t stream,
                                         hipEvent_t start, hipEvent_t stop);
extern "C" hipError_t tkh_launch_decode(const tkh::DecodeArgs *p, int dtype, int head_dim, int rows,
                                        int keys_per_lane, int waves, int64_t groups, int fused,
                                        hipStream_t stream, hipEvent_t start, hipEvent_t stop);

using namespace tkh_host;

namespace {

// The error code of a nonzero device status word.
uint32_t status_error(uint32_t st, tkh_error *err) {
    if (st & tkh::ST_SPLIT_TIMEOUT)
        return fail(err, TKH_DEVICE, "decode splits", 0, 0, 0,
                    "a decode merge timed out waiting for its key splits (status 0x%x)", st);
    // A non-finite input anywhere decides first (the reference checks every
    // input before computing).
    if (st & tkh::ST_NONFINITE_INPUT)
        return fail(err, TKH_NON_FINITE, "attention inputs", 0, 0, 0,
                    "non-finite value in attention inputs or scores (status 0x%x)", st);
    if (st & tkh::ST_NONFINITE_LOGIT)
        return fail(err, TKH_NON_FINITE, "output", 0, 0, 0,
                    "non-finite projected logit (status 0x%x)", st);
    if (st & tkh::ST_BAD_MASS)
        return fail(err, TKH_NON_FINITE, "attention probabilities", 0, 0, 0,
                    "softmax mass is not finite and positive (status 0x%x)", st);
    return fail(err, TKH_NON_FINITE, "attention context", 0, 0, 0,
                "non-finite value in attention context (status 0x%x)", st);
}

// Completes queued work and turns the status word into an error code.
uint32_t finish(tkh_context *ctx, tkh_error *err) {
    hipError_t e = hipMemcpyAsync(ctx->status_host, ctx->status_dev, sizeof(uint32_t),
                                  hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return device_error(e, "synchronize", err);
    uint32_t st = *ctx->status_host;
    if (st == 0) return ok(err);
    // Clear the sticky word so the next call starts clean.
    e = tkh_launch_fill_u32(ctx->status_dev, 0, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return device_error(e, "status reset", err);
    return status_error(st, err);
}

uint32_t after_launch(tkh_context *ctx, tkh_error *err) {
    if (ctx->synchronous) return finish(ctx, err);
    return ok(err);
}

// A launch plan: problems sharing head geometry, dtype and mask parameters.
// Its problems live in fixed storage, so planning a call allocates nothing:
// one inline problem for the single-problem entry points, or the context's
// batch store (kSlotProblems problems, allocated with the context) for the
// batched ones, which plan and launch their sessions a store at a time.
struct Plan {
    tkh::Problem one{};
    tkh::Problem *store = &one;
    size_t capacity = 1, count = 0;
    Plan() = default;
    Plan(const Plan &) = delete;
    Plan &operator=(const Plan &) = delete;
    void add(const tkh::Problem &p) { store[count++] = p; }  // count < capacity by construction
    tkh_dtype dtype = TKH_BF16;
    int64_t query_heads = 0, kv_heads = 0, head_dim = 0;
    bool has_window = false;
    int64_t window = 0;
    float scale = 1.0f;
    float softcap = 0.0f;
    int diag_mode = 0;
    float *scores = nullptr;
    float *probs = nullptr;
    const tkh::FusedDecode *fused = nullptr;  // decode with the producer folded in
};

// A run of problems launched together (a view into a Plan's problems, or a
// problem held on the caller's stack).
struct Problems {
    tkh::Problem *p;
    size_t n;
    tkh::Problem *begin() const { return p; }
    tkh::Problem *end() const { return p + n; }
    tkh::Problem *data() const { return p; }
    size_t size() const { return n; }
    tkh::Problem &operator[](size_t i) const { return p[i]; }
};

tkh::Problem make_problem(const void *q, float *out, int64_t q_row_stride, int64_t q_pos0,
                          int64_t k_pos0, int64_t keys, int64_t queries) {
    tkh::Problem p{};
    p.q = q;
    p.out = out;
    p.q_row_stride = q_row_stride;
    p.q_pos0 = q_pos0;
    p.k_pos0 = k_pos0;
    p.keys = keys;
    p.queries = (int32_t)queries;
    p.nseg = 0;
    p.splits = 1;
    p.split_keys = 0;
    p.row_blocks = 1;
    return p;
}

void add_segment(tkh::Problem &p, const void *k, const void *v, int64_t head_stride,
                 int64_t row_stride, int64_t keys, int64_t start) {
    tkh::Segment &s = p.seg[p.nseg++];
    s.k = k;
    s.v = v;
    s.head_stride = head_stride;
    s.row_stride = row_stride;
    s.keys = keys;
    s.start = start;
}

uint32_t upload(tkh_context *ctx, const tkh::Problem *probs, int count, tkh::Problem **dev,
                tkh_error *err) {
    int slot = ctx->ring_next;
    ctx->ring_next = (ctx->ring_next + 1) % kSlots;
    if (ctx->ring_used[slot]) HIP_TRY(hipEventSynchronize(ctx->ring_events[slot]), "problem ring");
    tkh::Problem *host = ctx->ring_host + (size_t)slot * kSlotProblems;
    *dev = ctx->ring_dev + (size_t)slot * kSlotProblems;
    std::memcpy(host, probs, sizeof(tkh::Problem) * count);
    HIP_TRY(hipMemcpyAsync(*dev, host, sizeof(tkh::Problem) * count, hipMemcpyHostToDevice,
                           ctx->stream),
            "problem upload");
    HIP_TRY(hipEventRecord(ctx->ring_events[slot], ctx->stream), "problem ring");
    ctx->ring_used[slot] = true;
    return TKH_OK;
}

// Fold finished event quads into the totals. Each launch slot holds the start
// and stop events of the attention kernel and of the combine kernel; the
// second pair is left unrecorded when the launch has no combine kernel.
uint32_t profile_drain(tkh_context *ctx, tkh_error *err) {
    if (ctx->prof_used == 0) return TKH_OK;
    HIP_TRY(hipStreamSynchronize(ctx->stream), "profile");
    for (size_t i = 0; i < ctx->prof_used; ++i) {
        hipEvent_t *ev = &ctx->prof_events[4 * i];
        float a = 0, c = 0;
        HIP_TRY(hipEventElapsedTime(&a, ev[0], ev[1]), "profile");
        if (ctx->prof_has_combine[i]) HIP_TRY(hipEventElapsedTime(&c, ev[2], ev[3]), "profile");
        ctx->prof_attention_ms += a;
        ctx->prof_combine_ms += c;
        ctx->prof_launches += 1;
    }
    ctx->prof_used = 0;
    return TKH_OK;
}

uint32_t profile_slot(tkh_context *ctx, hipEvent_t **ev, bool combine, tkh_error *err) {
    const size_t cap = 1024;
    if (ctx->prof_events.empty()) {
        ctx->prof_events.resize(4 * cap);
        ctx->prof_has_combine.resize(cap);
        for (auto &e : ctx->prof_events) HIP_TRY(hipEventCreate(&e), "profile");
    }
    if (ctx->prof_used == cap) TRY(profile_drain(ctx, err));
    ctx->prof_has_combine[ctx->prof_used] = combine;
    *ev = &ctx->prof_events[4 * ctx->prof_used++];
    return TKH_OK;
}

// Key range [lo, hi) visible to at least one query row of a problem.
void visible_union(const Plan &plan, tkh::Problem &p) {
    const int64_t pos_min = p.q_pos0, pos_max = p.q_pos0 + p.queries - 1;
    int64_t hi = std::min<int64_t>(pos_max - p.k_pos0 + 1, p.keys);
    int64_t lo = 0;
    if (plan.has_window) lo = std::max<int64_t>(0, pos_min - (plan.window - 1) - p.k_pos0);
    p.vis_lo = std::max<int64_t>(0, lo);
    p.vis_hi = std::max<int64_t>(p.vis_lo, hi);
}

tkh::Params base_params(tkh_context *ctx, const Plan &plan) {
    tkh::Params prm{};
    prm.query_heads = (int32_t)plan.query_heads;
    prm.kv_heads = (int32_t)plan.kv_heads;
    prm.head_dim = (int32_t)plan.head_dim;
    prm.group = (int32_t)(plan.query_heads / plan.kv_heads);
    prm.has_window = plan.has_window ? 1 : 0;
    prm.window = plan.window;
    prm.scale = plan.scale;
    prm.scale_log2 = plan.scale * 1.4426950408889634f;
    prm.softcap = plan.softcap;
    prm.softcap_inv = plan.softcap != 0.0f ? 1.0f / plan.softcap : 0.0f;
    prm.softcap_y = prm.scale * prm.softcap_inv;
    prm.softcap_log2 = plan.softcap * 1.4426950408889634f;
    prm.status = ctx->status_dev;
    return prm;
}

// Few query rows per KV head: the streaming decode kernel, one launch.
uint32_t launch_decode(tkh_context *ctx, const Plan &plan, Problems group,
                       int rows, tkh_error *err) {
    const int64_t D = plan.head_dim, Hkv = plan.kv_heads;
    const int R = rows <= 1 ? 1 : rows <= 2 ? 2 : rows <= 4 ? 4 : 8;
    double work = 0;
    int64_t max_span = 0;
    for (auto &p : group) {
        visible_union(plan, p);
        work += (double)Hkv * (double)(p.vis_hi - p.vis_lo);
        max_span = std::max<int64_t>(max_span, p.vis_hi - p.vis_lo);
    }
    // Two regimes.  Little work (a few sessions): latency decides, so one
    // round of wide workgroups (eight waves, one per CU).  Much work: the
    // stream decides, so many narrower workgroups (two per CU), which keeps
    // every CU streaming while others start or merge and evens out sessions
    // of different lengths.
    // With much work of even length (sessions of about the same span), one
    // round of one equal workgroup per CU suffices and keeps the splits and
    // their merges few (16 sessions at 8192 keys: 97 us against 100 us at two
    // per CU and 103-110 us at four to eight); spans of mixed lengths take
    // several rounds so the dispatcher can even them out.
    const bool bulk = work >= (double)ctx->decode_bulk_keys * ctx->cus;
    const bool even = work >= 0.9 * (double)Hkv * (double)max_span * (double)group.size();
    // Even spans at one workgroup per CU stream best with eight waves of two
    // keys per lane (16 sessions at 8192 keys: 96 us against 98 us at four
    // waves of four keys); mixed spans and latency-bound launches do not
    // (configs[2] 199 -> 219 us, configs[1] steps 11.9 -> 13.0 us).
    const int nw_max = std::min(!bulk ? ctx->decode_waves
                                      : (even ? ctx->decode_even_waves : ctx->decode_bulk_waves),
                                tkh_decode_max_waves((int)plan.dtype, (int)D, R));
    const double groups = !bulk ? ctx->decode_groups
                                : (even ? ctx->decode_even_groups : ctx->decode_bulk_groups);
    int nw = nw_max;
    const int u = tkh_decode_keys_per_lane((int)plan.dtype, (int)D, R,
                                           bulk && even ? ctx->decode_even_keys_per_lane
                                                        : ctx->decode_keys_per_lane);
    const int max_splits = std::min(ctx->decode_max_splits, tkh_decode_max_splits());
    const int64_t kpb = (int64_t)8 * u;  // keys per wave block
    // Keys per split: about decode_groups workgroups in all, at most
    // max_splits per KV head, in whole blocks, and at least one block for
    // each wave a split launch needs (its merge reads 64 outputs per wave);
    // then as many waves (up to nw) as the split has blocks, so no wave
    // starts without work.
    const int merge_waves = std::min(nw_max, (int)((R * D + 63) / 64));
    int64_t sk = (int64_t)std::ceil(work / groups);
    sk = std::max<int64_t>(sk, (max_span + max_splits - 1) / max_splits);
    if (sk < max_span) sk = std::max<int64_t>(sk, kpb * merge_waves);
    if (ctx->split_keys_override > 0) sk = ctx->split_keys_override;
    sk = std::max<int64_t>(kpb, (sk + kpb - 1) / kpb * kpb);
    // Splits never straddle a segment boundary, so a view of several segments
    // rounds each one up: grow the split size (in whole blocks) until every
    // problem fits the merge, which reads at most max_splits partials.
    auto seg_split_counts = [&](tkh::Problem &p, int64_t keys_per_split) {
        int64_t n_all = 0;
        for (int s = 0; s < 3; ++s) {
            int64_t n = 0;
            if (s < p.nseg) {
                const int64_t lo = std::max<int64_t>(p.vis_lo, p.seg[s].start);
                const int64_t hi = std::min<int64_t>(p.vis_hi, p.seg[s].start + p.seg[s].keys);
                if (hi > lo) n = (hi - lo + keys_per_split - 1) / keys_per_split;
            }
            p.seg_splits[s] = (int32_t)n;
            n_all += n;
        }
        if (n_all == 0) {  // nothing visible: one empty split reports the bad mass
            p.seg_splits[0] = 1;
            n_all = 1;
        }
        return n_all;
    };
    for (;;) {
        int64_t worst = 0;
        for (auto &p : group) worst = std::max<int64_t>(worst, seg_split_counts(p, sk));
        if (worst <= max_splits) break;
        sk = (sk * 2 + kpb - 1) / kpb * kpb;
    }
    if (sk > INT32_MAX) return fail(err, TKH_UNSUPPORTED, "keys", 0, 0, 0, "key range too large");
    nw = (int)std::min<int64_t>(nw, sk / kpb);

    // Splits of every problem, laid out segment by segment over its visible range.
    int64_t wgs = 0, slots = 0;
    for (size_t i = 0; i < group.size(); ++i) {
        auto &p = group[i];
        p.split_keys = (int32_t)sk;
        p.splits = (int32_t)seg_split_counts(p, sk);
        p.row_blocks = 1;
        p.tile_base = wgs;
        p.slot_base = slots;
        p.group_base = (int32_t)(i * Hkv);
        wgs += Hkv * p.splits;
        slots += Hkv * p.splits;
    }
    // The merging workgroup of a split launch reads 64 outputs per wave: one
    // wave per 64 outputs (within the kernel's limit) makes the merge one pass.
    bool any_split = false;
    for (auto &p : group) any_split |= p.splits > 1;
    if (any_split) nw = std::max(nw, merge_waves);

    // Decode partials: completion flags, then (max, mass) and contexts, in the
    // decode half of the workspace.
    const size_t flag_bytes = ((size_t)slots * sizeof(uint32_t) + 255) / 256 * 256;
    const size_t part_bytes = (size_t)slots * R * (D + 2) * sizeof(float);
    const size_t need = flag_bytes + part_bytes;
    if (need > decode_region_bytes(ctx))
        return fail(err, TKH_UNSUPPORTED, "workspace", 0, need, decode_region_bytes(ctx),
                    "decode needs %zu workspace bytes, context has %zu for it", need,
                    decode_region_bytes(ctx));
    // The merge addresses every partial through one buffer resource based at
    // the (max, mass) array, with 32-bit byte offsets below 2^31.
    if (part_bytes > (size_t)INT32_MAX)
        return fail(err, TKH_UNSUPPORTED, "workspace", 0, (size_t)INT32_MAX, part_bytes,
                    "decode partials of %zu bytes exceed the merge's 2 GiB range", part_bytes);

    // Up to DECODE_BATCH_MAX single-token sessions laid out as tkh_decode_batch
    // lays them out (Q/context rows consecutive, K and V at one offset from
    // common bases) travel in the kernel arguments; other launches of several
    // problems upload their descriptors.
    tkh::DecodeArgs args{};
    tkh::DecodeBatch &cb = args.b;
    if (group.size() > 1 && group.size() <= (size_t)tkh::DECODE_BATCH_MAX && !plan.fused) {
        const tkh::Problem &p0 = group[0];
        const int64_t es = esize(plan.dtype), row = plan.query_heads * D;
        bool compact = true;
        for (size_t i = 0; i < group.size() && compact; ++i) {
            const tkh::Problem &p = group[i];
            const int64_t dk = (const uint8_t *)p.seg[0].k - (const uint8_t *)p0.seg[0].k;
            const int64_t dv = (const uint8_t *)p.seg[0].v - (const uint8_t *)p0.seg[0].v;
            compact = p.nseg == 1 && p.queries == 1 && p.k_pos0 == 0 && p.seg[0].start == 0 &&
                      p.seg[0].row_stride == D && p.keys == p.seg[0].keys &&
                      p.q_pos0 == p.keys - 1 && p.vis_lo == 0 && p.vis_hi == p.keys &&
                      p.keys <= UINT32_MAX && p.seg[0].head_stride <= UINT32_MAX &&
                      p.tile_base <= UINT32_MAX && p.slot_base == p.tile_base &&
                      (const uint8_t *)p.q == (const uint8_t *)p0.q + (int64_t)i * row * es &&
                      p.out == p0.out + (int64_t)i * row && dk == dv && dk % es == 0;
            if (compact) {
                tkh::DecodeBatchEntry &e = cb.e[i];
                e.kv_offset = dk / es;
                e.head_stride = (uint32_t)p.seg[0].head_stride;
                e.keys = (uint32_t)p.keys;
                e.tile_base = (uint32_t)p.tile_base;
                e.splits = (uint32_t)p.splits;
            }
        }
        if (compact) {
            cb.q = p0.q;
            cb.out = p0.out;
            cb.k = p0.seg[0].k;
            cb.v = p0.seg[0].v;
            cb.count = (int32_t)group.size();
            cb.split_keys = (int32_t)sk;
        }
    }
    tkh::Problem *dev = nullptr;
    if (group.size() > 1 && cb.count == 0) TRY(upload(ctx, group.data(), (int)group.size(), &dev, err));
    tkh::Params &prm = args.p;
    prm = base_params(ctx, plan);
    prm.problems = dev;
    if (group.size() == 1) prm.single = group[0];
    prm.nproblems = (int32_t)group.size();
    prm.total_tiles = wgs;
    bool split = false;
    for (auto &p : group) split |= p.splits > 1;
    if (split && ++ctx->epoch == 0) {
        // The epoch wrapped: clear every flag so no stale one can match again.
        HIP_TRY(tkh_launch_zero_u64(reinterpret_cast<uint64_t *>(decode_region(ctx)),
                                    (int64_t)(decode_region_bytes(ctx) / sizeof(uint64_t)), ctx->stream),
                "decode workspace clear");
        ctx->epoch = 1;
    }
    prm.epoch = ctx->epoch;
    // The merging split waits for this launch's epoch; the test hook makes it
    // wait for one that no split stores, to exercise the bounded wait.
    prm.wait_epoch = ctx->epoch + (ctx->test_flag_skew ? 1u : 0u);
    prm.split_wait_ticks = ctx->split_wait_ticks;
    // Much work streams at the HBM limit, where nontemporal loads raise the
    // rate (configs[2] 200 -> 184 us, 16 sessions at 8192 keys 96 -> 86 us);
    // a latency-bound launch is 0.4 us slower with them (one session at 8192
    // keys 15.3 -> 15.7 us), so it keeps plain loads.
    prm.stream_nt = ctx->decode_stream_nt < 0 ? (bulk ? 1 : 0) : ctx->decode_stream_nt;
    prm.flags = reinterpret_cast<uint32_t *>(decode_region(ctx));
    float *ws = reinterpret_cast<float *>(decode_region(ctx) + flag_bytes);
    prm.part_ml = ws;
    prm.part_o = ws + (size_t)slots * R * 2;

    // A single problem with little work (one session's decode step) leaves
    // the combine to a second launch: every split stores its partial and
    // exits, and the kernel boundary orders the stores, instead of the
    // in-kernel merge's three memory round trips between workgroups.
    // (The bounded-wait test hook exercises the in-kernel merge.)
    const bool merge_batch = split && cb.count > 0 && ctx->decode_merge_batch && !ctx->test_flag_skew;
    const bool merge_launch = merge_batch || (split && group.size() == 1 && !bulk &&
                                              ctx->decode_merge_launch && !ctx->test_flag_skew);
    prm.merge_launch = merge_launch ? 1 : 0;
    hipEvent_t *ev = nullptr;
    if (ctx->profiling) TRY(profile_slot(ctx, &ev, merge_launch, err));
    if (plan.fused) prm.fused = *plan.fused;
    hipError_t e = tkh_launch_decode(&args, (int)plan.dtype, (int)D, R, u, nw, wgs,
                                     plan.fused ? 1 : 0, ctx->stream, ev ? ev[0] : nullptr,
                                     ev ? ev[1] : nullptr);
    if (e != hipSuccess) return device_error(e, "decode launch", err);
    if (merge_batch) {
        e = tkh_launch_decode_merge_batch(&args, (int)D, R, ctx->stream, ev ? ev[2] : nullptr,
                                          ev ? ev[3] : nullptr);
        if (e != hipSuccess) return device_error(e, "decode merge launch", err);
    } else if (merge_launch) {
        e = tkh_launch_decode_merge(&prm, (int)D, R, (int)Hkv, ctx->stream, ev ? ev[2] : nullptr,
                                    ev ? ev[3] : nullptr);
        if (e != hipSuccess) return device_error(e, "decode merge launch", err);
    }
    return TKH_OK;
}

// Planned chunks of one shape (equal query counts, one segment from key 0
// ending at the chunk, no key splits, Q and contexts at one stride, K and V at
// the same offset from the first chunk's) as a compact batch in the kernel's
// arguments; false when the group does not have that shape.
bool compact_prefill(const Plan &plan, const Problems &group, tkh::PrefillBatch *b) {
    if (group.size() < 2 || group.size() > (size_t)tkh::PREFILL_BATCH_MAX) return false;
    const int64_t D = plan.head_dim, es = esize(plan.dtype), row = plan.query_heads * D;
    const tkh::Problem &p0 = group[0];
    const int64_t step = (int64_t)p0.queries * row;
    const uint8_t *k0 = static_cast<const uint8_t *>(p0.seg[0].k);
    const uint8_t *v0 = static_cast<const uint8_t *>(p0.seg[0].v);
    for (size_t i = 0; i < group.size(); ++i) {
        const tkh::Problem &p = group[i];
        const tkh::Segment &sg = p.seg[0];
        if (p.nseg != 1 || p.splits != 1 || p.queries != p0.queries || p.row_blocks != p0.row_blocks ||
            p.k_pos0 != 0 || sg.start != 0 || sg.keys != p.keys || sg.row_stride != D ||
            p.q_row_stride != row || p.q_pos0 + p.queries != p.keys || p.vis_lo != 0 ||
            p.vis_hi != p.keys)
            return false;
        if (static_cast<const uint8_t *>(p.q) != static_cast<const uint8_t *>(p0.q) + (int64_t)i * step * es ||
            p.out != p0.out + (int64_t)i * step)
            return false;
        const int64_t dk = static_cast<const uint8_t *>(sg.k) - k0;
        const int64_t dv = static_cast<const uint8_t *>(sg.v) - v0;
        if (dk != dv || dk % es != 0) return false;
        b->e[i] = tkh::PrefillBatchEntry{dk / es, sg.head_stride, p.q_pos0, p.tile_base};
    }
    b->q = p0.q;
    b->out = p0.out;
    b->k = k0;
    b->v = v0;
    b->q_step = step;
    b->count = (int32_t)group.size();
    b->tokens = p0.queries;
    b->row_blocks = p0.row_blocks;
    b->split_keys = p0.split_keys;
    return true;
}

// Many query rows per KV head (bf16/f16): the MFMA flash kernel, one launch.
uint32_t launch_prefill(tkh_context *ctx, const Plan &plan, Problems group,
                        tkh_error *err) {
    const int64_t D = plan.head_dim, Hkv = plan.kv_heads, G = plan.query_heads / plan.kv_heads;
    // Eight-wave (256-row) workgroups where the head_dim has them and their row
    // blocks alone fill the device (the target is set in 128-row workgroups);
    // four-wave ones otherwise.
    int waves = tkh_prefill_waves((int)D, 0);
    {
        const int wide = tkh_prefill_waves((int)D, 1);
        int64_t wide_groups = 0;
        for (auto &p : group) wide_groups += Hkv * (((int64_t)p.queries * G + 32 * wide - 1) / (32 * wide));
        if (wide != waves && wide_groups >= ctx->prefill_fill_groups * 128 / (32 * wide)) waves = wide;
        if (ctx->prefill_waves == 4 || ctx->prefill_waves == wide) waves = ctx->prefill_waves;
    }
    // Four-wave launches at head_dim 128 and 256 take the 16-row kernel, by
    // default with four waves (64-row blocks), which doubles a chunk's
    // workgroups at the same partial volume: configs[3] session chunks 5.76-5.79
    // -> 5.32-5.39 ms, configs[1] chunk kernels 14.3-14.7 -> 13.1-13.5 us
    // (alternating runs).  Eight-wave launches (row blocks that fill the
    // device, configs[4]) keep the 32-row kernel: the 16-row one reads each
    // K/V operand for half as many rows and measured slower there.
    const bool rows16 = ctx->prefill16 != 0 && waves == 4 && (D == 128 || D == 256);
    const int waves16 = ctx->prefill16_waves;
    const int64_t rows_per = rows16 ? 16 * waves16 : 32 * waves;
    int64_t base_groups = 0;
    int64_t max_span = 0;
    for (auto &p : group) {
        visible_union(plan, p);
        p.row_blocks = (int32_t)(((int64_t)p.queries * G + rows_per - 1) / rows_per);
        base_groups += Hkv * p.row_blocks;
        max_span = std::max<int64_t>(max_span, p.vis_hi - p.vis_lo);
    }
    // Too few row-block workgroups to fill the device: split the keys.  The
    // target is set in 128-row workgroups and scaled to this head_dim's size.
    // The 16-row kernel takes its own target: 64 gave configs[3] and configs[1]
    // their best times with 64-row blocks (5.32-5.39 against 5.39-5.46 ms at
    // 128; configs[1] session prefill 0.60-0.62 against 0.60-0.65 ms).
    const int64_t target =
        std::max<int64_t>(1, (rows16 ? ctx->prefill16_groups : ctx->prefill_groups) * 128 / rows_per);
    int64_t splits = 1;
    if (base_groups < target) {
        splits = (target + base_groups - 1) / base_groups;
        splits = std::min<int64_t>(splits, ctx->prefill_max_splits);
        splits = std::min<int64_t>(splits, std::max<int64_t>(1, max_span / ctx->prefill_min_keys));
    }
    int64_t sk = (max_span + splits - 1) / splits;
    sk = std::max<int64_t>(32, (sk + 31) / 32 * 32);
    if (ctx->split_keys_override > 0) sk = (ctx->split_keys_override + 31) / 32 * 32;
    // Splits are laid out segment by segment and never straddle a segment
    // boundary (one base pointer per workgroup), so a view of several segments
    // needs at least one split each; grow the split size until every problem
    // fits the merge limit.
    auto seg_split_counts = [&](tkh::Problem &p, int64_t keys_per_split) {
        int64_t n_all = 0;
        for (int sgi = 0; sgi < 3; ++sgi) {
            int64_t n = 0;
            if (sgi < p.nseg) {
                const int64_t lo = std::max<int64_t>(p.vis_lo, p.seg[sgi].start);
                const int64_t hi = std::min<int64_t>(p.vis_hi, p.seg[sgi].start + p.seg[sgi].keys);
                if (hi > lo) n = (hi - lo + keys_per_split - 1) / keys_per_split;
            }
            p.seg_splits[sgi] = (int32_t)n;
            n_all += n;
        }
        if (n_all == 0) {  // nothing visible: one empty split reports the bad mass
            p.seg_splits[0] = 1;
            n_all = 1;
        }
        return n_all;
    };
    // The partials of a split launch must also fit the workspace: fewer, longer
    // splits until they do (a launch without splits writes none).
    auto partial_bytes = [&](int64_t keys_per_split) {
        size_t n_slots = 0;
        for (auto &p : group) {
            const int64_t n = seg_split_counts(p, keys_per_split);
            if (n > 1) n_slots += (size_t)(Hkv * p.row_blocks * n);
        }
        return n_slots * (size_t)rows_per * (size_t)(D + 2) * sizeof(float);
    };
    for (;;) {
        int64_t worst = 0;
        for (auto &p : group) worst = std::max<int64_t>(worst, seg_split_counts(p, sk));
        const bool fits = worst == 1 || partial_bytes(sk) <= split_region_bytes(ctx);
        if (worst <= tkh_prefill_max_splits() && (fits || sk >= max_span)) break;
        sk *= 2;
    }
    // Splits of one row block are combined by a second kernel, in merge blocks
    // of a few rows; Problem::part_base is the problem's first merge block.
    const int64_t merge_per_rb = tkh_prefill_merge_blocks_per_row_block((int)D, (int)rows_per);
    int64_t wgs = 0, slots = 0, merge_blocks = 0;
    for (auto &p : group) {
        if (sk > INT32_MAX) return fail(err, TKH_UNSUPPORTED, "keys", 0, 0, 0, "key range too large");
        p.split_keys = (int32_t)sk;
        p.splits = (int32_t)seg_split_counts(p, sk);
        p.tile_base = wgs;
        p.slot_base = slots;
        p.part_base = merge_blocks;
        const int64_t g = Hkv * p.row_blocks;
        wgs += g * p.splits;
        if (p.splits > 1) {
            slots += g * p.splits;
            merge_blocks += g * merge_per_rb;
        }
    }
    const size_t need = (size_t)slots * rows_per * (D + 2) * sizeof(float);
    if (need > split_region_bytes(ctx))
        return fail(err, TKH_UNSUPPORTED, "workspace", 0, need, split_region_bytes(ctx),
                    "attention needs %zu workspace bytes, context has %zu for it", need,
                    split_region_bytes(ctx));
    tkh::PrefillArgs args{};
    tkh::Problem *dev = nullptr;
    if (group.size() > 1 && !(ctx->prefill_compact && compact_prefill(plan, group, &args.b)))
        TRY(upload(ctx, group.data(), (int)group.size(), &dev, err));
    tkh::Params &prm = args.p;
    prm = base_params(ctx, plan);
    prm.problems = dev;
    if (group.size() == 1) prm.single = group[0];
    prm.nproblems = (int32_t)group.size();
    prm.total_tiles = wgs;
    float *ws = reinterpret_cast<float *>(ctx->workspace);
    prm.part_ml = ws;
    prm.part_o = ws + (size_t)slots * rows_per * 2;

    hipEvent_t *ev = nullptr;
    if (ctx->profiling) TRY(profile_slot(ctx, &ev, merge_blocks > 0, err));
    hipError_t e = rows16 ? tkh_launch_prefill16(&args, (int)plan.dtype, (int)D, waves16, wgs, ctx->stream,
                                                 ev ? ev[0] : nullptr, ev ? ev[1] : nullptr)
                          : tkh_launch_prefill(&args, (int)plan.dtype, (int)D, waves, wgs, ctx->stream,
                                               ev ? ev[0] : nullptr, ev ? ev[1] : nullptr);
    if (e != hipSuccess) return device_error(e, "prefill launch", err);
    if (merge_blocks > 0) {
        e = tkh_launch_prefill_merge(&prm, (int)D, (int)rows_per, merge_blocks, ctx->stream,
                                     ev ? ev[2] : nullptr, ev ? ev[3] : nullptr);
        if (e != hipSuccess) return device_error(e, "prefill merge launch", err);
    }
    return TKH_OK;
}

// Launch one group of problems (<= kSlotProblems) through the workspace.
uint32_t launch_group(tkh_context *ctx, const Plan &plan, Problems group,
                      tkh_error *err) {
    const int64_t D = plan.head_dim, Hq = plan.query_heads, Hkv = plan.kv_heads;
    const int64_t G = Hq / Hkv;
    {
        int64_t max_rows = 0;
        for (auto &p : group) max_rows = std::max<int64_t>(max_rows, (int64_t)p.queries * G);
        const int limit = tkh_decode_max_rows((int)plan.dtype, (int)D);
        if (plan.fused) {
            // The softcap build of the fused decode exists at head_dim 256.
            if (limit <= 0 || max_rows > limit || plan.diag_mode != 0 ||
                (plan.softcap != 0.0f && D != 256))
                return fail(err, TKH_UNSUPPORTED, "fused decode", 0, limit, max_rows,
                            "fused producer decode needs the streaming decode kernel");
            return launch_decode(ctx, plan, group, (int)max_rows, err);
        }
        if (!ctx->force_generic && !ctx->decode_disable && plan.diag_mode == 0 && limit > 0 &&
            max_rows <= limit)
            return launch_decode(ctx, plan, group, (int)max_rows, err);
        if (!ctx->force_generic && plan.diag_mode == 0 &&
            (plan.dtype == TKH_BF16 || plan.dtype == TKH_F16) && (D == 64 || D == 128 || D == 256))
            return launch_prefill(ctx, plan, group, err);
    }
    // FP32, odd head sizes and diagnostics: one wave per (query, head), then a
    // combine launch that publishes the context.
    const size_t ws_floats = split_region_bytes(ctx) / sizeof(float);
    {
        size_t need = 0;
        for (auto &p : group) need += (size_t)p.queries * Hq * (D + 2);
        if (need > ws_floats)
            return fail(err, TKH_UNSUPPORTED, "workspace", 0, need * 4, split_region_bytes(ctx),
                        "attention needs %zu workspace bytes, context has %zu for it", need * 4,
                        split_region_bytes(ctx));
    }
    int64_t tiles = 0, rows = 0, part_rows = 0;
    for (auto &p : group) {
        p.tile_base = tiles;
        p.part_base = rows;
        p.splits = 1;
        p.row_blocks = 1;
        tiles += (int64_t)p.queries * Hq;
        p.slot_base = part_rows;
        rows += (int64_t)p.queries * Hq;
        part_rows += (int64_t)p.queries * Hq;
    }

    tkh::Problem *dev = nullptr;
    if (group.size() > 1) TRY(upload(ctx, group.data(), (int)group.size(), &dev, err));

    tkh::Params prm{};
    prm.problems = dev;
    if (group.size() == 1) prm.single = group[0];
    prm.nproblems = (int32_t)group.size();
    prm.query_heads = (int32_t)Hq;
    prm.kv_heads = (int32_t)Hkv;
    prm.head_dim = (int32_t)D;
    prm.group = (int32_t)G;
    prm.has_window = plan.has_window ? 1 : 0;
    prm.window = plan.window;
    prm.scale = plan.scale;
    prm.scale_log2 = plan.scale * 1.4426950408889634f;
    prm.softcap = plan.softcap;
    prm.softcap_inv = plan.softcap != 0.0f ? 1.0f / plan.softcap : 0.0f;
    prm.softcap_y = prm.scale * prm.softcap_inv;
    prm.softcap_log2 = plan.softcap * 1.4426950408889634f;
    prm.total_tiles = tiles;
    prm.part_ml = reinterpret_cast<float *>(ctx->workspace);
    prm.part_o = reinterpret_cast<float *>(ctx->workspace) + 2 * part_rows;
    prm.status = ctx->status_dev;
    prm.scores = plan.scores;
    prm.probs = plan.probs;
    prm.diag_mode = plan.diag_mode;

    hipEvent_t *ev = nullptr;
    if (ctx->profiling) TRY(profile_slot(ctx, &ev, true, err));
    hipError_t e = tkh_launch_generic(&prm, (int)plan.dtype, ctx->stream, ev ? ev[0] : nullptr,
                                      ev ? ev[1] : nullptr);
    if (e != hipSuccess) return device_error(e, "attention launch", err);
    e = tkh_launch_combine(&prm, rows, ctx->stream, ev ? ev[2] : nullptr, ev ? ev[3] : nullptr);
    if (e != hipSuccess) return device_error(e, "combine launch", err);
    return TKH_OK;
}

// Launch `count` problems in groups of at most kSlotProblems (their planning
// fields are filled in place).
uint32_t launch_all(tkh_context *ctx, const Plan &plan, tkh::Problem *probs, size_t count,
                    tkh_error *err) {
    if (hipSetDevice(ctx->device) != hipSuccess)
        return fail(err, TKH_DEVICE, "device", 0, 0, 0, "hipSetDevice failed");
    for (size_t i = 0; i < count; i += kSlotProblems) {
        const size_t n = std::min<size_t>(kSlotProblems, count - i);
        TRY(launch_group(ctx, plan, Problems{probs + i, n}, err));
    }
    return TKH_OK;
}

uint32_t run(tkh_context *ctx, Plan &plan, tkh_error *err) {
    TRY(launch_all(ctx, plan, plan.store, plan.count, err));
    return after_launch(ctx, err);
}


// The planner's settings of a context on `device`: the defaults, each
// overridable by a TKH_* environment variable, and the device's CU count.
void init_tuning(tkh_context *ctx, int device) {
    ctx->split_keys_override = env_int("TKH_SPLIT_KEYS", 0);
    ctx->force_generic = env_int("TKH_FORCE_GENERIC", 0);
    ctx->decode_waves = std::min(8, std::max(1, env_int("TKH_DECODE_WAVES", 8)));
    ctx->decode_keys_per_lane = std::max(1, env_int("TKH_DECODE_KEYS_PER_LANE", 4));
    // One round of decode workgroups: with eight waves and the register
    // budget of the kernel, one workgroup fits per CU.
    {
        hipDeviceProp_t prop;
        int cus = 256;
        if (hipGetDeviceProperties(&prop, device) == hipSuccess && prop.multiProcessorCount > 0)
            cus = prop.multiProcessorCount;
        ctx->cus = cus;
        ctx->decode_groups = std::max(1, env_int("TKH_DECODE_GROUPS", cus));
        ctx->decode_bulk_groups = std::max(1, env_int("TKH_DECODE_BULK_GROUPS", 8 * cus));
        ctx->decode_even_groups = std::max(1, env_int("TKH_DECODE_EVEN_GROUPS", cus));
    }
    ctx->decode_bulk_waves = std::min(8, std::max(1, env_int("TKH_DECODE_BULK_WAVES", 4)));
    ctx->decode_even_waves = std::min(8, std::max(1, env_int("TKH_DECODE_EVEN_WAVES", 8)));
    ctx->decode_even_keys_per_lane = std::max(1, env_int("TKH_DECODE_EVEN_KEYS_PER_LANE", 2));
    ctx->decode_bulk_keys = std::max(1, env_int("TKH_DECODE_BULK_KEYS", 2048));
    ctx->decode_stream_nt = std::min(1, std::max(-1, env_int("TKH_DECODE_STREAM_NT", -1)));
    // Test hooks for the decode merge's bounded wait (s_memrealtime ticks,
    // 100 MHz; default half a second) and a flag value no split stores.
    ctx->split_wait_ticks = (uint64_t)std::max(1, env_int("TKH_TEST_SPLIT_WAIT_TICKS", 50000000));
    ctx->test_flag_skew = env_int("TKH_TEST_SPLIT_FLAG_SKEW", 0) != 0;
    ctx->decode_max_splits = std::max(1, env_int("TKH_DECODE_MAX_SPLITS", 64));
    ctx->decode_disable = env_int("TKH_DECODE_DISABLE", 0);
    ctx->decode_merge_launch = env_int("TKH_DECODE_MERGE_LAUNCH", 1) != 0;
    ctx->decode_merge_batch = env_int("TKH_DECODE_MERGE_BATCH", 0) != 0;
    // Split target: 128 workgroups.  At configs[1] chunk sizes (16 row blocks)
    // that is 8 key splits instead of the 16 a 512 target gave: half the
    // partials to write and merge, 21.7 -> 21.0 us per chunk for the two
    // kernels; configs[3] (8 row blocks) keeps 16 splits.
    ctx->prefill_groups = std::max(1, env_int("TKH_PREFILL_GROUPS", 128));
    ctx->prefill_fill_groups = std::max(1, env_int("TKH_PREFILL_FILL_GROUPS", 512));
    ctx->prefill_max_splits =
        std::min(tkh_prefill_max_splits(), std::max(1, env_int("TKH_PREFILL_MAX_SPLITS", 16)));
    // 64: configs[3] prefill 8.8 -> 7.5 ms and configs[1] chunks 17.9 -> 15.8 us
    // against 256 (128: 7.6 ms, 16.1 us; 32: no better).
    ctx->prefill_min_keys = std::max(32, env_int("TKH_PREFILL_MIN_KEYS", 64));
    ctx->prefill_waves = env_int("TKH_PREFILL_WAVES", 0);
    ctx->prefill_compact = env_int("TKH_PREFILL_COMPACT", 1) != 0;
    ctx->prefill16 = env_int("TKH_PREFILL16", 1);
    ctx->prefill16_groups = std::max(1, env_int("TKH_PREFILL16_GROUPS", 64));
    ctx->prefill16_waves = env_int("TKH_PREFILL16_WAVES", 4) == 8 ? 8 : 4;
}

// First visible key (absolute) of a query at `position` (window_attention.rs:105-107).
uint64_t first_visible(uint64_t key_start, uint64_t position, bool has_window, uint64_t window) {
    if (!has_window) return key_start;
    uint64_t lower = position >= window - 1 ? position - (window - 1) : 0;
    return std::max(key_start, lower);
}

}  // namespace

extern "C" {

uint32_t tkh_abi_version(void) { return TKH_ABI_VERSION; }

uint32_t tkh_context_create(int device, void *stream, size_t workspace_bytes, int synchronous,
                            tkh_context **out, tkh_error *err) {
    if (!out) return invalid("context output", err);
    *out = nullptr;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count == 0)
        return fail(err, TKH_DEVICE, "device", 0, 0, 0, "no HIP device is available");
    if (device < 0 || device >= count) return invalid("device ordinal", err);
    HIP_TRY(hipSetDevice(device), "hipSetDevice");
    auto *ctx = new tkh_context();
    ctx->device = device;
    ctx->synchronous = synchronous != 0;
    ctx->workspace_bytes = workspace_bytes ? workspace_bytes : (size_t)256 << 20;
    init_tuning(ctx, device);
    auto cleanup = [&](hipError_t e, const char *where) {
        tkh_context_destroy(ctx);
        return device_error(e, where, err);
    };
    hipError_t e;
    // The caller's stream, or the device's null stream: work is ordered with
    // whatever the caller queued there (no private stream, no priorities).
    ctx->stream = reinterpret_cast<hipStream_t>(stream);
    if ((e = hipMalloc(&ctx->status_dev, 256)) != hipSuccess) return cleanup(e, "status");
    if ((e = hipMemset(ctx->status_dev, 0, 256)) != hipSuccess) return cleanup(e, "status");
    if ((e = hipHostMalloc(&ctx->status_host, sizeof(uint32_t), hipHostMallocDefault)) != hipSuccess)
        return cleanup(e, "status");
    if ((e = hipMalloc(&ctx->workspace, ctx->workspace_bytes)) != hipSuccess)
        return cleanup(e, "workspace");
    // Decode tags start at 0, which no launch epoch equals.
    if ((e = hipMemset(decode_region(ctx), 0, decode_region_bytes(ctx))) != hipSuccess)
        return cleanup(e, "workspace");
    ctx->batch_store = new (std::nothrow) tkh::Problem[kSlotProblems];
    if (!ctx->batch_store) return cleanup(hipErrorOutOfMemory, "batch plan store");
    size_t ring = sizeof(tkh::Problem) * kSlots * kSlotProblems;
    if ((e = hipMalloc(&ctx->ring_dev, ring)) != hipSuccess) return cleanup(e, "problem ring");
    if ((e = hipHostMalloc(&ctx->ring_host, ring, hipHostMallocDefault)) != hipSuccess)
        return cleanup(e, "problem ring");
    for (int i = 0; i < kSlots; ++i)
        if ((e = hipEventCreateWithFlags(&ctx->ring_events[i], hipEventDisableTiming)) != hipSuccess)
            return cleanup(e, "problem ring");
    *out = ctx;
    return ok(err);
}

void tkh_context_destroy(tkh_context *ctx) {
    if (!ctx) return;
    delete[] ctx->batch_store;
    hipSetDevice(ctx->device);
    if (ctx->stream) hipStreamSynchronize(ctx->stream);
    for (int i = 0; i < kSlots; ++i)
        if (ctx->ring_events[i]) hipEventDestroy(ctx->ring_events[i]);
    for (auto &e : ctx->prof_events)
        if (e) hipEventDestroy(e);
    if (ctx->ring_host) hipHostFree(ctx->ring_host);
    if (ctx->ring_dev) hipFree(ctx->ring_dev);
    if (ctx->workspace) hipFree(ctx->workspace);
    if (ctx->status_host) hipHostFree(ctx->status_host);
    if (ctx->status_dev) hipFree(ctx->status_dev);
    delete ctx;
}

uint32_t tkh_context_synchronize(tkh_context *ctx, tkh_error *err) {
    if (!ctx) return invalid("context", err);
    return finish(ctx, err);
}

void *tkh_context_stream(tkh_context *ctx) { return ctx ? (void *)ctx->stream : nullptr; }

uint32_t tkh_context_profile(tkh_context *ctx, int enable, tkh_error *err) {
    if (!ctx) return invalid("context", err);
    TRY(profile_drain(ctx, err));
    ctx->profiling = enable != 0;
    ctx->prof_launches = 0;
    ctx->prof_attention_ms = 0;
    ctx->prof_combine_ms = 0;
    return ok(err);
}

uint32_t tkh_context_profile_read(tkh_context *ctx, tkh_profile *out, tkh_error *err) {
    if (!ctx || !out) return invalid("context", err);
    TRY(profile_drain(ctx, err));
    out->launches = ctx->prof_launches;
    out->attention_ms = ctx->prof_attention_ms;
    out->combine_ms = ctx->prof_combine_ms;
    return ok(err);
}

// ---------------------------------------------------------------- operators

}  // extern "C"

namespace {

// Sizes of an attention_cached call, checked in src/cpu/attention.rs:218-245's
// order up to the context length.
struct CachedDims {
    uint64_t end, q_stride, head_stride;
};
uint32_t check_cached(const tkh_cached_shape &s, uint64_t q_len, uint64_t k_len, uint64_t v_len,
                      uint64_t context_len, CachedDims *d, tkh_error *err) {
    TRY(nonzero(s.tokens, "tokens", err));
    TRY(nonzero(s.query_heads, "query_heads", err));
    TRY(nonzero(s.kv_heads, "kv_heads", err));
    TRY(nonzero(s.head_dim, "head_dim", err));
    TRY(nonzero(s.capacity, "cache capacity", err));
    if (s.query_heads % s.kv_heads != 0) return invalid("query_heads must be divisible by kv_heads", err);
    TRY(add(s.offset, s.tokens, &d->end, err));
    if (d->end > s.capacity) return invalid("cache capacity exceeded", err);
    uint64_t q_count, kv_count;
    TRY(product(s.query_heads, s.head_dim, &d->q_stride, err));
    TRY(product(s.tokens, d->q_stride, &q_count, err));
    TRY(product(s.capacity, s.head_dim, &d->head_stride, err));
    TRY(product(s.kv_heads, d->head_stride, &kv_count, err));
    TRY(length("q", q_len, q_count, err));
    TRY(length("k cache", k_len, kv_count, err));
    TRY(length("v cache", v_len, kv_count, err));
    TRY(length("attention context", context_len, q_count, err));
    return TKH_OK;
}

void cached_plan(const tkh_cached_shape &s, tkh_dtype dtype, Plan *plan) {
    plan->dtype = dtype;
    plan->query_heads = (int64_t)s.query_heads;
    plan->kv_heads = (int64_t)s.kv_heads;
    plan->head_dim = (int64_t)s.head_dim;
    plan->scale = 1.0f / std::sqrt((float)s.head_dim);
}

}  // namespace

extern "C" {

uint32_t tkh_attention_cached(tkh_context *ctx, const tkh_cached_shape *shape, tkh_dtype dtype,
                              const void *q, uint64_t q_len, const void *k, uint64_t k_len,
                              const void *v, uint64_t v_len, float *context,
                              uint64_t context_len, float *scores, uint64_t scores_len,
                              float *probabilities, uint64_t probabilities_len, tkh_error *err) {
    if (!valid_dtype(dtype)) return invalid("dtype", err);
    if (!shape) return invalid("shape", err);
    const tkh_cached_shape s = *shape;
    // src/cpu/attention.rs:218-251, in order.
    CachedDims d;
    TRY(check_cached(s, q_len, k_len, v_len, context_len, &d, err));
    if (scores) TRY(length("attention scores", scores_len, s.capacity, err));
    if (probabilities) TRY(length("attention probabilities", probabilities_len, s.capacity, err));
    if (s.head_dim > 512) return fail(err, TKH_UNSUPPORTED, "head_dim", 0, 0, 0, "head_dim above 512");
    if (!ctx) return invalid("context", err);
    Plan plan;
    cached_plan(s, dtype, &plan);
    plan.diag_mode = (scores || probabilities) ? 2 : 0;
    plan.scores = scores;
    plan.probs = probabilities;
    tkh::Problem p = make_problem(q, context, d.q_stride, s.offset, 0, d.end, s.tokens);
    add_segment(p, k, v, d.head_stride, s.head_dim, d.end, 0);
    plan.add(p);
    return run(ctx, plan, err);
}

}  // extern "C"

// ---------------------------------------------------------------- fixed scratch

namespace {

// The device memory of tkh_attention_cached_static: the status word (the first
// 256 bytes), then a workspace laid out as a context's (split-K partials of
// the prefill and generic kernels, then the decode kernel's completion flags
// and partials).  Each GPU the library runs on holds its own copy, at its own
// address, until the process ends.
constexpr size_t kStaticStatusBytes = 256;
__device__ __align__(256) uint8_t scratch[TKH_STATIC_SCRATCH_BYTES];

constexpr int kStaticMaxDevices = 64;
struct StaticDevice {
    bool ready = false;
    uint8_t *ptr = nullptr;  // this device's address of `scratch` (never the symbol itself)
    tkh_context ctx;         // planner settings and decode epoch; views into ptr, owns nothing
};
std::mutex g_static_mutex;
StaticDevice g_static[kStaticMaxDevices];

// Once per device, with that device current: the array's address, the
// planner settings, and a cleared array (status 0; decode flags 0, which no
// launch epoch equals).
uint32_t static_device(int device, hipStream_t stream, StaticDevice **out, tkh_error *err) {
    if (device < 0 || device >= kStaticMaxDevices) return invalid("device ordinal", err);
    StaticDevice &sd = g_static[device];
    if (!sd.ready) {
        int count = 0;
        if (hipGetDeviceCount(&count) != hipSuccess || device >= count)
            return fail(err, TKH_DEVICE, "device", 0, 0, 0, "HIP device %d is not available", device);
        HIP_TRY(hipSetDevice(device), "hipSetDevice");
        void *ptr = nullptr;
        HIP_TRY(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "scratch address");
        sd.ptr = static_cast<uint8_t *>(ptr);
        tkh_context &c = sd.ctx;
        c.device = device;
        c.synchronous = false;
        c.workspace = sd.ptr + kStaticStatusBytes;
        c.workspace_bytes = TKH_STATIC_SCRATCH_BYTES - kStaticStatusBytes;
        init_tuning(&c, device);
        HIP_TRY(tkh_launch_zero_u64(reinterpret_cast<uint64_t *>(sd.ptr),
                                    (int64_t)(TKH_STATIC_SCRATCH_BYTES / sizeof(uint64_t)), stream),
                "scratch clear");
        sd.ready = true;
    }
    *out = &sd;
    return TKH_OK;
}

}  // namespace

extern "C" {

uint32_t tkh_attention_cached_static(int device, void *stream, const tkh_cached_shape *shape,
                                     tkh_dtype dtype, const void *q, uint64_t q_len, const void *k,
                                     uint64_t k_len, const void *v, uint64_t v_len, float *context,
                                     uint64_t context_len, uint32_t *status, tkh_error *err) {
    if (!valid_dtype(dtype)) return invalid("dtype", err);
    if (!shape) return invalid("shape", err);
    const tkh_cached_shape s = *shape;
    CachedDims d;
    TRY(check_cached(s, q_len, k_len, v_len, context_len, &d, err));
    if (s.head_dim > 512) return fail(err, TKH_UNSUPPORTED, "head_dim", 0, 0, 0, "head_dim above 512");
    std::lock_guard<std::mutex> lock(g_static_mutex);
    StaticDevice *sd = nullptr;
    TRY(static_device(device, reinterpret_cast<hipStream_t>(stream), &sd, err));
    tkh_context &c = sd->ctx;
    c.stream = reinterpret_cast<hipStream_t>(stream);
    c.status_dev = status ? status : reinterpret_cast<uint32_t *>(sd->ptr);
    HIP_TRY(hipSetDevice(device), "hipSetDevice");
    if (!status) HIP_TRY(tkh_launch_fill_u32(c.status_dev, 0, c.stream), "status clear");
    Plan plan;
    cached_plan(s, dtype, &plan);
    tkh::Problem p = make_problem(q, context, d.q_stride, s.offset, 0, d.end, s.tokens);
    add_segment(p, k, v, d.head_stride, s.head_dim, d.end, 0);
    tkh_error launch_err{};
    const uint32_t rc = launch_all(&c, plan, &p, 1, &launch_err);
    if (rc == TKH_UNSUPPORTED && std::strcmp(launch_err.tensor, "workspace") == 0)
        return fail(err, TKH_UNSUPPORTED, "scratch", 0, launch_err.actual, launch_err.expected,
                    "the call needs %llu bytes of split partials, the fixed scratch has %llu for them",
                    (unsigned long long)launch_err.expected, (unsigned long long)launch_err.actual);
    if (rc != TKH_OK) {
        if (err) *err = launch_err;
        return rc;
    }
    if (status) return ok(err);
    uint32_t word = 0;
    hipError_t e = hipMemcpyAsync(&word, c.status_dev, sizeof word, hipMemcpyDeviceToHost, c.stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c.stream);
    if (e != hipSuccess) return device_error(e, "synchronize", err);
    return word ? status_error(word, err) : ok(err);
}

}  // extern "C"

// attention_cached for one new token whose producer (RMSNorm, rotary, rounding,
// cache append) runs inside the decode kernel (session decode steps).  The
// shape is validated as tkh_attention_cached validates it.
uint32_t tkh_host::attention_cached_fused(tkh_context *ctx, const tkh_cached_shape *shape,
                                          tkh_dtype dtype, const void *k, const void *v,
                                          float *context, const tkh::FusedDecode &fused,
                                          tkh_error *err) {
    if (!valid_dtype(dtype)) return invalid("dtype", err);
    if (!shape || !ctx) return invalid("shape", err);
    const tkh_cached_shape s = *shape;
    TRY(nonzero(s.tokens, "tokens", err));
    TRY(nonzero(s.query_heads, "query_heads", err));
    TRY(nonzero(s.kv_heads, "kv_heads", err));
    TRY(nonzero(s.head_dim, "head_dim", err));
    TRY(nonzero(s.capacity, "cache capacity", err));
    if (s.tokens != 1) return invalid("fused decode takes one token", err);
    if (s.query_heads % s.kv_heads != 0) return invalid("query_heads must be divisible by kv_heads", err);
    uint64_t end;
    TRY(add(s.offset, s.tokens, &end, err));
    if (end > s.capacity) return invalid("cache capacity exceeded", err);
    Plan plan;
    plan.dtype = dtype;
    plan.query_heads = s.query_heads;
    plan.kv_heads = s.kv_heads;
    plan.head_dim = s.head_dim;
    plan.scale = 1.0f / std::sqrt((float)s.head_dim);
    plan.fused = &fused;
    tkh::Problem p = make_problem(nullptr, context, s.query_heads * s.head_dim, s.offset, 0, end, 1);
    add_segment(p, k, v, s.capacity * s.head_dim, s.head_dim, end, 0);
    plan.add(p);
    return run(ctx, plan, err);
}

uint32_t tkh_host::span_attention_fused(tkh_context *ctx, const tkh_span_shape *shape,
                                        tkh_dtype dtype, const tkh_segment segments[3],
                                        float *context, const tkh::FusedDecode &fused,
                                        tkh_error *err) {
    if (!valid_dtype(dtype)) return invalid("dtype", err);
    if (!ctx || !shape || !segments) return invalid("shape", err);
    const tkh_span_shape s = *shape;
    if (s.queries != 1) return invalid("fused decode takes one token", err);
    TRY(nonzero(s.keys, "keys", err));
    TRY(nonzero(s.query_heads, "query_heads", err));
    TRY(nonzero(s.kv_heads, "kv_heads", err));
    TRY(nonzero(s.head_dim, "head_dim", err));
    if (s.query_heads % s.kv_heads != 0 || (s.has_window && s.window == 0) ||
        !std::isfinite(s.scale) || s.scale <= 0.0f)
        return invalid("segmented attention heads/window/scale", err);
    if (s.softcap != 0.0f && (!std::isfinite(s.softcap) || s.softcap < 0.0f))
        return invalid("attention score softcap", err);
    // The new key is the view's last (fused.new_key counts from the view's
    // first key, as its segments do), at the query's position; -1: no new
    // row to make (the view's keys are all stored; the Q rows alone are made).
    if ((fused.new_key != -1 && fused.new_key != (int64_t)(s.keys - 1)) ||
        s.query_start + 1 != s.key_start + s.keys)
        return invalid("fused decode: the new key must end the view", err);
    Plan plan;
    plan.dtype = dtype;
    plan.query_heads = s.query_heads;
    plan.kv_heads = s.kv_heads;
    plan.head_dim = s.head_dim;
    plan.has_window = s.has_window != 0;
    plan.window = (int64_t)s.window;
    plan.scale = s.scale;
    plan.softcap = s.softcap;
    plan.fused = &fused;
    tkh::Problem p = make_problem(nullptr, context, s.query_heads * s.head_dim, s.query_start,
                                  s.key_start, s.keys, 1);
    uint64_t logical = 0;
    for (int i = 0; i < 3; ++i) {
        const tkh_segment &seg = segments[i];
        if (seg.keys == 0) continue;
        add_segment(p, seg.k, seg.v, seg.head_stride, s.head_dim, seg.keys, logical);
        logical += seg.keys;
    }
    if (logical != s.keys) return invalid("attention segment keys", err);
    plan.add(p);
    return run(ctx, plan, err);
}

extern "C" {

uint32_t tkh_attention(tkh_context *ctx, const tkh_attention_shape *shape, tkh_dtype dtype,
                       const void *q, uint64_t q_len, const void *k, uint64_t k_len,
                       const void *v, uint64_t v_len, float *context, uint64_t context_len,
                       float *scores, uint64_t scores_len, float *probabilities,
                       uint64_t probabilities_len, tkh_error *err) {
    if (!valid_dtype(dtype)) return invalid("dtype", err);
    if (!shape) return invalid("shape", err);
    const tkh_attention_shape s = *shape;
    // src/cpu/attention.rs:102-134, in order.
    TRY(nonzero(s.tokens, "tokens", err));
    TRY(nonzero(s.query_heads, "query_heads", err));
    TRY(nonzero(s.kv_heads, "kv_heads", err));
    TRY(nonzero(s.head_dim, "head_dim", err));
    if (s.query_heads % s.kv_heads != 0) return invalid("query_heads must be divisible by kv_heads", err);
    uint64_t q_stride, kv_stride, q_count, kv_count, tmp, score_count;
    TRY(product(s.query_heads, s.head_dim, &q_stride, err));
    TRY(product(s.kv_heads, s.head_dim, &kv_stride, err));
    TRY(product(s.tokens, q_stride, &q_count, err));
    TRY(product(s.tokens, kv_stride, &kv_count, err));
    TRY(product(s.query_heads, s.tokens, &tmp, err));
    TRY(product(tmp, s.tokens, &score_count, err));
    TRY(length("q", q_len, q_count, err));
    TRY(length("k", k_len, kv_count, err));
    TRY(length("v", v_len, kv_count, err));
    TRY(length("attention context", context_len, q_count, err));
    if (scores) TRY(length("attention scores", scores_len, score_count, err));
    if (probabilities) TRY(length("attention probabilities", probabilities_len, score_count, err));
    if (s.head_dim > 512) return fail(err, TKH_UNSUPPORTED, "head_dim", 0, 0, 0, "head_dim above 512");
    if (!ctx) return invalid("context", err);
    Plan plan;
    plan.dtype = dtype;
    plan.query_heads = s.query_heads;
    plan.kv_heads = s.kv_heads;
    plan.head_dim = s.head_dim;
    plan.scale = 1.0f / std::sqrt((float)s.head_dim);
    plan.diag_mode = (scores || probabilities) ? 1 : 0;
    plan.scores = scores;
    plan.probs = probabilities;
    tkh::Problem p = make_problem(q, context, q_stride, 0, 0, s.tokens, s.tokens);
    add_segment(p, k, v, s.head_dim, kv_stride, s.tokens, 0);
    plan.add(p);
    return run(ctx, plan, err);
}

uint32_t tkh_window_attention(tkh_context *ctx, const tkh_window_shape *shape, tkh_dtype dtype,
                              const void *q, uint64_t q_len, const void *k, uint64_t k_len,
                              const void *v, uint64_t v_len, float *context,
                              uint64_t context_len, float *scores, uint64_t scores_len,
                              float *probabilities, uint64_t probabilities_len, tkh_error *err) {
    if (!valid_dtype(dtype)) return invalid("dtype", err);
    if (!shape) return invalid("shape", err);
    const tkh_window_shape s = *shape;
    // src/cpu/window_attention.rs:45-115, in order.
    TRY(nonzero(s.queries, "queries", err));
    TRY(nonzero(s.keys, "keys", err));
    TRY(nonzero(s.query_heads, "query_heads", err));
    TRY(nonzero(s.kv_heads, "kv_heads", err));
    TRY(nonzero(s.head_dim, "head_dim", err));
    if (s.keys > s.capacity || s.query_heads % s.kv_heads != 0)
        return invalid("attention capacity/head mapping", err);
    if ((s.has_window && s.window == 0) || !std::isfinite(s.scale) || s.scale <= 0.0f)
        return invalid("attention window/scale", err);
    if (s.softcap != 0.0f && (!std::isfinite(s.softcap) || s.softcap < 0.0f))
        return invalid("attention score softcap", err);
    uint64_t key_end, query_last;
    TRY(add(s.key_start, s.keys - 1, &key_end, err));
    TRY(add(s.query_start, s.queries - 1, &query_last, err));
    uint64_t query_stride, query_count, kv_stride, kv_count, tmp, scratch_count;
    TRY(product(s.query_heads, s.head_dim, &query_stride, err));
    TRY(product(s.queries, query_stride, &query_count, err));
    TRY(product(s.capacity, s.head_dim, &kv_stride, err));
    TRY(product(s.kv_heads, kv_stride, &kv_count, err));
    TRY(product(s.query_heads, s.queries, &tmp, err));
    TRY(product(tmp, s.keys, &scratch_count, err));
    TRY(length("attention query", q_len, query_count, err));
    TRY(length("attention key", k_len, kv_count, err));
    TRY(length("attention value", v_len, kv_count, err));
    TRY(length("attention context", context_len, query_count, err));
    if (scores) TRY(length("attention scores", scores_len, scratch_count, err));
    if (probabilities) TRY(length("attention probabilities", probabilities_len, scratch_count, err));
    for (uint64_t query = 0; query < s.queries; ++query) {
        uint64_t position = s.query_start + query;
        uint64_t first = first_visible(s.key_start, position, s.has_window, s.window);
        uint64_t last = std::min(key_end, position);
        if (first > last)
            return fail(err, TKH_FULLY_MASKED, nullptr, query, 0, 0, "softmax row %llu is entirely masked",
                        (unsigned long long)query);
    }
    if (s.head_dim > 512) return fail(err, TKH_UNSUPPORTED, "head_dim", 0, 0, 0, "head_dim above 512");
    if (!ctx) return invalid("context", err);
    Plan plan;
    plan.dtype = dtype;
    plan.query_heads = s.query_heads;
    plan.kv_heads = s.kv_heads;
    plan.head_dim = s.head_dim;
    plan.has_window = s.has_window != 0;
    plan.window = (int64_t)s.window;
    plan.scale = s.scale;
    plan.softcap = s.softcap;
    plan.diag_mode = (scores || probabilities) ? 1 : 0;
    plan.scores = scores;
    plan.probs = probabilities;
    tkh::Problem p = make_problem(q, context, query_stride, s.query_start, s.key_start, s.keys,
                                  s.queries);
    add_segment(p, k, v, kv_stride, s.head_dim, s.keys, 0);
    plan.add(p);
    return run(ctx, plan, err);
}

uint32_t tkh_span_attention(tkh_context *ctx, const tkh_span_shape *shape, tkh_dtype dtype,
                            const void *q, uint64_t q_len, const tkh_segment segments[3],
                            float *context, uint64_t context_len, float *scores,
                            uint64_t scores_len, float *probabilities, uint64_t probabilities_len,
                            tkh_error *err) {
    if (!valid_dtype(dtype)) return invalid("dtype", err);
    if (!shape || !segments) return invalid("shape", err);
    const tkh_span_shape s = *shape;
    // src/cpu/span_attention.rs:50-138, in order.
    TRY(nonzero(s.queries, "queries", err));
    TRY(nonzero(s.keys, "keys", err));
    TRY(nonzero(s.query_heads, "query_heads", err));
    TRY(nonzero(s.kv_heads, "kv_heads", err));
    TRY(nonzero(s.head_dim, "head_dim", err));
    if (s.query_heads % s.kv_heads != 0 || (s.has_window && s.window == 0) ||
        !std::isfinite(s.scale) || s.scale <= 0.0f)
        return invalid("segmented attention heads/window/scale", err);
    if (s.softcap != 0.0f && (!std::isfinite(s.softcap) || s.softcap < 0.0f))
        return invalid("attention score softcap", err);
    uint64_t key_end, query_last;
    TRY(add(s.key_start, s.keys - 1, &key_end, err));
    TRY(add(s.query_start, s.queries - 1, &query_last, err));
    uint64_t query_stride, query_count, tmp, scratch_count;
    TRY(product(s.query_heads, s.head_dim, &query_stride, err));
    TRY(product(s.queries, query_stride, &query_count, err));
    TRY(product(s.query_heads, s.queries, &tmp, err));
    TRY(product(tmp, s.keys, &scratch_count, err));
    TRY(length("attention query", q_len, query_count, err));
    TRY(length("attention context", context_len, query_count, err));
    if (scores) TRY(length("attention scores", scores_len, scratch_count, err));
    if (probabilities) TRY(length("attention probabilities", probabilities_len, scratch_count, err));
    uint64_t keys = 0;
    for (int i = 0; i < 3; ++i) {
        const tkh_segment &seg = segments[i];
        uint64_t rows, expected = 0;
        TRY(product(seg.keys, s.head_dim, &rows, err));
        if (seg.keys != 0) {
            if (seg.head_stride < rows) return invalid("attention segment heads overlap", err);
            uint64_t start;
            TRY(add(s.key_start, keys, &start, err));
            if (seg.key_start != start) return invalid("attention segment logical origin", err);
            uint64_t heads_part;
            TRY(product(s.kv_heads - 1, seg.head_stride, &heads_part, err));
            TRY(add(heads_part, rows, &expected, err));
        }
        TRY(length("attention segment key", seg.k_len, expected, err));
        TRY(length("attention segment value", seg.v_len, expected, err));
        TRY(add(keys, seg.keys, &keys, err));
    }
    TRY(length("attention segment keys", keys, s.keys, err));
    for (uint64_t query = 0; query < s.queries; ++query) {
        uint64_t position = s.query_start + query;
        uint64_t first = first_visible(s.key_start, position, s.has_window, s.window);
        uint64_t last = std::min(key_end, position);
        if (first > last)
            return fail(err, TKH_FULLY_MASKED, nullptr, query, 0, 0, "softmax row %llu is entirely masked",
                        (unsigned long long)query);
    }
    if (s.head_dim > 512) return fail(err, TKH_UNSUPPORTED, "head_dim", 0, 0, 0, "head_dim above 512");
    if (!ctx) return invalid("context", err);
    Plan plan;
    plan.dtype = dtype;
    plan.query_heads = s.query_heads;
    plan.kv_heads = s.kv_heads;
    plan.head_dim = s.head_dim;
    plan.has_window = s.has_window != 0;
    plan.window = (int64_t)s.window;
    plan.scale = s.scale;
    plan.softcap = s.softcap;
    plan.diag_mode = (scores || probabilities) ? 1 : 0;
    plan.scores = scores;
    plan.probs = probabilities;
    tkh::Problem p = make_problem(q, context, query_stride, s.query_start, s.key_start, s.keys,
                                  s.queries);
    uint64_t logical = 0;
    for (int i = 0; i < 3; ++i) {
        const tkh_segment &seg = segments[i];
        if (seg.keys == 0) continue;
        add_segment(p, seg.k, seg.v, seg.head_stride, s.head_dim, seg.keys, logical);
        logical += seg.keys;
    }
    plan.add(p);
    return run(ctx, plan, err);
}

uint32_t tkh_project_greedy(tkh_context *ctx, uint64_t rows, uint64_t hidden, uint64_t vocab,
                            const float *context, uint64_t context_len, const float *weights,
                            uint64_t weights_len, float *logits, uint64_t logits_len,
                            uint32_t *tokens, uint64_t tokens_len, tkh_error *err) {
    // src/cpu/mod.rs:192-201 in order, then src/sampling.rs:6-9.
    TRY(nonzero(rows, "tokens", err));
    TRY(nonzero(hidden, "in_features", err));
    TRY(nonzero(vocab, "out_features", err));
    uint64_t n;
    TRY(product(rows, hidden, &n, err));
    TRY(length("input", context_len, n, err));
    TRY(product(vocab, hidden, &n, err));
    TRY(length("weights", weights_len, n, err));
    TRY(product(rows, vocab, &n, err));
    if (logits) TRY(length("output", logits_len, n, err));
    TRY(length("tokens", tokens_len, rows, err));
    if (vocab - 1 > (uint64_t)UINT32_MAX) return invalid("vocabulary IDs must fit u32", err);
    if (!ctx) return invalid("context", err);
    if (!context || !weights || !tokens) return invalid("projection buffers", err);
    const int64_t per = tkh_project_vocab_per_block();
    const uint64_t vblocks = (vocab + per - 1) / per;
    if (vblocks > (uint64_t)INT32_MAX || rows > (uint64_t)UINT32_MAX || rows / 16 >= 65535)
        return fail(err, TKH_UNSUPPORTED, "projection", 0, 0, 0, "projection grid too large");
    uint64_t need;
    TRY(product(rows, vblocks * sizeof(uint64_t), &need, err));
    if (need > split_region_bytes(ctx))
        return fail(err, TKH_UNSUPPORTED, "workspace", 0, need, split_region_bytes(ctx),
                    "projection needs %llu workspace bytes, context has %zu for it",
                    (unsigned long long)need, split_region_bytes(ctx));
    tkh::ProjectParams p{};
    p.context = context;
    p.weights = weights;
    p.logits = logits;
    p.pairs = reinterpret_cast<uint64_t *>(ctx->workspace);
    p.tokens = tokens;
    p.rows = (int64_t)rows;
    p.hidden = (int64_t)hidden;
    p.vocab = (int64_t)vocab;
    p.vblocks = (int32_t)vblocks;
    p.status = ctx->status_dev;
    HIP_TRY(hipSetDevice(ctx->device), "hipSetDevice");
    hipEvent_t *ev = nullptr;
    if (ctx->profiling) TRY(profile_slot(ctx, &ev, false, err));
    HIP_TRY(tkh_launch_project(&p, ctx->stream, ev ? ev[0] : nullptr, ev ? ev[1] : nullptr),
            "projection launch");
    return after_launch(ctx, err);
}

uint32_t tkh_logit_softcap(tkh_context *ctx, float *logits, uint64_t len, float cap,
                           tkh_error *err) {
    // src/cpu/softcap.rs:17-23
    TRY(nonzero(len, "logit softcap width", err));
    if (!std::isfinite(cap) || cap <= 0.0f) return invalid("logit softcap", err);
    if (!ctx) return invalid("context", err);
    HIP_TRY(hipSetDevice(ctx->device), "hipSetDevice");
    HIP_TRY(tkh_launch_softcap(logits, (int64_t)len, cap, ctx->status_dev, ctx->stream), "softcap");
    return after_launch(ctx, err);
}

namespace {
uint32_t batch_common(tkh_context *ctx, uint64_t batch, uint64_t tokens, uint64_t query_heads,
                      uint64_t kv_heads, uint64_t head_dim, tkh_dtype dtype, float scale,
                      tkh_error *err) {
    if (!valid_dtype(dtype)) return invalid("dtype", err);
    TRY(nonzero(batch, "batch", err));
    TRY(nonzero(tokens, "tokens", err));
    TRY(nonzero(query_heads, "query_heads", err));
    TRY(nonzero(kv_heads, "kv_heads", err));
    TRY(nonzero(head_dim, "head_dim", err));
    if (query_heads % kv_heads != 0) return invalid("query_heads must be divisible by kv_heads", err);
    if (!std::isfinite(scale) || scale <= 0.0f) return invalid("attention scale", err);
    if (head_dim > 512) return fail(err, TKH_UNSUPPORTED, "head_dim", 0, 0, 0, "head_dim above 512");
    if (!ctx) return invalid("context", err);
    return TKH_OK;
}
}  // namespace

uint32_t tkh_decode_batch(tkh_context *ctx, uint64_t batch, uint64_t query_heads,
                          uint64_t kv_heads, uint64_t head_dim, tkh_dtype dtype, const void *q,
                          const void *k_base, const void *v_base, const uint64_t *offsets,
                          const uint64_t *head_strides, const uint64_t *lengths, float scale,
                          float *context, tkh_error *err) {
    TRY(batch_common(ctx, batch, 1, query_heads, kv_heads, head_dim, dtype, scale, err));
    if (!offsets || !head_strides || !lengths) return invalid("batch descriptors", err);
    Plan plan;
    plan.dtype = dtype;
    plan.query_heads = query_heads;
    plan.kv_heads = kv_heads;
    plan.head_dim = head_dim;
    plan.scale = scale;
    const int64_t es = esize(dtype);
    const int64_t row = (int64_t)(query_heads * head_dim);
    for (uint64_t b = 0; b < batch; ++b) {
        if (lengths[b] == 0) return fail(err, TKH_ZERO_DIMENSION, "lengths", b, 0, 0, "session %llu has no keys", (unsigned long long)b);
        if (head_strides[b] < lengths[b] * head_dim) return invalid("attention segment heads overlap", err);
    }
    plan.store = ctx->batch_store;
    plan.capacity = kSlotProblems;
    for (uint64_t b0 = 0; b0 < batch; b0 += kSlotProblems) {
        plan.count = 0;
        for (uint64_t b = b0; b < std::min<uint64_t>(batch, b0 + kSlotProblems); ++b) {
            tkh::Problem p = make_problem((const uint8_t *)q + b * row * es, context + b * row, row,
                                          (int64_t)lengths[b] - 1, 0, (int64_t)lengths[b], 1);
            add_segment(p, (const uint8_t *)k_base + offsets[b] * es,
                        (const uint8_t *)v_base + offsets[b] * es, (int64_t)head_strides[b],
                        (int64_t)head_dim, (int64_t)lengths[b], 0);
            plan.add(p);
        }
        TRY(launch_all(ctx, plan, plan.store, plan.count, err));
    }
    return after_launch(ctx, err);
}

uint32_t tkh_prefill_batch(tkh_context *ctx, uint64_t batch, uint64_t tokens,
                           uint64_t query_heads, uint64_t kv_heads, uint64_t head_dim,
                           tkh_dtype dtype, const void *q, const void *k_base,
                           const void *v_base, const uint64_t *offsets,
                           const uint64_t *head_strides, const uint64_t *positions, float scale,
                           float *context, tkh_error *err) {
    TRY(batch_common(ctx, batch, tokens, query_heads, kv_heads, head_dim, dtype, scale, err));
    if (!offsets || !head_strides || !positions) return invalid("batch descriptors", err);
    Plan plan;
    plan.dtype = dtype;
    plan.query_heads = query_heads;
    plan.kv_heads = kv_heads;
    plan.head_dim = head_dim;
    plan.scale = scale;
    const int64_t es = esize(dtype);
    const int64_t row = (int64_t)(query_heads * head_dim);
    for (uint64_t b = 0; b < batch; ++b) {
        const uint64_t keys = positions[b] + tokens;
        if (head_strides[b] < keys * head_dim) return invalid("attention segment heads overlap", err);
    }
    plan.store = ctx->batch_store;
    plan.capacity = kSlotProblems;
    for (uint64_t b0 = 0; b0 < batch; b0 += kSlotProblems) {
        plan.count = 0;
        for (uint64_t b = b0; b < std::min<uint64_t>(batch, b0 + kSlotProblems); ++b) {
            const int64_t keys = (int64_t)(positions[b] + tokens);
            tkh::Problem p = make_problem((const uint8_t *)q + b * tokens * row * es,
                                          context + b * tokens * row, row, (int64_t)positions[b], 0,
                                          keys, (int64_t)tokens);
            add_segment(p, (const uint8_t *)k_base + offsets[b] * es,
                        (const uint8_t *)v_base + offsets[b] * es, (int64_t)head_strides[b],
                        (int64_t)head_dim, keys, 0);
            plan.add(p);
        }
        TRY(launch_all(ctx, plan, plan.store, plan.count, err));
    }
    return after_launch(ctx, err);
}

}  // extern "C"

// ---------------------------------------------------------------- KV owners


namespace {

std::atomic<uint64_t> g_next_owner{1};

// capacity::KvOwner::at_capacity (src/capacity.rs:49-80) with copies and no guards.
uint32_t owner_bytes(uint64_t heads, uint64_t head_dim, uint64_t capacity, bool has_window,
                     uint64_t window, tkh_dtype storage, uint64_t copies, uint64_t *total,
                     uint64_t *per_array, tkh_error *err) {
    TRY(nonzero(capacity, "KV capacity", err));
    TRY(nonzero(heads, "KV heads", err));
    TRY(nonzero(head_dim, "KV head dimension", err));
    TRY(nonzero(copies, "KV physical owners", err));
    uint64_t retained = capacity;
    if (has_window) {
        TRY(nonzero(window, "KV window", err));
        retained = std::min(capacity, window);
    }
    uint64_t elements, bytes, pair;
    TRY(product(heads, retained, &elements, err));
    TRY(product(elements, head_dim, &elements, err));
    TRY(product(elements, (uint64_t)esize(storage), &bytes, err));
    if (bytes > (uint64_t)INT64_MAX) return fail(err, TKH_SIZE_OVERFLOW, nullptr, 0, 0, 0, "tensor size arithmetic overflow");
    TRY(product(bytes, 2, &pair, err));
    TRY(product(pair, copies, total, err));
    if (per_array) *per_array = bytes;
    return TKH_OK;
}

// WindowKvCache::admit_tokens (src/model/window_cache.rs:214-237).
uint32_t admit_tokens(const tkh_kv *kv, uint64_t tokens, uint64_t *elements, tkh_error *err) {
    TRY(nonzero(tokens, "KV new tokens", err));
    uint64_t after;
    TRY(add(kv->offset, tokens, &after, err));
    uint64_t limit = kv->has_window ? kv->max_positions : std::min(kv->capacity, kv->max_positions);
    if (after > limit)
        return fail(err, TKH_CAPACITY, "KV cache", kv->offset, limit, after,
                    "offset %llu plus %llu tokens exceeds limit %llu",
                    (unsigned long long)kv->offset, (unsigned long long)tokens,
                    (unsigned long long)limit);
    if (kv->generation == UINT64_MAX) return fail(err, TKH_SIZE_OVERFLOW, nullptr, 0, 0, 0, "KV generation exhausted");
    uint64_t e;
    TRY(product(kv->heads, tokens, &e, err));
    TRY(product(e, kv->dims, &e, err));
    *elements = e;
    return TKH_OK;
}

// WindowKvCache::validate (src/model/window_cache.rs:239-254).
uint32_t validate_frame(const tkh_kv *kv, const tkh_kv_frame *f, tkh_error *err) {
    if (f->owner != kv->owner || f->generation != kv->generation || f->offset != kv->offset)
        return fail(err, TKH_INVALID_CONFIG, "KV frame", 0, 0, 0, "stale or foreign KV proposal");
    uint64_t elements;
    return admit_tokens(kv, f->tokens, &elements, err);
}

// window_rows (src/model/window_rows.rs:24-88).
uint64_t view_start(uint64_t offset, bool has_window, uint64_t window) {
    if (!has_window) return 0;
    return offset >= window - 1 ? offset - (window - 1) : 0;
}
void old_spans(uint64_t capacity, uint64_t offset, bool has_window, uint64_t window, uint64_t out[6]) {
    uint64_t start = view_start(offset, has_window, window);
    uint64_t old = offset - start;
    uint64_t slot = start % capacity;
    uint64_t first = std::min(old, capacity - slot);
    out[0] = start; out[1] = slot; out[2] = first;
    out[3] = start + first; out[4] = 0; out[5] = old - first;
}
void copy_runs(uint64_t capacity, uint64_t offset, uint64_t tokens, bool sliding, uint64_t out[6]) {
    uint64_t first_new = sliding ? (tokens > capacity ? tokens - capacity : 0) : 0;
    uint64_t slot = sliding ? (offset % capacity + first_new % capacity) % capacity : offset;
    uint64_t count = tokens - first_new;
    uint64_t first = std::min(count, capacity - slot);
    out[0] = first_new; out[1] = slot; out[2] = first;
    out[3] = first_new + first; out[4] = 0; out[5] = count - first;
}

}  // namespace

extern "C" {

uint32_t tkh_kv_planned_bytes(uint64_t heads, uint64_t head_dim, uint64_t capacity,
                              uint32_t has_window, uint64_t window, tkh_dtype storage,
                              uint64_t copies, uint64_t *total_bytes, tkh_error *err) {
    if (!total_bytes) return invalid("total_bytes", err);
    if (!valid_dtype(storage)) return invalid("dtype", err);
    TRY(owner_bytes(heads, head_dim, capacity, has_window != 0, window, storage, copies,
                    total_bytes, nullptr, err));
    return ok(err);
}

uint32_t tkh_kv_create(tkh_context *ctx, uint64_t heads, uint64_t dims, uint64_t capacity,
                       uint64_t max_positions, uint32_t has_window, uint64_t window,
                       tkh_dtype storage, tkh_kv **out, tkh_error *err) {
    if (!ctx) return invalid("context", err);
    if (!out) return invalid("kv output", err);
    if (!valid_dtype(storage)) return invalid("dtype", err);
    *out = nullptr;
    // WindowKvCache::planned_bytes (src/model/window_cache.rs:62-97).
    TRY(nonzero(heads, "KV heads", err));
    TRY(nonzero(dims, "KV head width", err));
    TRY(nonzero(capacity, "KV capacity", err));
    TRY(nonzero(max_positions, "KV maximum positions", err));
    if (capacity > max_positions || (has_window && (window == 0 || window != capacity)))
        return fail(err, TKH_INVALID_CONFIG, "KV capacity/window", 0, 0, 0, "invalid KV capacity/window");
    uint64_t total, per_array;
    TRY(owner_bytes(heads, dims, capacity, has_window != 0, window, storage, 1, &total, &per_array, err));
    HIP_TRY(hipSetDevice(ctx->device), "hipSetDevice");
    auto *kv = new tkh_kv();
    kv->ctx = ctx;
    kv->device = ctx->device;
    kv->heads = heads;
    kv->dims = dims;
    kv->capacity = capacity;
    kv->max_positions = max_positions;
    kv->has_window = has_window != 0;
    kv->window = window;
    kv->storage = storage;
    hipError_t e = hipMalloc(&kv->k, per_array);
    if (e == hipSuccess) e = hipMalloc(&kv->v, per_array);
    if (e == hipSuccess) e = hipMemsetAsync(kv->k, 0, per_array, ctx->stream);
    if (e == hipSuccess) e = hipMemsetAsync(kv->v, 0, per_array, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        tkh_kv_destroy(kv);
        return device_error(e, "KV allocation", err);
    }
    kv->allocated_bytes = total;
    kv->owner = g_next_owner.fetch_add(1);
    *out = kv;
    return ok(err);
}

void tkh_kv_destroy(tkh_kv *kv) {
    if (!kv) return;
    // The owning context is not touched: it may already be destroyed.  hipFree
    // waits for work still using the memory.
    hipSetDevice(kv->device);
    if (kv->k) hipFree(kv->k);
    if (kv->v) hipFree(kv->v);
    delete kv;
}

uint32_t tkh_kv_info_get(const tkh_kv *kv, tkh_kv_info *info) {
    if (!kv || !info) return TKH_INVALID_PARAMETER;
    info->heads = kv->heads;
    info->dims = kv->dims;
    info->capacity = kv->capacity;
    info->max_positions = kv->max_positions;
    info->window = kv->window;
    info->offset = kv->offset;
    info->generation = kv->generation;
    info->owner = kv->owner;
    info->has_window = kv->has_window ? 1 : 0;
    info->storage = kv->storage;
    info->k = kv->k;
    info->v = kv->v;
    info->allocated_bytes = kv->allocated_bytes;
    return TKH_OK;
}

uint32_t tkh_kv_append(tkh_kv *kv, uint64_t offset, uint64_t tokens, tkh_dtype src_dtype,
                       const void *k, const void *v, tkh_error *err) {
    if (!kv) return invalid("kv", err);
    if (!valid_dtype(src_dtype)) return invalid("dtype", err);
    if (kv->has_window) return fail(err, TKH_INVALID_CONFIG, "KV cache", 0, 0, 0, "append needs a full-retention cache; use prepare/commit");
    TRY(nonzero(tokens, "KV new tokens", err));
    uint64_t end;
    TRY(add(offset, tokens, &end, err));
    if (end > kv->capacity)
        return fail(err, TKH_CAPACITY, "KV cache", offset, kv->capacity, end, "cache capacity exceeded");
    if (src_dtype != TKH_F32 && src_dtype != kv->storage) return invalid("append source dtype", err);
    tkh_context *ctx = kv->ctx;
    HIP_TRY(hipSetDevice(ctx->device), "hipSetDevice");
    HIP_TRY(tkh_launch_kv_append((int)src_dtype, (int)kv->storage, k, v, kv->k, kv->v,
                                 (int64_t)tokens, (int)kv->heads, (int)kv->dims,
                                 (int64_t)kv->capacity, (int64_t)offset, ctx->status_dev,
                                 ctx->stream),
            "KV append");
    return after_launch(ctx, err);
}

uint32_t tkh_kv_prepare(const tkh_kv *kv, const void *k, uint64_t k_len, const void *v,
                        uint64_t v_len, uint64_t tokens, tkh_kv_frame *frame, tkh_error *err) {
    if (!kv || !frame) return invalid("kv", err);
    uint64_t elements;
    TRY(admit_tokens(kv, tokens, &elements, err));
    TRY(length("new KV keys", k_len, elements, err));
    TRY(length("new KV values", v_len, elements, err));
    tkh_context *ctx = kv->ctx;
    HIP_TRY(hipSetDevice(ctx->device), "hipSetDevice");
    HIP_TRY(tkh_launch_check_finite((int)kv->storage, k, v, (int64_t)elements, ctx->status_dev,
                                    ctx->stream),
            "KV prepare");
    uint32_t rc = after_launch(ctx, err);
    if (rc != TKH_OK) return rc;
    frame->k = k;
    frame->v = v;
    frame->owner = kv->owner;
    frame->generation = kv->generation;
    frame->offset = kv->offset;
    frame->tokens = tokens;
    return ok(err);
}

uint32_t tkh_kv_view(const tkh_kv *kv, const tkh_kv_frame *frame, uint64_t query_heads,
                     float scale, tkh_segment segments[3], tkh_span_shape *shape,
                     tkh_error *err) {
    if (!kv || !frame || !segments || !shape) return invalid("kv", err);
    TRY(validate_frame(kv, frame, err));
    const uint64_t es = (uint64_t)esize(kv->storage);
    const uint64_t stride = kv->capacity * kv->dims;
    uint64_t spans[6];
    old_spans(kv->capacity, kv->offset, kv->has_window, kv->window, spans);
    for (int i = 0; i < 2; ++i) {
        uint64_t position = spans[3 * i], slot = spans[3 * i + 1], rows = spans[3 * i + 2];
        tkh_segment &s = segments[i];
        if (rows == 0) {
            s = tkh_segment{nullptr, 0, nullptr, 0, 0, 0, kv->offset};
            continue;
        }
        uint64_t begin = slot * kv->dims;
        uint64_t len = (kv->heads - 1) * stride + rows * kv->dims;
        s.k = (const uint8_t *)kv->k + begin * es;
        s.v = (const uint8_t *)kv->v + begin * es;
        s.k_len = len;
        s.v_len = len;
        s.keys = rows;
        s.head_stride = stride;
        s.key_start = position;
    }
    uint64_t len = kv->heads * frame->tokens * kv->dims;
    segments[2] = tkh_segment{frame->k, len, frame->v, len, frame->tokens,
                              frame->tokens * kv->dims, kv->offset};
    uint64_t start = view_start(kv->offset, kv->has_window, kv->window);
    // KvView::attention_shape (src/model/window_cache.rs:392-406).
    shape->queries = frame->tokens;
    shape->keys = kv->offset + frame->tokens - start;
    shape->query_heads = query_heads;
    shape->kv_heads = kv->heads;
    shape->head_dim = kv->dims;
    shape->query_start = kv->offset;
    shape->key_start = start;
    shape->has_window = kv->has_window ? 1 : 0;
    shape->window = kv->window;
    shape->scale = scale;
    shape->softcap = 0.0f;
    return ok(err);
}

}  // extern "C"

// commit_batch with an optional device gate: the copies of a gated commit run
// only while the status word is clean, and the last one records
// `committed_value` in `committed` (queued sessions read it back after a
// failure to learn which chunks reached the rings).
uint32_t tkh_host::commit_frames(tkh_kv *const *kvs, const tkh_kv_frame *frames, uint64_t count,
                                 const uint32_t *gate, uint64_t *committed,
                                 uint64_t committed_value, tkh_error *err) {
    if (count && (!kvs || !frames)) return invalid("kv batch", err);
    for (uint64_t i = 0; i < count; ++i) {
        if (!kvs[i]) return invalid("kv", err);
        TRY(validate_frame(kvs[i], &frames[i], err));
    }
    for (uint64_t i = 0; i < count; ++i)
        for (uint64_t j = i + 1; j < count; ++j)
            if (kvs[i] == kvs[j])
                return fail(err, TKH_INVALID_CONFIG, "KV frame", 0, 0, 0, "duplicate KV owner in commit");
    // No fallible arithmetic remains: copy only the final min(tokens, W) rows.
    // Consecutive rings of one context and stream go out in one launch (up to
    // COPY_BATCH_MAX each); the last launch records the committed length.
    // A ring's offset and generation advance once its copy is queued.
    tkh::CopyBatch batch{};
    tkh_context *batch_ctx = nullptr;
    std::pair<tkh_kv *, uint64_t> pending[tkh::COPY_BATCH_MAX];
    auto flush = [&](bool last) -> uint32_t {
        if (batch.count == 0) return TKH_OK;
        batch.gate = gate;
        batch.committed = last ? committed : nullptr;
        batch.committed_value = committed_value;
        HIP_TRY(hipSetDevice(batch_ctx->device), "hipSetDevice");
        HIP_TRY(tkh_launch_copy_batch(&batch, batch_ctx->stream), "KV commit");
        for (int j = 0; j < batch.count; ++j) {
            pending[j].first->offset += pending[j].second;
            pending[j].first->generation += 1;
        }
        batch.count = 0;
        return TKH_OK;
    };
    for (uint64_t i = 0; i < count; ++i) {
        tkh_kv *kv = kvs[i];
        const tkh_kv_frame &f = frames[i];
        if (batch.count == tkh::COPY_BATCH_MAX || (batch_ctx && (kv->ctx->device != batch_ctx->device ||
                                                                  kv->ctx->stream != batch_ctx->stream)))
            TRY(flush(false));
        batch_ctx = kv->ctx;
        uint64_t runs[6];
        copy_runs(kv->capacity, kv->offset, f.tokens, kv->has_window, runs);
        tkh::CopyRunsEntry &e = batch.e[batch.count++];
        e.src_k = static_cast<const uint8_t *>(f.k);
        e.src_v = static_cast<const uint8_t *>(f.v);
        e.dst_k = static_cast<uint8_t *>(kv->k);
        e.dst_v = static_cast<uint8_t *>(kv->v);
        e.tokens = (int64_t)f.tokens;
        e.row_bytes = (int64_t)(kv->dims * esize(kv->storage));
        e.capacity = (int64_t)kv->capacity;
        for (int j = 0; j < 6; ++j) e.runs[j] = (int64_t)runs[j];
        e.heads = (int32_t)kv->heads;
        pending[batch.count - 1] = {kv, f.tokens};
    }
    TRY(flush(true));
    for (uint64_t i = 0; i < count; ++i)
        if (kvs[i]->ctx->synchronous) HIP_TRY(hipStreamSynchronize(kvs[i]->ctx->stream), "KV commit");
    return ok(err);
}

extern "C" {

uint32_t tkh_kv_commit_batch(tkh_kv *const *kvs, const tkh_kv_frame *frames, uint64_t count,
                             tkh_error *err) {
    return commit_frames(kvs, frames, count, nullptr, nullptr, 0, err);
}

uint32_t tkh_kv_reset_batch(tkh_kv *const *kvs, uint64_t count, tkh_error *err) {
    if (count && !kvs) return invalid("kv batch", err);
    for (uint64_t i = 0; i < count; ++i) {
        if (!kvs[i]) return invalid("kv", err);
        if (kvs[i]->generation == UINT64_MAX)
            return fail(err, TKH_INVALID_CONFIG, "KV cache", 0, 0, 0, "KV reset generation exhausted");
    }
    for (uint64_t i = 0; i < count; ++i) {
        kvs[i]->offset = 0;
        kvs[i]->generation += 1;
    }
    return ok(err);
}

}  // extern "C"
