"""Benchmark of the session attention path on one MI355X.

The line's workload is the metric's decode configuration, configs[2] of
64 independent sessions at Qwen3 shape (16 query heads, 8 KV
heads, head_dim 128), f16 KV, lengths drawn U[512, 8192], one query token per
session per step (one batched decode launch).  A step is one such launch over
all 64 sessions; inputs are resident in HBM before timing.  `value` is decode
attention GB/s over the timed steps (algorithmic bytes: visible keys x
2*Hkv*D*2 + Q/O bytes), `roofline` the decode kernel's rate from HIP events on
its stream, with HBM traffic from the committed rocprofv3 counter passes.

Also on the line: `prefill_roofline` on configs[4] (32 sessions x (4096 cached
+ 128 new) with Q/K rotated at theta 500000, the MFMA-bound prefill), the CPU
baselines of both on BASELINE.md's subsets (the oracle on one host core),
configs[0] (FP32 session, GPU and CPU
tokens/s, and the device o-projection + greedy pick), configs[1] (Qwen3
session job), configs[3] (Gemma local/global session), decode at 8192 keys for
one and 16 sessions, and the host CPU model.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_HBM_GBS = 8000.0
PEAK_BF16_TFLOPS = 2500.0
# Idle seconds before each workload after the first: the chip's clock depends on
# the heat the previous workload left (configs[4]'s kernel measured 375 us right
# after configs[2] and 349-352 us on its own), so each workload starts cool.
SETTLE_S = 3.0


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--no-north-star", action="store_true",
                    help="run only the headline configs[2] and configs[4]")
    ap.add_argument("--only", choices=["c1", "c2", "c3", "c4", "c5", "d8k", "d8kb", "copy"], default=None,
                    help="run a single workload (for profiling); `copy` runs a plain 1 GiB "
                         "device copy that calibrates the FETCH_SIZE/WRITE_SIZE counters")
    return ap.parse_args()


# ---------------------------------------------------------------- inputs

def qk_producer(torch, x, weight, positions, theta):
    """Per-head RMSNorm (FP32, eps 1e-6) then split-half RoPE; x: [T, H, D] fp32."""
    d = x.shape[-1]
    rms = torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6)
    x = x * rms * weight
    half = d // 2
    freq = theta ** (-(2.0 * torch.arange(half, device=x.device, dtype=torch.float64)) / d)
    ang = positions.to(torch.float64)[:, None] * freq[None, :]
    sin = torch.sin(ang).float()[:, None, :]
    cos = torch.cos(ang).float()[:, None, :]
    a, b = x[..., :half], x[..., half:]
    return torch.cat([a * cos - b * sin, b * cos + a * sin], dim=-1)


class C2:
    """Qwen3-shaped single session driven through the native session
    (tkh_session_evaluate): per prefill chunk and layer, the producer (per-head
    RMSNorm, rotary 1e6, bf16 rounding, K/V append) and the attention kernel; per
    decode step, one decode launch with the producer folded in."""
    hq, hkv, d = 16, 8, 128
    prefill, chunk, decode = 2048, 128, 256

    def __init__(self, torch, ops, sessmod, ctx, seed=1234):
        self.torch, self.ops, self.ctx, self.sessmod = torch, ops, ctx, sessmod
        g = torch.Generator(device="cuda").manual_seed(seed)
        total = self.prefill + self.decode
        self.total = total
        # Projections (the producer's inputs) resident in HBM, N(0, 1); norm weights N(1, 0.02).
        self.q_proj = torch.randn(total, self.hq, self.d, generator=g, device="cuda")
        self.k_proj = torch.randn(total, self.hkv, self.d, generator=g, device="cuda")
        self.v_proj = torch.randn(total, self.hkv, self.d, generator=g, device="cuda")
        self.wq = 1.0 + 0.02 * torch.randn(self.d, generator=g, device="cuda")
        self.wk = 1.0 + 0.02 * torch.randn(self.d, generator=g, device="cuda")
        self.out = torch.zeros(total, self.hq * self.d, dtype=torch.float32, device="cuda")
        self.session = sessmod.Session(ctx, sessmod.Options(
            capacity=total, prefill_chunk_size=self.chunk, vocab_size=151936, layers=1,
            query_heads=self.hq, kv_heads=self.hkv, head_dim=self.d, storage="bf16",
            norm_epsilon=1e-6, theta=1e6))
        self.io = [sessmod.LayerIo(self.q_proj, self.k_proj, self.v_proj, self.out, self.wq,
                                   self.wk)]
        self.tokens = torch.randint(0, 151936, (total,), generator=torch.Generator().manual_seed(seed)).tolist()

    def run_prefill(self):
        self.session.reset()
        self.session.set_tokens(self.tokens[:self.prefill])
        self.session.evaluate(self.io)

    def run_decode(self):
        self.session.append(self.tokens[self.prefill:])
        self.session.evaluate(self.io, chunk_limit=1)

    def prefill_flops(self):
        pairs = sum(sum(start + t + 1 for t in range(self.chunk))
                    for start in range(0, self.prefill, self.chunk))
        return 4.0 * self.hq * self.d * pairs

    def decode_bytes_per_step(self, keys):
        return keys * 2 * self.hkv * self.d * 2 + self.hq * self.d * 2 + self.hq * self.d * 4

    def decode_bytes(self):
        return sum(self.decode_bytes_per_step(p + 1) for p in range(self.prefill, self.total))


def time_region(torch, fn, steps, warmup):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for _ in range(steps):
        fn()
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return start.elapsed_time(end) / 1e3, wall


def timed_profiled(torch, ctx, fn, steps):
    """time_region with the kernels' dispatch-recorded durations taken on the
    timed launches themselves, for workloads whose step is one long launch
    (the events cost microseconds against hundreds)."""
    torch.cuda.synchronize()
    ctx.profile(True)
    s, wall = time_region(torch, fn, steps, 0)
    prof = ctx.profile_read()
    ctx.profile(False)
    ctx.synchronize()
    return s, prof


def profiled(torch, ctx, fn, steps):
    """The attention kernels' dispatch-recorded durations over `steps` calls of
    fn, in a pass separate from the timed region (the events add work)."""
    torch.cuda.synchronize()
    ctx.profile(True)
    for _ in range(steps):
        fn()
    prof = ctx.profile_read()
    ctx.profile(False)
    ctx.synchronize()
    return prof


def bench_c2(torch, ops, sessmod, ctx, steps, warmup):
    w = C2(torch, ops, sessmod, ctx)
    log("c2: qwen3 16/8/128 bf16, prefill 2048 in 128-token chunks + 256 decode steps "
        "(native session: producer + attention per chunk)")

    def step():
        w.run_prefill()
        w.run_decode()
        w.session.synchronize()
    job_s, job_wall = time_region(torch, step, steps, warmup)
    # Phase timing (same calls, no event recording: the phase rates).
    pre_s = dec_s = 0.0
    for _ in range(steps):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        w.run_prefill()
        w.session.synchronize()
        pre_s += time.perf_counter() - t0
        t0 = time.perf_counter()
        w.run_decode()
        w.session.synchronize()
        dec_s += time.perf_counter() - t0
    # Kernel durations: a second pass with the attention kernels'
    # dispatch-recorded events (which add host and queue work of their own).
    pre_prof = {"attention_ms": 0.0, "combine_ms": 0.0, "launches": 0}
    dec_prof = dict(pre_prof)
    for _ in range(steps):
        ctx.profile(True)
        w.run_prefill()
        w.session.synchronize()
        p = ctx.profile_read()
        ctx.profile(True)
        w.run_decode()
        w.session.synchronize()
        d = ctx.profile_read()
        for acc, src in ((pre_prof, p), (dec_prof, d)):
            for k in acc:
                acc[k] += src[k]
    ctx.profile(False)
    flops = w.prefill_flops()
    dbytes = w.decode_bytes()
    res = {
        "job_ms_per_step": job_s / steps * 1e3,
        "tokens_per_s": (w.total * steps) / job_s,
        "prefill_ms": pre_s / steps * 1e3,
        "prefill_tflops": flops * steps / pre_s / 1e12,
        "prefill_kernel_tflops": flops * steps / ((pre_prof["attention_ms"] + pre_prof["combine_ms"]) / 1e3) / 1e12,
        "prefill_kernel_us": pre_prof["attention_ms"] / max(1, pre_prof["launches"]) * 1e3,
        "prefill_merge_us": pre_prof["combine_ms"] / max(1, pre_prof["launches"]) * 1e3,
        "decode_ms": dec_s / steps * 1e3,
        "decode_gbs": dbytes * steps / dec_s / 1e9,
        "decode_us_per_token": dec_s / steps / w.decode * 1e6,
        "decode_kernel_us": dec_prof["attention_ms"] / dec_prof["launches"] * 1e3,
        "decode_combine_us": dec_prof["combine_ms"] / dec_prof["launches"] * 1e3,
        "decode_kernel_gbs": dbytes * steps / (dec_prof["attention_ms"] / 1e3) / 1e9,
        "decode_launches": dec_prof["launches"],
        "decode_bytes_per_step_avg": dbytes / w.decode,
    }
    return res, w


def bench_decode_batch(torch, ops, ctx, steps, warmup, *, batch, lmin, lmax, dtype, seed=7):
    """batched decode, per-session L ~ U[lmin, lmax], one new token per step."""
    hq, hkv, d = 16, 8, 128
    g = torch.Generator().manual_seed(seed)
    lengths = torch.randint(lmin, lmax + 1, (batch,), generator=g).tolist()
    caps = [l + steps + warmup + 8 for l in lengths]
    offsets, acc = [], 0
    for c in caps:
        offsets.append(acc)
        acc += hkv * c * d
    gd = torch.Generator(device="cuda").manual_seed(seed)
    # One scale per (session, KV head), applied to that head's K and V rows and
    # to the query heads of its group.
    scales = torch.empty(batch, hkv, device="cuda").uniform_(0.5, 2.0, generator=gd)
    kpool = torch.empty(acc, dtype=dtype, device="cuda")
    vpool = torch.empty(acc, dtype=dtype, device="cuda")
    for b in range(batch):
        n = hkv * caps[b] * d
        for pool in (kpool, vpool):
            x = torch.randn(hkv, caps[b] * d, generator=gd, device="cuda") * scales[b][:, None]
            pool[offsets[b]:offsets[b] + n] = x.reshape(-1).to(dtype)
    q = (torch.randn(batch, hq, d, generator=gd, device="cuda") *
         scales.repeat_interleave(hq // hkv, dim=1)[:, :, None]).to(dtype)
    out = torch.zeros(batch * hq * d, dtype=torch.float32, device="cuda")
    head_strides = [c * d for c in caps]
    scale = 1.0 / math.sqrt(d)
    cur = list(lengths)

    def step():
        for b in range(batch):
            cur[b] += 1
        ops.decode_batch(ctx, q, kpool, vpool, offsets, head_strides, cur, out, query_heads=hq,
                         kv_heads=hkv, head_dim=d, scale=scale)

    bytes_of = lambda ls: sum(l * 2 * hkv * d * kpool.element_size() for l in ls) + \
        batch * hq * d * (kpool.element_size() + 4)
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    start_lengths = list(cur)
    s, _ = time_region(torch, step, steps, 0)
    total_bytes = sum(bytes_of([l + i + 1 for l in start_lengths]) for i in range(steps))
    # Kernel durations over the same lengths, in a pass of their own.
    cur[:] = start_lengths
    prof = profiled(torch, ctx, step, steps)
    res = {
        "batch": batch, "sum_keys": sum(start_lengths), "dtype": str(dtype).replace("torch.", ""),
        "ms_per_step": s / steps * 1e3,
        "gbs": total_bytes / s / 1e9,
        "kernel_us": prof["attention_ms"] / max(1, prof["launches"]) * 1e3,
        "combine_us": prof["combine_ms"] / max(1, prof["launches"]) * 1e3,
        "kernel_gbs": total_bytes / (prof["attention_ms"] / 1e3) / 1e9,
        "kernel_frac_hbm": total_bytes / (prof["attention_ms"] / 1e3) / 1e9 / PEAK_HBM_GBS,
        "bytes_per_step": total_bytes / steps,
    }
    state = {"q": q, "k": kpool, "v": vpool, "offsets": offsets, "caps": caps,
             "lengths": start_lengths, "hq": hq, "hkv": hkv, "d": d, "bytes_of": bytes_of}
    return res, state


def bench_prefill_batch(torch, ops, ctx, steps, warmup, *, batch=32, cached=4096, tokens=128,
                        seed=11, dtype=None):
    """32 sessions x (4096 cached + 128 new causal), Llama-3-8B heads, bf16.
    Inputs (untimed): per session N(0, 1) FP32 Q/K/V projections, 5% of K rows x8,
    through the library's producer with split-half rotary theta 500000 (the cached
    positions into the session's cache, then the new ones: Q for the batch, K/V
    appended)."""
    hq, hkv, d, theta = 32, 8, 128, 5e5
    gd = torch.Generator(device="cuda").manual_seed(seed)
    cap = cached + tokens
    per = hkv * cap * d
    dtype = dtype or torch.bfloat16
    k = torch.empty(batch * per, dtype=dtype, device="cuda")
    v = torch.empty_like(k)
    q = torch.empty(batch, tokens, hq, d, dtype=dtype, device="cuda")
    q_prefix = torch.zeros(cached, hq, d, device="cuda")  # the cached positions' Q is not used
    q_scratch = torch.empty(cached, hq, d, dtype=dtype, device="cuda")
    for b in range(batch):
        kp = torch.randn(cap, hkv, d, generator=gd, device="cuda")
        mask = torch.rand(cap, hkv, 1, generator=gd, device="cuda") < 0.05
        kp = torch.where(mask, kp * 8.0, kp)
        vp = torch.randn(cap, hkv, d, generator=gd, device="cuda")
        qp = torch.randn(tokens, hq, d, generator=gd, device="cuda")
        kb, vb = k[b * per:(b + 1) * per], v[b * per:(b + 1) * per]
        ops.produce_qkv(ctx, ops.ProducerShape(cached, hq, hkv, d, 0, theta=theta), q_prefix,
                        kp[:cached], vp[:cached], None, None, q_scratch, kb, vb, cap * d)
        ops.produce_qkv(ctx, ops.ProducerShape(tokens, hq, hkv, d, cached, theta=theta), qp,
                        kp[cached:], vp[cached:], None, None, q[b], kb[cached * d:], vb[cached * d:],
                        cap * d)
    ctx.synchronize()
    del q_prefix, q_scratch
    out = torch.zeros(batch * tokens * hq * d, dtype=torch.float32, device="cuda")
    offsets = [b * per for b in range(batch)]
    strides = [cap * d] * batch
    positions = [cached] * batch

    def step():
        ops.prefill_batch(ctx, q, k, v, offsets, strides, positions, out, tokens=tokens,
                          query_heads=hq, kv_heads=hkv, head_dim=d, scale=1.0 / math.sqrt(d))

    pairs = batch * sum(cached + t + 1 for t in range(tokens))
    flops = 4.0 * hq * d * pairs
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    # One launch per step: its duration is recorded on the timed launches (a
    # separate pass after them would run on a chip their heat has slowed).
    s, prof = timed_profiled(torch, ctx, step, steps)
    kernel_s = (prof["attention_ms"] + prof["combine_ms"]) / 1e3
    res = {
        "sessions": batch, "cached": cached, "new": tokens,
        "ms_per_step": s / steps * 1e3,
        "tflops": flops * steps / s / 1e12,
        "kernel_us": prof["attention_ms"] / max(1, prof["launches"]) * 1e3,
        "merge_us": prof["combine_ms"] / max(1, prof["launches"]) * 1e3,
        "kernel_tflops": flops * steps / kernel_s / 1e12,
        "kernel_frac_mfma": flops * steps / kernel_s / 1e12 / PEAK_BF16_TFLOPS,
        "gflop_per_step": flops / 1e9,
    }
    state = {"q": q, "k": k, "v": v, "per": per, "cap": cap, "cached": cached, "tokens": tokens,
             "hq": hq, "hkv": hkv, "d": d, "flops_per_session": flops / batch}
    return res, state


def bench_c4(torch, ops, sessmod, ctx, steps, warmup, softcap=50.0, seed=5):
    """Gemma3-style 6-layer group (5 sliding W=1024 + 1 global), 8/4/256 bf16,
    scale 1/16, score softcap 50, through the native session: prefill 4096 in 128-token
    chunks, then 128 single-token decode steps."""
    hq, hkv, d, W, prompt, dec, layers = 8, 4, 256, 1024, 4096, 128, 6
    total = prompt + dec
    g = torch.Generator(device="cuda").manual_seed(seed)
    io, outs = [], []
    for _ in range(layers):
        out = torch.zeros(total, hq * d, dtype=torch.float32, device="cuda")
        io.append(sessmod.LayerIo(torch.randn(total, hq, d, generator=g, device="cuda"),
                                  torch.randn(total, hkv, d, generator=g, device="cuda"),
                                  torch.randn(total, hkv, d, generator=g, device="cuda"), out))
        outs.append(out)
    windows = [W] * 5 + [0]
    sess = sessmod.Session(ctx, sessmod.Options(
        capacity=total, prefill_chunk_size=128, vocab_size=262144, layers=layers, query_heads=hq,
        kv_heads=hkv, head_dim=d, storage="bf16", score_scale=1.0 / 16.0, softcap=softcap,
        theta=1e6, layer_windows=windows))
    tokens = [1] * total

    def prefill():
        sess.reset()
        sess.set_tokens(tokens[:prompt])
        sess.evaluate(io)
        sess.synchronize()

    def decode():
        sess.append(tokens[prompt:])
        sess.evaluate(io, chunk_limit=1)
        sess.synchronize()

    for _ in range(warmup):
        prefill()
        decode()
    pre_s = dec_s = 0.0
    for _ in range(steps):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        prefill()
        pre_s += time.perf_counter() - t0
        t0 = time.perf_counter()
        decode()
        dec_s += time.perf_counter() - t0
    pairs_global = sum(p + 1 for p in range(prompt))
    pairs_sliding = sum(min(p + 1, W) for p in range(prompt))
    flops = 4.0 * hq * d * (pairs_global + 5 * pairs_sliding)
    per_key = 2 * hkv * d * 2
    dbytes = sum(per_key * ((p + 1) + 5 * min(p + 1, W)) + layers * hq * d * 6
                 for p in range(prompt, total))
    return {
        "layers": "5 sliding (W=1024) + 1 global", "softcap": softcap,
        "prefill_ms": pre_s / steps * 1e3,
        "prefill_tflops": flops * steps / pre_s / 1e12,
        "prefill_gflop": flops / 1e9,
        "decode_ms": dec_s / steps * 1e3,
        "decode_us_per_token": dec_s / steps / dec * 1e6,
        "decode_gbs": dbytes * steps / dec_s / 1e9,
        "tokens_per_s": total * steps / (pre_s + dec_s),
    }


def copy_calibration(torch, nbytes=1 << 30, reps=3):
    """A plain device copy of known size: its FETCH_SIZE/WRITE_SIZE per dispatch
    (rocprofv3 --pmc) against nbytes gives the counters' scale factor."""
    src = torch.ones(nbytes // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    t = []
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        dst.copy_(src)
        b.record()
        torch.cuda.synchronize()
        t.append(a.elapsed_time(b) / 1e3)
    return {"copy_bytes_read": nbytes, "copy_bytes_written": nbytes,
            "copy_gbs": 2 * nbytes / min(t) / 1e9}


def measured_traffic(key):
    """HBM bytes per launch of a workload's dominant kernel, from the committed
    rocprofv3 --pmc summary (FETCH_SIZE and WRITE_SIZE passes of this script,
    each scaled by what the counter reads for a plain copy of known size)."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            entry = json.load(f).get(key)
    except (OSError, ValueError):
        return None, None
    if not entry:
        return None, None
    return entry.get("bytes_per_launch"), entry


def host_info():
    """The host CPU the baselines ran on: model name and visible CPUs."""
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": model, "cpus_visible": os.cpu_count()}


def cpu_baseline_decode_batch(state, seconds=10.0, steps=2):
    """The reference's CPU path for configs[2] on BASELINE.md's subset (2 decode steps
    of all 64 sessions), restated by the oracle on one thread: attention_cached per
    session (FP32 dot, FP64 softmax) over FP32 copies of the stored f16 K/V, repeated
    in passes until `seconds` have been measured.  Reported as GB/s of the same
    algorithmic bytes the GPU line counts (f16 K/V bytes + Q/O)."""
    import numpy as np

    import oracle

    oracle.lib()
    hq, hkv, d = state["hq"], state["hkv"], state["d"]
    kh = state["k"].float().cpu().numpy()
    vh = state["v"].float().cpu().numpy()
    qh = state["q"].float().cpu().numpy()
    offsets, lengths = state["offsets"], state["lengths"]
    nbytes_pass = sum(state["bytes_of"]([l + i + 1 for l in lengths]) for i in range(steps))
    passes, t0 = 0, time.perf_counter()
    while True:
        for i in range(steps):
            for b, l0 in enumerate(lengths):
                L = l0 + i + 1
                cap = state["caps"][b]  # rows per head of the session's cache; [0, L) are keys
                kb = kh[offsets[b]:offsets[b] + hkv * cap * d]
                vb = vh[offsets[b]:offsets[b] + hkv * cap * d]
                oracle.attention_cached(qh[b].reshape(-1), kb, vb, 1, hq, hkv, d, cap, L - 1)
        passes += 1
        dt = time.perf_counter() - t0
        if dt >= seconds:
            break
    return {
        "value": nbytes_pass * passes / dt / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
        "sample": f"configs[2] subset: {steps} decode steps of all {len(lengths)} sessions "
                  f"(sum of lengths {sum(lengths)}), oracle attention_cached (FP32 dot, FP64 "
                  f"softmax) on FP32 copies of the f16 K/V, x {passes} passes, {dt:.2f} s; bytes "
                  f"counted as the GPU's f16 bytes",
        "seconds": dt,
    }


def cpu_threads():
    """Host threads for the all-core CPU baselines: the job's CPU share
    (OMP_NUM_THREADS when the launcher sets it, else the affinity mask), at most 16."""
    n = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or len(os.sched_getaffinity(0))
    return max(1, min(16, n))


def cpu_baseline_decode_batch_threads(state, seconds=8.0, steps=2):
    """cpu_baseline_decode_batch with the same calls spread over cpu_threads() host
    threads (one session's attention_cached per task; the oracle's C calls run
    without the interpreter lock)."""
    import numpy as np  # noqa: F401
    from concurrent.futures import ThreadPoolExecutor

    import oracle

    oracle.lib()
    hq, hkv, d = state["hq"], state["hkv"], state["d"]
    kh = state["k"].float().cpu().numpy()
    vh = state["v"].float().cpu().numpy()
    qh = state["q"].float().cpu().numpy()
    offsets, lengths = state["offsets"], state["lengths"]
    nbytes_pass = sum(state["bytes_of"]([l + i + 1 for l in lengths]) for i in range(steps))
    tasks = [(i, b) for i in range(steps) for b in range(len(lengths))]

    def one(task):
        i, b = task
        cap = state["caps"][b]
        kb = kh[offsets[b]:offsets[b] + hkv * cap * d]
        vb = vh[offsets[b]:offsets[b] + hkv * cap * d]
        oracle.attention_cached(qh[b].reshape(-1), kb, vb, 1, hq, hkv, d, cap, lengths[b] + i)

    n = cpu_threads()
    passes, t0 = 0, time.perf_counter()
    with ThreadPoolExecutor(max_workers=n) as pool:
        while True:
            list(pool.map(one, tasks))
            passes += 1
            dt = time.perf_counter() - t0
            if dt >= seconds:
                break
    return {
        "value": nbytes_pass * passes / dt / 1e9, "unit": "GB/s", "cores": n, "kind": "port",
        "sample": f"the single-thread line's subset and calls ({steps} decode steps of all "
                  f"{len(lengths)} sessions), one session per task over {n} host threads, x {passes} "
                  f"passes, {dt:.2f} s",
        "seconds": dt,
    }


def cpu_baseline_prefill_batch(state, seconds=10.0):
    """The reference's CPU path for configs[4] on BASELINE.md's subset (1 of 32
    sessions: 128 new rows over 4224 keys, all 32 heads), restated by the oracle on
    one thread, in passes until `seconds` have been measured; TFLOP/s of the same
    algorithmic FLOPs (4 Hq D per visible pair) as the GPU line."""
    import oracle

    oracle.lib()
    hq, hkv, d, per, cap = state["hq"], state["hkv"], state["d"], state["per"], state["cap"]
    kb = state["k"][:per].float().cpu().numpy()
    vb = state["v"][:per].float().cpu().numpy()
    qb = state["q"][0].float().cpu().numpy().reshape(-1)
    passes, t0 = 0, time.perf_counter()
    while True:
        oracle.attention_cached(qb, kb, vb, state["tokens"], hq, hkv, d, cap, state["cached"])
        passes += 1
        dt = time.perf_counter() - t0
        if dt >= seconds:
            break
    return {
        "value": state["flops_per_session"] * passes / dt / 1e12, "unit": "TFLOP/s", "cores": 1,
        "kind": "port",
        "sample": f"configs[4] subset: session 0 of 32 (128 new rows x {hq} heads over {cap} keys), "
                  f"oracle attention_cached on FP32 copies of the bf16 K/V, x {passes} passes, "
                  f"{dt:.2f} s",
        "seconds": dt,
    }


def cpu_baseline_prefill_batch_threads(state, seconds=8.0, sessions=4):
    """cpu_baseline_prefill_batch over cpu_threads() host threads: the first
    `sessions` sessions, each split by KV head (its query-head group against its K/V
    rows) into one oracle call per task."""
    from concurrent.futures import ThreadPoolExecutor

    import oracle

    oracle.lib()
    hq, hkv, d, per, cap = state["hq"], state["hkv"], state["d"], state["per"], state["cap"]
    T, G = state["tokens"], hq // hkv
    work = []
    for b in range(sessions):
        kb = state["k"][b * per:(b + 1) * per].float().cpu().numpy().reshape(hkv, cap * d)
        vb = state["v"][b * per:(b + 1) * per].float().cpu().numpy().reshape(hkv, cap * d)
        qb = state["q"][b].float().cpu().numpy().reshape(T, hq, d)
        for h in range(hkv):
            work.append((qb[:, h * G:(h + 1) * G, :].copy().reshape(-1), kb[h].copy(), vb[h].copy()))

    def one(item):
        q, k, v = item
        oracle.attention_cached(q, k, v, T, G, 1, d, cap, state["cached"])

    n = cpu_threads()
    passes, t0 = 0, time.perf_counter()
    with ThreadPoolExecutor(max_workers=n) as pool:
        while True:
            list(pool.map(one, work))
            passes += 1
            dt = time.perf_counter() - t0
            if dt >= seconds:
                break
    return {
        "value": state["flops_per_session"] * sessions * passes / dt / 1e12, "unit": "TFLOP/s",
        "cores": n, "kind": "port",
        "sample": f"configs[4] subset: sessions 0-{sessions - 1} of 32, one (session, KV head) per "
                  f"task over {n} host threads, oracle attention_cached on FP32 copies of the bf16 "
                  f"K/V, x {passes} passes, {dt:.2f} s",
        "seconds": dt,
    }


def bench_c1(torch, ops, sessmod, ctx, steps, warmup, seed=3):
    """Qwen2.5-0.5B-shaped attention on the FP32 path (14/2/64, rotary 1e6,
    scale 1/8), one session: a 128-token prompt then 32 decode steps, through the
    native session (producer + attention per chunk or step).  One step = that whole
    job.  The greedy token of every row over a seeded 896 x 151936 projection runs
    after the timed region, on the device, and is reported separately.  The CPU line
    runs the oracle's rotary + attention for the same job on one thread."""
    import numpy as np

    import oracle

    hq, hkv, d, prompt, dec = 14, 2, 64, 128, 32
    total = prompt + dec
    g = torch.Generator(device="cuda").manual_seed(seed)
    qp = torch.randn(total, hq, d, generator=g, device="cuda")
    kp = torch.randn(total, hkv, d, generator=g, device="cuda")
    vp = torch.randn(total, hkv, d, generator=g, device="cuda")
    out = torch.zeros(total, hq * d, dtype=torch.float32, device="cuda")
    sess = sessmod.Session(ctx, sessmod.Options(
        capacity=total, prefill_chunk_size=128, vocab_size=151936, layers=1, query_heads=hq,
        kv_heads=hkv, head_dim=d, storage="f32", theta=1e6))
    io = [sessmod.LayerIo(qp, kp, vp, out)]

    def step():
        sess.reset()
        sess.set_tokens([1] * prompt)
        sess.evaluate(io)
        sess.append([2] * dec)
        sess.evaluate(io, chunk_limit=1)
        sess.synchronize()

    s, _ = time_region(torch, step, steps, warmup)
    # The step after: o-projection + greedy pick of every row (untimed above).
    w = torch.randn(151936, hq * d, generator=g, device="cuda")
    tokens = torch.zeros(total, dtype=torch.int32, device="cuda")
    ops.project_greedy(ctx, out, w, tokens)
    torch.cuda.synchronize()
    t_rows, _ = time_region(torch, lambda: ops.project_greedy(ctx, out, w, tokens), 5, 1)
    one = torch.zeros(1, dtype=torch.int32, device="cuda")
    t_one, _ = time_region(torch, lambda: ops.project_greedy(ctx, out[-1:], w, one), 20, 2)
    # CPU: the oracle's producer (rotary) and attention for the same job, one thread.
    oracle.lib()
    qh, kh, vh = qp.cpu().numpy(), kp.cpu().numpy(), vp.cpu().numpy()
    passes, t0 = 0, time.perf_counter()
    while True:
        q = oracle.rotary(qh.reshape(-1), total, hq, d, 0, 1e6)
        k = oracle.rotary(kh.reshape(-1), total, hkv, d, 0, 1e6).reshape(total, hkv, d)
        kc = np.zeros((hkv, total, d), np.float32)
        vc = np.zeros((hkv, total, d), np.float32)
        kc[:, :prompt] = k[:prompt].transpose(1, 0, 2)
        vc[:, :prompt] = vh[:prompt].transpose(1, 0, 2)
        oracle.attention_cached(q[:prompt * hq * d], kc, vc, prompt, hq, hkv, d, total, 0)
        for p in range(prompt, total):
            kc[:, p] = k[p]
            vc[:, p] = vh[p]
            oracle.attention_cached(q[p * hq * d:(p + 1) * hq * d], kc, vc, 1, hq, hkv, d, total, p)
        passes += 1
        dt = time.perf_counter() - t0
        if dt >= 2.0:
            break
    sess.close()
    return {
        "tokens_per_s": total * steps / s,
        "ms_per_job": s / steps * 1e3,
        "projection_greedy_us_160_rows": t_rows / 5 * 1e6,
        "projection_greedy_us_1_row": t_one / 20 * 1e6,
        "projection_1_row_gbs": 151936 * hq * d * 4 / (t_one / 20) / 1e9,
        "cpu_baseline": {"value": total * passes / dt, "unit": "tokens/s", "cores": 1, "kind": "port",
                         "sample": f"the same job (rotary + 128-token prefill + 32 decode steps) x "
                                   f"{passes} passes, {dt:.2f} s"},
    }


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus must be 1",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    import torch

    from toklet_amd import ops
    from toklet_amd import session as sessmod

    assert torch.cuda.is_available(), "bench.py needs the MI355X"
    if args.only == "copy":
        print(json.dumps(copy_calibration(torch)))
        return
    ctx = ops.Context(0, synchronous=False)
    run = lambda name: args.only in (None, name) and (args.only == name or not args.no_north_star
                                                      or name in ("c3", "c5"))
    result, states = {}, {}
    started = [False]

    def settle():
        if started[0]:
            torch.cuda.synchronize()
            time.sleep(SETTLE_S)
        started[0] = True

    if run("c3"):
        settle()
        c3, states["c3"] = bench_decode_batch(torch, ops, ctx, args.steps, args.warmup, batch=64,
                                              lmin=512, lmax=8192, dtype=torch.float16)
        log("c3 (configs[2] batched decode): " + json.dumps(c3))
        result["c3"] = c3
    if run("c5"):
        settle()
        c5, states["c5"] = bench_prefill_batch(torch, ops, ctx, 10, 2)
        log("c5 (configs[4] batched prefill): " + json.dumps(c5))
        result["c5"] = c5
    if run("c1"):
        settle()
        c1 = bench_c1(torch, ops, sessmod, ctx, 10, 2)
        log("c1 (configs[0] FP32 session): " + json.dumps(c1))
        result["c1"] = c1
    if run("c2"):
        settle()
        c2, _ = bench_c2(torch, ops, sessmod, ctx, 5, 1)
        log("c2 (configs[1] session job): " + json.dumps(c2))
        result["c2"] = c2
    if run("c4"):
        settle()
        c4 = bench_c4(torch, ops, sessmod, ctx, 2, 1)
        log("c4 (configs[3] Gemma session): " + json.dumps(c4))
        result["c4"] = c4
    if run("d8k"):
        settle()
        d8k, _ = bench_decode_batch(torch, ops, ctx, 50, 5, batch=1, lmin=8192, lmax=8192,
                                    dtype=torch.bfloat16)
        log("single-session decode at 8192: " + json.dumps(d8k))
        result["decode_8k"] = d8k
    if run("d8kb"):
        settle()
        d8kb, _ = bench_decode_batch(torch, ops, ctx, 20, 3, batch=16, lmin=8192, lmax=8192,
                                     dtype=torch.bfloat16)
        log("sustained decode at 8192, 16 sessions: " + json.dumps(d8kb))
        result["decode_8k_batch16"] = d8kb
    if args.only is not None and args.only not in ("c3",):
        print(json.dumps(result))
        return

    c3 = result["c3"]
    traffic, traffic_entry = measured_traffic("c3_decode")
    line = {
        "metric": "decode attn GB/s (% HBM peak); prefill attn TFLOPS (% MFMA peak)",
        "value": round(c3["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(c3["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded N(0,1) Q/K/V times a U[0.5, 2] scale per (session, KV head))",
        "config": {"workload": "configs[2] batched decode: 64 independent sessions, L ~ U[512, 8192] "
                               "(seeded), one query token per session per step, Qwen3 16q/8kv/d128, "
                               "f16 KV, FP32 accumulation",
                   "sessions": 64, "query_heads": 16, "kv_heads": 8, "head_dim": 128,
                   "sum_keys_first_step": c3["sum_keys"]},
        "decode_frac_hbm": round(c3["gbs"] / PEAK_HBM_GBS, 5),
        "roofline": {
            "bound": "hbm",
            "kernel": "attn_decode<f16, D=128, 2 rows, 4 keys per lane> (configs[2], one launch "
                      "per step)",
            "achieved": round(c3["kernel_gbs"], 2),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(c3["kernel_gbs"] / PEAK_HBM_GBS, 5),
            "traffic": traffic,
            "traffic_source": (traffic_entry or {}).get("source"),
            "avg_kernel_us": round(c3["kernel_us"], 3),
            "algorithmic_bytes_per_launch": round(c3["bytes_per_step"]),
            "timing": "hipExtLaunchKernelGGL start/stop events on the library's stream",
        },
    }
    if "c5" in result:
        c5 = result["c5"]
        ptraffic, ptraffic_entry = measured_traffic("c5_prefill")
        line["prefill_tflops"] = round(c5["tflops"], 2)
        line["prefill_roofline"] = {
            "bound": "mfma",
            "kernel": "attn_prefill<bf16, D=128, 8 waves> (configs[4]: 32 sessions x (4096 cached "
                      "+ 128 new), 32q/8kv/d128, Q/K rotary theta 5e5)",
            "achieved": round(c5["kernel_tflops"], 2),
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(c5["kernel_frac_mfma"], 5),
            "traffic": ptraffic,
            "traffic_source": (ptraffic_entry or {}).get("source"),
            "avg_kernel_us": round(c5["kernel_us"], 3),
            "algorithmic_flops_per_launch": round(c5["gflop_per_step"] * 1e9),
            "timing": "hipExtLaunchKernelGGL start/stop events on the library's stream, recorded "
                      "on the timed launches",
        }
    line["configs"] = {k: result[k] for k in ("c1", "c2", "c4", "decode_8k", "decode_8k_batch16", "c5")
                       if k in result}
    line["configs"]["c3"] = c3
    line["host"] = host_info()
    if not args.no_cpu:
        log("cpu baselines: the oracle on one host core, then on the job's host threads")
        line["cpu_baseline"] = cpu_baseline_decode_batch(states["c3"])
        line["cpu_baseline_all_cores"] = cpu_baseline_decode_batch_threads(states["c3"])
        if "c5" in states:
            line["prefill_cpu_baseline"] = cpu_baseline_prefill_batch(states["c5"])
            line["prefill_cpu_baseline_all_cores"] = cpu_baseline_prefill_batch_threads(states["c5"])
    print(json.dumps(line))


if __name__ == "__main__":
    main()
