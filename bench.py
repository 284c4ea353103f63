"""Benchmark of the session attention path on one MI355X.

Default workload (Qwen3-shaped single session):
16 query heads, 8 KV heads, head_dim 128, bf16 KV (and Q stored as bf16),
per-head RMSNorm (weights N(1, 0.02)) and RoPE (theta 1e6) on seeded N(0,1)
Q/K, causal prefill of 2048 tokens in 128-token chunks, then 256 decode
steps at context 2049..2304.  One step = that whole job for one layer:
16 x (KV append + chunk attention) + 256 x (KV append + decode attention),
every call through the C ABI.  Inputs are resident in HBM before timing.

Reported (one JSON line): decode attention GB/s over the decode phase as
`value` (algorithmic bytes: visible keys x 2*Hkv*D*2 + Q/O bytes), prefill
attention TFLOPS (4*Hq*D per visible (query, key) pair), the roofline of the
decode attention kernel from HIP events on its stream, the north-star
configurations (single-session and 16-session decode at 8192 keys,
configs[2] batched decode, configs[3] Gemma local/global, configs[4] batched
prefill), and the CPU oracle timed on this host as the baseline.
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


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--no-north-star", action="store_true", help="skip configs[2]/[4]")
    ap.add_argument("--only", choices=["c2", "c3", "c4", "c5", "d8k", "d8kb", "copy"], default=None,
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
    return {
        "batch": batch, "sum_keys": sum(start_lengths), "dtype": str(dtype).replace("torch.", ""),
        "ms_per_step": s / steps * 1e3,
        "gbs": total_bytes / s / 1e9,
        "kernel_us": prof["attention_ms"] / max(1, prof["launches"]) * 1e3,
        "combine_us": prof["combine_ms"] / max(1, prof["launches"]) * 1e3,
        "kernel_gbs": total_bytes / (prof["attention_ms"] / 1e3) / 1e9,
        "kernel_frac_hbm": total_bytes / (prof["attention_ms"] / 1e3) / 1e9 / PEAK_HBM_GBS,
    }


def bench_prefill_batch(torch, ops, ctx, steps, warmup, *, batch=32, cached=4096, tokens=128,
                        seed=11, dtype=None):
    """32 sessions x (4096 cached + 128 new causal), Llama-3-8B heads, bf16."""
    hq, hkv, d = 32, 8, 128
    gd = torch.Generator(device="cuda").manual_seed(seed)
    cap = cached + tokens
    per = hkv * cap * d
    k = torch.randn(batch, hkv, cap, d, generator=gd, device="cuda")
    mask = torch.rand(batch, hkv, cap, 1, generator=gd, device="cuda") < 0.05
    dtype = dtype or torch.bfloat16
    k = torch.where(mask, k * 8.0, k).to(dtype).reshape(-1)
    v = torch.randn(batch * per, generator=gd, device="cuda").to(dtype)
    q = torch.randn(batch, tokens, hq, d, generator=gd, device="cuda").to(dtype)
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
    s, _ = time_region(torch, step, steps, 0)
    prof = profiled(torch, ctx, step, steps)
    kernel_s = (prof["attention_ms"] + prof["combine_ms"]) / 1e3
    return {
        "sessions": batch, "cached": cached, "new": tokens,
        "ms_per_step": s / steps * 1e3,
        "tflops": flops * steps / s / 1e12,
        "kernel_us": prof["attention_ms"] / max(1, prof["launches"]) * 1e3,
        "merge_us": prof["combine_ms"] / max(1, prof["launches"]) * 1e3,
        "kernel_tflops": flops * steps / kernel_s / 1e12,
        "kernel_frac_mfma": flops * steps / kernel_s / 1e12 / PEAK_BF16_TFLOPS,
        "gflop_per_step": flops / 1e9,
    }


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


def cpu_baseline(w, torch, seconds=10.0, max_passes=20):
    """The reference's CPU path for configs[1]'s decode steps, restated by the oracle
    (single thread): per step rmsnorm + rotary of the new Q/K rows (FP64), append into
    FP32 head-major caches (the reference's CPU storage), attention_cached (FP32 dot,
    FP64 softmax).  All 256 steps after an untimed 2048-token prefix, run as repeated
    passes (each pass rewrites the same rows with the same values) until at least
    `seconds` of CPU time have been measured, so the sample is about 10 s of work."""
    import numpy as np

    import oracle

    oracle.lib()
    hq, hkv, d, cap, pre = w.hq, w.hkv, w.d, w.total, w.prefill
    qp = w.q_proj.cpu().numpy()
    kp = w.k_proj.cpu().numpy()
    vp = w.v_proj.cpu().numpy()
    wq = w.wq.cpu().numpy()
    wk = w.wk.cpu().numpy()

    def produce(x, wt, t0, n, heads):
        y = oracle.rmsnorm(x[t0:t0 + n].reshape(-1), wt, n * heads, d, 1e-6)
        return oracle.rotary(y, n, heads, d, t0, 1e6).reshape(n, heads, d)

    kc = np.zeros((hkv, cap, d), np.float32)
    vc = np.zeros((hkv, cap, d), np.float32)
    kc[:, :pre] = produce(kp, wk, 0, pre, hkv).transpose(1, 0, 2)
    vc[:, :pre] = vp[:pre].transpose(1, 0, 2)
    positions = list(range(pre, cap))
    passes = 0
    t0 = time.perf_counter()
    while True:
        for p in positions:
            q = produce(qp, wq, p, 1, hq)
            kc[:, p] = produce(kp, wk, p, 1, hkv)[0]
            vc[:, p] = vp[p]
            oracle.attention_cached(q.reshape(-1), kc, vc, 1, hq, hkv, d, cap, p)
        passes += 1
        dt = time.perf_counter() - t0
        if dt >= seconds or passes >= max_passes:
            break
    steps = passes * len(positions)
    nbytes = passes * sum(w.decode_bytes_per_step(p + 1) for p in positions)
    return {
        "value": nbytes / dt / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
        "sample": f"configs[1] decode, 1 layer, all {len(positions)} steps (context {positions[0] + 1}.."
                  f"{positions[-1] + 1}) x {passes} passes: oracle rmsnorm + rotary + append + "
                  f"attention_cached (FP32 KV, FP64 softmax), {dt:.2f} s; bytes counted as the "
                  f"GPU's bf16 bytes",
        "seconds": dt,
        "us_per_token": dt / steps * 1e6,
        "host_cpus": os.cpu_count(),
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
    result = {}
    w = None
    if args.only in (None, "c2"):
        c2, w = bench_c2(torch, ops, sessmod, ctx, args.steps, args.warmup)
        log(json.dumps(c2))
        result["c2"] = c2
    if not args.no_north_star and args.only in (None, "d8k"):
        d8k = bench_decode_batch(torch, ops, ctx, 50, 5, batch=1, lmin=8192, lmax=8192,
                                 dtype=torch.bfloat16)
        log("single-session decode at 8192: " + json.dumps(d8k))
        result["decode_8k"] = d8k
    if not args.no_north_star and args.only in (None, "d8kb"):
        d8kb = bench_decode_batch(torch, ops, ctx, 20, 3, batch=16, lmin=8192, lmax=8192,
                                  dtype=torch.bfloat16)
        log("sustained decode at 8192, 16 sessions: " + json.dumps(d8kb))
        result["decode_8k_batch16"] = d8kb
    if not args.no_north_star and args.only in (None, "c3"):
        c3 = bench_decode_batch(torch, ops, ctx, 20, 3, batch=64, lmin=512, lmax=8192,
                                dtype=torch.float16)
        log("c3: " + json.dumps(c3))
        result["c3"] = c3
    if not args.no_north_star and args.only in (None, "c4"):
        c4 = bench_c4(torch, ops, sessmod, ctx, 2, 1)
        log("c4: " + json.dumps(c4))
        result["c4"] = c4
    if not args.no_north_star and args.only in (None, "c5"):
        c5 = bench_prefill_batch(torch, ops, ctx, 10, 2)
        log("c5: " + json.dumps(c5))
        result["c5"] = c5
    if args.only is not None and args.only != "c2":
        print(json.dumps(result))
        return

    c2 = result["c2"]
    traffic, traffic_entry = measured_traffic("c2_decode")
    line = {
        "metric": "decode attn GB/s (% HBM peak); prefill attn TFLOPS (% MFMA peak)",
        "value": round(c2["decode_gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(c2["job_ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) Q/K/V, per-head RMSNorm N(1,0.02) weights, RoPE 1e6)",
        "config": {"workload": "configs[1] Qwen3 16q/8kv/d128 bf16 KV, prefill 2048 in 128-token "
                               "chunks + 256 decode steps, 1 layer per step",
                   "query_heads": 16, "kv_heads": 8, "head_dim": 128, "prefill": 2048, "chunk": 128,
                   "decode_steps": 256},
        "prefill_tflops": round(c2["prefill_tflops"], 3),
        "prefill_frac_mfma": round(c2["prefill_tflops"] / PEAK_BF16_TFLOPS, 5),
        "decode_frac_hbm": round(c2["decode_gbs"] / PEAK_HBM_GBS, 5),
        "tokens_per_s": round(c2["tokens_per_s"], 1),
        "decode_us_per_token": round(c2["decode_us_per_token"], 3),
        "roofline": {
            "bound": "hbm",
            "kernel": "attn_decode<bf16, D=128, 2 rows, producer folded in> (the 256 decode "
                      "launches of configs[1])",
            "achieved": round(c2["decode_kernel_gbs"], 2),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(c2["decode_kernel_gbs"] / PEAK_HBM_GBS, 5),
            "traffic": traffic,
            "traffic_source": (traffic_entry or {}).get("source"),
            "avg_kernel_us": round(c2["decode_kernel_us"], 3),
            "algorithmic_bytes_per_launch": round(c2["decode_bytes_per_step_avg"]),
            "timing": "hipExtLaunchKernelGGL start/stop events on the library's stream",
        },
        "prefill_roofline": {
            "bound": "mfma", "achieved": round(c2["prefill_kernel_tflops"], 3),
            "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
            "frac": round(c2["prefill_kernel_tflops"] / PEAK_BF16_TFLOPS, 5),
        },
        "north_star": {k: result[k] for k in ("decode_8k", "decode_8k_batch16", "c3", "c4", "c5")
                       if k in result},
        "detail": c2,
    }
    if not args.no_cpu and w is not None:
        log("cpu baseline: oracle on the host cores")
        line["cpu_baseline"] = cpu_baseline(w, torch)
    print(json.dumps(line))


if __name__ == "__main__":
    main()
