#!/usr/bin/env python3
"""Decode-attention benchmark for the SunShape compressed-KV path on MI355X.

Workload (BASELINE.json metric, config 2 at T_kv = 32768): batch 1, 32 query
heads / 8 KV heads, head_dim 128, 1-bit/dim SunShape keys (uint8 indices
(8, 32768, 16)) and fp16 values N(0,1); one fp16 query token per step;
codebook fit on 4096 N(0,1) keys with a per-dim scale in [0.5, 4].

A step is one fused decode-attention launch over the whole cache (all 32
query heads).  The timed region rotates over enough cache copies (> 3x the
256 MB Infinity Cache) that every step reads its indices and values from
HBM.  ``value`` is algorithmic HBM bytes per step / time per step.

Prints one JSON line on stdout; progress goes to stderr.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "decode attention µs/step and achieved HBM GB/s (% of peak) at T_kv=32K"
HBM_PEAK_GBS = 8000.0
MALL_BYTES = 256 << 20


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--t-kv", type=int, default=32768)
    p.add_argument("--batch", type=int, default=1)
    p.add_argument("--splits", type=int, default=0, help="token splits (0 = library choice)")
    p.add_argument("--copies", type=int, default=0, help="cache copies rotated (0 = auto)")
    p.add_argument("--launch", choices=("eager", "graph"), default="eager")
    p.add_argument("--layout", choices=("il8", "dense"), default="il8",
                   help="value cache layout: 8-token interleaved (MFMA kernel) or token-major")
    p.add_argument("--cpu-seconds", type=float, default=12.0,
                   help="budget for the CPU baseline (0 disables it)")
    p.add_argument("--traffic-file", default=os.path.join(ROOT, "profiles",
                                                          "decode_fp16v_t32k_traffic.json"))
    p.add_argument("--layers", type=int, default=28, help="config5: decoder layers per step")
    p.add_argument("--reference-mixed", action="store_true",
                   help="config5: drop the heavy blocks from the scores as the reference does "
                        "(default: keep them in fp16 and score them exactly)")
    p.add_argument("--t-q", type=int, default=4096, help="prefill: prompt tokens")
    p.add_argument("--workload", choices=("metric", "hybrid", "encode", "turboquant", "config5",
                                          "fit", "prefill", "scores"),
                   default="metric",
                   help="metric: the headline metric decode (fp16 values, B=1); hybrid: config 4 "
                        "(B=8, 2-bit grouped values, g=64, fp16 scale/zero); encode: config 3 "
                        "(65,536 fp16 keys block-VQ encoded); turboquant: the config-4 shape "
                        "with 2-bit TurboQuant values; config5: 28 layers x B=16, "
                        "T_kv=131072, mixed-precision keys, SunShape values; prefill: one "
                        "causal prompt of --t-q tokens against its own cache; scores: the "
                        "score-only path (LUT + one gather over all heads) at the config-4 "
                        "shape")
    p.add_argument("--calibrate-copy", type=int, default=0, metavar="MB",
                   help="only run a plain device copy of MB megabytes --steps times (the "
                        "known-size kernel that scales rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    return p.parse_args()


def calibrate_copy(mb: int, steps: int) -> int:
    import torch

    n = mb * (1 << 20) // 4
    src = torch.randn(n, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(steps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calibrate_copy_bytes_read": n * 4, "calibrate_copy_bytes_written": n * 4,
                      "dispatches": steps}), flush=True)
    return 0


def algorithmic_bytes(b, hq, hkv, d, t_kv, nb, v_bytes=2, q_bytes=2, out_bytes=2) -> int:
    """Bytes one step must move at minimum: every key index row and value row
    once per (batch, KV head), the query in and the output out.  Centroids
    (128 KB, cache-resident), split partials and GQA re-reads excluded."""
    return b * hkv * t_kv * (nb + d * v_bytes) + b * hq * d * (q_bytes + out_bytes)


def time_launches(fn, argv, steps, warmup, hip):
    """Mean µs per launch over ``steps`` back-to-back launches (after
    ``warmup``), rotating over the argument tuples, plus per-launch event
    durations."""
    import numpy as np
    import torch

    for i in range(warmup):
        hip.check(fn(*argv[i % len(argv)]))
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record()
    for i in range(steps):
        rc = fn(*argv[i % len(argv)])
        if rc:
            hip.check(rc)
    ev1.record()
    torch.cuda.synchronize()
    us = ev0.elapsed_time(ev1) * 1e3 / steps
    n_pl = min(steps, 100)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(n_pl)]
    for i, (e0, e1) in enumerate(evs):
        e0.record()
        hip.check(fn(*argv[i % len(argv)]))
        e1.record()
    torch.cuda.synchronize()
    per = np.array([e0.elapsed_time(e1) * 1e3 for e0, e1 in evs])
    return us, per


def stream_ceiling(nbytes: int, steps: int, warmup: int, hip, n_workgroups: int = 512) -> dict:
    """Per-launch time of the library's read-ceiling kernel (plain 16-byte
    loads, ss_stream_read) over ``nbytes`` rotated across enough copies that
    every launch reads HBM: the fastest one launch can read a decode step's
    bytes on this device."""
    import torch

    lib = hip.load_library()
    n16 = (nbytes + 15) // 16 * 16
    n_copies = max(2, math.ceil(3 * MALL_BYTES / n16))
    bufs = [torch.randint(0, 1 << 30, (n16 // 4,), dtype=torch.int32, device="cuda:0")
            for _ in range(n_copies)]
    sink = torch.zeros(16, dtype=torch.int32, device="cuda:0")
    st = torch.cuda.current_stream().cuda_stream
    argv = [(b.data_ptr(), n16, n_workgroups, sink.data_ptr(), st) for b in bufs]
    us, per = time_launches(lib.ss_stream_read, argv, steps, warmup, hip)
    del bufs
    return {"us_per_launch": round(us, 3), "gbs": round(nbytes / (us * 1e-6) / 1e9, 2),
            "bytes": nbytes, "workgroups": n_workgroups, "copies": n_copies,
            "kernel": "ss_stream_read (plain 16-byte non-temporal loads, 4 in flight per thread)"}


def time_api_steps(pkg, caches, q, scale, steps, warmup, kv_step=None) -> dict:
    """The drop-in path per decode step over caches built through the API,
    rotated so every step reads HBM: ``sunshape_sdpa`` alone, or (with
    ``kv_step`` = (keys, values) of one token) ``update_and_fetch`` of that
    token first, as mlx-lm runs a decode step.  HIP events bracket all the
    steps; the host clock gives the Python time per step."""
    import torch

    n = len(caches)

    def one(i):
        c = caches[i % n]
        if kv_step is not None:
            c.update_and_fetch(*kv_step)
        pkg.sunshape_sdpa(q, c, scale)

    for i in range(warmup):
        one(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    h0 = time.perf_counter()
    for i in range(steps):
        one(i)
    h1 = time.perf_counter()
    e1.record()
    torch.cuda.synchronize()
    return {"us_per_step": round(e0.elapsed_time(e1) * 1e3 / steps, 3),
            "host_us_per_step": round((h1 - h0) * 1e6 / steps, 3),
            "backend": caches[0].codec.last_score_backend}


def cpu_threads() -> int:
    """Host threads the CPU baseline uses: the CPUs this process may run on,
    capped at 16 (one GPU's share of the box)."""
    return max(1, min(len(os.sched_getaffinity(0)), 16))


def run_hybrid(args) -> int:
    """Config 4: B=8 hybrid cache, 1-bit/dim keys (uniform u8 indices), values
    2-bit grouped (g=64) with fp16 scale/zero, one fp16 query token per step
    for 32 query heads; one fused grouped-value decode launch per step."""
    import numpy as np
    import torch

    import __graft_entry__

    pkg = __graft_entry__.load_package()
    hip = pkg._hip
    lib = hip.load_library()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    b, hq, hkv, d, t_kv, nb = 8, 32, 8, 128, args.t_kv, 16
    bits, group = 2, 64
    scale = 1.0 / math.sqrt(d)
    g = torch.Generator(device=dev).manual_seed(4)
    cents = torch.randn((nb, 256, 8), generator=g, device=dev)
    perm = torch.randperm(d, generator=g, device=dev).to(torch.int32)
    idx0 = torch.randint(0, 256, (b, hkv, t_kv, nb), generator=g, device=dev).to(torch.uint8)
    v = torch.randn((b, hkv, t_kv, d), generator=g, device=dev).to(torch.float16)
    pd, ng = d * bits // 32, d // group
    packed0 = torch.empty((b, hkv, t_kv, pd), dtype=torch.int32, device=dev)
    sc0 = torch.empty((b, hkv, t_kv, ng), dtype=torch.float16, device=dev)
    ze0 = torch.empty((b, hkv, t_kv, ng), dtype=torch.float16, device=dev)
    hip.quantize_values_grouped(v, bits, group, packed0, sc0, ze0)
    # the cache's code layout: token-interleaved (16 tokens of one dim per word)
    il0 = torch.empty((b, hkv, t_kv * bits // 32, d), dtype=torch.int32, device=dev)
    hip.pack_grouped_il(packed0, bits, il0, 0)
    q = torch.randn((b, hq, 1, d), generator=g, device=dev).to(torch.float16)
    del v
    per_copy = idx0.numel() + il0.numel() * 4 + (sc0.numel() + ze0.numel()) * 2
    n_copies = args.copies or max(2, math.ceil(3 * MALL_BYTES / per_copy))
    bufs = [(idx0, il0, sc0, ze0)] + [tuple(t.clone() for t in (idx0, il0, sc0, ze0))
                                      for _ in range(n_copies - 1)]
    torch.cuda.synchronize()
    log(f"hybrid cache ready: {n_copies} copies x {per_copy / 1e6:.1f} MB")
    splits, ws_bytes = hip.decode_plan(hip.KIND_IL8, b, hq, hkv, 1, d, t_kv, args.splits)
    ws = torch.zeros(max(ws_bytes, 256), dtype=torch.uint8, device=dev)
    out = torch.empty((b, hq, 1, d), dtype=torch.float16, device=dev)
    stream = torch.cuda.current_stream().cuda_stream
    fn = lib.ss_decode_attn_grouped_il
    cb = hip.codebook_f16x2(cents)
    argv = [(q.data_ptr(), hip.SS_F16, b, hq, hkv, 1, d, scale, perm.data_ptr(), cb.data_ptr(),
             nb, 256, t[0].data_ptr(), t[1].data_ptr(), t[2].data_ptr(), t[3].data_ptr(), hip.SS_F16,
             bits, group, t_kv, t_kv, 0, 0, out.data_ptr(), hip.SS_F16, ws.data_ptr(), ws_bytes,
             splits, stream) for t in bufs]
    us, per = time_launches(fn, argv, args.steps, args.warmup, hip)
    nbytes = b * hkv * t_kv * (nb + pd * 4 + ng * 2 * 2) + b * hq * d * 4
    gbs = nbytes / (us * 1e-6) / 1e9
    log(f"hybrid: {us:.2f} us/step, {gbs:.1f} GB/s (splits={splits})")

    check = None
    if args.cpu_seconds > 0:  # output check of one (b, KV head) against the oracle
        from oracle import sunshape_oracle as O

        hip.check(fn(*argv[0]))
        torch.cuda.synchronize()
        bi, hi = 3, 5
        vals = O.dequantize_values(packed0[bi, hi].cpu().numpy().view(np.uint32),
                                   sc0[bi, hi].float().cpu().numpy(), ze0[bi, hi].float().cpu().numpy(),
                                   d, bits, group)
        qh = q[bi:bi + 1, hi * 4:(hi + 1) * 4].cpu().numpy()
        ref = O.sdpa(qh, idx0[bi:bi + 1, hi:hi + 1].cpu().numpy(), vals[None, None],
                     cents.cpu().numpy(), perm.cpu().numpy(), scale)
        got = out[bi, hi * 4:(hi + 1) * 4].float().cpu().numpy().reshape(ref.shape)
        check = float(np.abs(got - ref).max() / np.abs(ref).max())

    # ---- the drop-in path: hybrid caches built through the API (default
    # 128-token fp16 buffer, 2-bit grouped values, fp16 scale/zero), rotated;
    # sunshape_sdpa alone, then whole decode steps (update_and_fetch of one
    # token: stored, the oldest buffered token encoded and quantised) ----
    del bufs, argv, packed0, il0
    codec = pkg.codec.SunShapeBlockCodec(d, device=dev)
    codec.load_state_dict({"centroids": cents.cpu().numpy(), "permutation": perm.cpu().numpy()})
    kk = torch.randn((b, hkv, t_kv, d), generator=g, device=dev).to(torch.float16)
    vv = torch.randn((b, hkv, t_kv, d), generator=g, device=dev).to(torch.float16)
    caches = []
    for _ in range(n_copies):
        c = pkg.cache.create_kv_cache(codec, n_kv_heads=hkv, value_backend="grouped",
                                      value_bits=bits, value_group_size=group,
                                      value_scale_dtype=torch.float16, max_tokens=t_kv + 1024)
        c.update_and_fetch(kk, vv)
        caches.append(c)
    del kk, vv
    torch.cuda.synchronize()
    sdpa = time_api_steps(pkg, caches, q, scale, args.steps, args.warmup)
    log(f"hybrid sunshape_sdpa end to end: {sdpa['us_per_step']:.2f} us/step "
        f"(host {sdpa['host_us_per_step']:.1f} us/call, {sdpa['backend']})")
    k1 = torch.randn((b, hkv, 1, d), generator=g, device=dev).to(torch.float16)
    v1 = torch.randn((b, hkv, 1, d), generator=g, device=dev).to(torch.float16)
    n_step = min(args.steps, 1024 * n_copies // 2)
    step = time_api_steps(pkg, caches, q, scale, n_step, args.warmup, kv_step=(k1, v1))
    step["t_kv_range"] = [t_kv, caches[0].offset]
    log(f"hybrid decode step end to end: {step['us_per_step']:.2f} us/step "
        f"(host {step['host_us_per_step']:.1f} us/step, {step['backend']})")
    # the same steps with the flush and buffer store as their own launch
    # (fuse_steps off)
    for c in caches:
        c.fuse_steps = False
    sep = time_api_steps(pkg, caches, q, scale, n_step, args.warmup, kv_step=(k1, v1))
    step["separate_append"] = {k_: sep[k_] for k_ in ("us_per_step", "host_us_per_step")}
    log(f"  ... with the step launched separately: {sep['us_per_step']:.2f} us/step")
    del caches

    traffic = None  # HBM bytes per launch from the committed counter runs
    tf = os.path.join(ROOT, "profiles", "decode_grouped2b_t32k_traffic.json")
    if os.path.exists(tf):
        with open(tf) as f:
            tr = json.load(f)
        if tr.get("t_kv") == t_kv and tr.get("batch") == b:
            traffic = tr.get("hbm_bytes_per_launch")

    line = {
        "metric": "hybrid decode attention µs/step and achieved HBM GB/s (config 4)",
        "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(us * 1e-3, 6), "us_per_step": round(us, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "decode B=8 Hq=32 Hkv=8 D=128 T_kv=32768, u8 key indices, 2-bit "
                               "grouped values g=64 with fp16 scale/zero (codes token-interleaved), "
                               "fp16 query/output",
                   "t_kv": t_kv, "splits": splits, "cache_copies": n_copies,
                   "algorithmic_bytes_per_step": nbytes},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic},
        "per_launch_us": {"mean": round(float(np.mean(per)), 3),
                          "median": round(float(np.median(per)), 3)},
        "check_max_rel_err_vs_oracle": check,
        "sdpa_end_to_end": sdpa,
        "decode_step_end_to_end": step,
    }
    print(json.dumps(line), flush=True)
    return 0


def run_prefill(args) -> int:
    """Prefill: one prompt of T tokens (B=1, 32 query / 8 KV heads, D=128)
    attended causally against the cache that holds the same T tokens (u8
    key indices, fp16 values 8-token interleaved), as mlx-lm's prefill does
    after update_and_fetch: sunshape_sdpa(q, cache, scale, mask="causal"),
    whose fused path is one ss_prefill_attn_il8 launch.  Reported
    as µs per prompt and attention TFLOP/s (QK^T and P.V over the causal
    half, 4 * B * Hq * D * T^2 / 2 flops); the decode-shaped kernel's time on
    the same prompt is reported beside it."""
    import numpy as np
    import torch

    import __graft_entry__

    pkg = __graft_entry__.load_package()
    hip = pkg._hip
    lib = hip.load_library()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    b, hq, hkv, d, nb = 1, 32, 8, 128, 16
    t = args.t_q
    scale = 1.0 / math.sqrt(d)
    g = torch.Generator(device=dev).manual_seed(6)
    cents = torch.randn((nb, 256, 8), generator=g, device=dev)
    perm = torch.randperm(d, generator=g, device=dev).to(torch.int32)
    idx = torch.randint(0, 256, (b, hkv, t, nb), generator=g, device=dev).to(torch.uint8)
    v = torch.randn((b, hkv, t, d), generator=g, device=dev).to(torch.float16)
    v8 = torch.zeros((b, hkv, t // 8, d, 8), dtype=torch.float16, device=dev)
    hip.append_values_il8(v, v8, 0)
    q = torch.randn((b, hq, t, d), generator=g, device=dev).to(torch.float16)
    out = torch.empty((b, hq, t, d), dtype=torch.float16, device=dev)
    stream = torch.cuda.current_stream().cuda_stream
    cb = hip.codebook_f16x2(cents)
    fn = lib.ss_prefill_attn_il8
    argv = [(q.data_ptr(), hip.SS_F16, b, hq, hkv, t, d, scale, perm.data_ptr(), cb.data_ptr(),
             nb, 256, idx.data_ptr(), v8.data_ptr(), hip.SS_F16, t, t, 1, 0, out.data_ptr(),
             hip.SS_F16, stream)]
    steps, warmup = max(1, args.steps // 10), max(1, args.warmup // 4)
    us, per = time_launches(fn, argv, steps, warmup, hip)
    flops = 4 * b * hq * d * t * t // 2
    tflops = flops / (us * 1e-6) / 1e12
    log(f"prefill T={t}: {us:.1f} us/prompt, {tflops:.2f} TFLOP/s")
    # the decode-shaped kernel on the same prompt, for comparison
    splits, ws_bytes = hip.decode_plan(hip.KIND_IL8, b, hq, hkv, t, d, t, args.splits)
    ws = torch.zeros(max(ws_bytes, 256), dtype=torch.uint8, device=dev)
    out_dec = torch.empty_like(out)
    argv_dec = [(q.data_ptr(), hip.SS_F16, b, hq, hkv, t, d, scale, perm.data_ptr(), cb.data_ptr(),
                 nb, 256, idx.data_ptr(), v8.data_ptr(), hip.SS_F16, t, t, 1, 0,
                 out_dec.data_ptr(), hip.SS_F16, ws.data_ptr(), ws_bytes, splits, stream)]
    us_dec, _ = time_launches(lib.ss_decode_attn_il8, argv_dec, max(1, steps // 4), 1, hip)
    log(f"decode-shaped kernel on the same prompt: {us_dec:.1f} us")

    check = None
    if args.cpu_seconds > 0:  # one (KV head, query head) of the last 64 rows vs the oracle
        from oracle import sunshape_oracle as O

        hip.check(fn(*argv[0]))
        torch.cuda.synchronize()
        hi, rows = 5, slice(t - 64, t)
        qh = q[:, hi * 4:hi * 4 + 1, rows].cpu().numpy()
        # the last 64 rows see keys 0 .. t-64+i: the oracle's causal mask
        # over a (64, t) score block with offset t - 64
        ref = O.sdpa(qh, idx[:, hi:hi + 1].cpu().numpy(), v[:, hi:hi + 1].cpu().numpy(),
                     cents.cpu().numpy(), perm.cpu().numpy(), scale, mask="causal")
        got = out[:, hi * 4:hi * 4 + 1, rows].float().cpu().numpy()
        check = float(np.abs(got - ref).max() / np.abs(ref).max())

    cache = pkg.create_kv_cache(pkg.SunShapeBlockCodec(d, device=dev), n_kv_heads=hkv)
    cache.codec.load_state_dict({"centroids": cents.cpu().numpy(), "permutation": perm.cpu().numpy()})
    cache.update_and_fetch(torch.zeros((b, hkv, t, d), dtype=torch.float16, device=dev),
                           v)  # encode cost not timed; indices replaced below
    cache._key_indices[:, :, :t] = idx
    torch.cuda.synchronize()
    for _ in range(warmup):
        pkg.sunshape_sdpa(q, cache, scale, mask="causal")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        o2 = pkg.sunshape_sdpa(q, cache, scale, mask="causal")
    torch.cuda.synchronize()
    sdpa_us = (time.perf_counter() - t0) * 1e6 / steps
    same = bool(torch.equal(o2, out))

    # the same prompt through a hybrid cache: 2-bit grouped values (g=64,
    # fp16 scale/zero), a 128-token fp16 buffer -- config 4's cache kind.
    # The prompt's keys are encoded by the cache (update_and_fetch, not
    # timed); the kernel then scores T - 128 positions from the codebook and
    # the buffered 128 from the whole keys.
    hcache = pkg.create_kv_cache(pkg.SunShapeBlockCodec(d, device=dev), n_kv_heads=hkv,
                                 value_backend="grouped", value_bits=2,
                                 value_scale_dtype=torch.float16, buffer_size=128)
    hcache.codec.load_state_dict({"centroids": cents.cpu().numpy(),
                                  "permutation": perm.cpu().numpy()})
    keys = torch.randn((b, hkv, t, d), generator=g, device=dev).to(torch.float16)
    hcache.update_and_fetch(keys, v)
    torch.cuda.synchronize()
    vil8, rows, fac, t_raw0 = hcache.prefill_operands()
    hc = hcache.codec
    hkw = dict(causal=True, q_offset=0)

    def hybrid_kernel():
        hip.prefill_attn_il8_hybrid(q, scale, hc.permutation, hc.kernel_codebook(), 256,
                                    hcache._key_indices, vil8, t, rows, fac, t_raw0, **hkw)
        return 0

    h_us, h_per = time_launches(hybrid_kernel, [()], steps, warmup, hip)
    for _ in range(warmup):
        pkg.sunshape_sdpa(q, hcache, scale, mask="causal")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        oh = pkg.sunshape_sdpa(q, hcache, scale, mask="causal")
    torch.cuda.synchronize()
    h_sdpa_us = (time.perf_counter() - t0) * 1e6 / steps
    h_backend = hcache.codec.last_score_backend
    log(f"hybrid 2-bit grouped cache: kernel {h_us:.1f} us, sdpa {h_sdpa_us:.1f} us "
        f"({h_backend}), {h_us / us:.2f}x the fp16 prefill kernel")
    h_check = None
    if args.cpu_seconds > 0:  # one query head, the last 64 rows, vs the reference's two passes
        from oracle import sunshape_oracle as O

        hi, rows_ = 5, slice(t - 64, t)
        ref = O.sdpa_two_pass(q[:, hi * 4:hi * 4 + 1, rows_].cpu().numpy(), scale,
                              perm.cpu().numpy(), cents.cpu().numpy(),
                              hcache.key_indices[:, hi:hi + 1].cpu().numpy(),
                              hcache.buffer_keys[:, hi:hi + 1].float().cpu().numpy(),
                              hcache.values[:, hi:hi + 1].float().cpu().numpy(),
                              mask="causal")
        got = oh[:, hi * 4:hi * 4 + 1, rows_].float().cpu().numpy()
        h_check = float(np.abs(got - ref).max() / np.abs(ref).max())

    line = {
        "metric": "causal prefill attention µs/prompt and TFLOP/s",
        "value": round(tflops, 3), "unit": "TFLOP/s", "n_gpus": 1, "steps": steps,
        "warmup": warmup, "ms_per_step": round(us * 1e-3, 6), "us_per_step": round(us, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": f"prefill B=1 Hq=32 Hkv=8 D=128 T_q=T_kv={t} causal, u8 key "
                               "indices, fp16 values (il8), fp16 query/output",
                   "t": t, "attention_flops": flops, "kernel": "ss_prefill_attn_il8"},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 3), "peak": 2500.0,
                     "unit": "TFLOP/s", "frac": round(tflops / 2500.0, 5), "traffic": None},
        "per_launch_us": {"mean": round(float(np.mean(per)), 3),
                          "median": round(float(np.median(per)), 3)},
        "sdpa_end_to_end": {"us_per_prompt": round(sdpa_us, 1), "same_output": same,
                            "backend": cache.codec.last_score_backend},
        "decode_shaped_kernel_us": round(us_dec, 1),
        "check_max_rel_err_vs_oracle": check,
        "hybrid_grouped2_buffer128": {
            "kernel_us": round(h_us, 1), "x_fp16_prefill": round(h_us / us, 3),
            "per_launch_median_us": round(float(np.median(h_per)), 3),
            "sdpa_end_to_end_us": round(h_sdpa_us, 1), "backend": h_backend,
            "check_max_rel_err_vs_oracle": h_check},
    }
    print(json.dumps(line), flush=True)
    return 0


def run_turboquant(args) -> int:
    """Config-4 shape (B=8, 32/8 heads, D=128, T_kv=32768, u8 key indices)
    with 2-bit TurboQuant values (codes + fp32 norm per token): one
    ss_decode_attn_turboquant_il call per step (matrix-core decode kernel,
    split merge and output-row rotation on one stream), the vector-ALU
    ss_decode_attn_turboquant timed beside it."""
    import numpy as np
    import torch

    import __graft_entry__

    pkg = __graft_entry__.load_package()
    hip = pkg._hip
    lib = hip.load_library()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    b, hq, hkv, d, t_kv, nb, bits = 8, 32, 8, 128, args.t_kv, 16, 2
    scale = 1.0 / math.sqrt(d)
    g = torch.Generator(device=dev).manual_seed(6)
    cents = torch.randn((nb, 256, 8), generator=g, device=dev)
    perm = torch.randperm(d, generator=g, device=dev).to(torch.int32)
    idx0 = torch.randint(0, 256, (b, hkv, t_kv, nb), generator=g, device=dev).to(torch.uint8)
    pd = d * bits // 32
    pk0 = torch.randint(-2 ** 31, 2 ** 31 - 1, (b, hkv, t_kv, pd), generator=g, device=dev,
                        dtype=torch.int64).to(torch.int32)
    nm0 = torch.rand((b, hkv, t_kv), generator=g, device=dev) * 3 + 0.1
    tq = pkg.TurboQuantValueCodec(head_dim=d, bits=bits, seed=43, device=dev)
    levels = tq.levels_host()
    lv_host = (ctypes.c_float * len(levels))(*levels)
    rot = tq.rotation.contiguous()
    q = torch.randn((b, hq, 1, d), generator=g, device=dev).to(torch.float16)
    per_copy = idx0.numel() + pk0.numel() * 4 + nm0.numel() * 4
    n_copies = args.copies or max(2, math.ceil(3 * MALL_BYTES / per_copy))
    bufs = [(idx0, pk0, nm0)] + [tuple(t.clone() for t in (idx0, pk0, nm0))
                                 for _ in range(n_copies - 1)]
    torch.cuda.synchronize()
    log(f"turboquant cache ready: {n_copies} copies x {per_copy / 1e6:.1f} MB")
    ws_bytes = lib.ss_decode_turboquant_workspace_bytes(b, hq, hkv, 1, d, t_kv, 0, args.splits)
    splits = lib.ss_decode_default_splits(b, hq, hkv, 1, d, t_kv) if args.splits <= 0 else args.splits
    ws = torch.zeros(max(ws_bytes, 256), dtype=torch.uint8, device=dev)
    out = torch.empty((b, hq, 1, d), dtype=torch.float16, device=dev)
    stream = torch.cuda.current_stream().cuda_stream
    lv_ptr = ctypes.cast(lv_host, ctypes.c_void_p).value
    # the hybrid cache's layout for 2-bit codes: token-interleaved words
    # (ss_pack_grouped_il of the packed rows), read by the matrix-core kernel
    cb16 = hip.codebook_f16x2(cents)
    ils = []
    for t in bufs:
        il = torch.empty((b, hkv, t_kv // 16, d), dtype=torch.int32, device=dev)
        hip.pack_grouped_il(t[1], bits, il, 0)
        ils.append(il)
    torch.cuda.synchronize()
    fn = lib.ss_decode_attn_turboquant_il
    argv = [(q.data_ptr(), hip.SS_F16, b, hq, hkv, 1, d, scale, perm.data_ptr(), cb16.data_ptr(),
             nb, 256, t[0].data_ptr(), il.data_ptr(), t[2].data_ptr(), lv_ptr, rot.data_ptr(),
             t_kv, t_kv, None, None, 0, 0, 0, 0, 0, None, None, 0, 0, 0, out.data_ptr(),
             hip.SS_F16, ws.data_ptr(), ws_bytes, args.splits, stream) for t, il in zip(bufs, ils)]
    us, per = time_launches(fn, argv, args.steps, args.warmup, hip)
    nbytes = b * hkv * t_kv * (nb + pd * 4 + 4) + b * hq * d * 4
    gbs = nbytes / (us * 1e-6) / 1e9
    log(f"turboquant (matrix cores): {us:.2f} us/step, {gbs:.1f} GB/s")
    # the vector-ALU kernel over the reference's packed rows
    fn_v = lib.ss_decode_attn_turboquant
    argv_v = [(q.data_ptr(), hip.SS_F16, b, hq, hkv, 1, d, scale, perm.data_ptr(), cents.data_ptr(),
               nb, 256, t[0].data_ptr(), t[1].data_ptr(), t[2].data_ptr(), lv_ptr, rot.data_ptr(),
               bits, t_kv, t_kv, None, None, 0, 0, 0, 0, 0, None, None, 0, 0, 0, out.data_ptr(),
               hip.SS_F16, ws.data_ptr(), ws_bytes, args.splits, stream) for t in bufs]
    us_v, _ = time_launches(fn_v, argv_v, max(args.steps // 4, 5), args.warmup, hip)
    log(f"turboquant (vector ALUs, packed rows): {us_v:.2f} us/step")

    check = None
    if args.cpu_seconds > 0:  # output check of one (b, KV head) against the oracle
        from oracle import sunshape_oracle as O

        bi, hi = 2, 6
        vals = O.turboquant_decode(pk0[bi, hi].cpu().numpy().view(np.uint32),
                                   nm0[bi, hi].cpu().numpy(), rot.cpu().numpy(),
                                   np.asarray(levels, np.float32), d, bits)
        qh = q[bi:bi + 1, hi * 4:(hi + 1) * 4].cpu().numpy()
        ref = O.sdpa(qh, idx0[bi:bi + 1, hi:hi + 1].cpu().numpy(), vals[None, None],
                     cents.cpu().numpy(), perm.cpu().numpy(), scale)
        check = 0.0
        for f_, a_ in ((fn, argv[0]), (fn_v, argv_v[0])):
            hip.check(f_(*a_))
            torch.cuda.synchronize()
            got = out[bi, hi * 4:(hi + 1) * 4].float().cpu().numpy().reshape(ref.shape)
            check = max(check, float(np.abs(got - ref).max() / np.abs(ref).max()))

    traffic = None  # HBM bytes per call from the committed counter runs
    tf = os.path.join(ROOT, "profiles", "decode_attn_mfma_turboquant2b_t32k_traffic.json")
    if os.path.exists(tf):
        with open(tf) as f:
            tr = json.load(f)
        if tr.get("t_kv") == t_kv and tr.get("batch") == b:
            traffic = tr.get("hbm_bytes_per_launch")

    line = {
        "metric": "TurboQuant-value decode attention µs/step and achieved HBM GB/s",
        "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(us * 1e-3, 6), "us_per_step": round(us, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "decode B=8 Hq=32 Hkv=8 D=128 T_kv=32768, u8 key indices, 2-bit "
                               "TurboQuant values (token-interleaved codes + fp32 norm), fp16 "
                               "query/output",
                   "t_kv": t_kv, "splits": splits, "cache_copies": n_copies,
                   "algorithmic_bytes_per_step": nbytes},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic},
        "per_launch_us": {"mean": round(float(np.mean(per)), 3),
                          "median": round(float(np.median(per)), 3)},
        "valu_kernel_us": round(us_v, 3),
        "check_max_rel_err_vs_oracle": check,
    }
    print(json.dumps(line), flush=True)
    return 0


def run_config5(args) -> int:
    """Config 5: one decode step of a 28-layer Qwen-style 4B model's attention
    (32 query / 8 KV heads, D=128, B=16, T_kv=131072 per layer).  Keys: a
    profileperm_mixed_precision codec's 16 uint8 indices per token (the 4
    heavy blocks' centroids zero) plus those 4 blocks' 32 dims in fp16,
    scored exactly (the config's "4 heaviest blocks fp16"; --reference-mixed
    drops them, as the reference does); values: SunShape block-VQ,
    block_dim 4, 256 centroids (32 index bytes per token), permutation
    transform.  Random N(0,1) codebooks, keys and uniform indices; 28 distinct
    layer caches (52.6 GB), one ss_decode_attn_sunshape_v call per layer."""
    import numpy as np
    import torch

    import __graft_entry__

    pkg = __graft_entry__.load_package()
    hip = pkg._hip
    lib = hip.load_library()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    layers = args.layers
    b, hq, hkv, d, t_kv, nb, vbd = 16, 32, 8, 128, args.t_kv, 16, 4
    nbv = d // vbd
    scale = 1.0 / math.sqrt(d)
    g = torch.Generator(device=dev).manual_seed(5)
    cents = torch.randn((nb, 256, 8), generator=g, device=dev)
    heavy = torch.randperm(nb, generator=g, device=dev)[:4]
    cents[heavy] = 0.0  # mixed-precision heavy blocks: zero centroids
    heavy_fp16 = not args.reference_mixed
    hd = torch.sort(heavy).values
    heavy_dims = (hd[:, None] * 8 + torch.arange(8, device=dev)[None]).flatten().to(torch.int32)
    nhd = heavy_dims.numel() if heavy_fp16 else 0
    perm = torch.randperm(d, generator=g, device=dev).to(torch.int32)
    v_cents = torch.randn((nbv, 256, vbd), generator=g, device=dev)
    vperm = torch.randperm(d, generator=g, device=dev)
    inv = torch.argsort(vperm)
    v_transform = torch.zeros((d, d), dtype=torch.float32, device=dev)
    v_transform[inv, torch.arange(d, device=dev)] = 1.0
    caches = []
    for _ in range(layers):
        caches.append((torch.randint(0, 256, (b, hkv, t_kv, nb), generator=g, device=dev,
                                     dtype=torch.uint8),
                       torch.randint(0, 256, (b, hkv, t_kv, nbv), generator=g, device=dev,
                                     dtype=torch.uint8),
                       torch.randn((b, hkv, t_kv, nhd), generator=g, device=dev).half()
                       if heavy_fp16 else None))
    q = torch.randn((b, hq, 1, d), generator=g, device=dev).to(torch.float16)
    torch.cuda.synchronize()
    per_layer = b * hkv * t_kv * (nb + nbv + 2 * nhd)
    log(f"config 5 caches ready: {layers} layers x {per_layer / 1e6:.1f} MB")
    ws_bytes = lib.ss_decode_turboquant_workspace_bytes(b, hq, hkv, 1, d, t_kv, 0, args.splits)
    splits = lib.ss_decode_default_splits(b, hq, hkv, 1, d, t_kv) if args.splits <= 0 else args.splits
    ws = torch.zeros(max(ws_bytes, 256), dtype=torch.uint8, device=dev)
    out = torch.empty((b, hq, 1, d), dtype=torch.float16, device=dev)
    stream = torch.cuda.current_stream().cuda_stream
    fn = lib.ss_decode_attn_sunshape_v
    argv = [(q.data_ptr(), hip.SS_F16, b, hq, hkv, 1, d, scale, perm.data_ptr(), cents.data_ptr(),
             nb, 256, ki.data_ptr(), vi.data_ptr(), v_cents.data_ptr(), vbd, 256,
             v_transform.data_ptr(), kh.data_ptr() if kh is not None else None,
             heavy_dims.data_ptr(), nhd, t_kv, t_kv, None, None, 0, 0, 0, 0, 0, 0, 0,
             out.data_ptr(), hip.SS_F16, ws.data_ptr(), ws_bytes, args.splits, stream)
            for ki, vi, kh in caches]

    def step():
        for a in argv:
            rc = fn(*a)
            if rc:
                hip.check(rc)

    steps, warmup = max(1, args.steps // 20), max(1, args.warmup // 10)
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record()
    for _ in range(steps):
        step()
    ev1.record()
    torch.cuda.synchronize()
    us = ev0.elapsed_time(ev1) * 1e3 / steps
    nbytes = layers * (per_layer + b * hq * d * 4)
    gbs = nbytes / (us * 1e-6) / 1e9
    log(f"config 5: {us:.1f} us/step ({us / layers:.1f} us/layer), {gbs:.1f} GB/s")

    check = None
    if args.cpu_seconds > 0:  # output check of one (b, KV head) of layer 0 against the oracle
        from oracle import sunshape_oracle as O

        hip.check(fn(*argv[0]))
        torch.cuda.synchronize()
        bi, hi = 11, 3
        ki, vi, kh = caches[0]
        vals = O.dequantize_blockvq(vi[bi, hi].cpu().numpy(), v_cents.cpu().numpy(),
                                    inv.cpu().numpy())
        qh = q[bi:bi + 1, hi * 4:(hi + 1) * 4].cpu().numpy()
        ref = O.sdpa_two_pass(qh, scale, perm.cpu().numpy(), cents.cpu().numpy(),
                              ki[bi:bi + 1, hi:hi + 1].cpu().numpy(), None, vals[None, None],
                              heavy_keys=(kh[bi:bi + 1, hi:hi + 1].cpu().numpy()
                                          if kh is not None else None),
                              heavy_dims=heavy_dims.cpu().numpy())
        got = out[bi, hi * 4:(hi + 1) * 4].float().cpu().numpy().reshape(ref.shape)
        check = float(np.abs(got - ref).max() / np.abs(ref).max())

    traffic = None  # HBM bytes per layer launch from the committed counter runs
    tf = os.path.join(ROOT, "profiles", "decode_sunshape_v_config5_traffic.json")
    if heavy_fp16 and os.path.exists(tf):
        with open(tf) as f:
            tr = json.load(f)
        if tr.get("t_kv") == t_kv and tr.get("batch") == b:
            traffic = tr.get("hbm_bytes_per_launch")

    line = {
        "metric": "28-layer decode step attention µs/step and achieved HBM GB/s (config 5)",
        "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": round(us * 1e-3, 6), "us_per_step": round(us, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": f"{layers} layers x decode B=16 Hq=32 Hkv=8 D=128 T_kv={t_kv}, "
                               + ("mixed-precision keys (16 u8 indices + 4 heavy blocks' 32 dims "
                                  "fp16, scored exactly), " if heavy_fp16 else
                                  "mixed-precision keys (16 u8 indices, 4 heavy blocks zero as in "
                                  "the reference), ") +
                               "SunShape values block_dim 4 / 256 centroids (32 u8 indices), "
                               "fp16 query/output",
                   "t_kv": t_kv, "layers": layers, "splits": splits,
                   "algorithmic_bytes_per_step": nbytes},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "traffic_per": "one layer's decode launch"},
        "check_max_rel_err_vs_oracle": check,
    }
    print(json.dumps(line), flush=True)
    return 0


def run_scores(args) -> int:
    """The score-only path (attention_scores, the two-pass fallback's
    compressed scores, attention.py:44-73 / codec.py:575-637) at the config-4
    shape: B=8, 32 query / 8 KV heads (4 query rows per KV head), T=32768,
    16 uint8 indices per token.  One LUT build for all 256 rows, then one
    score-gather launch over every (batch, KV head); the gather is the
    HBM-bound kernel (indices in, 4 fp32 scores per token out)."""
    import numpy as np
    import torch

    import __graft_entry__

    pkg = __graft_entry__.load_package()
    hip = pkg._hip
    lib = hip.load_library()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    b, hq, hkv, d, t_kv, nb, nc = 8, 32, 8, 128, args.t_kv, 16, 256
    rows = hq // hkv
    g = torch.Generator(device=dev).manual_seed(8)
    cents = torch.randn((nb, nc, 8), generator=g, device=dev)
    perm = torch.randperm(d, generator=g, device=dev).to(torch.int32)
    q = torch.randn((b * hq, d), generator=g, device=dev).to(torch.float16)
    per_copy = b * hkv * t_kv * (nb + rows * 4)
    n_copies = args.copies or max(2, math.ceil(3 * MALL_BYTES / per_copy))
    idxs = [torch.randint(0, nc, (b, hkv, t_kv, nb), generator=g, device=dev).to(torch.uint8)
            for _ in range(n_copies)]
    outs = [torch.empty((b, hkv, rows, t_kv), dtype=torch.float32, device=dev)
            for _ in range(n_copies)]
    lut = hip.build_lut(q, perm, 1.0 / math.sqrt(d), cents).reshape(b, hkv, rows, nb, nc)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream().cuda_stream
    fn = lib.ss_score_gather_heads
    argv = [(lut.data_ptr(), rows, nb, nc, ix.data_ptr(), b, hkv, ix.stride(0), ix.stride(1),
             ix.stride(2), t_kv, o.data_ptr(), stream) for ix, o in zip(idxs, outs)]
    us, per = time_launches(fn, argv, args.steps, args.warmup, hip)
    nbytes = b * hkv * t_kv * nb + b * hkv * rows * t_kv * 4 + b * hkv * rows * nb * nc * 4
    gbs = nbytes / (us * 1e-6) / 1e9
    log(f"score gather: {us:.2f} us/launch, {gbs:.1f} GB/s ({n_copies} copies)")
    # the whole score call as the two-pass path makes it (LUT build + gather)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(args.steps):
        lt = hip.build_lut(q, perm, 1.0 / math.sqrt(d), cents).reshape(b, hkv, rows, nb, nc)
        hip.score_gather_heads(lt, idxs[i % n_copies])
    e1.record()
    torch.cuda.synchronize()
    whole = e0.elapsed_time(e1) * 1e3 / args.steps
    check = None
    if args.cpu_seconds > 0:  # one head against the oracle's gather
        from oracle import sunshape_oracle as O

        hip.check(fn(*argv[0]))
        torch.cuda.synchronize()
        ref = O.gather_scores(lut[3, 5].cpu().numpy(), idxs[0][3, 5].cpu().numpy())
        got = outs[0][3, 5].cpu().numpy()
        check = float(np.abs(got - ref).max() / np.abs(ref).max())
    traffic = None  # HBM bytes per launch from the committed counter runs
    tf = os.path.join(ROOT, "profiles", "score_gather4_config4_traffic.json")
    if os.path.exists(tf):
        with open(tf) as f:
            tr = json.load(f)
        if tr.get("t_kv") == t_kv:
            traffic = tr.get("hbm_bytes_per_launch")
    line = {
        "metric": "compressed score gather µs/launch and achieved HBM GB/s (config-4 shape)",
        "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(us * 1e-3, 6), "us_per_step": round(us, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": f"score gather B=8 Hkv=8 rows=4 per KV head T={t_kv}, u8 indices "
                               "(16 blocks x 256 centroids), f32 scores; one launch over all "
                               "heads", "t_kv": t_kv, "cache_copies": n_copies,
                   "algorithmic_bytes_per_launch": nbytes},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic},
        "per_launch_us": {"mean": round(float(np.mean(per)), 3),
                          "median": round(float(np.median(per)), 3)},
        "lut_plus_gather_us": round(whole, 3),
        "check_max_rel_err_vs_oracle": check,
    }
    print(json.dumps(line), flush=True)
    return 0


def run_fit(args) -> int:
    """Codec fit of config 1 (seed 42: q_cal (1024, 128) and k_cal (2048, 128)
    N(0,1), profileperm_baseline, 15 k-means iterations): the per-block
    k-means of every block in one ss_kmeans_blocks launch, timed with HIP
    events, beside the NumPy k-means loop of the same fit on the host."""
    import numpy as np
    import torch

    import __graft_entry__

    pkg = __graft_entry__.load_package()
    hip = pkg._hip
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    rng = np.random.default_rng(42)
    k_cal = rng.standard_normal((2048, 128)).astype(np.float32)
    nb, bd, k, iters = 16, 8, 256, 15
    data = torch.from_numpy(np.ascontiguousarray(k_cal.reshape(2048, nb, bd).transpose(1, 0, 2))).to(dev)
    init = torch.stack([data[b][torch.from_numpy(np.random.RandomState(42 + b).permutation(2048)[:k])
                                .to(dev)] for b in range(nb)])
    for _ in range(2):
        hip.kmeans_blocks(data, init, iters)
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    n = max(3, args.steps // 20)
    ev0.record()
    for _ in range(n):
        out = hip.kmeans_blocks(data, init, iters)
    ev1.record()
    torch.cuda.synchronize()
    ms = ev0.elapsed_time(ev1) / n
    t0 = time.perf_counter()
    ref = [pkg.codec._kmeans(data[b].cpu().numpy(), k, n_iters=iters, seed=42 + b) for b in range(nb)]
    cpu_ms = (time.perf_counter() - t0) * 1e3
    x = data.cpu().numpy().astype(np.float64)

    def inertia(c):
        return float(np.mean([((x[b][:, None] - np.asarray(c[b], np.float64)[None]) ** 2)
                              .sum(-1).min(1).mean() for b in range(nb)]))

    flops = nb * iters * 2048 * k * bd * 2
    line = {
        "metric": "codec fit k-means ms (config 1: 16 blocks, 2048 points, 256 centroids, 15 iterations)",
        "value": round(ms, 4), "unit": "ms", "n_gpus": 1, "steps": n, "warmup": 2,
        "ms_per_step": round(ms, 4), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "ss_kmeans_blocks over the 16 blocks of k_cal (2048 x 128, seed 42)",
                   "assignment_flops_per_step": flops},
        "roofline": {"bound": "valu", "achieved": round(flops / (ms * 1e-3) / 1e12, 3),
                     "peak": FP32_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(flops / (ms * 1e-3) / 1e12 / FP32_PEAK_TFLOPS, 4),
                     "traffic": None},
        "cpu_baseline": {"value": round(cpu_ms, 2), "unit": "ms", "cores": 1, "kind": "port",
                         "sample": "the same 16-block k-means in NumPy (codec._kmeans), once"},
        "inertia": {"gpu": round(inertia(out.cpu().numpy()), 6), "numpy": round(inertia(ref), 6)},
    }
    print(json.dumps(line), flush=True)
    return 0


# MI355X's published fp32 peak (157.3 TFLOP/s); the fp32 vector issue rate
# without packed fp32 instructions (which this build does not emit) is half
# of it: 256 CUs x 4 SIMDs x 16 lanes x 2 flops x 2.4 GHz = 78.6 TFLOP/s
FP32_PEAK_TFLOPS = 157.3
VALU_FP32_UNPACKED_TFLOPS = 78.6


def run_encode(args) -> int:
    """Config 3: 65,536 fp16 keys (8 x 8192 x 128, per-dim scale
    exp(U[ln .25, ln 8]), seed 3) block-VQ encoded against a codebook fit on
    4096 draws of the same distribution; one ss_encode_blockvq launch per step.
    VALU-bound (direct-form distances, N*16*256*8*3 flops); GB/s reported
    beside TFLOP/s."""
    import numpy as np
    import torch

    import __graft_entry__

    pkg = __graft_entry__.load_package()
    hip = pkg._hip
    lib = hip.load_library()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    n_h, n_t, d, nb = 8, 8192, 128, 16
    rng = np.random.default_rng(3)
    s = np.exp(rng.uniform(np.log(0.25), np.log(8.0), d)).astype(np.float32)
    k_cal = (rng.standard_normal((4096, d)) * s).astype(np.float32)
    q_cal = (rng.standard_normal((4096, d)) * s).astype(np.float32)
    t0 = time.time()
    codec = pkg.codec.SunShapeBlockCodec(d, device=dev).fit(q_cal, k_cal, kmeans_iters=15, seed=3)
    log(f"codec fit {time.time() - t0:.1f}s")
    keys0 = torch.from_numpy((rng.standard_normal((n_h, n_t, d)) * s).astype(np.float16)).to(dev)
    per_copy = keys0.numel() * 2
    n_copies = args.copies or max(2, math.ceil(3 * MALL_BYTES / per_copy))
    keys = [keys0] + [keys0.clone() for _ in range(n_copies - 1)]
    outs = [torch.empty((n_h, n_t, nb), dtype=torch.uint8, device=dev) for _ in range(n_copies)]
    stream = torch.cuda.current_stream().cuda_stream
    prep = codec.encode_codebook()
    fn = lib.ss_encode_blockvq_prepared
    base = [(keys[i].data_ptr(), hip.SS_F16, 1, n_h, n_t, n_h * n_t * d, n_t * d, d, d,
             codec.permutation.data_ptr(), codec.centroids.data_ptr(), nb, 256, 8,
             outs[i].data_ptr(), n_h * n_t * nb, n_t * nb, nb) for i in range(n_copies)]
    argv = [a + (prep.data_ptr(), stream) for a in base]
    us, per = time_launches(fn, argv, args.steps, args.warmup, hip)
    # the plain (vector-ALU, direct-form) encoder on the same keys
    us_plain, _ = time_launches(lib.ss_encode_blockvq, [a + (stream,) for a in base],
                                max(args.steps // 4, 5), args.warmup, hip)
    n_tok = n_h * n_t
    nbytes = n_tok * d * 2 + n_tok * nb
    flops = n_tok * nb * 256 * 8 * 3
    gbs = nbytes / (us * 1e-6) / 1e9
    tflops = flops / (us * 1e-6) / 1e12
    log(f"encode: {us:.2f} us/step, {gbs:.1f} GB/s, {tflops:.1f} TFLOP/s direct-form equivalent "
        f"(plain encoder {us_plain:.2f} us)")
    # matrix-core work actually issued: 16 centroid tiles x 16 blocks per 16
    # tokens, one 16x16x32 fp16 product each
    mfma_flops = (n_tok // 16) * nb * 16 * 16 * 16 * 32 * 2
    check = None
    if args.cpu_seconds > 0:  # bit-exact check of 512 tokens against the oracle
        from oracle import sunshape_oracle as O

        hip.check(fn(*argv[0]))
        torch.cuda.synchronize()
        kk = keys0[0, :512].float().cpu().numpy()
        ref, near = O.encode_blockvq_c(kk, codec.centroids.cpu().numpy(),
                                       codec.permutation.cpu().numpy())
        got = outs[0][0, :512].cpu().numpy()
        check = int(((got != ref) & ~near).sum())
    line = {
        "metric": "block-VQ encode throughput (config 3)", "value": round(n_tok / (us * 1e-6), 1),
        "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(us * 1e-3, 6), "us_per_step": round(us, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "encode 8 x 8192 fp16 keys, D=128, 16 blocks x 256 centroids "
                               "(codec fit on 4096 draws), exact L2 argmin (matrix-core bound "
                               "filter, exact ranking of unresolved blocks)",
                   "tokens": n_tok, "cache_copies": n_copies, "bytes_per_step": nbytes,
                   "flops_per_step": flops},
        "roofline": {"bound": "valu", "achieved": round(tflops, 2), "peak": FP32_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tflops / FP32_PEAK_TFLOPS, 4),
                     "frac_of_unpacked_fp32": round(tflops / VALU_FP32_UNPACKED_TFLOPS, 4),
                     "mfma_tflops_issued": round(mfma_flops / (us * 1e-6) / 1e12, 2),
                     "traffic": None, "hbm_gbs": round(gbs, 2)},
        "plain_encoder_us": round(us_plain, 3),
        "per_launch_us": {"mean": round(float(np.mean(per)), 3),
                          "median": round(float(np.median(per)), 3)},
        "check_mismatches_vs_oracle_512_tokens": check,
    }
    print(json.dumps(line), flush=True)
    return 0


def main() -> int:
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported "
              "(the decode path would shard by KV head, with no exchange between GPUs)",
              file=sys.stderr)
        return 2
    if args.calibrate_copy:
        return calibrate_copy(args.calibrate_copy, args.steps)
    if args.workload == "hybrid":
        return run_hybrid(args)
    if args.workload == "fit":
        return run_fit(args)
    if args.workload == "config5":
        if args.t_kv == 32768 and "--t-kv" not in sys.argv:
            args.t_kv = 131072
        return run_config5(args)
    if args.workload == "turboquant":
        return run_turboquant(args)
    if args.workload == "encode":
        return run_encode(args)
    if args.workload == "prefill":
        return run_prefill(args)
    if args.workload == "scores":
        return run_scores(args)

    import numpy as np
    import torch

    import __graft_entry__

    pkg = __graft_entry__.load_package()
    hip = pkg._hip
    lib = hip.load_library()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    b, hq, hkv, d, t_kv = args.batch, 32, 8, 128, args.t_kv
    nb = d // 8
    scale = 1.0 / math.sqrt(d)

    # ---- codebook: fit on anisotropic N(0,1) * s calibration data ----
    rng = np.random.default_rng(2)
    s = rng.uniform(0.5, 4.0, d).astype(np.float32)
    k_cal = (rng.standard_normal((4096, d)) * s).astype(np.float32)
    q_cal = (rng.standard_normal((4096, d)) * s).astype(np.float32)
    t0 = time.time()
    codec = pkg.codec.SunShapeBlockCodec(d, device=dev).fit(q_cal, k_cal, kmeans_iters=15,
                                                            seed=2)
    log(f"codec fit {time.time() - t0:.1f}s")

    # ---- cache: encode fresh keys on the GPU; fp16 values ----
    g = torch.Generator(device=dev).manual_seed(2)
    s_t = torch.from_numpy(s).to(dev)
    keys = (torch.randn((b, hkv, t_kv, d), generator=g, device=dev) * s_t).to(torch.float16)
    idx0 = torch.empty((b, hkv, t_kv, nb), dtype=torch.uint8, device=dev)
    hip.encode_blockvq(keys, codec.permutation, codec.centroids, idx0, 8)
    v0 = torch.randn((b, hkv, t_kv, d), generator=g, device=dev).to(torch.float16)
    q = torch.randn((b, hq, 1, d), generator=g, device=dev).to(torch.float16)
    del keys
    if args.layout == "il8":
        # the cache's value layout: 8-token interleaved (append kernel)
        vbuf = torch.zeros((b, hkv, t_kv // 8, d, 8), dtype=torch.float16, device=dev)
        hip.append_values_il8(v0, vbuf, 0)
        fn, kind = lib.ss_decode_attn_il8, hip.KIND_IL8
    else:
        vbuf = v0
        fn, kind = lib.ss_decode_attn_dense, hip.KIND_DENSE
    per_copy = idx0.numel() + vbuf.numel() * 2
    n_copies = args.copies or max(2, math.ceil(3 * MALL_BYTES / per_copy))
    idxs = [idx0] + [idx0.clone() for _ in range(n_copies - 1)]
    vals = [vbuf] + [vbuf.clone() for _ in range(n_copies - 1)]
    torch.cuda.synchronize()
    log(f"cache ready: {n_copies} copies x {per_copy / 1e6:.1f} MB, layout {args.layout}")

    # ---- lean launcher: prebuilt C-ABI argument tuples, one per copy ----
    splits, ws_bytes = hip.decode_plan(kind, b, hq, hkv, 1, d, t_kv, args.splits)
    ws = torch.zeros(max(ws_bytes, 256), dtype=torch.uint8, device=dev)
    out = torch.empty((b, hq, 1, d), dtype=torch.float16, device=dev)

    # the il8 kernel reads the codec's split-fp16 codebook (prepared once per codec)
    cb = codec.kernel_codebook() if args.layout == "il8" else codec.centroids

    def arg_tuples(stream_handle):
        return [(q.data_ptr(), hip.SS_F16, b, hq, hkv, 1, d, scale, codec.permutation.data_ptr(),
                 cb.data_ptr(), nb, 256, idxs[i].data_ptr(), vals[i].data_ptr(),
                 hip.SS_F16, t_kv, t_kv, 0, 0, out.data_ptr(), hip.SS_F16, ws.data_ptr(),
                 ws_bytes, splits, stream_handle) for i in range(n_copies)]

    argv = arg_tuples(torch.cuda.current_stream().cuda_stream)

    def run(n, start=0):
        for i in range(start, start + n):
            rc = fn(*argv[i % n_copies])
            if rc:
                hip.check(rc)

    run(args.warmup)
    torch.cuda.synchronize()
    log(f"warmup {args.warmup} steps done (splits={splits}, workspace={ws_bytes} B)")

    if args.launch == "graph":
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            argv = arg_tuples(torch.cuda.current_stream().cuda_stream)
            run(n_copies)
        torch.cuda.synchronize()
        reps = max(1, args.steps // n_copies)
        steps = reps * n_copies
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        ev0.record()
        for _ in range(reps):
            graph.replay()
        ev1.record()
        torch.cuda.synchronize()
    else:
        steps = args.steps
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        ev0.record()
        run(steps)
        ev1.record()
        torch.cuda.synchronize()
    ms_total = ev0.elapsed_time(ev1)
    ms_step = ms_total / steps
    log(f"timed {steps} steps: {ms_step * 1e3:.2f} us/step")

    # per-launch durations (events bracket each launch on the launch stream)
    argv = arg_tuples(torch.cuda.current_stream().cuda_stream)
    n_pl = min(steps, 100)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(n_pl)]
    for i, (e0, e1) in enumerate(evs):
        e0.record()
        hip.check(fn(*argv[i % n_copies]))
        e1.record()
    torch.cuda.synchronize()
    per = np.array([e0.elapsed_time(e1) * 1e3 for e0, e1 in evs])

    nbytes = algorithmic_bytes(b, hq, hkv, d, t_kv, nb)
    gbs = nbytes / (ms_step * 1e-3) / 1e9
    # roofline: algorithmic bytes over the kernel's average launch duration
    # over the timed region (events on the launch stream bracket the region;
    # one C-ABI call is one launch on the il8 path, the kernel merges its
    # splits itself)
    kernel_gbs = gbs

    # ---- the drop-in path end to end: sunshape_sdpa on caches built through
    # the API (create_kv_cache + update_and_fetch), rotated like the kernel;
    # then whole decode steps (update_and_fetch of one token, then
    # sunshape_sdpa) on the same caches ----
    sdpa = step = None
    if args.layout == "il8":
        caches = []
        for i in range(n_copies):
            cache = pkg.cache.create_kv_cache(codec, n_kv_heads=hkv, max_tokens=t_kv + 1024)
            g2 = torch.Generator(device=dev).manual_seed(100 + i)
            kk = (torch.randn((b, hkv, t_kv, d), generator=g2, device=dev) * s_t).to(torch.float16)
            cache.update_and_fetch(kk, v0)
            caches.append(cache)
            del kk
        torch.cuda.synchronize()
        sdpa = time_api_steps(pkg, caches, q, scale, steps, args.warmup)
        sdpa["gbs"] = round(nbytes / (sdpa["us_per_step"] * 1e-6) / 1e9, 2)
        log(f"sunshape_sdpa end to end: {sdpa['us_per_step']:.2f} us/step "
            f"(host {sdpa['host_us_per_step']:.1f} us/call, {sdpa['backend']})")
        k1 = (torch.randn((b, hkv, 1, d), generator=g, device=dev) * s_t).to(torch.float16)
        v1 = torch.randn((b, hkv, 1, d), generator=g, device=dev).to(torch.float16)
        n_step = min(steps, 1024 * n_copies // 2)
        step = time_api_steps(pkg, caches, q, scale, n_step, args.warmup, kv_step=(k1, v1))
        step["t_kv_range"] = [t_kv, caches[0].offset]
        log(f"decode step end to end (update_and_fetch of one token + sunshape_sdpa): "
            f"{step['us_per_step']:.2f} us/step (host {step['host_us_per_step']:.1f} us/step, "
            f"{step['backend']})")
        # the same steps with the append as its own launch (fuse_steps off)
        for c in caches:
            c.fuse_steps = False
        sep = time_api_steps(pkg, caches, q, scale, n_step, args.warmup, kv_step=(k1, v1))
        step["separate_append"] = {k_: sep[k_] for k_ in ("us_per_step", "host_us_per_step")}
        log(f"  ... with the append launched separately: {sep['us_per_step']:.2f} us/step")
        del caches
    ceiling = stream_ceiling(nbytes, steps, args.warmup, hip)
    log(f"read ceiling: {ceiling['us_per_launch']:.2f} us ({ceiling['gbs']:.0f} GB/s)")

    traffic = None
    if os.path.exists(args.traffic_file):
        with open(args.traffic_file) as f:
            tr = json.load(f)
        if tr.get("t_kv") == t_kv and tr.get("batch") == b:
            traffic = tr.get("hbm_bytes_per_launch")

    # ---- output check + CPU baseline (oracle restatement, host cores) ----
    cpu = None
    check = None
    if args.cpu_seconds > 0:
        from threadpoolctl import threadpool_limits

        from oracle import sunshape_oracle as O

        hip.check(fn(*argv[0]))
        torch.cuda.synchronize()
        gpu_out = out.float().cpu().numpy().reshape(b, hq, d)
        perm = codec.permutation.cpu().numpy()
        cents = codec.centroids.cpu().numpy()
        q_np = q.cpu().numpy()
        q_t = O.apply_permutation(O.scale_query(q_np, scale), perm).astype(np.float32)
        q_t = q_t.reshape(b, hkv, hq // hkv, d)
        idx_np = idx0.cpu().numpy()
        v_np = v0.cpu().numpy()
        n_thr = cpu_threads()
        with threadpool_limits(1):
            forms = {}
            for name, fnc, budget in (
                    ("parallel", lambda *a: O.decode_cpu_parallel(*a, n_threads=n_thr), 0.6),
                    ("vectorised", O.decode_cpu_vectorised, 0.25),
                    ("reference_shaped", O.decode_cpu_reference_shaped, 0.15)):
                n_run, t_start, res = 0, time.perf_counter(), None
                while True:
                    res = fnc(q_t, cents, idx_np, v_np)
                    n_run += 1
                    if time.perf_counter() - t_start > args.cpu_seconds * budget:
                        break
                dt = (time.perf_counter() - t_start) / n_run
                forms[name] = (dt, n_run, res)
                log(f"cpu {name}: {dt * 1e3:.1f} ms/step over {n_run} steps")
        dt, n_run, res = forms["parallel"]
        check = float(np.abs(gpu_out - res).max() / np.abs(res).max())
        cpu = {
            "value": round(nbytes / dt / 1e9, 3),
            "unit": "GB/s",
            "cores": n_thr,
            "kind": "port",
            "sample": (f"{n_run} full steps of the metric workload by the NumPy float32 "
                       f"restatement on {n_thr} host threads (oracle.decode_cpu_parallel: "
                       f"(KV head, 4096-token chunk) units merged by log-sum-exp, 1 BLAS "
                       f"thread per worker), {dt * 1e3:.1f} ms/step; on one thread the "
                       f"head-vectorised form takes {forms['vectorised'][0] * 1e3:.1f} ms/step "
                       f"and the reference-shaped per-(b,h,r) loop "
                       f"{forms['reference_shaped'][0] * 1e3:.1f} ms/step"),
            "ms_per_step": round(dt * 1e3, 3),
            "host_cpus_visible": len(os.sched_getaffinity(0)),
            "blas_threads_per_worker": 1,
            "ms_per_step_1thread_vectorised": round(forms["vectorised"][0] * 1e3, 3),
            "ms_per_step_1thread_reference_shaped": round(forms["reference_shaped"][0] * 1e3, 3),
        }

    line = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 6),
        "us_per_step": round(ms_step * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "decode B=1 Hq=32 Hkv=8 D=128 T_kv=32768, 1-bit/dim SunShape keys "
                        "(u8 idx), fp16 values, fp16 query/output, f32 accumulate",
            "batch": b, "n_q_heads": hq, "n_kv_heads": hkv, "head_dim": d, "t_kv": t_kv,
            "splits": splits, "launch": args.launch, "cache_copies": n_copies,
            "value_layout": args.layout,
            "algorithmic_bytes_per_step": nbytes,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(kernel_gbs, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(kernel_gbs / HBM_PEAK_GBS, 4),
            "traffic": traffic,
        },
        "per_launch_us": {"mean": round(float(np.mean(per)), 3),
                          "median": round(float(np.median(per)), 3),
                          "p10": round(float(np.percentile(per, 10)), 3),
                          "p90": round(float(np.percentile(per, 90)), 3), "n": int(n_pl)},
        "cpu_baseline": cpu,
        "check_max_rel_err_vs_cpu": check,
        "sdpa_end_to_end": sdpa,
        "decode_step_end_to_end": step,
        "stream_ceiling": ceiling,
        "frac_of_stream_ceiling": round(ceiling["us_per_launch"] / (ms_step * 1e3), 4),
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
