"""Benchmark: forward token loop (prefill) and greedy decode on one MI355X.

Headline (`value`): prefill tok/s of the 7B shape (dim 4096, hidden 11008,
32 layers, 32 heads x 128, vocab 32000), seq 512, batch 1, fp16 weights and
activations with fp32 accumulation; one step = one forward + cross-entropy
loss over a batch whose tokens are already resident in HBM.  Weights are
N(0, 0.02) generated on the device, tokens uniform random.

The same JSON line carries:
  roofline      the dominant kernel (the W1|W3 GEMM + SwiGLU epilogue):
                algorithmic FLOPs per launch / mean launch time, timed with
                HIP events on the context stream inside the timed region
  forward_mfma  whole-forward algorithmic FLOPs / step time vs the fp16 peak
  decode        batch-1 greedy decode at ctx 2048 -> 2303 (graph replay) with
                its HBM roofline (compulsory bytes / step time vs 8 TB/s)
  prefill_batches / decode_batches / prefill_configs
                the same measurements at batch 4 and 16, and batch-1 prefill
                of the 600M and 5B shapes
  scheduler     32 forward requests through the request scheduler
  cpu_baseline  the CPU oracle (fp32 restatement of the reference forward)
                timed on the host cores over a bounded sample; likewise
                cpu_baseline_decode for one KV-cached greedy step
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_FP16_TFLOPS = 2516.6   # MI355X dense fp16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--seq", type=int, default=512)
    ap.add_argument("--config", default="7b", choices=["7b", "600m", "5b", "tiny"])
    ap.add_argument("--decode-steps", type=int, default=256)
    ap.add_argument("--decode-ctx", type=int, default=2048)
    ap.add_argument("--decode-batch", type=int, default=1)
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-extra", action="store_true",
                    help="only the headline configuration (no extra batches or model shapes)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--extra-batches", default="4,16", help="also time these prefill batches ('' for none)")
    ap.add_argument("--extra-decode-batches", default="16",
                    help="also time greedy decode at these batches ('' for none)")
    ap.add_argument("--extra-configs", default="600m,5b",
                    help="also time batch-1 prefill of these model shapes ('' for none)")
    ap.add_argument("--decode-only", action="store_true", help="skip the prefill timing")
    ap.add_argument("--train-only", action="store_true",
                    help="time only the training step (forward + backward)")
    ap.add_argument("--train-steps", type=int, default=5)
    ap.add_argument("--train-batches", default="1,4", help="batches of the training-step timing")
    ap.add_argument("--train-max-batch", type=int, default=10,
                    help="context batch capacity in --train-only runs (>= 10 adds the accum-10 train step)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run three 256 MiB device-to-device copies (a known-size kernel "
                         "for scaling hardware byte counters)")
    ap.add_argument("--decode-eager", action="store_true",
                    help="decode with eager launches instead of graph replay (profilers that "
                         "cannot follow graph capture)")
    ap.add_argument("--vendor-gemm", action="store_true",
                    help="only time hipBLASLt (torch.mm) at the 7B prefill GEMM shapes of batch 1, 4 and 16, "
                         "for reference")
    ap.add_argument("--no-graphs", action="store_true",
                    help="eager launches everywhere, prefill included (profilers that cannot follow "
                         "graph capture)")
    args = ap.parse_args()
    if args.vendor_gemm:
        print(json.dumps({"vendor_gemm": run_vendor_gemm()}), flush=True)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported in this build "
              "(multi-GPU sharding is design-only).", file=sys.stderr)
        sys.exit(2)

    from rustane_amd import hip_bridge as hb
    from rustane_amd import hip_rt
    from rustane_amd import engine as E

    cfg = {"7b": E.cfg_7b, "600m": E.cfg_600m, "5b": E.cfg_5b_deep, "tiny": E.tiny_config}[args.config]()
    cfg.seq = args.seq
    if args.no_extra:
        args.extra_batches = args.extra_decode_batches = args.extra_configs = ""
    extra = [int(x) for x in args.extra_batches.split(",") if x]
    extra_dec = [] if args.no_decode else [int(x) for x in args.extra_decode_batches.split(",") if x]
    train_b = [int(x) for x in args.train_batches.split(",") if x] if (args.train_only or not args.no_extra) else []
    max_batch = max([args.batch, args.decode_batch] + extra + extra_dec + train_b +
                    ([args.train_max_batch] if args.train_only else []))
    max_ctx = 0 if args.no_decode else args.decode_ctx + args.decode_steps
    log(f"[bench] config={args.config} B={args.batch} S={cfg.seq} max_ctx={max_ctx}")
    t0 = time.time()
    ctx = hb.Context(cfg.to_rh(), 0, max_batch, max_ctx)
    ctx.init_normal(seed=1234, std=0.02)
    if args.no_graphs:
        args.decode_eager = True
        ctx.set_graphs(False)
    log(f"[bench] context + weights ready in {time.time() - t0:.1f}s")

    stream = ctx.stream

    def run_prefill(B, steps, warmup, profile=True):
        rng = np.random.default_rng(99 + B)
        toks = rng.integers(0, cfg.vocab, size=(B, cfg.seq + 1)).astype(np.uint32)
        tok = hip_rt.DeviceArray.from_numpy(toks[:, :-1])
        tgt = hip_rt.DeviceArray.from_numpy(toks[:, 1:])
        mean = hip_rt.DeviceArray((B,), np.float32)
        for _ in range(warmup):  # the first call captures the forward's graph
            ctx.forward_dev(tok.ptr, tgt.ptr, B, cfg.seq, None, None, mean.ptr)
        ctx.sync()

        def timed_steps():
            ev0, ev1 = hip_rt.Event(), hip_rt.Event()
            hip_rt.synchronize()
            ev0.record(stream)
            t = time.perf_counter()
            for _ in range(steps):
                ctx.forward_dev(tok.ptr, tgt.ptr, B, cfg.seq, None, None, mean.ptr)
            ev1.record(stream)
            ctx.sync()
            hip_rt.synchronize()
            return ev0.elapsed_ms(ev1), time.perf_counter() - t

        # the timed region: one graph launch per step (eager with --no-graphs)
        ms, wall = timed_steps()
        loss = mean.numpy()
        k_ms, k_n, eager_ms = 0.0, 0, None
        if profile:
            # The W1|W3 GEMM's own duration: the same steps launched eagerly
            # with a HIP event pair attached to each of its dispatches (a
            # graph replays the same kernels with the same arguments).
            ctx.profile_enable(hb.K_GEMM_W13, True)
            eager_ms, _ = timed_steps()
            k_ms, k_n = ctx.profile_read(hb.K_GEMM_W13)
            ctx.profile_enable(hb.K_GEMM_W13, False)
        return ms, wall, k_ms, k_n, loss, eager_ms

    if args.copy_calibration:
        nb = 256 << 20
        src, dst = hip_rt.DeviceArray((nb,), np.uint8), hip_rt.DeviceArray((nb,), np.uint8)
        for _ in range(3):
            hip_rt.copy_d2d(dst, src, nb)
        hip_rt.synchronize()
        del src, dst
        log(f"[bench] copy calibration: 3 x {nb} bytes device-to-device")

    if args.decode_only:
        print(json.dumps({"decode": run_decode(ctx, cfg, args, hb, E, hip_rt, stream)}), flush=True)
        return
    if args.train_only:
        tr = {f"B{b}": run_train_step(ctx, cfg, args, E, b) for b in train_b}
        out = {"train_step": tr, "optimizer": run_optimizer(ctx, cfg, hb)}
        if ctx.max_batch >= 10:
            out["train_step_accum10"] = run_train_full(ctx, cfg, hb, E)
        print(json.dumps(out), flush=True)
        return

    B = args.batch
    ms, wall, k_ms, k_n, loss, eager_ms = run_prefill(B, args.steps, args.warmup)
    ms_step = ms / args.steps
    tok_s = B * cfg.seq * args.steps / (ms / 1e3)
    fl = E.prefill_flops(cfg, cfg.seq, B)
    w13_launch_flops = fl["w13_per_launch"]
    w13_avg_s = (k_ms / k_n) / 1e3 if k_n else float("nan")
    w13_tflops = w13_launch_flops / w13_avg_s / 1e12
    fwd_tflops = fl["total"] / (ms_step / 1e3) / 1e12
    log(f"[bench] prefill B={B}: {ms_step:.3f} ms/step ({'eager' if args.no_graphs else 'graph'}; "
        f"eager {eager_ms / args.steps if eager_ms else float('nan'):.3f}), {tok_s:.0f} tok/s, loss {loss}, "
        f"W13 GEMM {w13_avg_s * 1e6:.1f} us ({w13_tflops:.0f} TFLOP/s), forward {fwd_tflops:.0f} TFLOP/s")

    extra_lines = {}
    for eb in extra:
        e_ms, _, ek_ms, ek_n, _, _ = run_prefill(eb, max(3, args.steps // max(1, eb // 2)), 1)
        esteps = max(3, args.steps // max(1, eb // 2))
        efl = E.prefill_flops(cfg, cfg.seq, eb)
        ew13_us = (ek_ms / ek_n) * 1e3 if ek_n else None
        ew13_tf = efl["w13_per_launch"] / (ew13_us * 1e-6) / 1e12 if ew13_us else None
        extra_lines[f"B{eb}"] = {
            "tok_s": eb * cfg.seq * esteps / (e_ms / 1e3),
            "ms_per_step": e_ms / esteps,
            "forward_mfma_frac": efl["total"] / (e_ms / esteps / 1e3) / 1e12 / PEAK_FP16_TFLOPS,
            "w13_gemm_us": ew13_us,
            "roofline": None if ew13_tf is None else {
                "bound": "mfma", "kernel": "gemm_kernel<..., EPI_SWIGLU> (W1|W3 GEMM + SwiGLU)",
                "achieved": round(ew13_tf, 1), "peak": PEAK_FP16_TFLOPS, "unit": "TFLOP/s",
                "frac": round(ew13_tf / PEAK_FP16_TFLOPS, 4), "traffic": measured_traffic(args.config, eb, cfg.seq),
                "flops_per_launch": efl["w13_per_launch"], "mean_launch_us": round(ew13_us, 2),
                "traffic_source": "rocprofv3 FETCH_SIZE/WRITE_SIZE passes recorded in profiles/"},
        }
        log(f"[bench] prefill B={eb}: {extra_lines[f'B{eb}']}")

    sched = None
    if not args.no_extra and max_batch >= 16:
        sched = run_scheduler(ctx, cfg, hb, requests=32, max_batch=16)

    train = {f"B{b}": run_train_step(ctx, cfg, args, E, b) for b in train_b} if train_b else None
    optim = run_optimizer(ctx, cfg, hb) if train_b else None
    train_full = run_train_full(ctx, cfg, hb, E) if (train_b and max_batch >= 10) else None

    decode = None
    decode_lines = {}
    if not args.no_decode:
        decode = run_decode(ctx, cfg, args, hb, E, hip_rt, stream)
        for db in extra_dec:
            decode_lines[f"B{db}"] = run_decode(ctx, cfg, args, hb, E, hip_rt, stream, batch=db)
    ctx.close()

    config_lines = {}
    for name in [x for x in args.extra_configs.split(",") if x]:
        config_lines[name] = other_config_prefill(name, args, hb, E, hip_rt)

    cpu = None if args.no_cpu else cpu_baseline(cfg, args)
    cpu_dec = None if (args.no_cpu or args.no_decode) else cpu_baseline_decode(cfg, args)
    cpu_train = None if (args.no_cpu or not train_b) else cpu_baseline_train(cfg, args)

    line = {
        "metric": "prefill tok/s @7B seq512 fp16 (%MFMA); decode tok/s @7B b1 ctx2048 (%HBM)",
        "value": round(tok_s, 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic: weights N(0,0.02) from a device Philox generator, uniform random token ids",
        "config": {"workload": f"{args.config} prefill forward + CE loss", "dim": cfg.dim,
                   "hidden": cfg.hidden, "nlayers": cfg.nlayers, "heads": cfg.heads,
                   "head_dim": cfg.hd, "vocab": cfg.vocab, "seq_len": cfg.seq, "batch": B,
                   "global_batch": B, "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "mfma", "kernel": "gemm_kernel<..., EPI_SWIGLU> (W1|W3 GEMM + SwiGLU)",
                     "achieved": round(w13_tflops, 1), "peak": PEAK_FP16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(w13_tflops / PEAK_FP16_TFLOPS, 4),
                     "traffic": measured_traffic(args.config, B, cfg.seq),
                     "flops_per_launch": w13_launch_flops,
                     "mean_launch_us": round(w13_avg_s * 1e6, 2), "launches": k_n,
                     "timing": "HIP event pair attached to each W1|W3 GEMM dispatch, over the same steps "
                               "launched eagerly right after the timed region",
                     "traffic_source": "rocprofv3 FETCH_SIZE/WRITE_SIZE passes recorded in profiles/"},
        "forward_mfma": {"achieved_tflops": round(fwd_tflops, 1),
                         "frac": round(fwd_tflops / PEAK_FP16_TFLOPS, 4),
                         "flops_per_step": fl["total"]},
        "loss": float(loss[0]),
        "wall_s_timed": round(wall, 3),
        "launch": "eager" if args.no_graphs else "hip graph per forward",
        "eager_ms_per_step": round(eager_ms / args.steps, 4) if eager_ms else None,
    }
    if extra_lines:
        line["prefill_batches"] = extra_lines
    if decode:
        line["decode"] = decode
    if decode_lines:
        line["decode_batches"] = decode_lines
    if sched:
        line["scheduler"] = sched
    if train:
        line["train_step"] = train
    if optim:
        line["optimizer"] = optim
    if train_full:
        line["train_step_accum10"] = train_full
    if config_lines:
        line["prefill_configs"] = config_lines
    if cpu:
        line["cpu_baseline"] = cpu
    if cpu_dec:
        line["cpu_baseline_decode"] = cpu_dec
    if cpu_train:
        line["cpu_baseline_train"] = cpu_train
    print(json.dumps(line), flush=True)


def run_train_step(ctx, cfg, args, E, B):
    """One training step = zero the gradients, then forward + backward over
    one batch of B sequences (the weights do not change), timed by wall clock
    around rh_zero_grads + rh_forward_backward (each call synchronises)."""
    S = cfg.seq
    rng = np.random.default_rng(7)
    toks = rng.integers(0, cfg.vocab, size=(B, S + 1)).astype(np.uint32)
    tok, tgt = np.ascontiguousarray(toks[:, :-1]), np.ascontiguousarray(toks[:, 1:])
    t0 = time.perf_counter()
    ctx.forward_backward(tok, tgt)  # first call allocates gradients and transposed weights
    first = time.perf_counter() - t0
    ctx.forward_backward(tok, tgt)
    t = time.perf_counter()
    for _ in range(args.train_steps):
        ctx.zero_grads()
        loss = ctx.forward_backward(tok, tgt)
    ms = (time.perf_counter() - t) * 1e3 / args.train_steps
    flops = E.train_step_flops(cfg, S, B)
    tf = flops / (ms / 1e3) / 1e12
    out = {"tok_s": round(B * S / (ms / 1e3), 1), "ms_per_step": round(ms, 3), "steps": args.train_steps,
           "batch": B, "seq_len": S, "flops_per_step": flops, "achieved_tflops": round(tf, 1),
           "mfma_frac": round(tf / PEAK_FP16_TFLOPS, 4), "loss": float(loss[0]),
           "first_call_s": round(first, 3)}
    log(f"[bench] train step B={B}: {out}")
    return out


def run_optimizer(ctx, cfg, hb, steps=3):
    """The optimizer half of a training step over every parameter: the
    global gradient norm (a read of the fp32 gradients) and the fused AdamW
    update (per parameter: fp32 grad, m, v, master read; m, v, master written;
    fp16 device copy written = 30 bytes), timed by wall clock (each call
    synchronises)."""
    P = cfg.param_count() - cfg.dim * (2 * cfg.nlayers + 1)  # matrices + embedding
    G = cfg.param_count()                                      # + gammas
    tc = hb.train_config()
    ctx.update_weights(1, 1e-4, tc, 1.0)  # allocates the optimizer state
    t = time.perf_counter()
    for i in range(steps):
        ctx.update_weights(2 + i, 1e-4, tc, 1.0)
    upd_ms = (time.perf_counter() - t) * 1e3 / steps
    t = time.perf_counter()
    for _ in range(steps):
        ctx.grad_norm()
    norm_ms = (time.perf_counter() - t) * 1e3 / steps
    upd_bytes = 30 * P + 28 * (G - P)
    out = {"update_ms": round(upd_ms, 3), "update_bytes": upd_bytes,
           "update_gb_s": round(upd_bytes / (upd_ms / 1e3) / 1e9, 1),
           "update_hbm_frac": round(upd_bytes / (upd_ms / 1e3) / 1e9 / PEAK_HBM_GBS, 4),
           "grad_norm_ms": round(norm_ms, 3), "grad_norm_gb_s": round(4 * G / (norm_ms / 1e3) / 1e9, 1),
           "params": G}
    log(f"[bench] optimizer: {out}")
    return out


def run_train_full(ctx, cfg, hb, E, steps=3):
    """rh_train_step with TrainConfig's defaults (accum_steps 10: ten
    sequences per optimizer step, run as one batch, then the norm, clip and
    AdamW) over a synthetic uint16 token file, timed by wall clock."""
    import tempfile
    tc = hb.train_config()
    n = max(64 * cfg.seq, 200000)
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "train.bin")
        np.random.default_rng(8).integers(0, cfg.vocab, size=n).astype("<u2").tofile(path)
        data = hb.TokenData(path)
        ctx.train_step(data, 0, tc)  # warm-up (and state allocation)
        t = time.perf_counter()
        for s in range(1, steps + 1):
            loss, norm = ctx.train_step(data, s, tc)
        ms = (time.perf_counter() - t) * 1e3 / steps
        data.close()
    toks = tc.accum_steps * cfg.seq
    flops = E.train_step_flops(cfg, cfg.seq, tc.accum_steps)
    out = {"ms_per_step": round(ms, 2), "tok_s": round(toks / (ms / 1e3), 1), "accum_steps": tc.accum_steps,
           "tokens_per_step": toks, "achieved_tflops": round(flops / (ms / 1e3) / 1e12, 1),
           "mfma_frac": round(flops / (ms / 1e3) / 1e12 / PEAK_FP16_TFLOPS, 4), "loss": round(loss, 4),
           "grad_norm": round(norm, 4)}
    log(f"[bench] train_step (accum {tc.accum_steps}): {out}")
    return out


def run_scheduler(ctx, cfg, hb, requests, max_batch):
    """Forward requests (seq 512) submitted at once to the request scheduler
    (the multistream ForwardScheduler analogue): served in batches of up to
    max_batch; whole-run tok/s from the host clock, loss per request."""
    rng = np.random.default_rng(21)
    reqs = []
    for i in range(requests):
        t = rng.integers(0, cfg.vocab, size=cfg.seq + 1).astype(np.uint32)
        reqs.append((i, t[:-1], t[1:]))
    with hb.Scheduler(ctx, max_batch=max_batch, max_wait_us=2000) as s:
        s.run_batch(reqs[:max_batch])  # warm-up
        t = time.perf_counter()
        res = s.run_batch(reqs)
        wall = time.perf_counter() - t
    bad = [r.request_id for r in res if r.status != 0]
    out = {"requests": requests, "max_batch": max_batch, "seq_len": cfg.seq,
           "tok_s": round(requests * cfg.seq / wall, 1), "wall_s": round(wall, 4),
           "mean_batch": round(float(np.mean([r.batch for r in res])), 2),
           "mean_total_ms": round(float(np.mean([r.total_ms for r in res])), 2), "failed": bad}
    log(f"[bench] scheduler: {out}")
    return out


def other_config_prefill(name, args, hb, E, hip_rt, steps=10, warmup=2):
    """Batch-1 seq-512 prefill of another model shape (own context, device
    weights N(0, 0.02)): tok/s and whole-forward MFMA fraction."""
    cfg = {"7b": E.cfg_7b, "600m": E.cfg_600m, "5b": E.cfg_5b_deep, "tiny": E.tiny_config}[name]()
    cfg.seq = 512
    with hb.Context(cfg.to_rh(), 0, 1, 0) as c:
        c.init_normal(seed=4321, std=0.02)
        c.set_graphs(not args.no_graphs)
        rng = np.random.default_rng(11)
        toks = rng.integers(0, cfg.vocab, size=(1, cfg.seq + 1)).astype(np.uint32)
        tok = hip_rt.DeviceArray.from_numpy(toks[:, :-1])
        tgt = hip_rt.DeviceArray.from_numpy(toks[:, 1:])
        mean = hip_rt.DeviceArray((1,), np.float32)
        for _ in range(warmup):
            c.forward_dev(tok.ptr, tgt.ptr, 1, cfg.seq, None, None, mean.ptr)
        c.sync()
        ev0, ev1 = hip_rt.Event(), hip_rt.Event()
        ev0.record(c.stream)
        for _ in range(steps):
            c.forward_dev(tok.ptr, tgt.ptr, 1, cfg.seq, None, None, mean.ptr)
        ev1.record(c.stream)
        c.sync()
        ms = ev0.elapsed_ms(ev1) / steps
    fl = E.prefill_flops(cfg, cfg.seq, 1)["total"]
    out = {"dim": cfg.dim, "hidden": cfg.hidden, "nlayers": cfg.nlayers, "heads": cfg.heads,
           "vocab": cfg.vocab, "seq_len": cfg.seq, "tok_s": round(cfg.seq / (ms / 1e3), 1),
           "ms_per_step": round(ms, 4), "flops_per_step": fl,
           "forward_mfma_frac": round(fl / (ms / 1e3) / 1e12 / PEAK_FP16_TFLOPS, 4)}
    log(f"[bench] prefill {name}: {out}")
    return out


def measured_traffic(config, batch, seq):
    """HBM bytes per launch of the W1|W3 GEMM from the rocprofv3 FETCH_SIZE /
    WRITE_SIZE passes recorded in profiles/ (null when that workload has not
    been profiled)."""
    path = os.path.join(ROOT, "profiles", "gemm_w13_traffic.json")
    try:
        with open(path) as f:
            rec = json.load(f)
        return rec.get(f"{config}_b{batch}_s{seq}")
    except (OSError, ValueError):
        return None


def measured_decode_traffic(config, batch, ctx_start, mean_ctx):
    """HBM bytes per decode step at the run's mean context from the rocprofv3
    counter passes recorded in profiles/ (null when that workload has not
    been profiled)."""
    try:
        with open(os.path.join(ROOT, "profiles", "decode_traffic.json")) as f:
            rec = json.load(f).get(f"{config}_b{batch}_ctx{ctx_start}")
    except (OSError, ValueError):
        return None
    if not rec:
        return None
    pts = sorted((float(c), v) for c, v in rec["per_step_bytes_at_ctx"].items())
    return int(round(float(np.interp(mean_ctx, [c for c, _ in pts], [v for _, v in pts]))))


def run_decode(ctx, cfg, args, hb, E, hip_rt, stream, batch=None):
    B = batch or args.decode_batch
    ctx.set_graphs(not args.decode_eager)
    rng = np.random.default_rng(7)
    prompt = rng.integers(0, cfg.vocab, size=(B, args.decode_ctx)).astype(np.uint32)
    t = time.time()
    nxt, _ = ctx.prefill(prompt)
    log(f"[bench] decode prefill ctx={args.decode_ctx} B={B} in {time.time() - t:.2f}s")
    # warm-up: capture the step graph on a short run, then re-prefill
    ctx.decode(nxt, 4)
    nxt, _ = ctx.prefill(prompt)
    ev0, ev1 = hip_rt.Event(), hip_rt.Event()
    hip_rt.synchronize()
    ev0.record(stream)
    toks = ctx.decode(nxt, args.decode_steps)
    ev1.record(stream)
    ev1.synchronize()
    ms = ev0.elapsed_ms(ev1)
    ms_tok = ms / args.decode_steps
    mean_ctx = args.decode_ctx + (args.decode_steps - 1) / 2.0
    by = E.decode_bytes(cfg, mean_ctx, B)
    gbs = by["total"] / (ms_tok / 1e3) / 1e9
    # per-kernel HBM rate of the W1|W3 GEMV: a short eager pass with event timing
    nxt2, _ = ctx.prefill(prompt)
    ctx.set_graphs(False)
    ctx.profile_enable(hb.K_GEMV_W13, True)
    ctx.decode(nxt2, 8)
    k_ms, k_n = ctx.profile_read(hb.K_GEMV_W13)
    ctx.profile_enable(hb.K_GEMV_W13, False)
    ctx.set_graphs(not args.decode_eager)
    w13_bytes = 2 * cfg.hidden * cfg.dim * 2
    w13_gbs = w13_bytes / ((k_ms / k_n) / 1e3) / 1e9 if k_n else None
    out = {
        "tok_s": round(B * args.decode_steps / (ms / 1e3), 1),
        "ms_per_token_step": round(ms_tok, 4),
        "batch": B, "ctx_start": args.decode_ctx, "steps": args.decode_steps,
        "bytes_per_step": by["total"],
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4),
                     "traffic": measured_decode_traffic(args.config, B, args.decode_ctx, mean_ctx),
                     "traffic_source": "rocprofv3 FETCH_SIZE/WRITE_SIZE per decode kernel, summed over one step, "
                                       "recorded in profiles/decode_traffic.json"},
        "gemv_w13": {"bytes_per_launch": w13_bytes,
                     "mean_launch_us": round((k_ms / k_n) * 1e3, 2) if k_n else None,
                     "achieved_gbs": round(w13_gbs, 1) if w13_gbs else None},
        "first_tokens": [int(x) for x in toks[:8, 0]],
        "launch": "eager" if args.decode_eager else "hip graph per step",
    }
    log(f"[bench] decode B={B}: {out}")
    return out


CPU_METHOD = "1 warm-up + 3 timed runs, median (tests/bench_fwd_only_scale.rs:117-131)"


def median_time(fn, warmup=1, reps=3):
    """The reference's probe methodology: warm-up runs, then the median of
    the timed runs (tests/bench_fwd_only_scale.rs:117-131)."""
    for _ in range(warmup):
        fn()
    ts = []
    for _ in range(reps):
        t = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t)
    return float(np.median(ts))


def _oracle_layer_weights(rng, D, F):
    def mat(*s):
        return (rng.standard_normal(s, dtype=np.float32) * np.float32(0.02))

    return [mat(D, D), mat(D, D), mat(D, D), mat(D, D), mat(D, F), mat(D, F), mat(D, F),
            np.ones(D, np.float32), np.ones(D, np.float32)], mat


def cpu_host_info(L):
    return {"cores": int(L.orc_num_threads()), "omp_num_threads": os.environ.get("OMP_NUM_THREADS"),
            "nproc": os.cpu_count(), "method": CPU_METHOD}


def cpu_full_forward(oracle, E, name):
    """Full oracle forward + CE loss of a whole (small) model config, timed by
    the reference's method: the tiny config of the reference's CPU path
    (dim 512 / 8 layers / vocab 8192, seq 256) and the 600M shape at seq 512."""
    cfg = {"tiny": E.tiny_config, "600m": E.cfg_600m}[name]()
    D, F, V, S = cfg.dim, cfg.hidden, cfg.vocab, cfg.seq
    rng = np.random.default_rng(9)
    lw, mat = _oracle_layer_weights(rng, D, F)
    ocfg = oracle.make_config(D, F, cfg.heads, cfg.nlayers, V, head_dim=cfg.hd)
    w = oracle.Weights(mat(V, D), np.ones(D, np.float32), [lw] * cfg.nlayers)
    tok = rng.integers(0, V, size=(1, S + 1)).astype(np.uint32)
    a, b = np.ascontiguousarray(tok[:, :-1]), np.ascontiguousarray(tok[:, 1:])
    t = median_time(lambda: oracle.forward(ocfg, w, a, b, want_logits=False))
    return {"tok_s": round(S / t, 2), "ms_per_forward": round(t * 1e3, 2), "dim": D, "hidden": F,
            "nlayers": cfg.nlayers, "vocab": V, "seq_len": S}


def cpu_baseline(cfg, args):
    """Oracle forward at the benchmark shape over a bounded sample: 1 and 2
    layers (+ embedding, final norm, logits, CE) at seq 512, each timed by the
    reference's method, extrapolated linearly in the layer count; plus full
    forwards of the tiny and 600M configs."""
    try:
        import oracle
        from rustane_amd import engine as E
    except Exception as e:  # pragma: no cover
        log(f"[bench] no oracle: {e}")
        return None
    oracle.build()
    L = oracle.lib()
    D, F, V, S = cfg.dim, cfg.hidden, cfg.vocab, cfg.seq
    rng = np.random.default_rng(5)
    lw, mat = _oracle_layer_weights(rng, D, F)
    embed = mat(V, D)
    tok = rng.integers(0, V, size=(1, S + 1)).astype(np.uint32)
    a, b = np.ascontiguousarray(tok[:, :-1]), np.ascontiguousarray(tok[:, 1:])
    times = {}
    for nl in (1, 2):
        ocfg = oracle.make_config(D, F, cfg.heads, nl, V, head_dim=cfg.hd)
        w = oracle.Weights(embed, np.ones(D, np.float32), [lw] * nl)
        times[nl] = median_time(lambda: oracle.forward(ocfg, w, a, b, want_logits=False))
    t_layer = max(times[2] - times[1], 1e-9)
    t_total = times[1] + (cfg.nlayers - 1) * t_layer
    out = {"value": round(S / t_total, 2), "unit": "tok/s", "kind": "port", **cpu_host_info(L),
           "sample": f"oracle fp32 forward at dim {D}/hidden {F}/vocab {V}/seq {S} with 1 and 2 layers "
                     f"(medians {times[1]:.3f}s, {times[2]:.3f}s), extrapolated linearly to {cfg.nlayers} "
                     f"layers ({t_total:.2f}s per forward)"}
    out["full_forward"] = {name: cpu_full_forward(oracle, E, name) for name in ("tiny", "600m")}
    log(f"[bench] cpu baseline: {out}")
    return out


def cpu_baseline_train(cfg, args):
    """Oracle forward + backward (fp32, all host cores) at the same shape over
    a bounded sample: 1 and 2 layers at seq 512, extrapolated linearly."""
    try:
        import oracle
    except Exception as e:  # pragma: no cover
        log(f"[bench] no oracle: {e}")
        return None
    oracle.build()
    D, F, V, S = cfg.dim, cfg.hidden, cfg.vocab, cfg.seq
    rng = np.random.default_rng(6)

    def mat(*s):
        return (rng.standard_normal(s, dtype=np.float32) * np.float32(0.02))

    lw, mat = _oracle_layer_weights(rng, D, F)
    embed = mat(V, D)
    tok = rng.integers(0, V, size=(1, S + 1)).astype(np.uint32)
    a, b = np.ascontiguousarray(tok[:, :-1]), np.ascontiguousarray(tok[:, 1:])
    times = {}
    for nl in (1, 2):
        ocfg = oracle.make_config(D, F, cfg.heads, nl, V, head_dim=cfg.hd)
        w = oracle.Weights(embed, np.ones(D, np.float32), [lw] * nl)
        times[nl] = median_time(lambda: oracle.forward_backward(ocfg, w, a, b))
    t_layer = max(times[2] - times[1], 1e-9)
    t_total = times[1] + (cfg.nlayers - 1) * t_layer
    return {"value": round(S / t_total, 2), "unit": "tok/s", "kind": "port", **cpu_host_info(oracle.lib()),
            "sample": f"oracle fp32 forward + backward at dim {D}/hidden {F}/vocab {V}/seq {S} with 1 and 2 "
                      f"layers (medians {times[1]:.2f}s, {times[2]:.2f}s), extrapolated linearly to "
                      f"{cfg.nlayers} layers ({t_total:.1f}s per step)"}


def cpu_baseline_decode(cfg, args, steps=4):
    """Oracle KV-cached greedy step at the same width over a bounded sample:
    1 and 2 layers, a 2048-token prompt, median of a few steps, extrapolated
    linearly in the layer count (the tied-logits GEMV is in both samples)."""
    try:
        import oracle
    except Exception as e:  # pragma: no cover
        log(f"[bench] no oracle: {e}")
        return None
    oracle.build()
    L = oracle.lib()
    D, F, V = cfg.dim, cfg.hidden, cfg.vocab
    ctx_len = args.decode_ctx
    rng = np.random.default_rng(6)

    def mat(*s):
        return (rng.standard_normal(s, dtype=np.float32) * np.float32(0.02))

    lw, mat = _oracle_layer_weights(rng, D, F)
    embed = mat(V, D)
    prompt = rng.integers(0, V, size=ctx_len).astype(np.uint32)
    step_s = {}
    for nl in (1, 2):
        ocfg = oracle.make_config(D, F, cfg.heads, nl, V, head_dim=cfg.hd)
        w = oracle.Weights(embed, np.ones(D, np.float32), [lw] * nl)
        kv = oracle.KV(ocfg, ctx_len + steps + 2)
        lg = kv.prefill(w, prompt)
        state = {"tok": int(np.argmax(lg))}

        def one():
            state["tok"], _ = kv.step(w, state["tok"])

        step_s[nl] = median_time(one, warmup=1, reps=steps - 1)
    t_layer = max(step_s[2] - step_s[1], 1e-9)
    t_step = step_s[1] + (cfg.nlayers - 1) * t_layer
    return {"value": round(1.0 / t_step, 3), "unit": "tok/s", "kind": "port", "batch": 1, **cpu_host_info(L),
            "sample": f"oracle fp32 KV-cached greedy step at dim {D}/hidden {F}/vocab {V}, ctx {ctx_len}, "
                      f"1 and 2 layers (1 warm-up step, median of {steps - 1}: {step_s[1] * 1e3:.1f} ms, "
                      f"{step_s[2] * 1e3:.1f} ms), extrapolated linearly to {cfg.nlayers} layers "
                      f"({t_step * 1e3:.0f} ms per token)"}


def run_vendor_gemm(iters=30, rows=(512, 2048, 8192)):
    """hipBLASLt through torch.mm at the 7B prefill GEMM shapes for batch 1,
    4 and 16 of 512 tokens (M = 512, 2048, 8192; fp16 operands, fp16 output,
    weights [N, K] as the library stores them), each weight rotated over more
    than 1 GiB of copies so every launch reads it from HBM past the 256 MB
    last-level cache, as the forward does.  A reference point for the
    library's GEMMs, which also fuse their epilogues (RoPE and the cache
    scatter, SwiGLU, residual + RMSNorm)."""
    import torch
    shapes = {"QKV": (12288, 4096), "W1|W3": (22016, 4096), "W2": (4096, 11008), "Wo": (4096, 4096),
              "logits": (32000, 4096)}
    out = {}
    for M in rows:
        for name, (N, K) in shapes.items():
            g = torch.Generator(device="cuda").manual_seed(5)
            a = torch.randn(M, K, device="cuda", dtype=torch.float16, generator=g)
            nrot = (1 << 30) // (N * K * 2) + 2
            ws = [torch.randn(N, K, device="cuda", dtype=torch.float16, generator=g) for _ in range(nrot)]
            for w in ws[:2]:
                torch.mm(a, w.t())
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for i in range(iters):
                torch.mm(a, ws[i % nrot].t())
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / iters
            tf = 2.0 * M * N * K / us / 1e6
            out[f"{name} M{M}"] = {"M": M, "N": N, "K": K, "us": round(us, 2), "tflops": round(tf, 1),
                                   "mfma_frac": round(tf / PEAK_FP16_TFLOPS, 4)}
            log(f"[bench] hipBLASLt {name} {M}x{N}x{K}: {us:.2f} us, {tf:.0f} TFLOP/s")
            del ws
    return out


if __name__ == "__main__":
    main()
