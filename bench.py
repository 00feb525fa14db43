#!/usr/bin/env python3
"""Throughput of the quantized GEMV hot path on one MI355X.

Default workload: one Phi-4-mini decoder layer's projections as Q4_0 GEMVs at
batch 1 (qkv 3072->5120, o_proj 3072->3072, gate_up 3072->16384,
down 8192->3072), FP32 activations N(0,1), synthetic seeded weights.  One
step = the four GEMVs over one copy of the layer's weights.  Steps rotate
over distinct weight copies (> 512 MB in total) so every launch streams its
weights from HBM rather than from the 256 MB Infinity Cache.

    python bench.py [--steps K] [--warmup W] [--gpus 1]

Prints one JSON line (stdout).  Progress goes to stderr.
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

HBM_PEAK_GBS = 8000.0
PREFILL_LAUNCHES_PER_PLAN = 8
METRIC = "quantized GEMV HBM GB/s (% of 8 TB/s); decode tok/s at Phi-4-mini shape"

# (name, rows = output features, cols = input features)
LAYER_Q4_0 = [("qkv", 5120, 3072), ("o_proj", 3072, 3072), ("gate_up", 16384, 3072), ("down", 3072, 8192)]
CONFIGS = {
    "layer_q4_0": ("Phi-4-mini decoder layer projections as Q4_0 GEMVs, batch 1", 2, LAYER_Q4_0),
    "q8_0_3072": ("single Q8_0 3072x3072 GEMV, batch 1", 8, [("matvec", 3072, 3072)]),
}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def synth_weights(fmt: int, rows: int, cols: int, rng: np.random.Generator) -> np.ndarray:
    """GGUF blocks with the workload's distributions (numpy RNG)."""
    from sharpinference_amd import native
    nb = rows * cols // 32
    if fmt == native.Q4_0:
        d = (np.abs(rng.standard_normal(nb) * 0.02) / 8).astype(np.float16)
        q = rng.integers(0, 256, size=(nb, 16), dtype=np.uint8)
        out = np.empty((nb, 18), np.uint8)
        out[:, :2] = d.view(np.uint8).reshape(nb, 2)
        out[:, 2:] = q
        return out.reshape(-1)
    if fmt == native.Q8_0:
        d = (np.abs(rng.standard_normal(nb) * 0.02) / 127).astype(np.float16)
        q = rng.integers(-127, 128, size=(nb, 32), dtype=np.int8)
        out = np.empty((nb, 34), np.uint8)
        out[:, :2] = d.view(np.uint8).reshape(nb, 2)
        out[:, 2:] = q.view(np.uint8)
        return out.reshape(-1)
    raise ValueError(fmt)


def plan_schedule(n: int, copies: int) -> list:
    """Plan launches of n layer-set steps: ("round",) for each whole round of
    `copies` steps (one plan holding the round), then ("rest", r) for the r
    remaining steps (one plan holding them)."""
    full, rest = divmod(n, copies)
    return [("round",)] * full + ([("rest", rest)] if rest else [])


def one_plan_schedule(n: int, copies: int) -> list:
    """Plan launches of n steps with one plan per step: ("one", c) for the
    step over weight copy c."""
    return [("one", i % copies) for i in range(n)]


def warmup_schedule(steps: int, warmup: int, copies: int) -> list:
    """Untimed launches before timing: the warm-up steps themselves, every
    plan the timed region launches that they did not, then every one-step
    plan once, so that no plan is launched for the first time while timed."""
    keys = plan_schedule(max(warmup, 1), copies)
    for key in plan_schedule(steps, copies) + one_plan_schedule(min(steps, copies), copies):
        if key not in keys:
            keys.append(key)
    return keys


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--config", default="layer_q4_0", choices=sorted(CONFIGS))
    ap.add_argument("--copies", type=int, default=0, help="weight copies to rotate (0: enough for 640 MB)")
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="bounded CPU-baseline budget")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-prefill", action="store_true", help="skip the batched prefill (MFMA) measurement")
    ap.add_argument("--no-decode", action="store_true", help="skip the Phi-4-mini decode-step measurement")
    ap.add_argument("--no-rwkv", action="store_true", help="skip the RWKV-7 token-step measurement")
    ap.add_argument("--no-ceiling", action="store_true", help="skip the plain-read ceiling leg")
    ap.add_argument("--no-legs", action="store_true",
                    help="skip the single-matrix legs (Q8_0 and F16 3072x3072, F16 head) and the F16 decode step")
    ap.add_argument("--decode-only", action="store_true",
                    help="only the Phi-4 and RWKV-7 token loops (one token at a time, no back-to-back "
                         "replays, no CPU leg); prints their JSON; for kernel-trace profiles")
    ap.add_argument("--eager", action="store_true",
                    help="with --decode-only: launch each step kernel by kernel instead of replaying its graph; "
                         "with --prefill-only: launch the four products --rounds times back to back, no graph")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only the batched prefill leg (M = 512, Q4_0 layer shapes); prints its JSON")
    ap.add_argument("--rounds", type=int, default=400,
                    help="with --prefill-only --eager: rounds of the four products (the first ~30 ms of work "
                         "run at lower clocks; a kernel trace takes the later launches)")
    ap.add_argument("--copy-calibration-mib", type=int, default=0,
                    help="before timing, copy this many MiB device-to-device once (a plain copy of "
                         "known size that scales the HBM byte counters of a profiler run)")
    ap.add_argument("--batch-ops", action="store_true",
                    help="only the batched prefill operators at 16 rows (the Phi-4 Q4_K layer mat-vecs and the "
                         "attention chain), launched eagerly and event-timed: a kernel trace of this run sees "
                         "every launch")
    ap.add_argument("--prefill-vendor", action="store_true",
                    help="only torch's dense bf16 linear (hipBLASLt) at the prefill shapes with bf16 W (no "
                         "dequant): a library reference, not a product path; torch's own HIP runtime does "
                         "not share a process with this library's, so the leg runs alone")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported in this build "
              "(the GEMV would shard by output rows, each GPU taking one slice of W's rows; "
              "this bench measures one GPU's share)", file=sys.stderr)
        return 2
    if args.steps < 1 or args.warmup < 0:
        print("--steps must be >= 1 and --warmup >= 0", file=sys.stderr)
        return 2

    if args.prefill_vendor:   # before this library is loaded
        print(json.dumps({"vendor_dense_bf16": bench_vendor_dense()}), flush=True)
        return 0

    from sharpinference_amd import native

    if args.prefill_only:
        hip = native.HipContext(0)
        rng = np.random.default_rng(20250101)
        res = prefill_eager(hip, rng, args.rounds) if args.eager else bench_prefill(hip, rng)
        hip.close()
        print(json.dumps({"prefill": res}), flush=True)
        return 0

    if args.batch_ops:
        hip = native.HipContext(0)
        res = bench_batch_ops(hip)
        hip.close()
        print(json.dumps({"batch_ops": res}), flush=True)
        return 0

    if args.decode_only:
        hip = native.HipContext(0)
        res = {"decode": None if args.no_decode else bench_decode(hip, cpu=False, replay_timing=False,
                                                                   eager=args.eager),
               "decode_rwkv7": None if args.no_rwkv else bench_rwkv_decode(hip, cpu=False, replay_timing=False,
                                                                           eager=args.eager)}
        hip.close()
        print(json.dumps(res), flush=True)
        return 0

    desc, fmt, shapes = CONFIGS[args.config]
    rng = np.random.default_rng(20250101)
    bytes_per_step = 0
    host_w = []
    for name, rows, cols in shapes:
        w = synth_weights(fmt, rows, cols, rng)
        assert w.nbytes == native.tensor_bytes(fmt, rows, cols)
        host_w.append(w)
        bytes_per_step += w.nbytes + 4 * (rows + cols)
    wbytes_per_copy = sum(w.nbytes for w in host_w)
    copies = args.copies or max(2, -(-640 * 2 ** 20 // wbytes_per_copy))
    log(f"{desc}: {bytes_per_step} algorithmic bytes/step, {copies} weight copies "
        f"({copies * wbytes_per_copy / 2 ** 20:.0f} MiB)")

    hip = native.HipContext(0)
    xs = {}
    for name, rows, cols in shapes:
        if cols not in xs:
            xs[cols] = hip.to_device(rng.standard_normal(cols).astype(np.float32))
    ys = {name: hip.alloc(rows * 4) for name, rows, cols in shapes}
    dev_w = []
    for c in range(copies):
        per = []
        for w in host_w:
            b = hip.alloc(w.nbytes)
            b.upload(w)
            per.append(b)
        dev_w.append(per)

    def record_steps(first: int, n: int):
        def body():
            for i in range(n):
                for (name, rows, cols), wb in zip(shapes, dev_w[(first + i) % copies]):
                    hip.gemv(fmt, wb.ptr, xs[cols].ptr, ys[name].ptr, rows, cols)
        return hip.record(body)

    # Submission: one recorded plan holds a round of `copies` steps (each step
    # = the layer's GEMVs, in order on the stream, over one weight copy), as
    # a model's layers share one submission; a remainder of steps uses
    # one plan holding those steps.  Launching one small plan per step instead
    # adds a plan-launch gap to every step, reported as `one_plan_per_step`.
    round_plan = record_steps(0, copies)
    plans = [record_steps(c, 1) for c in range(copies)]
    rest_plans = {}
    for key in warmup_schedule(args.steps, args.warmup, copies):
        if key[0] == "rest" and key[1] not in rest_plans:
            rest_plans[key[1]] = record_steps(0, key[1])

    def plan_of(key):
        if key[0] == "round":
            return round_plan
        return rest_plans[key[1]] if key[0] == "rest" else plans[key[1]]

    def launch(keys) -> None:
        """Launches the plans named by `keys`, in order, on the library's stream."""
        if keys:
            hip.launch_sequence([plan_of(k) for k in keys], len(keys))

    # per-shape plans (rotation over copies) for the per-kernel breakdown
    shape_plans = {}
    for k, (name, rows, cols) in enumerate(shapes):
        def body(k=k, name=name, rows=rows, cols=cols):
            for c in range(copies):
                hip.gemv(fmt, dev_w[c][k].ptr, xs[cols].ptr, ys[name].ptr, rows, cols)
        shape_plans[name] = hip.record(body)

    if args.copy_calibration_mib > 0:
        n = args.copy_calibration_mib * 2 ** 20
        src, dst = hip.alloc(n), hip.alloc(n)
        hip.fill_u32(src.ptr, 0x3F800000, n // 4)
        hip.copy(dst.ptr, src.ptr, n)
        hip.sync()
        src.free()
        dst.free()
        log(f"calibration copy of {args.copy_calibration_mib} MiB done")

    # warm-up: the W steps, then every plan the timed region launches that
    # those steps did not (a graph's first launch pays its upload and the
    # first touch of its kernels), then every one-step plan
    log(f"warmup {args.warmup} steps + every plan the timed region launches")
    launch(warmup_schedule(args.steps, args.warmup, copies))
    hip.sync()

    log(f"timing {args.steps} steps")
    hip.sync()
    hip.timer_begin()
    launch(plan_schedule(args.steps, copies))
    ms = hip.timer_end()
    hip.sync()
    s_per_step = ms / 1e3 / args.steps
    gbs = bytes_per_step / s_per_step / 1e9
    log(f"{ms:.3f} ms for {args.steps} steps -> {s_per_step * 1e6:.2f} us/step, {gbs:.1f} GB/s")
    hip.timer_begin()
    launch(one_plan_schedule(args.steps, copies))
    ms1 = hip.timer_end()
    one_plan = {"us_per_step": round(ms1 * 1e3 / args.steps, 3),
                "GBs": round(bytes_per_step / (ms1 / 1e3 / args.steps) / 1e9, 1)}
    log(f"one plan per step: {one_plan['us_per_step']:.2f} us/step, {one_plan['GBs']:.1f} GB/s")

    kernels = {}
    for k, (name, rows, cols) in enumerate(shapes):
        plan = shape_plans[name]
        plan.measure_us(4)
        samples = sorted(plan.measure_us(16) for _ in range(9))
        us = samples[4] / copies          # median, per launch
        b = host_w[k].nbytes + 4 * (rows + cols)
        kernels[name] = {"rows": rows, "cols": cols, "bytes": b, "us_per_launch": round(us, 3),
                         "GBs": round(b / us / 1e3, 1), "frac": round(b / us / 1e3 / HBM_PEAK_GBS, 4)}
        log(f"  {name:8s} {rows}x{cols}: {us:.3f} us/launch, {b / us / 1e3:.1f} GB/s")

    batched, batched_plan = bench_batched_form(hip, shapes, copies, dev_w, xs, ys, fmt, bytes_per_step)
    plans[0].launch()   # the outputs the CPU parity check reads come from the timed path's kernels again
    hip.sync()

    ceiling = None if args.no_ceiling else bench_read_ceiling(hip, shapes, copies, dev_w, host_w)

    legs = None if args.no_legs else bench_matvec_legs(hip, rng)
    prefill = None if args.no_prefill else bench_prefill(hip, rng)
    decode = None if args.no_decode else bench_decode(hip, cpu=not args.no_cpu)
    decode_f16 = None if args.no_decode or args.no_legs else bench_decode_dense(hip)
    rwkv = None if args.no_rwkv else bench_rwkv_decode(hip, cpu=not args.no_cpu)

    # dispatch floor: the same graph mechanism with 64 one-wave fill kernels
    scratch = hip.alloc(4096)
    floor_plan = hip.record(lambda: [hip.fill_u32(scratch.ptr, 0, 64) for _ in range(64)])
    floor_plan.measure_us(2)
    floor_us = sorted(floor_plan.measure_us(8) for _ in range(5))[2] / 64
    floor_plan.destroy()
    scratch.free()
    log(f"dispatch floor: {floor_us:.3f} us per dependent launch")

    result = {
        "metric": METRIC,
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(s_per_step * 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded numpy; GGUF blocks, weights resident in HBM)",
        "config": {
            "workload": desc,
            "weights": native.FORMAT_NAMES[fmt],
            "shapes": [[n, r, c] for n, r, c in shapes],
            "batch": 1,
            "weight_copies_rotated": copies,
            "steps_per_plan": copies,
            "parallelism": "single GPU",
        },
        "one_plan_per_step": one_plan,
        "independent_products_batched": batched,
        "hbm_fraction": round(gbs / HBM_PEAK_GBS, 4),
        "kernels": kernels,
        "dispatch_floor_us": round(floor_us, 3),
        "plain_read_ceiling": ceiling,
        "matvec_legs": legs,
        "prefill": prefill,
        "decode": decode,
        "decode_f16": decode_f16,
        "decode_rwkv7": rwkv,
        "roofline": {
            "bound": "hbm",
            "achieved": round(gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4),
            "traffic": committed_traffic(args.config),
            "kernel": f"gemv_fast_kernel ({native.FORMAT_NAMES[fmt]}), launch-averaged over the step's "
                      f"{len(shapes)} GEMVs",
            # event-timed average launch of the step's GEMVs: the kernel's
            # duration plus whatever gap separates consecutive launches
            # (a kernel trace of the same run gives the duration alone)
            "launch_us": round(s_per_step * 1e6 / len(shapes), 3),
            "dispatch_floor_us": round(floor_us, 3),
        },
    }

    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(fmt, shapes, host_w, xs, ys, hip, bytes_per_step, args.cpu_seconds)

    for plan in plans + [round_plan, batched_plan] + list(shape_plans.values()) + list(rest_plans.values()):
        plan.destroy()
    hip.close()
    print(json.dumps(result), flush=True)
    return 0


def time_rotated_gemv(hip, fmt, host, rows, cols, copies, rng):
    """Median event-timed microseconds per launch of one GEMV shape: a plan
    of `copies` dependent launches over distinct weight copies."""
    from sharpinference_amd import native
    dev = []
    for _ in range(copies):
        b = hip.alloc(host.nbytes)
        b.upload(host)
        dev.append(b)
    x = hip.to_device(rng.standard_normal(cols).astype(np.float32))
    y = hip.alloc(4 * rows)
    plan = hip.record(lambda: [hip.gemv(fmt, b.ptr, x.ptr, y.ptr, rows, cols) for b in dev])
    plan.measure_us(2)
    us = sorted(plan.measure_us(8) for _ in range(7))[3] / copies
    plan.destroy()
    for b in dev + [x, y]:
        b.free()
    nbytes = host.nbytes + 4 * (rows + cols)
    return {"format": native.FORMAT_NAMES[fmt], "rows": rows, "cols": cols, "bytes": nbytes,
            "weight_copies_rotated": copies, "us_per_launch": round(us, 3), "GBs": round(nbytes / us / 1e3, 1),
            "frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4)}


def bench_batched_form(hip, shapes, copies, dev_w, xs, ys, fmt, bytes_per_step):
    """The layer set's four products through si_hip_gemv_batch.  Their
    synthetic activations are independent inputs, so the three 3072-column
    products can share one launch and down takes a second: a step is two
    launches instead of four.  This is not the decode's order (there qkv,
    attention, o_proj, gate_up and down each need the one before); it shows
    the kernels' rate with half the dependent-launch floors per byte.  The
    plan (one step per weight copy) is returned for the caller to destroy at
    the end of the run."""
    from sharpinference_amd import native
    ops = [[native.gemv_op(fmt, dev_w[c][k].ptr, xs[cols].ptr, ys[name].ptr, rows, cols)
            for k, (name, rows, cols) in enumerate(shapes)] for c in range(copies)]
    paths = []
    plan = hip.record(lambda: [paths.append(hip.gemv_batch(ops[c])) for c in range(copies)])
    settle(lambda: plan.measure_us(4))
    us = sorted(plan.measure_us(8) for _ in range(5))[2] / copies
    gbs = bytes_per_step / us / 1e3
    log(f"independent products batched (2 launches per step): {us:.2f} us/step, {gbs:.1f} GB/s "
        f"({gbs / HBM_PEAK_GBS * 100:.1f}% of HBM)")
    return {"us_per_step": round(us, 3), "GBs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
            "launches_per_step": 2, "paths": paths[0] if paths else None,
            "form": "si_hip_gemv_batch: qkv, o_proj and gate_up in one launch, down in a second; "
                    "the step's products as independent inputs (not the decode's dependent order)"}, plan


def bench_read_ceiling(hip, shapes, copies, dev_w, host_w):
    """Plain-read ceiling: the same bytes, read once by a streaming kernel
    (si_hip_checksum), in the same plan structure (one launch per weight
    tensor, the step's four in order, rotating over the copies)."""
    from sharpinference_amd import native
    acc = hip.alloc(4 * native.CHECKSUM_PARTS)
    read_plan = hip.record(lambda: [hip.checksum(dev_w[c][k].ptr, host_w[k].nbytes, acc.ptr)
                                    for c in range(copies) for k in range(len(shapes))])
    read_plan.measure_us(2)
    read_us = sorted(read_plan.measure_us(8) for _ in range(5))[2] / copies
    read_w = sum(w.nbytes for w in host_w)
    read_shapes = {}
    for k, (name, rows, cols) in enumerate(shapes):
        plan = hip.record(lambda k=k: [hip.checksum(dev_w[c][k].ptr, host_w[k].nbytes, acc.ptr)
                                       for c in range(copies)])
        plan.measure_us(2)
        us = sorted(plan.measure_us(8) for _ in range(5))[2] / copies
        read_shapes[name] = {"bytes": host_w[k].nbytes, "us_per_launch": round(us, 3),
                             "GBs": round(host_w[k].nbytes / us / 1e3, 1)}
        plan.destroy()
    read_plan.destroy()
    acc.free()
    ceiling = {"kernel": "checksum_kernel (streaming 16-byte reads, one partial per workgroup)", "us_per_step": round(read_us, 3),
               "GBs": round(read_w / read_us / 1e3, 1), "frac": round(read_w / read_us / 1e3 / HBM_PEAK_GBS, 4),
               "shapes": read_shapes}
    log(f"plain-read ceiling of the same weights: {read_us:.2f} us/step, {read_w / read_us / 1e3:.0f} GB/s")
    return ceiling


def bench_matvec_legs(hip, rng):
    """Single-matrix lines beside the layer set: the minimum slice (Q8_0
    3072x3072, weights uniform in [-127, 127], d = |N(0, 0.02)| / 127), the
    reference's own F16 weights at the same shape, and the F16 200064 x 3072
    tied vocabulary head of the reference's Phi-4 model.  Copies rotate
    through > 512 MB so every launch reads HBM."""
    from sharpinference_amd import native
    from sharpinference_amd.synth import synth_blocks
    out = {}
    for key, fmt, rows, cols in (("q8_0_3072x3072", native.Q8_0, 3072, 3072),
                                 ("f16_3072x3072", native.F16, 3072, 3072),
                                 ("f16_head_200064x3072", native.F16, 200064, 3072)):
        host = synth_blocks(fmt, rows, cols, rng)
        copies = max(1, -(-640 * 2 ** 20 // host.nbytes))
        out[key] = time_rotated_gemv(hip, fmt, host, rows, cols, copies, rng)
        log(f"  {key}: {out[key]['us_per_launch']:.3f} us/launch, {out[key]['GBs']:.1f} GB/s "
            f"({100 * out[key]['frac']:.1f}% of HBM)")
    return out


def bench_decode_dense(hip, context: int = 2048):
    """The Phi-4-mini decode step in the reference model's own storage: F16
    layer weights and the tied F16 token_embd table as embedding and head
    (Phi4TextModel.cs:53,95-105), fp16 KV cache with `context` tokens."""
    from sharpinference_amd import native, phi4
    cfg = phi4.Phi4Config(weight_format=native.F16, embed_format=native.F16, head_format=native.F16)
    t0 = time.time()
    weights = phi4.synth_weights(cfg, seed=11, distinct_layers=4, tied=True)
    sess = phi4.Phi4DecodeSession(hip, cfg, weights)
    kv = phi4.synth_kv(phi4.Phi4Config(layers=1, capacity=cfg.capacity), context, seed=12)[0]
    for l in range(cfg.layers):
        sess.load_kv(l, *kv)
    log(f"decode f16: model on device in {time.time() - t0:.1f} s")
    sess.set_control(1, context)
    sess.plan.launch()
    hip.sync()
    settle(lambda: sess.plan.measure_us(4))
    us = sorted(sess.plan.measure_us(16) for _ in range(5))[2]
    sess.close()
    del weights
    step_bytes = cfg.weight_bytes_per_token() + cfg.kv_bytes(context + 1)
    gbs = step_bytes / us / 1e3
    log(f"decode f16: {us:.1f} us/token ({1e6 / us:.0f} tok/s, {gbs:.0f} GB/s)")
    return {"workload": "Phi-4-mini decode step, 32 layers, F16 layers, tied F16 embedding/head 200064x3072, "
                        f"fp16 KV cache with {context} tokens, batch 1",
            "us_per_token": r1(us), "tok_s": r1(1e6 / us), "bytes_per_token": step_bytes, "GBs": r1(gbs),
            "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "roofline_tok_s": round(HBM_PEAK_GBS * 1e9 / step_bytes, 1),
            "layer_weights": "4 distinct layers uploaded as 32 separate device copies"}


SETTLE_S = 0.04


def settle(replay, seconds: float = SETTLE_S) -> None:
    """Calls `replay` (untimed replays of what is measured next) at least
    once and until `seconds` have passed: after the host-side uploads between measurements the GPU's
    clocks start low and reach their loaded state only after tens of
    milliseconds of work (a prefill product timed right after an upload
    measured 36.8 us, the same product 30 ms of replays later 33.7 us)."""
    t0 = time.perf_counter()
    while True:
        replay()
        if time.perf_counter() - t0 >= seconds:
            break


def bench_prefill(hip, rng, m: int = 512):
    """Batched prefill product at the same layer shapes: M = 512 tokens of
    bf16 activations against the Q4_0 projections (MFMA), FP32 out.  Every
    plan is replayed untimed for 40 ms before it is timed (steady clocks)."""
    from sharpinference_amd import native
    MFMA_BF16_PEAK_TFLOPS = 2500.0
    out = {"tokens": m, "shapes": {}}
    total_flops, total_us, total_us_single = 0.0, 0.0, 0.0
    bufs = []
    reps = PREFILL_LAUNCHES_PER_PLAN
    for name, rows, cols in LAYER_Q4_0:
        w = hip.to_device(synth_weights(native.Q4_0, rows, cols, rng))
        xb = rng.standard_normal(m * cols).astype(np.float32).view(np.uint32)
        xb = ((xb + 0x7FFF + ((xb >> 16) & 1)) >> 16).astype(np.uint16)
        x = hip.to_device(xb)
        y = hip.alloc(m * rows * 4)
        bufs.append((w, x, y, rows, cols))
        flops = 2.0 * m * rows * cols
        # one plan holds `reps` launches of the product back to back (as the
        # layer set's plan holds a round of steps); replayed, warmed first
        plan = hip.record(lambda: [hip.gemm_prefill(native.Q4_0, w.ptr, x.ptr, y.ptr, m, rows, cols)
                                   for _ in range(reps)])
        settle(lambda: plan.measure_us(4))
        us = sorted(plan.measure_us(4) for _ in range(5))[2] / reps
        plan.destroy()
        # the same product as a one-launch plan replayed `reps` times: each
        # launch then also carries a plan-launch gap
        plan = hip.record(lambda: hip.gemm_prefill(native.Q4_0, w.ptr, x.ptr, y.ptr, m, rows, cols))
        settle(lambda: plan.measure_us(4))
        us_single = sorted(plan.measure_us(reps) for _ in range(5))[2]
        plan.destroy()
        total_flops += flops
        total_us += us
        total_us_single += us_single
        out["shapes"][name] = {"us": round(us, 2), "TFLOPs": round(flops / us / 1e6, 1),
                               "us_one_launch_plans": round(us_single, 2)}
        log(f"  prefill {name:8s} m={m} {rows}x{cols}: {us:.1f} us, {flops / us / 1e6:.1f} TFLOP/s "
            f"({us_single:.1f} us as one-launch plans)")
    tflops = total_flops / total_us / 1e6
    out.update({"us_total": round(total_us, 1), "TFLOPs": round(tflops, 1),
                "mfma_bf16_frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4),
                "form": f"each product's {reps} launches recorded in one plan, per-launch average, "
                        f"after {SETTLE_S * 1e3:.0f} ms of untimed replays",
                "one_launch_plans": {"us_total": round(total_us_single, 1),
                                     "TFLOPs": round(total_flops / total_us_single / 1e6, 1)}})

    # the same four products recorded as one plan, a layer's submission
    # (no gap between separate plan launches inside it)
    def layer():
        for w, x, y, rows, cols in bufs:
            hip.gemm_prefill(native.Q4_0, w.ptr, x.ptr, y.ptr, m, rows, cols)
    plan = hip.record(layer)
    settle(lambda: plan.measure_us(4))
    layer_us = sorted(plan.measure_us(8) for _ in range(5))[2]
    plan.destroy()
    for w, x, y, _, _ in bufs:
        for b in (w, x, y):
            b.free()
    out["layer_plan"] = {"us": round(layer_us, 1), "TFLOPs": round(total_flops / layer_us / 1e6, 1),
                         "form": "the four products in one recorded plan, replayed 8 times back to back"}
    log(f"  prefill layer plan m={m}: {layer_us:.1f} us, {total_flops / layer_us / 1e6:.1f} TFLOP/s")
    return out


def prefill_eager(hip, rng, rounds: int, m: int = 512):
    """The prefill leg's four products launched one by one, `rounds` times
    back to back with no plan (for kernel traces and counters, which then
    see every launch); wall time per round after a final synchronize."""
    from sharpinference_amd import native
    bufs = []
    for name, rows, cols in LAYER_Q4_0:
        w = hip.to_device(synth_weights(native.Q4_0, rows, cols, rng))
        xb = rng.standard_normal(m * cols).astype(np.float32).view(np.uint32)
        xb = ((xb + 0x7FFF + ((xb >> 16) & 1)) >> 16).astype(np.uint16)
        bufs.append((w, hip.to_device(xb), hip.alloc(m * rows * 4), rows, cols))
    hip.sync()
    t0 = time.perf_counter()
    for r in range(rounds):
        for w, x, y, rows, cols in bufs:
            hip.gemm_prefill(native.Q4_0, w.ptr, x.ptr, y.ptr, m, rows, cols)
        if r % 100 == 99:
            hip.sync()
            log(f"prefill eager: {r + 1} rounds, {(time.perf_counter() - t0) * 1e3:.0f} ms")
    hip.sync()
    ms = (time.perf_counter() - t0) * 1e3
    for bb in bufs:
        for b in bb[:3]:
            b.free()
    return {"tokens": m, "rounds": rounds, "ms": round(ms, 2), "us_per_round": round(ms * 1e3 / max(rounds, 1), 1),
            "form": "the four products launched eagerly, no plan"}


def bench_batch_ops(hip, rows: int = 16, context: int = 4096):
    """The batched prefill operators of the op-by-op program at 16 rows,
    launched eagerly (no plan): the four Phi-4-mini Q4_K layer mat-vecs
    (batch_matvec) and the attention chain (scores, causal softmax, values,
    and the three fused into two launches) over an fp16 cache of `context`
    positions, 24 query and 8 KV heads, for
    batches starting at 0 and at context / 2 - 16.  Each op event-timed,
    median of 5 samples of 20 back-to-back launches."""
    from sharpinference_amd import native, phi4
    cfg = phi4.Phi4Config()
    rng = np.random.default_rng(11)

    def timed(fn):
        fn()
        samples = []
        for _ in range(5):
            hip.timer_begin()
            for _ in range(20):
                fn()
            samples.append(hip.timer_end() * 1e3 / 20)
        return sorted(samples)[2]

    ctl = hip.to_device(np.array([0, rows], np.int32))
    out = {"rows": rows, "matvec_us": {}, "attention_us": {}}
    flops, total = 0.0, 0.0
    for name, (r, c) in cfg.layer_shapes().items():
        w = hip.to_device(phi4.synth_blocks(cfg.weight_format, r, c, rng))
        x = hip.to_device(rng.standard_normal((rows, c)).astype(np.float32))
        y = hip.alloc(rows * r * 4)
        us = timed(lambda: hip.batch_matvec(cfg.weight_format, w.ptr, x.ptr, ctl.ptr, y.ptr, rows, r, c))
        out["matvec_us"][name] = r1(us)
        flops += 2.0 * rows * r * c
        total += us
        for b in (w, x, y):
            b.free()
    out["matvec_layer_us"] = r1(total)
    out["matvec_tflops"] = r1(flops / total / 1e6)
    heads, kv, head = cfg.heads, cfg.kv_heads, cfg.head_dim
    q = hip.to_device(rng.standard_normal((rows, heads * head)).astype(np.float32))
    kc = hip.to_device(rng.standard_normal((context, kv, head)).astype(np.float16))
    vc = hip.to_device(rng.standard_normal((context, kv, head)).astype(np.float16))
    sc, pr = hip.alloc(4 * rows * heads * context), hip.alloc(4 * rows * heads * context)
    att = hip.alloc(4 * rows * heads * head)
    ws = hip.alloc(native.batch_values_workspace_bytes(rows, heads, context))
    for start in (0, context // 2 - 16):
        ctl.upload(np.array([start, rows], np.int32))
        a_s = native.BatchAttentionArgs(q.ptr, pr.ptr, kc.ptr, ctl.ptr, sc.ptr, ws.ptr, native.F16, rows, heads, kv,
                                        head, context)
        a_v = native.BatchAttentionArgs(q.ptr, pr.ptr, vc.ptr, ctl.ptr, att.ptr, ws.ptr, native.F16, rows, heads, kv,
                                        head, context)
        a_f = native.BatchAttentionArgs(q.ptr, 0, kc.ptr, ctl.ptr, att.ptr, ws.ptr, native.F16, rows, heads, kv,
                                        head, context)
        out["attention_us"][str(start)] = {
            "scores": r1(timed(lambda: hip.batch_gqa_scores(a_s))),
            "softmax": r1(timed(lambda: hip.batch_causal_softmax(sc.ptr, ctl.ptr, pr.ptr, rows, heads, context))),
            "values": r1(timed(lambda: hip.batch_gqa_values(a_v))),
            "fused": r1(timed(lambda: hip.batch_gqa_attention(a_f, vc.ptr)))}
    for b in (ctl, q, kc, vc, sc, pr, att, ws):
        b.free()
    log("batch ops: mat-vec " + ", ".join(f"{k} {v} us" for k, v in out["matvec_us"].items())
        + f" ({out['matvec_layer_us']} us, {out['matvec_tflops']} TFLOP/s); attention "
        + "; ".join(f"start {k}: " + ", ".join(f"{n} {v} us" for n, v in d.items())
                    for k, d in out["attention_us"].items()))
    return out


def bench_vendor_dense(m: int = 512):
    """The vendor library's dense bf16 product at the prefill shapes:
    torch.nn.functional.linear (hipBLASLt) of bf16 X [m, K] by bf16 W [N, K]
    (four weight copies rotated), bf16 out, timed with events on torch's
    stream (median of 5 samples of 20 launches, after 40 ms of untimed
    launches).  W here is already dense
    bf16 (3.6x the bytes of Q4_0 and no decode), so this is a reference
    for what a plain GEMM reaches at these shapes, not a product path."""
    import torch
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(7)
    out = {"library": "torch.nn.functional.linear (hipBLASLt), bf16 in / out", "tokens": m, "shapes": {}}
    total_flops, total_us = 0.0, 0.0
    for name, rows, cols in LAYER_Q4_0:
        x = torch.randn(m, cols, device=dev, dtype=torch.bfloat16, generator=gen)
        ws = [torch.randn(rows, cols, device=dev, dtype=torch.bfloat16, generator=gen) for _ in range(4)]
        def replay():
            for i in range(8):
                torch.nn.functional.linear(x, ws[i % 4])
            torch.cuda.synchronize()
        settle(replay)
        samples = []
        for _ in range(5):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            for i in range(20):
                torch.nn.functional.linear(x, ws[i % 4])
            b.record()
            b.synchronize()
            samples.append(a.elapsed_time(b) * 1e3 / 20)
        us = sorted(samples)[2]
        flops = 2.0 * m * rows * cols
        total_flops += flops
        total_us += us
        out["shapes"][name] = {"us": round(us, 2), "TFLOPs": round(flops / us / 1e6, 1)}
        log(f"  vendor dense bf16 {name:8s} m={m} {rows}x{cols}: {us:.1f} us, {flops / us / 1e6:.1f} TFLOP/s")
        del x, ws
    out.update({"us_total": round(total_us, 1), "TFLOPs": round(total_flops / total_us / 1e6, 1)})
    log(f"vendor dense bf16 total: {total_us:.1f} us, {out['TFLOPs']} TFLOP/s")
    return out


def cpu_threads() -> int:
    return int(os.environ.get("OMP_NUM_THREADS", "0")) or min(16, os.cpu_count() or 1)


def r1(v):
    """Rounded value, None for a measurement that was not taken (NaN)."""
    return None if v != v else round(v, 1)


def time_cpu_steps(step, samples: int = 3) -> float:
    """Median seconds of `samples` oracle token steps after one warm-up."""
    step()
    times = []
    for _ in range(samples):
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    return sorted(times)[len(times) // 2]


def bench_decode(hip, context: int = 2048, tokens: int = 64, cpu: bool = True, replay_timing: bool = True,
                 eager: bool = False):
    """Phi-4-mini-shaped decode step (32 layers, Q4_K layers, Q8_0 embedding
    and head, fp16 KV cache holding `context` tokens), one new token per
    step.  Steady state: the recorded step replayed back to back at position
    `context`; loop: forward_token (control upload, replay, next-token
    readback) over `tokens` consecutive positions.  CPU: the oracle's decode
    step (CpuVm restatement) on the same weights and cache."""
    from sharpinference_amd import phi4
    cfg = phi4.Phi4Config()
    t0 = time.time()
    weights = phi4.synth_weights(cfg, seed=7, distinct_layers=4)
    sess = phi4.Phi4DecodeSession(hip, cfg, weights)
    kv = phi4.synth_kv(phi4.Phi4Config(layers=1, capacity=cfg.capacity), context, seed=8)[0]
    for l in range(cfg.layers):
        sess.load_kv(l, *kv)
    log(f"decode: model on device in {time.time() - t0:.1f} s")
    sess.set_control(1, context)
    if eager:   # warm-up without a plan replay: kernel-trace profiles of this run contain no graph launch
        hip.phi4_decode(sess.model)
    else:
        sess.plan.launch()
    hip.sync()
    if replay_timing:
        settle(lambda: sess.plan.measure_us(4))
    us = sorted(sess.plan.measure_us(16) for _ in range(5))[2] if replay_timing else float("nan")
    step_bytes = cfg.weight_bytes_per_token() + cfg.kv_bytes(context + 1)
    gbs = step_bytes / us / 1e3
    t0 = time.perf_counter()
    tok = 1
    for i in range(tokens):
        if eager:   # the same step launched kernel by kernel instead of as one graph replay
            sess.set_control(tok, context + i)
            hip.phi4_decode(sess.model)
            tok = int(sess.next_token.readback(np.int32, 1)[0])
        else:
            tok = sess.forward_token(tok, context + i)
    loop_s = (time.perf_counter() - t0) / tokens
    sess.close()
    log(f"decode: {us:.1f} us/token on device ({1e6 / us:.0f} tok/s, {gbs:.0f} GB/s), "
        f"{loop_s * 1e6:.1f} us/token with host round trips")
    op_program = None
    if replay_timing:
        # the same model as the reference's program form: 292 separate
        # dispatches through the C++ host executor
        from sharpinference_amd import host_program
        prog = host_program.Phi4OpProgram(cfg, weights, cache_fp16=True, prompt_rows=context)
        for l in range(cfg.layers):
            prog.load_kv(l, *kv)
        prog.forward_token(1, context)
        settle(lambda: prog.measure_us(4))
        op_us = sorted(prog.measure_us(8) for _ in range(5))[2]
        # prefill_fused_16: one batch of 16 prompt rows; attention cost grows
        # linearly with the batch's start, so the batch starting halfway
        # through a `context`-token prompt prices the prompt's average batch
        prog.upload("fused_embeddings", np.random.default_rng(9).standard_normal(
            (context, cfg.hidden)).astype(np.float32) * 0.05)
        prefill = {}
        for start in (0, context // 2 - 8, context - 16):
            prog.upload("control", np.array([start, 16], np.int32))
            settle(lambda: prog.measure_us(2, "prefill_fused_16"))
            prefill[start] = sorted(prog.measure_us(4, "prefill_fused_16") for _ in range(3))[1]
        mid = prefill[context // 2 - 8]
        op_program = {"us_per_token": r1(op_us), "tok_s": r1(1e6 / op_us), "dispatches": prog.dispatch_count(),
                      "form": "transformer.* / quant.mat-vec instructions, one launch each (two for attention)",
                      "prefill_fused_16": {
                          "us_per_batch_by_start": {str(k): r1(v) for k, v in prefill.items()},
                          "prompt_tok_s": r1(16e6 / mid), "dispatches": prog.dispatch_count("prefill_fused_16"),
                          "workload": f"16 prompt rows per batch; rate at the middle batch of a {context}-token "
                                      "prompt (the prompt average: attention is linear in the start)"}}
        prog.close()
        log(f"decode op-by-op program: {op_us:.1f} us/token ({1e6 / op_us:.0f} tok/s); prefill_fused_16 "
            + ", ".join(f"start {k}: {v:.0f} us" for k, v in prefill.items()) + f" ({16e6 / mid:.0f} prompt tok/s)")
    out = {"workload": "Phi-4-mini decode step, 32 layers, Q4_K layers, Q8_0 embedding/head 200064x3072, "
                       f"fp16 KV cache with {context} tokens, batch 1",
           "us_per_token": r1(us), "tok_s": r1(1e6 / us),
           "bytes_per_token": step_bytes, "GBs": r1(gbs), "hbm_frac": None if gbs != gbs else round(gbs / HBM_PEAK_GBS, 4),
           "roofline_tok_s": round(HBM_PEAK_GBS * 1e9 / step_bytes, 1),
           "loop_us_per_token": round(loop_s * 1e6, 1), "loop_tok_s": round(1.0 / loop_s, 1),
           "layer_weights": "4 distinct layers uploaded as 32 separate device copies",
           "op_program": op_program}
    if cpu:
        import oracle as orc
        model = orc.Phi4Oracle(cfg, weights)
        for l in range(cfg.layers):
            model.k[l][...] = kv[0]
            model.v[l][...] = kv[1]
        threads = cpu_threads()
        sec = time_cpu_steps(lambda: model.step(1, context, threads))
        out["cpu"] = {"tok_s": round(1.0 / sec, 3), "ms_per_token": round(sec * 1e3, 1), "cores": threads,
                      "kind": "port", "sample": "1 warm-up + 3 oracle decode steps (median) at position "
                                                f"{context}, same weights and cache"}
        log(f"decode cpu: {sec * 1e3:.1f} ms/token on {threads} threads")
        if op_program is not None:
            # the prompt batch's 16 rows as 16 oracle token steps at the
            # middle batch's positions (each step also computes the vocabulary
            # head, which the batched program computes once per batch)
            mid = context // 2 - 8
            t0 = time.perf_counter()
            for r in range(16):
                model.step(1, mid + r, threads)
            batch_s = time.perf_counter() - t0
            op_program["prefill_fused_16"]["cpu"] = {
                "prompt_tok_s": round(16.0 / batch_s, 2), "ms_per_batch": round(batch_s * 1e3, 1), "cores": threads,
                "kind": "port", "sample": f"16 oracle token steps at positions {mid}..{mid + 15} (one batch), each "
                                          "with the vocabulary head"}
            log(f"prefill_fused_16 cpu: {batch_s * 1e3:.0f} ms per 16-row batch on {threads} threads "
                f"({16.0 / batch_s:.1f} prompt tok/s)")
        del model
    del weights
    return out


def bench_rwkv_decode(hip, tokens: int = 64, cpu: bool = True, replay_timing: bool = True, eager: bool = False):
    """RWKV-7-shaped token step (24 layers, width 2048 in 32 heads of 64,
    FFN 8192, Q8_0 projections and LoRA, Q8_0 embedding/head 65536x2048,
    FP32 state with WKV matrices N(0, 0.1)).  Steady state: the recorded step
    replayed back to back; loop: forward_token over `tokens` tokens.  CPU:
    the oracle's token step on the same weights and state."""
    from sharpinference_amd import rwkv7
    cfg = rwkv7.Rwkv7Config()
    t0 = time.time()
    weights = rwkv7.synth_weights(cfg, seed=9, distinct_layers=4)
    state = rwkv7.synth_state(cfg, seed=10)
    sess = rwkv7.Rwkv7DecodeSession(hip, cfg, weights, state)
    log(f"rwkv7: model on device in {time.time() - t0:.1f} s")
    sess.control.upload(np.array([1], np.int32))
    if eager:
        hip.rwkv7_decode(sess.model)
    else:
        sess.plan.launch()
    hip.sync()
    if replay_timing:
        settle(lambda: sess.plan.measure_us(4))
    us = sorted(sess.plan.measure_us(16) for _ in range(5))[2] if replay_timing else float("nan")
    step_bytes = cfg.weight_bytes_per_token()
    gbs = step_bytes / us / 1e3
    t0 = time.perf_counter()
    tok = 1
    for _ in range(tokens):
        if eager:
            sess.control.upload(np.array([tok], np.int32))
            hip.rwkv7_decode(sess.model)
            tok = int(sess.next_token.readback(np.int32, 1)[0])
        else:
            tok = sess.forward_token(tok)
    loop_s = (time.perf_counter() - t0) / tokens
    sess.close()
    log(f"rwkv7: {us:.1f} us/token on device ({1e6 / us:.0f} tok/s, {gbs:.0f} GB/s), "
        f"{loop_s * 1e6:.1f} us/token with host round trips")
    graph = None
    if replay_timing:
        # the same model as the reference's portable graph: built from the tensor catalog, lowered
        # to a HIP VM program and run operator by operator through the C++ executor
        from sharpinference_amd import host_program
        prog = host_program.Rwkv7GraphProgram(cfg, weights, state)
        prog.forward_token(1)
        settle(lambda: prog.measure_us(1))
        g_us = sorted(prog.measure_us(4) for _ in range(3))[1]
        rep = prog.report()
        graph = {"us_per_token": r1(g_us), "tok_s": r1(1e6 / g_us), "dispatches": prog.dispatch_count(),
                 "definitions": rep["definitions"], "local_slots": rep["localSlots"],
                 "matvec_calls": rep["matvec"]["calls"], "nodes_lowered_to_views": rep["removedNodes"],
                 "form": "PortableRwkv7GraphProvider graph, one launch per lowered node (T0 / portable tensor "
                         "operators and quant.mat-vec)"}
        prog.close()
        log(f"rwkv7 portable graph: {g_us:.1f} us/token ({1e6 / g_us:.0f} tok/s), {graph['dispatches']} dispatches, "
            f"{graph['definitions']} definitions, {graph['local_slots']} local slots")
    out = {"workload": "RWKV-7 token step, 24 layers, width 2048 (32 heads x 64), FFN 8192, Q8_0 projections "
                       "and LoRA (ranks 96/96/64/256), Q8_0 embedding/head 65536x2048, batch 1",
           "us_per_token": r1(us), "tok_s": r1(1e6 / us), "bytes_per_token": step_bytes,
           "GBs": r1(gbs), "hbm_frac": None if gbs != gbs else round(gbs / HBM_PEAK_GBS, 4),
           "roofline_tok_s": round(HBM_PEAK_GBS * 1e9 / step_bytes, 1),
           "loop_us_per_token": round(loop_s * 1e6, 1), "loop_tok_s": round(1.0 / loop_s, 1),
           "layer_weights": "4 distinct layers uploaded as 24 separate device copies",
           "graph_program": graph}
    if cpu:
        import oracle as orc
        from types import SimpleNamespace
        ocfg = SimpleNamespace(**{k: getattr(cfg, k) for k in (
            "layers", "hidden", "heads", "head_size", "ffn", "vocab", "rank_w", "rank_a", "rank_v", "rank_g",
            "weight_format", "embed_format", "head_format")})
        model = orc.Rwkv7Oracle(ocfg, weights, state)
        threads = cpu_threads()
        sec = time_cpu_steps(lambda: model.step(1, threads))
        out["cpu"] = {"tok_s": round(1.0 / sec, 3), "ms_per_token": round(sec * 1e3, 1), "cores": threads,
                      "kind": "port", "sample": "1 warm-up + 3 oracle token steps (median), same weights and "
                                                "state"}
        log(f"rwkv7 cpu: {sec * 1e3:.1f} ms/token on {threads} threads")
    return out


def committed_traffic(config: str):
    """HBM bytes per launch measured by the FETCH_SIZE / WRITE_SIZE counter
    runs recorded in profiles/ for this workload (None when absent)."""
    path = os.path.join(ROOT, "profiles", {"layer_q4_0": "gemv_q4_0_layer_set.md"}.get(config, "-"))
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def cpu_baseline(fmt, shapes, host_w, xs, ys, hip, bytes_per_step, budget_s):
    """The oracle's CpuVm restatement (dequantise row -> FP32 dot, rows in
    parallel) timed on this host over a bounded sample of the same steps."""
    import oracle as orc
    threads = cpu_threads()
    x_host = {cols: xs[cols].readback(np.float32) for cols in xs}

    def step(n_threads):
        outs = {}
        for (name, rows, cols), w in zip(shapes, host_w):
            outs[name] = orc.gemv_cpuvm(fmt, w, x_host[cols], rows, cols, n_threads)
        return outs

    # parity of the GPU outputs of the timed steps (same weights, same x)
    outs = step(threads)
    parity = {}
    for name, rows, cols in shapes:
        g = ys[name].readback(np.float32, rows).astype(np.float64)
        c = outs[name].astype(np.float64)
        parity[name] = float(np.linalg.norm(g - c) / np.linalg.norm(c))
    log(f"cpu/gpu L2-relative difference per shape: {parity}")

    def median_step(n_threads, budget):
        """MatVecProfiler protocol: 4 warm-up batches, 9 timed batches, median."""
        t0 = time.perf_counter()
        step(n_threads)
        one = time.perf_counter() - t0
        reps = max(1, int(budget / 13 / max(one, 1e-6)))
        for _ in range(4):
            for _ in range(reps):
                step(n_threads)
        samples = []
        for _ in range(9):
            t0 = time.perf_counter()
            for _ in range(reps):
                step(n_threads)
            samples.append((time.perf_counter() - t0) / reps)
        return sorted(samples)[4], reps

    med, reps = median_step(threads, budget_s)
    gbs = bytes_per_step / med / 1e9
    log(f"cpu baseline: {med * 1e3:.2f} ms/step on {threads} threads -> {gbs:.2f} GB/s")
    med1, reps1 = median_step(1, budget_s / 2)
    log(f"cpu baseline: {med1 * 1e3:.2f} ms/step on 1 thread -> {bytes_per_step / med1 / 1e9:.2f} GB/s")
    cpu_model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu_model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {
        "value": round(gbs, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{reps} steps x 9 samples (median) of the same layer set, one weight copy, "
                  f"oracle CpuVm restatement (-O3 x86-64-v3, OpenMP rows); host {cpu_model}",
        "ms_per_step": round(med * 1e3, 3),
        "value_1thread": round(bytes_per_step / med1 / 1e9, 3),
        "ms_per_step_1thread": round(med1 * 1e3, 3),
        "host_cpus": os.cpu_count(),
        "gpu_vs_cpu_l2_rel": parity,
    }


if __name__ == "__main__":
    sys.exit(main())
