#!/usr/bin/env python3
"""LoRA fine-tuning step benchmark on one MI355X.

A step is the reference driver's optimizer step (gpt2_small_lora_finetune/
src/main.cpp:456-505): for each micro-batch forward → lm_cross_entropy →
backward with loss scaled by 1/accum, then global grad-norm clip, Adam on the
LoRA parameters and zero_grad — here one fused device-resident pass in
libmft_hip.so.  Default workload: BASELINE configs[0], GPT-2 small (the
configuration the benchmark's targets are stated on), batch 4 × seq 128,
LoRA r=8 α=16 on c_attn + attn c_proj, random-init weights N(0,0.02), LoRA
A ~ N(0,1/r), B ~ N(0,0.02), token ids uniform in [0, vocab) from the seed
(synthetic data; no dataset download).  --config names the others.

Prints ONE JSON line.  `value` = tokens/s of the whole job (accum·B·S tokens
per step / measured step time), inputs already resident in HBM.
`roofline` covers the dominant kernel family (the linear-layer GEMMs, fwd +
dX, with their split-K reductions), timed live with HIP events recorded by
the dispatches on the model's stream over a second region of up to 10 eager
steps right after the throughput region (events around every kernel add host
time, so `value` comes from the region without them).  `cpu_baseline` times
the CPU port (oracle/, BLAS-backed GEMMs) on the host: one warm-up step, then
the median of --cpu-steps (≥ 5) timed steps, on `nproc` threads.
"""
import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "LoRA fwd+bwd tokens/sec at 1 GPU; LoRA-linear & attention % of MFMA peak"
PEAK_FP32_MFMA = 157.3   # TFLOP/s, MI355X dense fp32 matrix
PEAK_FP16_MFMA = 2500.0  # TFLOP/s, MI355X dense fp16 matrix (fp16-stored W runs its GEMMs here)
PEAK_HBM = 8000.0        # GB/s, MI355X HBM3E


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="gpt2s",
                    help="gpt2s | gpt2m | gemma270m | qwen05b | gemma1b")
    ap.add_argument("--seed", type=int, default=1235)
    ap.add_argument("--lr", type=float, default=2e-4)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-api-bench", action="store_true",
                    help="skip the operators-API driver-loop line (GPT-2 small only)")
    ap.add_argument("--cpu-steps", type=int, default=5)
    ap.add_argument("--cpu-threads", type=int, default=0)
    ap.add_argument("--graph", action="store_true",
                    help="time the throughput region by replaying the captured step graph "
                         "instead of launching eagerly (the roofline region is always eager)")
    ap.add_argument("--no-timing", action="store_true",
                    help="skip the per-kernel HIP events (roofline becomes null)")
    ap.add_argument("--calibrate-copy-mb", type=int, default=0,
                    help="after the run, copy a buffer of this many MiB three times with a plain "
                         "device copy kernel: the reference reading for scaling HBM byte counters")
    ap.add_argument("--op", default=None, choices=["dequant_f16"],
                    help="time one standalone operator instead of the training step: "
                         "dequant_f16 = fp16 → fp32 widening of --elements values (HBM-bound)")
    ap.add_argument("--elements", type=int, default=256 << 20)
    ap.add_argument("--shard-budget-mb", type=float, default=0.0,
                    help="stream the frozen linear weights and the token embedding from pinned host "
                         "memory through an HBM pool of this size (the reference's --shard_budget_mb); "
                         "0 keeps every weight resident")
    ap.add_argument("--w-fp16", action="store_true",
                    help="store the frozen weights as fp16 (rounded to nearest even), as the reference's "
                         "sharder does with --shard_fp16_disk 1; the GEMMs then run on the fp16 matrix cores. "
                         "Changes the model's numerics: not the fp32 configs' headline")
    return ap.parse_args()


def op_bench(args):
    """Standalone operator: `--steps` launches timed with HIP events on the
    stream the library launches on (torch's current stream), after
    `--warmup` launches; the same bytes moved by a plain device copy are
    timed beside it as the achievable-bandwidth reference."""
    import torch

    from mobilefinetuner_amd import ops
    n = args.elements
    gen = torch.Generator(device="cuda").manual_seed(args.seed)
    src = (torch.randn(n, device="cuda", generator=gen) * 0.02).half()
    dst = torch.empty(n, device="cuda", dtype=torch.float32)
    run = lambda: ops.dequant_f16_into(src, dst)  # noqa: E731
    for _ in range(args.warmup):
        run()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        run()
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / args.steps
    nbytes = 6 * n  # 2 B read + 4 B written per element
    exact = bool(torch.equal(dst, src.float()))
    # reference: a device copy moving the same total bytes (half read, half written)
    cs = torch.empty(nbytes // 8, device="cuda")
    cd = torch.empty_like(cs)
    cd.copy_(cs)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(args.steps):
        cd.copy_(cs)
    e1.record()
    torch.cuda.synchronize()
    cus = e0.elapsed_time(e1) * 1e3 / args.steps
    gbs = nbytes / (us * 1e-6) / 1e9
    print(json.dumps({"op": "dequant_f16", "metric": "achieved HBM GB/s", "value": round(gbs, 1),
                      "unit": "GB/s", "higher_is_better": True, "elements": n,
                      "bytes_per_launch": nbytes, "avg_launch_us": round(us, 2),
                      "frac_of_peak": round(gbs / PEAK_HBM, 4), "peak": PEAK_HBM,
                      "copy_reference_GBps": round(nbytes / (cus * 1e-6) / 1e9, 1),
                      "bit_exact_vs_torch_half_to_float": exact, "steps": args.steps,
                      "warmup": args.warmup}))


def traffic_bytes(config_id):
    """HBM bytes per launch of the linear-GEMM family, from the two committed
    rocprofv3 --pmc runs (FETCH_SIZE, WRITE_SIZE, scaled by a plain-copy
    calibration) summarised under profiles/; counters cannot be read from
    inside this process, so the figure is the profiled one, or None."""
    path = os.path.join(ROOT, "profiles", f"gemm_linear_{config_id}_traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        t = json.load(f)
    return t.get("traffic_bytes_per_launch")


def host_cores():
    """`nproc` (the processing units this process may use: GNU nproc honours
    the affinity mask and OMP_NUM_THREADS), with os.cpu_count() beside it."""
    import subprocess
    try:
        n = int(subprocess.run(["nproc"], capture_output=True, text=True, check=True).stdout)
    except (OSError, ValueError, subprocess.CalledProcessError):
        n = len(os.sched_getaffinity(0))
    return n, os.cpu_count()


def cpu_baseline(rc, seed, steps, threads):
    """The CPU port (oracle/) with BLAS GEMMs, timed on the host."""
    import numpy as np

    import oracle as O
    nproc, online = host_cores()
    n = threads or nproc
    steps = max(steps, 5)
    O.lib().orc_set_threads(n)
    O.lib().orc_set_blas(1)
    backend = O.lib().orc_blas_backend().decode()
    mc = rc.model
    om = O.OracleModel(mc)
    rng = np.random.default_rng(seed)
    for p in om.params:
        name = p["name"]
        if name.endswith("lora_A"):
            v = rng.standard_normal(p["shape"], dtype=np.float32) / mc.lora_r
        elif "norm" in name or "ln_" in name:
            one = name.endswith("weight") and (mc.arch != 2)
            v = np.ones(p["shape"], np.float32) if one else np.zeros(p["shape"], np.float32)
        else:
            v = rng.standard_normal(p["shape"], dtype=np.float32) * 0.02
        if p["f16"]:
            v = v.astype(np.float16).view(np.uint16)
        om.set_param(name, v)
    B, S, acc = rc.batch, rc.seq, rc.accum
    ids = rng.integers(0, mc.vocab, (acc, B, S)).astype(np.int32)
    times = []
    for it in range(steps + 1):
        t0 = time.perf_counter()
        for a in range(acc):
            om.fwd_bwd(ids[a], None, ids[a], B, S, 1.0 / acc)
        om.opt_step(2e-4, clip=1.0)
        dt = time.perf_counter() - t0
        if it > 0:
            times.append(dt)
    med = statistics.median(times)
    return {"value": rc.tokens_per_step / med, "unit": "tokens/s", "cores": n, "kind": "port",
            "nproc": nproc, "cpu_count": online,
            "sample": f"median of {steps} timed optimizer steps (+1 warm-up) of the same workload "
                      f"({rc.tokens_per_step} tokens/step): {med:.3f} s/step "
                      f"(min {min(times):.3f}, max {max(times):.3f}); GEMMs via {backend}, "
                      f"{n} threads (nproc {nproc}, cpu_count {online})"}


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1 "
                          "(the multi-GPU sharding is a design, not built or run)"}))
        sys.exit(2)
    if args.op:
        return op_bench(args)
    # The operators API (the boundary the reference's drivers compile
    # against) timed by its own driver-loop program, run as a child process
    # before this process touches the GPU.
    api = None
    exe = os.path.join(ROOT, "mobilefinetuner_amd", "bin", "api_bench")
    if args.config == "gpt2s" and not args.no_api_bench and os.path.exists(exe):
        import subprocess
        r = subprocess.run([exe, "4", "128", "1", str(max(args.steps, 5)), str(max(args.warmup, 1))],
                           capture_output=True, text=True, timeout=600)
        if r.returncode != 0:
            raise RuntimeError("api_bench failed: " + r.stderr[-2000:])
        api = json.loads(r.stdout.strip().splitlines()[-1])
    import torch

    from mobilefinetuner_amd.configs import CONFIGS, step_flops
    from mobilefinetuner_amd.engine import (CLS_ATTN, CLS_CE, CLS_LINEAR, CLS_LMHEAD, CLS_RANK,
                                            Model)
    rc = CONFIGS[args.config]
    mc = rc.model
    if args.shard_budget_mb > 0 or args.w_fp16:
        import dataclasses
        if args.shard_budget_mb > 0:
            mc = dataclasses.replace(mc, shard_budget=int(args.shard_budget_mb * (1 << 20)))
        if args.w_fp16:
            mc = dataclasses.replace(mc, w_fp16=1)
    torch.cuda.set_device(0)
    tokens = rc.tokens_per_step
    model = Model(mc, tokens)
    model.init_params(args.seed, 0.02, 1.0 / mc.lora_r, 0.02)
    g = torch.Generator(device="cpu").manual_seed(args.seed)
    ids = torch.randint(0, mc.vocab, (tokens,), generator=g, dtype=torch.int32).cuda()
    labels = ids.clone()

    def step():
        model.train_step(ids, labels, n_micro=rc.accum, seqs_per_micro=rc.batch, S=rc.seq,
                         lr=args.lr, clip=1.0, graph=args.graph)

    # Throughput region: plain launches, no per-kernel events (each event pair
    # costs host time that would otherwise overlap the GPU work).
    for _ in range(max(1, args.warmup)):
        step()
    model.read_stats()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    loss, n_valid, gnorm = model.read_stats()
    ms = (t1 - t0) * 1000.0 / args.steps
    value = tokens / (ms / 1000.0)

    # Roofline region: the same steps launched eagerly with HIP events around
    # every kernel of interest, recorded on the model's stream.
    timing = not args.no_timing
    tsteps = min(args.steps, 10)
    ms_timed = None
    if timing:
        model.set_timing(True)
        model.train_step(ids, labels, n_micro=rc.accum, seqs_per_micro=rc.batch, S=rc.seq,
                         lr=args.lr, clip=1.0, graph=False)
        torch.cuda.synchronize()
        model.reset_timing()
        t2 = time.perf_counter()
        for _ in range(tsteps):
            model.train_step(ids, labels, n_micro=rc.accum, seqs_per_micro=rc.batch, S=rc.seq,
                             lr=args.lr, clip=1.0, graph=False)
        torch.cuda.synchronize()
        ms_timed = (time.perf_counter() - t2) * 1000.0 / tsteps
        model.set_timing(False)

    fl = step_flops(rc)
    result = {
        "metric": METRIC, "value": round(value, 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp32",
        "data": "synthetic (seeded uniform token ids; random-init weights)",
        "config": {"workload": f"{mc.name} LoRA r={mc.lora_r} alpha={mc.lora_alpha:g} "
                               f"targets_mask={mc.lora_mask:#x} fwd+bwd+clip+Adam",
                   "config_id": args.config, "batch": rc.batch, "seq_len": rc.seq,
                   "grad_accum": rc.accum, "tokens_per_step": tokens,
                   "weights": "fp16-stored frozen W" if mc.w_fp16 else "fp32",
                   "shard_budget_mb": args.shard_budget_mb or None},
        "algorithmic_tflop_per_step": round(sum(fl.values()) / 1e12, 4),
        "achieved_tflops_step": round(sum(fl.values()) / (ms / 1000.0) / 1e12, 2),
        "last_loss_mean": loss,
        "launch": "hip graph replay" if args.graph else "eager",
    }
    if timing:
        def cls(c):
            t_ms, work, n = model.timing(c)
            return t_ms, work, n
        t_ms, work, n = cls(CLS_LINEAR)
        ach = work / (t_ms / 1000.0) / 1e12 if t_ms > 0 else 0.0
        # fp16-stored W: the linear and LM-head GEMMs run on the fp16 matrix
        # cores (fp32 operand split into hi + lo fp16 halves, two fp16 products
        # per fp32 product), so their peak is the fp16 one; the fp32 fraction
        # is reported beside it.  Work is counted once (2·M·N·K per GEMM).
        peak_mm = PEAK_FP16_MFMA if mc.w_fp16 else PEAK_FP32_MFMA
        kname = ("linear-layer GEMMs (gemm_h_kernel: fp16 W on fp16 MFMA, fp32 operand as hi+lo fp16, "
                 "rank-r panel on fp32 MFMA; fwd + dX) with their split-K reductions" if mc.w_fp16 else
                 "linear-layer GEMMs (gemm_p_kernel / gemm_q_kernel, fwd + dX, merged LoRA "
                 "weights) with their split-K reductions")
        result["roofline"] = {
            "kernel": kname, "bound": "mfma",
            "achieved": round(ach, 2), "peak": peak_mm, "unit": "TFLOP/s",
            "frac": round(ach / peak_mm, 4), "traffic": traffic_bytes(args.config),
            "launches": n, "avg_launch_us": round(1000.0 * t_ms / max(n, 1), 2),
            "timed_steps": tsteps, "ms_per_step_with_events": round(ms_timed, 4)}
        if mc.w_fp16:
            result["roofline"].update({"peak_fp32": PEAK_FP32_MFMA,
                                       "frac_of_fp32_peak": round(ach / PEAK_FP32_MFMA, 4)})
        br = {}
        for name, c, unit in (("lm_head_gemm", CLS_LMHEAD, "TFLOP/s"), ("attention", CLS_ATTN, "TFLOP/s"),
                              ("cross_entropy", CLS_CE, "GB/s"), ("lora_rank_r", CLS_RANK, "GB/s")):
            t_ms, work, n = cls(c)
            if n == 0:
                continue
            rate = work / (t_ms / 1000.0) / (1e9 if unit == "GB/s" else 1e12)
            peak = PEAK_HBM if unit == "GB/s" else (
                peak_mm if c == CLS_LMHEAD else PEAK_FP32_MFMA)
            br[name] = {"ms_per_step": round(t_ms / tsteps, 4), "achieved": round(rate, 2),
                        "unit": unit, "frac_of_peak": round(rate / peak, 4), "peak": peak, "launches": n}
        lin_ms = model.timing(CLS_LINEAR)[0]
        br["linear_gemm"] = {"ms_per_step": round(lin_ms / tsteps, 4)}
        result["breakdown"] = br
    else:
        result["roofline"] = None
    if api is not None:
        result["operators_api"] = api
    if mc.shard_budget > 0:
        loads, hits, budget = model.shard_stats()
        result["shard_store"] = {"budget_bytes": budget, "loads": loads, "hits": hits}
    if args.calibrate_copy_mb:
        n = args.calibrate_copy_mb * (1 << 20) // 4
        src = torch.ones(n, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        result["copy_calibration_bytes"] = n * 4
        del src, dst
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(rc, args.seed, args.cpu_steps, args.cpu_threads)
    else:
        result["cpu_baseline"] = None
    model.close()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
