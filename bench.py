"""Benchmark of the shifted-window attention hot path on one MI355X.

Step = one SW-MSA attention half of a Swin block (SequentialSwinTransformer
.forward) on config c3 (the high-resolution ocean stage: B=1, 512x1024 tokens,
C=192, 6 heads, window 8, shift 4, ~30 % land folded into the mask), bf16,
inputs resident in HBM.  For this shape the drop-in runs the whole half-block
as one HIP kernel:

    [gather + LayerNorm + q/k/v + window attention + proj + residual + scatter]

`value` is tokens/s of the step.  The `roofline` object is for that kernel,
timed with HIP events on its launch stream over the timed steps: it is
MFMA-bound (1.80e11 flop against 403 MB of HBM traffic per launch), so
`achieved` is TFLOP/s against the dense bf16 peak.  `five_stage` reports the
same step through the unfused path (LN+partition gather, q/k/v GEMM, attention
kernel, proj GEMM, reverse+residual scatter) for comparison, with each of its
HIP kernels timed alone on the step's own arguments.  `attention_backward` is
the training path's attention-core backward on the step's q / k / v;
`mlp_half` the block's MLP half (SequentialMlp) as one kernel against the same
module through torch's ops, and `full_block` both halves together.

    python bench.py [--steps K] [--warmup W] [--no-cpu-baseline] [--config c1..c5|g1]

The other configurations (default c3) run the same measurement: c5 through
the 12-head fused kernel; c1, c2 and c4 (fp32, 7x7 windows, head dim 64)
through the five-stage path, whose roofline is then the attention core's
(HBM-bound), with the MLP half through torch's ops where no fused MLP kernel
serves the shape.
    python bench.py --mode kernels --steps 3     # the step's kernels only,
                                                 # plus a 192 MiB device copy
                                                 # (rocprofv3 counter calibration)
    python bench.py --mode training --steps 5    # the training step only
                                                 # (rocprofv3 kernel traces)
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E
MFMA_BF16_PEAK_TFLOPS = 2516.6  # dense bf16
METRIC = "window-attn fwd TFLOP/s & tokens/sec on 1 MI355X; % of MFMA/HBM roofline"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--config", default="c3", choices=("c1", "c2", "c3", "c4", "c5", "g1", "w32"))
    ap.add_argument("--prewarm-s", type=float, default=3.0,
                    help="seconds of untimed steps before the counted warm-up (clock settling)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="budget of the CPU baseline sample")
    ap.add_argument("--mode", choices=("step", "kernels", "training"), default="step",
                    help="step: the timed benchmark; kernels: run the step's HIP kernels --steps times "
                         "(for rocprofv3 counter passes) and a 192 MiB copy of known size; training: only the "
                         "training step (2 warm-up steps, then --steps timed ones; for rocprofv3 traces)")
    return ap.parse_args()


def measured_traffic(config):
    """HBM bytes per launch of the fused block kernel on `config` from the
    committed rocprofv3 counter summary profiles/swin_block_<config>_pmc.md
    (FETCH_SIZE + WRITE_SIZE, calibrated on a copy of known size), or None when
    there is no such summary."""
    try:
        with open(os.path.join(ROOT, "profiles", f"swin_block_{config}_pmc.md")) as f:
            for line in f:
                if line.strip().startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1].strip())
    except (OSError, ValueError):
        pass
    return None


def run_kernels(cfg, blk, x, steps):
    """The step's kernels on the step's own tensors, `steps` times: the fused
    block kernel, then the five-stage path's three HIP kernels, the plain
    partition kernel, then the
    attention backward on the same q / k / v, then the fused MLP half on the
    block's output; then a device copy of 192 MiB (the counter calibration)."""
    import torch

    from terra_amd import kernels, workloads

    B, L, C = x.shape
    geom = blk.geometry(B)
    grid = x.view(B, cfg.height, cfg.width, C)
    with torch.no_grad():
        for _ in range(steps):
            blk(x)
        win = kernels.swin_partition_ln(grid, geom, blk.norm1.weight, blk.norm1.bias, blk.norm1.eps)
        qkv = blk.attn.qkv(win)
        mask = blk.window_mask(geom)
        for _ in range(steps):
            win = kernels.swin_partition_ln(grid, geom, blk.norm1.weight, blk.norm1.bias, blk.norm1.eps)
            o = blk.attn.core(qkv[..., :C], qkv[..., C:2 * C], qkv[..., 2 * C:], mask=mask)
            kernels.swin_reverse(o, geom, residual=grid)
        for _ in range(steps):
            kernels.swin_partition(grid, geom)
        dqkv = torch.empty_like(qkv)
        table = blk.attn.relative_position_bias_table if blk.attn.use_relative_position_bias else None
        dbias = torch.zeros_like(table, dtype=torch.float32) if table is not None else None
        has_bwd = kernels.attention_backward_supported(qkv[..., :C], blk.attn.num_heads, blk.attn.window_size)
        for _ in range(steps if has_bwd else 0):
            kernels.window_attention_backward(qkv[..., :C], qkv[..., C:2 * C], qkv[..., 2 * C:], o, blk.attn.num_heads,
                                              blk.attn.window_size, blk.attn.scale,
                                              bias_table=table, mask=mask,
                                              dq=dqkv[..., :C], dk=dqkv[..., C:2 * C], dv=dqkv[..., 2 * C:],
                                              dbias=dbias)
        y = blk(x)
        mlp = workloads.mlp_for(cfg, 1).to(x.device).to(x.dtype)
        for _ in range(steps):
            mlp(y)
        src = torch.ones(192 << 20, dtype=torch.uint8, device=x.device)
        dst = torch.zeros_like(src)
        for _ in range(3):
            dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"mode": "kernels", "steps": steps, "calibration_copy_bytes": src.numel()}), flush=True)


def copy_peak_gbs(dev, mib: int = 512, reps: int = 5, per: int = 10) -> float:
    """The runtime's device-to-device copy rate (torch copy_ of a `mib` MiB
    buffer, read + write counted), reported beside the 8 TB/s peak.  Median
    over `reps` loops of `per` copies."""
    import torch
    n = mib << 20
    src = torch.ones(n, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    samples = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(per):
            dst.copy_(src)
        e1.record()
        torch.cuda.synchronize()
        samples.append(e0.elapsed_time(e1) * 1e-3 / per)
    del src, dst
    return 2 * n / statistics.median(samples) / 1e9


def cpu_model() -> str:
    """The host CPU's model name as lscpu prints it (else /proc/cpuinfo)."""
    try:
        out = subprocess.run(["lscpu"], stdout=subprocess.PIPE, stderr=subprocess.DEVNULL, text=True,
                             timeout=10).stdout
        for line in out.splitlines():
            if line.strip().lower().startswith("model name"):
                return line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_baseline(cfg, blk, land, budget_s: float):
    """The oracle's restatement of the reference block (torch CPU, fp32) on a
    bounded sample: a band of whole window rows of the same workload, timed
    with every thread torch uses and with one thread (two warm-up runs, then
    the median of up to 5 runs within the budget of each)."""
    import torch

    from oracle import swin_oracle as so
    from terra_amd import workloads

    params = {k: v.detach().float().cpu() for k, v in blk.state_dict().items() if k != "attn_mask"}
    # sample: the first `rows` token rows (whole window rows); the shift wraps within the band
    rows = min(cfg.height, max(cfg.window, (64 // cfg.window) * cfg.window))
    x = workloads.activations((1, rows * cfg.width, cfg.channels), 1000, torch.float32)
    land_s = land[:rows]
    tokens = rows * cfg.width

    def timed(threads: int, budget: float):
        prev = torch.get_num_threads()
        torch.set_num_threads(threads)
        try:
            times = []
            with torch.inference_mode():
                for _ in range(2):
                    so.swin_block_attention(x, rows, cfg.width, cfg.window, blk.shift_size, cfg.heads, params,
                                            land=land_s, use_attn_mask=cfg.attn_mask)
                t_end = time.perf_counter() + budget
                while len(times) < 5 and (time.perf_counter() < t_end or len(times) < 1):
                    t0 = time.perf_counter()
                    so.swin_block_attention(x, rows, cfg.width, cfg.window, blk.shift_size, cfg.heads, params,
                                            land=land_s, use_attn_mask=cfg.attn_mask)
                    times.append(time.perf_counter() - t0)
        finally:
            torch.set_num_threads(prev)
        return statistics.median(times), len(times)

    threads = torch.get_num_threads()
    t_all, n_all = timed(threads, budget_s)
    t_one, n_one = timed(1, budget_s)
    return {
        "value": tokens / t_all,
        "unit": "tokens/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{rows}x{cfg.width} band of {cfg.name}, fp32 oracle",
        "sample_tokens": tokens,
        "sample_windows": tokens // cfg.tokens,
        "ms_per_sample": t_all * 1e3,
        "runs": n_all,
        "value_1_thread": tokens / t_one,
        "ms_per_sample_1_thread": t_one * 1e3,
        "runs_1_thread": n_one,
        "os_cpu_count": os.cpu_count(),
        "torch_threads": threads,
        "cpu_model": cpu_model(),
        "what": "oracle restatement of the reference op sequence (torch CPU fp32, inference_mode)",
    }


def training_step_us(cfg, dev, warmup: int = 2, reps: int = 5):
    """Median time (us) of one fp32-parameter, bf16-autocast forward + backward
    of the attention half and the MLP half on `cfg` (see main)."""
    import torch

    from terra_amd import workloads

    land = workloads.land_mask(cfg.height, cfg.width, seed=42) if cfg.land else None
    blk = workloads.block_for(cfg, 1 if cfg.shift else 0, land=land).to(dev)
    mlp = workloads.mlp_for(cfg, 1).to(dev)
    x = workloads.activations((cfg.batch, cfg.height * cfg.width, cfg.channels), 1004).to(dev)
    gy = workloads.activations(tuple(x.shape), 1005).to(dev)
    params = list(blk.parameters()) + list(mlp.parameters())

    def step():
        xd = x.detach().requires_grad_(True)
        with torch.amp.autocast(device_type="cuda", dtype=torch.bfloat16):
            y = mlp(blk(xd))
        y.backward(gy)
        for p in params:
            p.grad = None

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    samples = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        step()
        e1.record()
        torch.cuda.synchronize()
        samples.append(1e3 * e0.elapsed_time(e1))
    return statistics.median(samples)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the multi-GPU sharding is designed, "
              "not built", file=sys.stderr)
        sys.exit(2)
    import torch

    from terra_amd import kernels, workloads
    import terra_amd._lib as lib

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(2)
    lib.load()
    dev = torch.device("cuda:0")
    cfg = workloads.CONFIGS[args.config]
    dtype = cfg.dtype
    land = workloads.land_mask(cfg.height, cfg.width, seed=42) if cfg.land else None
    blk = workloads.block_for(cfg, 1 if cfg.shift else 0, land=land).to(dev).to(dtype)
    x = workloads.activations((cfg.batch, cfg.height * cfg.width, cfg.channels), 1003, dtype).to(dev)
    if args.mode == "kernels":
        run_kernels(cfg, blk, x, args.steps)
        return
    if args.mode == "training":
        us = training_step_us(cfg, dev, warmup=2, reps=max(1, args.steps))
        print(json.dumps({"training_step_us": us, "config": args.config, "steps": max(1, args.steps)}), flush=True)
        return

    # Events around the fused kernel on its launch stream (torch's current
    # stream, which the C ABI receives as its hipStream_t).
    events = {"swin_block": [], "partition": [], "window_attention": [], "reverse": [], "proj_scatter": []}
    names = ("swin_block", "swin_partition_ln", "window_attention", "swin_reverse", "linear_residual")
    keys = ("swin_block", "partition", "window_attention", "reverse", "proj_scatter")
    orig = {n: getattr(kernels, n) for n in names}
    recording = {"on": False}
    last_call = {}

    def timed(key, fn):
        def wrapper(*a, **kw):
            if not recording["on"]:
                return fn(*a, **kw)
            s = torch.cuda.current_stream()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(s)
            out = fn(*a, **kw)
            e1.record(s)
            events[key].append((e0, e1))
            last_call[key] = (fn, a, kw)
            return out
        return wrapper

    for n, k in zip(names, keys):
        setattr(kernels, n, timed(k, orig[n]))

    prewarm = {"s": 0.0, "steps": 0}
    # c1 and c2 fit in L2 + the Infinity Cache: their steps are timed cold, a
    # 512 MiB write between steps (outside each step's event pair).
    flush = torch.empty(512 << 20, dtype=torch.uint8, device=dev) if args.config in ("c1", "c2") else None

    def steps_once(steps):
        """The step `steps` times; ms per step.  Cold configurations: a
        512 MiB write before each step and each step between its own events;
        otherwise all steps back to back between one event pair."""
        if flush is not None:
            pairs = []
            for i in range(steps):
                flush.fill_(i & 0xFF)
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                blk(x)
                e1.record()
                pairs.append((e0, e1))
            torch.cuda.synchronize()
            return sum(a.elapsed_time(b) for a, b in pairs) / steps
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        t0.record()
        for _ in range(steps):
            blk(x)
        t1.record()
        torch.cuda.synchronize()
        return t0.elapsed_time(t1) / steps

    def run(steps, warmup, prewarm_s=0.0):
        with torch.no_grad():
            # Time-based pre-warm: the step repeated for `prewarm_s` seconds,
            # so that the GPU clock has settled under this load before the
            # counted warm-up and the timed steps (a few launches from idle
            # run at a lower clock).
            t_end = time.perf_counter() + prewarm_s
            while time.perf_counter() < t_end:
                for _ in range(10):
                    blk(x)
                torch.cuda.synchronize()
                prewarm["steps"] += 10
            prewarm["s"] += prewarm_s
            for _ in range(warmup):
                blk(x)
            torch.cuda.synchronize()
            # The timed steps carry no per-launch events (an event pair around
            # every launch adds about 3 % to a step); the same number of steps
            # then runs again with events around each kernel launch, which
            # give the per-launch times of the roofline.
            ms = steps_once(steps)
            recording["on"] = True
            steps_once(steps)
            recording["on"] = False
        return ms

    def isolated_us(key, reps=5, per=20):
        """Median over `reps` loops of `per` back-to-back launches of one
        kernel on the arguments of its last call in the step, between two
        events (steady state of the kernel run repeatedly; any gap the host
        leaves between launches counts, so this errs on the slow side)."""
        fn, a, kw = last_call[key]
        with torch.no_grad():
            for _ in range(per):
                fn(*a, **kw)
            samples = []
            for _ in range(reps):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                for _ in range(per):
                    fn(*a, **kw)
                e1.record()
                torch.cuda.synchronize()
                samples.append(1e3 * e0.elapsed_time(e1) / per)
        return statistics.median(samples)

    try:
        ms = run(args.steps, args.warmup, args.prewarm_s)
        # The fused kernel serves bf16, 8x8 windows, head dim 32 (c3, c5); the
        # other configurations run the five-stage path as the step itself.
        fused = bool(events["swin_block"])
        if args.config == "c3" and not fused:
            raise RuntimeError("the fused block kernel did not serve the benchmark step")
        if fused:
            blk.use_fused_block = False  # the five-stage path, for comparison
            ms_five = run(max(5, args.steps // 2), 10)
            blk.use_fused_block = True
        else:
            ms_five = ms
        # At C = 1024 the step projects, reverses and adds the residual in one
        # linear-kernel launch; the reverse kernel alone is then timed on the
        # same windows and grid, and the launch against torch's proj (hipBLASLt)
        # followed by the reverse kernel.
        scatter = "proj_scatter" in last_call
        if scatter:
            fn, a, kw = last_call["proj_scatter"]
            o_, r_, geom_s = a[0], a[3], kw["geom"]
            last_call["reverse"] = (orig["swin_reverse"], (o_, geom_s), dict(residual=r_, out=torch.empty_like(r_)))
            pw, pb = blk.attn.proj.weight.detach(), blk.attn.proj.bias.detach()
            last_call["proj_torch"] = (lambda: orig["swin_reverse"](
                torch.nn.functional.linear(o_, pw, pb), geom_s, residual=r_), (), {})
        iso = {k: isolated_us(k) for k in ("partition", "window_attention", "reverse")}
        if scatter:
            iso["proj_scatter"] = isolated_us("proj_scatter")
            iso["proj_torch"] = isolated_us("proj_torch")
        # The plain gather (pad + roll + partition, no LayerNorm) on the same
        # frame: the partition kernel of a block whose LayerNorm is not fused.
        x_grid, geom_ = last_call["partition"][1][0], last_call["partition"][1][1]
        last_call["partition_plain"] = (kernels.swin_partition, (x_grid, geom_), {})
        iso["partition_plain"] = isolated_us("partition_plain")
        # The training-path backward of the same attention call (row f3): the
        # step's q / k / v, a synthetic output gradient, dq | dk | dv into one
        # [B_, N, 3C] buffer and the bias-table gradient.
        fn, a, kw = last_call["window_attention"]
        q_, k_, v_ = a[0], a[1], a[2]
        dout = torch.randn(q_.shape, generator=torch.Generator(device=q_.device).manual_seed(7), device=q_.device,
                           dtype=q_.dtype)
        dqkv = torch.empty(q_.shape[:-1] + (3 * q_.shape[-1],), device=q_.device, dtype=q_.dtype)
        C_ = q_.shape[-1]
        dbias = None if kw.get("bias_table") is None else torch.zeros_like(kw["bias_table"], dtype=torch.float32)
        last_call["attention_backward"] = (kernels.window_attention_backward, (q_, k_, v_, dout) + tuple(a[3:]), dict(
            bias_table=kw.get("bias_table"), mask=kw.get("mask"), dq=dqkv[..., :C_], dk=dqkv[..., C_:2 * C_],
            dv=dqkv[..., 2 * C_:], dbias=dbias))
        has_bwd = kernels.attention_backward_supported(q_, cfg.heads, (cfg.window, cfg.window), None)
        if has_bwd:
            iso["attention_backward"] = isolated_us("attention_backward")
        # The block's MLP half (row f4's buildable part): the SequentialMlp that
        # follows the attention half, on the step's output, as one kernel; and
        # the same module through torch's ops (the reference's norm2 / fc1 /
        # GELU / fc2 / add sequence) for comparison.
        mlp = workloads.mlp_for(cfg, 1).to(dev).to(dtype)
        with torch.no_grad():
            y_blk = blk(x)
            mlp_fused = mlp._fusable(y_blk)
            if args.config == "c3" and not mlp_fused:
                raise RuntimeError("the fused MLP kernel does not serve this configuration")
        if mlp_fused:  # bf16 with C in {128, 192, 384, 768}; other shapes run torch's sequence only
            last_call["mlp"] = (kernels.swin_mlp, (y_blk,), dict(out=torch.empty_like(y_blk), **mlp._fused_args()))
            iso["mlp"] = isolated_us("mlp")
        with torch.no_grad():
            mlp_gemm = (not mlp_fused) and mlp._gemm_path(y_blk)
        if mlp_gemm:  # C = 1024: HIP LayerNorm, fc1 + GELU on the linear kernel, fc2 + x on hipBLASLt
            last_call["mlp_gemm"] = (mlp, (y_blk,), {})
            iso["mlp_gemm"] = isolated_us("mlp_gemm")
        mlp.use_fused_mlp = False
        last_call["mlp_torch"] = (mlp, (y_blk,), {})
        iso["mlp_torch"] = isolated_us("mlp_torch")
        mlp.use_fused_mlp = True
        # A training step of the whole block (attention half + MLP half) as the
        # reference trains it (core/runtime/run_model.py:424-448): fp32 input
        # and parameters under bf16 autocast, forward then backward of a
        # synthetic output gradient (no optimizer update).  The LayerNorms and
        # their backward, partition / reverse and the attention core with its
        # backward run on the HIP kernels (the Linear bias gradients summed
        # inside the kernels that write the gradients); the projection, fc1 and
        # fc2 GEMMs and their backward on hipBLASLt through torch.  Median of
        # 10 steps after 3 warm-up steps (a step is 5-6 ms at c3).
        train = training_step_us(cfg, dev, warmup=3, reps=10) if has_bwd else None
    finally:
        for n in names:
            setattr(kernels, n, orig[n])

    B_, N, C = cfg.num_windows, cfg.tokens, cfg.channels
    elt = torch.tensor([], dtype=dtype).element_size()
    n_real = cfg.tokens  # square windows, no padded keys
    grid_bytes = float(cfg.batch * cfg.height * cfg.width * C * elt)
    block_bytes = 2.0 * grid_bytes                       # x read once, y written once
    flops_win = 2.0 * N * C * 3 * C + 4.0 * n_real * n_real * C + 2.0 * N * C * C
    block_flops = flops_win * B_
    core_flops = 4.0 * n_real * n_real * C * B_
    core_bytes = 4.0 * B_ * N * C * elt
    part_bytes = grid_bytes + B_ * N * C * elt
    bwd_bytes = 7.0 * B_ * N * C * elt
    bwd_flops = 10.0 * n_real * n_real * C * B_
    rev_bytes = B_ * N * C * elt + 2 * grid_bytes
    grid_tokens = cfg.batch * cfg.height * cfg.width
    mlp_flops = 2.0 * 2.0 * grid_tokens * C * (4 * C)    # fc1 + fc2
    mlp_bytes = 2.0 * grid_bytes                         # x read once, y written once

    def launch_us(name):
        """Per-launch durations (us) of a kernel over the timed steps: HIP
        events on its launch stream around each launch."""
        return [1e3 * a.elapsed_time(b) for a, b in events[name]]

    tokens = cfg.real_tokens
    if fused:
        per_launch = launch_us("swin_block")
        t_blk = statistics.mean(per_launch)
        blk_tflops = block_flops / (t_blk * 1e-6) / 1e12
        roofline = {
            "kernel": (("swin_block_w7_kernel" if cfg.window == 7 else
                        "swin_block_hd64_kernel" if cfg.channels == 768 else
                        "swin_block_dw_kernel" if cfg.heads == 6 else f"swin_block_kernel<{cfg.heads}>") +
                       " (fused LN + qkv + window attention + proj + residual, gather/scatter)"),
            "bound": "mfma",
            "achieved": blk_tflops,
            "peak": MFMA_BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": blk_tflops / MFMA_BF16_PEAK_TFLOPS,
            "traffic": measured_traffic(args.config),
            "algorithmic_flops_per_launch": block_flops,
            "algorithmic_bytes_per_launch": block_bytes,
            "avg_launch_us": t_blk,
            "median_launch_us": statistics.median(per_launch),
            "min_launch_us": min(per_launch),
            "max_launch_us": max(per_launch),
            "launches": len(per_launch),
            "hbm_GB_s": block_bytes / (t_blk * 1e-6) / 1e9,
            "hbm_frac": block_bytes / (t_blk * 1e-6) / 1e9 / HBM_PEAK_GBS,
        }
    elif N > 64:
        # Windows of more than 64 tokens (w32: 1024): the flash core does
        # 4 N^2 C flops per window on 4 N C elements, MFMA-bound.
        t_att = iso["window_attention"]
        roofline = {
            "kernel": "window_attn_flash_kernel<%d> (online-softmax core, five-stage path)" % (C // cfg.heads),
            "bound": "mfma",
            "achieved": core_flops / (t_att * 1e-6) / 1e12,
            "peak": MFMA_BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": core_flops / (t_att * 1e-6) / 1e12 / MFMA_BF16_PEAK_TFLOPS,
            "traffic": None,
            "algorithmic_flops_per_launch": core_flops,
            "algorithmic_bytes_per_launch": core_bytes,
            "avg_launch_us": t_att,
            "hbm_GB_s": core_bytes / (t_att * 1e-6) / 1e9,
        }
    else:
        # The step is the five-stage path; its dominant HIP kernel is the
        # window attention core, HBM-bound (N / elt flop per byte).
        t_att = iso["window_attention"]
        roofline = {
            "kernel": "window attention core (five-stage path)",
            "bound": "hbm",
            "achieved": core_bytes / (t_att * 1e-6) / 1e9,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": core_bytes / (t_att * 1e-6) / 1e9 / HBM_PEAK_GBS,
            "traffic": None,
            "algorithmic_bytes_per_launch": core_bytes,
            "algorithmic_flops_per_launch": core_flops,
            "avg_launch_us": t_att,
            "TFLOP_s": core_flops / (t_att * 1e-6) / 1e12,
        }
    res = {
        "metric": METRIC,
        "value": tokens / (ms * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "prewarm": {"seconds": prewarm["s"], "steps": prewarm["steps"],
                    "note": "untimed steps before the counted warm-up, so the clock has settled"},
        "ms_per_step": ms,
        "windows_per_s": B_ / (ms * 1e-3),
        "timing": ("the timed steps carry no per-launch events; a second pass of as many steps records events "
                   "around each kernel launch for the roofline's launch times"),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if dtype == torch.bfloat16 else "fp32",
        "data": "synthetic (seeded N(0,1) activations, trunc-normal(0.02) weights, seeded smoothed-noise land mask)",
        "config": {
            "workload": (f"{cfg.name}: {'SW' if cfg.shift else 'W'}-MSA attention half of a Swin block (LayerNorm, "
                         f"roll+partition, q/k/v, window attention"
                         + (f" with relative-position bias{' + shift' if cfg.shift else ''}"
                            f"{'/land' if cfg.land else ''} mask" if cfg.rel_bias or cfg.attn_mask else
                            " without relative-position bias or mask")
                         + ", proj, reverse+roll, "
                         f"residual) {'as one fused kernel' if fused else 'through the five-stage path'}, "
                         f"B={cfg.batch}, {cfg.height}x{cfg.width} tokens, C={C}, "
                         f"{cfg.heads} heads, window {cfg.window}, shift {cfg.shift}"
                         + (", ~30% land mask" if cfg.land else "")),
            "windows": B_,
            "tokens": tokens,
            "parallelism": "single GPU",
            "cache": ("cold: a 512 MiB write between steps, each step between its own events" if flush is not None
                      else "working set larger than L2 + Infinity Cache; steps back to back"),
        },
        "roofline": roofline,
        # The unfused path, for comparison.  Its kernels are timed alone, back to
        # back on the step's own arguments (median of 5 x 20 launches).
        "five_stage": {
            "ms_per_step": ms_five,
            "tokens_per_s": tokens / (ms_five * 1e-3),
            "window_attention": {
                "us": iso["window_attention"],
                "GB_s": core_bytes / (iso["window_attention"] * 1e-6) / 1e9,
                "hbm_frac": core_bytes / (iso["window_attention"] * 1e-6) / 1e9 / HBM_PEAK_GBS,
                "TFLOP_s": core_flops / (iso["window_attention"] * 1e-6) / 1e12,
            },
            "partition": {"us": iso["partition_plain"],
                          "GB_s": part_bytes / (iso["partition_plain"] * 1e-6) / 1e9,
                          "hbm_frac": part_bytes / (iso["partition_plain"] * 1e-6) / 1e9 / HBM_PEAK_GBS},
            "layernorm_partition": {"us": iso["partition"],
                                    "GB_s": part_bytes / (iso["partition"] * 1e-6) / 1e9,
                                    "hbm_frac": part_bytes / (iso["partition"] * 1e-6) / 1e9 / HBM_PEAK_GBS},
            "reverse_residual": {"us": iso["reverse"],
                                 "GB_s": rev_bytes / (iso["reverse"] * 1e-6) / 1e9,
                                 "hbm_frac": rev_bytes / (iso["reverse"] * 1e-6) / 1e9 / HBM_PEAK_GBS},
        },
        # Training path (row f3): backward of the attention core on the same
        # call, timed alone.  Algorithmic bytes: read q, k, v, dout and write
        # dq, dk, dv (7 N C elt per window); FLOPs: S recomputed, dP, dV, dQ,
        # dK (10 N^2 C per window).
        # Windows of more than 64 tokens: three MFMA-bound passes (row
        # statistics, dK / dV over query tiles, dQ over key tiles), so also
        # their fraction of the dense bf16 MFMA peak (on the 10 N^2 C
        # algorithmic FLOPs; the passes compute 18 N^2 C with the recomputed
        # forward).
        "attention_backward": {
            "kernel": ((f"window_attn_bwd_kernel<{cfg.channels // cfg.heads}, 1>" if cfg.channels // cfg.heads != 32
                        else "window_attn_bwd_kernel<32, 2>") if N <= 64 else
                       "flash backward: window_attn_flash_kernel<%d, 4, stats> + window_attn_flash_dkv_kernel<%d> + "
                       "window_attn_flash_dq_kernel<%d>" % ((cfg.channels // cfg.heads,) * 3)),
            "us": iso["attention_backward"],
            "GB_s": bwd_bytes / (iso["attention_backward"] * 1e-6) / 1e9,
            "hbm_frac": bwd_bytes / (iso["attention_backward"] * 1e-6) / 1e9 / HBM_PEAK_GBS,
            "TFLOP_s": bwd_flops / (iso["attention_backward"] * 1e-6) / 1e12,
            "algorithmic_bytes_per_launch": bwd_bytes,
            "algorithmic_flops_per_launch": bwd_flops,
            **({"mfma_frac": bwd_flops / (iso["attention_backward"] * 1e-6) / 1e12 / MFMA_BF16_PEAK_TFLOPS}
               if N > 64 else {}),
        } if has_bwd else {"kernel": None, "note": "no backward kernel at this shape"},
    }
    # The targets the hot path is held to, with this run's figures: the
    # attention core (HBM-bound) >= 70 % of HBM, partition and reverse >= 80 %,
    # and the fused kernel's fraction of the dense bf16 MFMA peak.
    fs = res["five_stage"]
    # HBM fractions are against the 8 TB/s peak; each also carries its rate
    # against the measured device-to-device copy of the runtime (torch
    # copy_, a hipMemcpy D2D), which the streaming kernels here exceed.
    copy_gbs = copy_peak_gbs(x.device)
    res["d2d_copy"] = {"GB_s": copy_gbs, "frac_of_peak": copy_gbs / HBM_PEAK_GBS,
                       "how": "torch copy_ of a 512 MiB device buffer, read + write counted, median of 5 x 10"}
    res["targets"] = {
        "attention_core_hbm_frac": {"value": fs["window_attention"]["hbm_frac"], "target": 0.70,
                                    "vs_d2d_copy": fs["window_attention"]["GB_s"] / copy_gbs},
        "partition_hbm_frac": {"value": fs["partition"]["hbm_frac"], "target": 0.80,
                               "vs_d2d_copy": fs["partition"]["GB_s"] / copy_gbs},
        "reverse_hbm_frac": {"value": fs["reverse_residual"]["hbm_frac"], "target": 0.80,
                             "vs_d2d_copy": fs["reverse_residual"]["GB_s"] / copy_gbs},
    }
    if fused:
        res["targets"]["fused_block_mfma_frac"] = {"value": res["roofline"]["frac"], "target": 0.50}
    t_attn_half = t_blk if fused else ms * 1e3
    if mlp_fused:
        res["mlp_half"] = {
            "kernel": ((f"swin_mlp_wide_kernel<{C}>" if C in (128, 768) else
                        f"swin_mlp_kernel<{C}, {'true' if C <= 192 else 'false'}>")
                       + " (LayerNorm + fc1 + exact GELU + fc2 + residual, hidden layer on chip)"),
            "us": iso["mlp"],
            "TFLOP_s": mlp_flops / (iso["mlp"] * 1e-6) / 1e12,
            "mfma_frac": mlp_flops / (iso["mlp"] * 1e-6) / 1e12 / MFMA_BF16_PEAK_TFLOPS,
            "GB_s": mlp_bytes / (iso["mlp"] * 1e-6) / 1e9,
            "torch_us": iso["mlp_torch"],
            "speedup_vs_torch": iso["mlp_torch"] / iso["mlp"],
            "algorithmic_flops_per_launch": mlp_flops,
            "algorithmic_bytes_per_launch": mlp_bytes,
        }
        t_mlp = iso["mlp"]
    elif mlp_gemm:
        res["mlp_half"] = {
            "kernel": "HIP LayerNorm over the token rows + linear_kernel (fc1 + exact GELU epilogue) + hipBLASLt fc2 + x",
            "us": iso["mlp_gemm"],
            "TFLOP_s": mlp_flops / (iso["mlp_gemm"] * 1e-6) / 1e12,
            "mfma_frac": mlp_flops / (iso["mlp_gemm"] * 1e-6) / 1e12 / MFMA_BF16_PEAK_TFLOPS,
            "torch_us": iso["mlp_torch"],
            "speedup_vs_torch": iso["mlp_torch"] / iso["mlp_gemm"],
            "algorithmic_flops_per_launch": mlp_flops,
        }
        t_mlp = iso["mlp_gemm"]
    else:
        res["mlp_half"] = {"kernel": None, "torch_us": iso["mlp_torch"],
                           "note": "no fused MLP kernel for this shape: torch's op sequence timed"}
        t_mlp = iso["mlp_torch"]
    if scatter:
        proj_flops = 2.0 * B_ * N * C * C
        proj_bytes = B_ * N * C * elt + 2 * grid_bytes  # O read, x read, y written
        res["proj_scatter"] = {
            "kernel": "linear_kernel<residual> (proj + bias, window reverse + inverse roll + residual, one launch)",
            "us": iso["proj_scatter"],
            "TFLOP_s": proj_flops / (iso["proj_scatter"] * 1e-6) / 1e12,
            "mfma_frac": proj_flops / (iso["proj_scatter"] * 1e-6) / 1e12 / MFMA_BF16_PEAK_TFLOPS,
            "GB_s": proj_bytes / (iso["proj_scatter"] * 1e-6) / 1e9,
            "torch_proj_then_reverse_us": iso["proj_torch"],
            "algorithmic_flops_per_launch": proj_flops,
            "algorithmic_bytes_per_launch": proj_bytes,
        }
    # The whole Swin block (attention half + MLP half).
    res["full_block"] = {"us": t_attn_half + t_mlp, "tokens_per_s": tokens / ((t_attn_half + t_mlp) * 1e-6)}
    res["training_step"] = {
        "us": train, "tokens_per_s": tokens / (train * 1e-6),
        "what": ("forward + backward of the attention half and the MLP half, fp32 input and parameters under bf16 "
                 "autocast (the reference's training mode), synthetic output gradient, no optimizer update; "
                 "median of 10 after 3 warm-up steps"),
    } if train is not None else {"us": None, "note": "no backward for windows of more than 64 tokens"}
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline(cfg, blk, land if land is not None else
                                           torch.zeros(cfg.height, cfg.width, dtype=torch.bool), args.cpu_seconds)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
