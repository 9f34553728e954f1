"""Benchmark: QuaternionMamba2Block forward on one MI355X.

    python bench.py [--gpus 1] [--steps 20] [--warmup 3]
                    [--mode full|ssm|ssm_b1|ssm_b1_whole|ssm_train|ssm_bwd|cumprod|cayley|qln|gemm|gemm_hipblaslt|fused_bc|bc_unfused|out_step|out_step_unfused|out_step_block|decode|decode_graph|block_long|train|copy]
                    [--preset small|base|large]

Workload (BASELINE configs[2]/[3] shape): one QuaternionMamba2Block forward,
batch 4, seq_len 2048, d_model 768, d_state 64, d_conv 4, expand_factor 2
(d_inner 1536); random-init weights (seed 0), bf16 storage with fp32
accumulation in the HIP kernels, synthetic x ~ N(0, 1) resident in HBM.

`value` is block-forward tokens/s (batch*seq_len*steps / timed seconds,
timed region bracketed by torch.cuda.synchronize()). `roofline` is the fused
SSM kernel (mqc_ssm_fused_fwd): algorithmic bytes per launch divided by its
mean launch duration, measured with HIP events on the stream it runs on.
`roofline_gemm` puts the kernel that holds most of the block's time, the B/C
projections fused with the SSM walk (mqc_ssm_fused_bc_fwd: both projections'
flops per launch), against the dense bf16 MFMA peak, with hipBLASLt's and this
library's standalone GEMMs of one projection beside it.
`cpu_baseline` times the CPU oracle (a restatement of the reference's
sequential torch path) on a bounded prefix of the same workload. `train_c4`
reports config 4 (block forward + backward under fp16 autocast) and the SSM's
training-forward and backward kernels at the same shape; `lm_c5` the base
preset LM forward (config 5).

The other modes run one kernel in a loop for rocprofv3 (no JSON contract).
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "block fwd tokens/s @B4 T2048 d768 s64; scan HBM GB/s as % of peak"
PEAK_HBM_GBS = 8000.0
PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
B, T, DM, DS, DCONV, EXPAND = 4, 2048, 768, 64, 4, 2
DI = DM * EXPAND


def ssm_bytes(b, t, d, s, el=2):
    """Algorithmic HBM bytes of one fused SSM launch: B and C read once,
    delta and s read once, Lambda (fp32, 4 per (d,k)) and D (fp32) read once,
    y written once."""
    return (2 * b * t * d * s * 4 * el + 2 * b * t * d * el + d * s * 4 * 4 + d * 4
            + b * t * d * 4 * el)


def qln_bytes(rows, d, el=2):
    return 2 * rows * d * 4 * el + d * 4 + d * 16


def ssm_bwd_bytes(b, t, d, s, el=2, ckpt_every=8):
    """Algorithmic HBM bytes of one SSM backward launch: reads delta, s, B, C,
    gy (storage dtype), the fp32 state checkpoints and Lambda/D; writes dB, dC
    (storage dtype), d_delta, d_s (fp32) and the per-batch parameter partials."""
    n_ckpt = -(-t // ckpt_every)
    reads = (2 * b * t * d * el + 2 * b * t * d * s * 4 * el + b * t * d * 4 * el
             + b * n_ckpt * d * s * 4 * 4 + d * s * 4 * 4 + d * 4)
    writes = 2 * b * t * d * s * 4 * el + 2 * b * t * d * 4 + b * d * s * 4 * 4 + b * d * 4
    return reads + writes


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def event_time_ms(fn, reps):
    """Mean duration of fn() over reps launches, each bracketed by events on the
    current stream (the stream the library launches on)."""
    import torch

    starts = [torch.cuda.Event(enable_timing=True) for _ in range(reps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(reps)]
    for i in range(reps):
        starts[i].record()
        fn()
        ends[i].record()
    torch.cuda.synchronize()
    return sum(s.elapsed_time(e) for s, e in zip(starts, ends)) / reps


def make_block(dtype):
    import torch
    import mambaqc_amd

    torch.manual_seed(0)
    with torch.device("cuda"):
        blk = mambaqc_amd.QuaternionMamba2Block(DM, d_state=DS, d_conv=DCONV, expand_factor=EXPAND)
    return blk.to(dtype).eval()


def ssm_inputs(blk, x):
    """The fused SSM's operands exactly as the block forms them for input x."""
    import torch
    import torch.nn.functional as F

    with torch.no_grad():
        xz = blk.in_proj(x)
        x_in, _ = xz.chunk(2, dim=-1)
        xa = F.silu(blk.conv1d(x_in))
        delta = F.softplus(blk.dt_proj(xa))
        Bq = blk.B_proj(xa).view(B, T, DI, DS, 4)
        Cq = blk.C_proj(xa).view(B, T, DI, DS, 4)
        s = torch.sigmoid(blk.gate_proj(xa)) * xa
    return delta, s, Bq, Cq, xa


def cpu_baseline(blk, x, t_sample=256):
    """Oracle block forward (fp32, CPU) on the first t_sample steps of the same
    input, with the same weights, on every core this process may run on. The
    sequential path's cost is linear in T."""
    import torch
    import oracle

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    sd = {k: v.detach().float().cpu() for k, v in blk.state_dict().items()}
    xs = x[:, :t_sample].float().cpu()
    oracle.block_forward_reference(sd, xs[:, :2], d_state=DS)  # warm-up
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        oracle.block_forward_reference(sd, xs, d_state=DS)
        times.append(time.perf_counter() - t0)
    med = sorted(times)[1]
    cpu = platform.processor() or ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": round(B * t_sample / med, 2),
        "unit": "tokens/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"oracle block forward (fp32 torch restatement of the reference's sequential "
                   f"CPU path) on x[:, :{t_sample}] of the B4 d768 s64 workload, median of 3; "
                   f"os.cpu_count()={os.cpu_count()}, cpu={cpu}"),
    }


def cpu_components():
    """The rest of the CPU baseline plan: the oracle (fp32 torch on the host's
    cores) on bounded samples of configs 1-3, median of 3 after one warm-up.
    GB/s figures use the same algorithmic bytes as the GPU kernels."""
    import torch
    import torch.nn.functional as F
    import mambaqc_amd
    import oracle

    def med(fn):
        fn()
        ts = []
        for _ in range(3):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return sorted(ts)[1]

    out = {}
    g = torch.Generator().manual_seed(0)
    # Config 1: the whole block, B1 T64 d64 s16.
    torch.manual_seed(0)
    blk = mambaqc_amd.QuaternionMamba2Block(64, d_state=16, d_conv=4, expand_factor=2)
    sd = blk.state_dict()
    x1 = torch.randn(1, 64, 64, generator=g)
    sec = med(lambda: oracle.block_forward_reference(sd, x1, d_state=16))
    out["c1_block_fwd_tokens_s"] = round(64 / sec, 1)
    # Config 2 on a slice of 96 of the 768 d's (all of B, T, S): Cayley, then the scan.
    shape = (2, 256, 96, 64)
    n = lambda: torch.randn(*shape, generator=g)
    z = torch.empty(*shape, 4)
    z[..., 0] = -torch.exp(n()) * F.softplus(n())
    for c in range(1, 4):
        z[..., c] = n() * F.softplus(n())
    nbytes = 2 * z.numel() * 4
    sec = med(lambda: oracle.cayley_reference(z))
    out["c2_cayley_GBs"] = round(nbytes / sec / 1e9, 3)
    q = oracle.cayley_reference(z)
    sec = med(lambda: oracle.cumprod_reference(q))
    out["c2_cumprod_GBs"] = round(nbytes / sec / 1e9, 3)
    del z, q
    # Config 3 SSM + QLN on B1, the first 32 steps, 64 of the 1536 d's (S = 64).
    Bt, Tt, Dt, St = 1, 32, 64, 64
    delta = F.softplus(torch.randn(Bt, Tt, Dt, generator=g) - 2)
    sv = torch.randn(Bt, Tt, Dt, generator=g)
    Bq = torch.randn(Bt, Tt, Dt, St, 4, generator=g) * 0.02
    Cq = torch.randn(Bt, Tt, Dt, St, 4, generator=g) * 0.02
    la = torch.randn(Dt, St, generator=g) * 0.5 + 1
    li = torch.randn(Dt, St, 3, generator=g) * 0.1
    Dv, gm, bt = torch.ones(Dt), torch.ones(Dt), torch.zeros(Dt, 4)
    sec = med(lambda: oracle.qln_reference(
        oracle.ssm_forward_dl_reference(delta, sv, Bq, Cq, la, li, Dv), gm, bt))
    lanes = Bt * Tt * Dt
    out["c3_ssm_qln_lane_steps_per_s"] = round(lanes * St / sec, 1)
    out["c3_ssm_qln_equiv_tokens_s"] = round(lanes * St / sec / (DI * DS), 3)
    out["samples"] = ("c1: whole block B1 T64 d64 s16; c2: [2,256,96,64,4] fp32 (96 of 768 d's) "
                      "Cayley then cumprod; c3: SSM+QLN on B1 T32, 64 of 1536 d's, S64, "
                      "equiv_tokens_s = (b,t,d,k) lane-steps per s / (1536 * 64)")
    return out


def read_traffic(name="ssm_fused_fwd_c3_traffic.txt", key="traffic_bytes_per_launch:"):
    """Bytes per launch leaving the L2 for a kernel, from a committed rocprofv3 PMC
    summary (FETCH_SIZE + WRITE_SIZE, scaled by the copy-kernel factor)."""
    p = ROOT / "profiles" / name
    if not p.exists():
        return None
    for line in p.read_text().splitlines():
        if line.startswith(key):
            return float(line.split(":", 1)[1])
    return None


def nat_aligned(t):
    from mambaqc_amd import _native as nat
    return nat.aligned16(t)


def mqc_gemm(x, w, out):
    """out = x @ w.T through the library's MFMA GEMM (bf16)."""
    from mambaqc_amd import _native as nat
    nat.call("mqc_gemm_nt", x, x.data_ptr(), w.data_ptr(), out.data_ptr(), x.shape[0],
             w.shape[0], x.shape[1], nat.BF16, nat.stream_of(x))
    return out


def box_copy_gbs(reps=20):
    """Read+write bandwidth of a 1 GiB device-to-device copy on this box. HBM
    throughput differs from box to box by up to ~15 %; this puts the SSM's
    figure beside what a plain copy gets on the same device."""
    import torch

    src = torch.empty(1 << 28, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    ms = event_time_ms(lambda: dst.copy_(src), reps)
    del src, dst
    torch.cuda.empty_cache()
    return 2 * (1 << 30) / (ms * 1e-3) / 1e9


FUSED_STAGE = "fused B/C projections + SSM (mqc_ssm_fused_bc_fwd)"


def flushed_time_ms(fn, reps):
    """Median duration of fn() over reps calls, each after a 1 GiB device copy
    that evicts L2 and the Infinity Cache; the copy occupies the device while fn's
    launches are queued, so the events around fn time its kernels, not the host."""
    import torch

    src = torch.empty(1 << 28, device="cuda")
    dst = torch.empty_like(src)
    fn()
    ts = []
    for _ in range(reps):
        dst.copy_(src)
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        fn()
        e1.record()
        torch.cuda.synchronize()
        ts.append(e0.elapsed_time(e1))
    del src, dst
    return sorted(ts)[len(ts) // 2]


def run_full(args):
    import torch
    from mambaqc_amd import kernels as K
    from mambaqc_amd.block import _out_proj, out_gate, out_proj_gate

    dtype = torch.bfloat16
    # Measured first, on a cold device, like the standalone copy mode.
    copy_gbs = box_copy_gbs()
    log(f"building block d_model={DM} d_state={DS} expand={EXPAND} on {torch.cuda.get_device_name(0)}")
    blk = make_block(dtype)
    g = torch.Generator(device="cuda").manual_seed(0)
    x = torch.randn(B, T, DM, generator=g, device="cuda").to(dtype)

    with torch.inference_mode():
        for i in range(args.warmup):
            blk(x)
        torch.cuda.synchronize()
        log(f"warmup {args.warmup} done")
        t0 = time.perf_counter()
        for _ in range(args.steps):
            out = blk(x)
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
    ms_step = elapsed * 1e3 / args.steps
    tokens_s = B * T * args.steps / elapsed
    log(f"block fwd: {ms_step:.3f} ms/step, {tokens_s:.0f} tokens/s")

    # Fused SSM kernel alone, on the block's own operands.
    delta, s, Bq, Cq, xa_in = ssm_inputs(blk, x)
    la, li, Dv = (blk.Lambda_alpha.detach().float(), blk.Lambda_imag.detach().float(),
                  blk.D.detach().float())
    fn = lambda: K.ssm_forward_fused_dl(delta, s, Bq, Cq, la, li, Dv, eps=1e-6)
    with torch.inference_mode():
        fn()
        ssm_ms = event_time_ms(fn, max(args.steps, 10))
    nbytes = ssm_bytes(B, T, DI, DS)
    achieved = nbytes / (ssm_ms * 1e-3) / 1e9
    log(f"ssm_fused_fwd: {ssm_ms:.3f} ms, {achieved:.0f} GB/s ({achieved / PEAK_HBM_GBS:.1%} of 8 TB/s)")

    # Per-stage breakdown of one block forward (events around each stage).
    stages = {}
    with torch.inference_mode():
        y = fn()
        stages["ssm_fused_fwd"] = ssm_ms
        stages["qln"] = event_time_ms(lambda: blk.norm(y), 10)
        stages["B_proj+C_proj GEMMs"] = event_time_ms(lambda: (blk.B_proj(s), blk.C_proj(s)), 5)
        # The block's path at this size: B/C projections fused into the SSM kernel.
        wbf, wcf = blk.B_proj.weight.detach(), blk.C_proj.weight.detach()
        stages["fused B/C projections + SSM (mqc_ssm_fused_bc_fwd)"] = event_time_ms(
            lambda: K.ssm_forward_fused_bc(xa_in, wbf, wcf, delta, s, la, li, Dv, eps=1e-6), 5)
        del y
        # A/B of the B projection alone: hipBLASLt (column blocks, the block's
        # path) against this library's MFMA GEMM (mqc_gemm_nt), same operands.
        xa = nat_aligned(s.reshape(-1, DI))
        wb = blk.B_proj.weight.detach()
        gemm_out = torch.empty(xa.shape[0], wb.shape[0], device="cuda", dtype=dtype)
        stages["B_proj GEMM hipBLASLt (column blocks)"] = event_time_ms(
            lambda: blk.B_proj(s), 5)
        stages["B_proj GEMM mqc_gemm_nt (MFMA, this library)"] = event_time_ms(
            lambda: mqc_gemm(xa, wb, gemm_out), 5)
        del gemm_out, xa
        # The block's inference paths on the same block and input, interleaved
        # (median over 6 rounds): the default (B/C projections fused into the SSM
        # kernel, output step as out_proj then the gate kernel), B/C unfused
        # (hipBLASLt GEMMs, then the SSM kernel), and the output step fused.
        variants = {
            "block forward (default: B/C fused into the SSM)": (None, None),
            "block forward, B/C unfused (hipBLASLt + SSM)": (False, None),
            "block forward, output step fused (mqc_out_proj_gate_fwd)": (None, True),
        }
        ab = {k: [] for k in variants}
        names = list(variants)
        for r in range(6):
            # The order rotates from round to round, so no variant always follows
            # the same one.
            for name in names[r % 3:] + names[:r % 3]:
                blk.fuse_bc, blk.fuse_out = variants[name]
                blk(x)
                ab[name].append(event_time_ms(lambda: blk(x), 3))
        blk.fuse_bc = blk.fuse_out = None
        for name, v in ab.items():
            stages[name] = sorted(v)[len(v) // 2]
        # The output step alone, fused and unfused, each call after a 1 GiB copy
        # that evicts its operands from the caches (as in the block, where the SSM's
        # traffic has evicted them); the copy keeps the device busy while the step
        # is queued, so the events time the step's kernels only.
        yq = blk.norm(K.ssm_forward_fused_bc(xa_in, wbf, wcf, delta, s, la, li, Dv, eps=1e-6))
        zq = torch.randn(B, T, 2 * DI, generator=g, device="cuda").to(dtype)[..., DI:]
        ow = blk.out_proj.weight.detach()
        stages["output step fused (mqc_out_proj_gate_fwd), caches flushed"] = flushed_time_ms(
            lambda: out_proj_gate(x, zq, yq, ow), 10)
        stages["output step unfused (out_proj + gate kernel), caches flushed"] = flushed_time_ms(
            lambda: out_gate(x, zq, _out_proj(blk.out_proj, yq)), 10)
        del yq, zq
        # The d-sliced B/C path on the same block and input (96 d's per slice:
        # 16 slices of two GEMMs and one chunked SSM each) against the whole
        # projections the block uses at this size.
        blk.bc_slice_d = 96
        stages["block forward, B/C in slices of 96 d's"] = event_time_ms(lambda: blk(x), 3)
        blk.bc_slice_d = None
    qln_gbs = qln_bytes(B * T, DI) / (stages["qln"] * 1e-3) / 1e9
    gemm_flop = 2 * B * T * DI * DI * DS * 4
    del delta, s, Bq, Cq, xa_in
    torch.cuda.empty_cache()
    log(f"box calibration: 1 GiB device copy {copy_gbs:.0f} GB/s; fused SSM at "
        f"{achieved / copy_gbs:.1%} of it")

    # Config 2 standalone: Cayley then cumprod, fp32 [2,256,768,64,4].
    shape = (2, 256, 768, 64)
    z = torch.empty(*shape, 4, device="cuda")
    n = lambda: torch.randn(*shape, generator=g, device="cuda")
    z[..., 0] = -torch.exp(n()) * torch.nn.functional.softplus(n())
    for c in range(1, 4):
        z[..., c] = n() * torch.nn.functional.softplus(n())
    with torch.inference_mode():
        q = K.cayley_discretization_fused(z)
        cay_ms = event_time_ms(lambda: K.cayley_discretization_fused(z), 10)
        K.parallel_scan_quaternion(q)
        scan_ms = event_time_ms(lambda: K.parallel_scan_quaternion(q), 10)
    c2_bytes = 2 * z.numel() * 4
    del z, q
    torch.cuda.empty_cache()

    long_ctx = None if args.block_only else long_context_timing(blk)
    train = None if args.block_only else train_timings(args)
    lm = None if args.block_only else lm_timing(args)

    base = None if args.no_cpu else cpu_baseline(blk, x)
    if base:
        log(f"cpu baseline: {base['value']} tokens/s on {base['cores']} threads")
        base["components"] = cpu_components()
        log(f"cpu components: {base['components']}")

    result = {
        "metric": METRIC,
        "value": round(tokens_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (x ~ N(0,1), random-init weights seed 0)",
        "config": {
            "workload": "QuaternionMamba2Block forward, bf16 storage / fp32 accumulate",
            "global_batch": B, "seq_len": T, "d_model": DM, "d_state": DS, "d_conv": DCONV,
            "expand_factor": EXPAND, "d_inner": DI, "parallelism": "single GPU",
        },
        "roofline": {
            "kernel": "mqc_ssm_fused_fwd (ssm_scan_kernel<bf16, delta-lambda>)",
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBS, 4),
            "traffic": read_traffic(),
            "algorithmic_bytes": nbytes,
            "mean_launch_ms": round(ssm_ms, 4),
            "box_copy_GBs": round(copy_gbs, 1),
            "frac_of_box_copy": round(achieved / copy_gbs, 4),
        },
        # Most of the block's time is the B/C projections, which at this size run
        # fused into the SSM kernel: its MFMA roofline (both projections' flops per
        # launch) beside the SSM's HBM one, with hipBLASLt's and this library's
        # standalone GEMMs for one projection.
        "roofline_gemm": {
            "kernel": "mqc_ssm_fused_bc_fwd (B/C projections + SSM walk, the block's path)",
            "bound": "mfma",
            "achieved": round(2 * gemm_flop / (stages[FUSED_STAGE] * 1e-3) / 1e12, 1),
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(2 * gemm_flop / (stages[FUSED_STAGE] * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
            "flop": 2 * gemm_flop,
            "traffic": read_traffic("fused_bc_ssm_c3.txt", "fused_traffic_bytes_per_launch:"),
            "mean_launch_ms": round(stages[FUSED_STAGE], 4),
            "hipblaslt_B_proj_TFLOPs": round(
                gemm_flop / (stages["B_proj GEMM hipBLASLt (column blocks)"] * 1e-3) / 1e12, 1),
            "mqc_gemm_nt_TFLOPs": round(
                gemm_flop / (stages["B_proj GEMM mqc_gemm_nt (MFMA, this library)"] * 1e-3) / 1e12, 1),
        },
        "stages_ms": {k: round(v, 4) for k, v in stages.items()},
        "components": {
            "qln_c3_GBs": round(qln_gbs, 1),
            "cayley_c2_GBs": round(c2_bytes / (cay_ms * 1e-3) / 1e9, 1),
            "cumprod_scan_c2_GBs": round(c2_bytes / (scan_ms * 1e-3) / 1e9, 1),
            "cayley_c2_ms": round(cay_ms, 4),
            "cumprod_scan_c2_ms": round(scan_ms, 4),
        },
        "long_context": long_ctx,
        "train_c4": train,
        "lm_c5": lm,
        "cpu_baseline": base,
    }
    print(json.dumps(result), flush=True)


LONG_T = 262144
LONG_TRAIN_T = 65536


def long_context_timing(blk):
    """The benchmark's block (config-3 width, bf16) on one sequence of LONG_T
    tokens. Whole B and C would take 2 x 206 GB. The block's inference path runs
    the fused B/C kernel in its split form (B and C never stored; two fp32 partial
    sums of y in a workspace); beside it, the d-sliced path (fuse_bc off: 8 d's per
    B/C slice of 2 GiB, each slice's SSM cut into time chunks)."""
    import torch
    from mambaqc_amd import block as bm

    g = torch.Generator(device="cuda").manual_seed(1)
    x = torch.randn(1, LONG_T, DM, generator=g, device="cuda").to(torch.bfloat16)
    width = bm.bc_slice_width(1, LONG_T, DI, DS, 2)

    def timed():
        torch.cuda.empty_cache()
        torch.cuda.reset_peak_memory_stats()
        base_mem = torch.cuda.memory_allocated()
        with torch.inference_mode():
            blk(x)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(2):
                blk(x)
            torch.cuda.synchronize()
        return ((time.perf_counter() - t0) * 1e3 / 2,
                (torch.cuda.max_memory_allocated() - base_mem) / 2**30)

    ms, peak = timed()
    blk.fuse_bc = False
    sliced_ms, sliced_peak = timed()
    blk.fuse_bc = None
    log(f"long context: B1 T{LONG_T} block forward {ms:.1f} ms ({LONG_T / ms * 1e3:.0f} tokens/s), "
        f"fused B/C (split), peak {peak:.1f} GiB beyond the inputs; d-sliced B/C "
        f"({width} d's per slice) {sliced_ms:.1f} ms, peak {sliced_peak:.1f} GiB")
    del x
    torch.cuda.empty_cache()
    # Training at LONG_TRAIN_T tokens: slices recomputed in the backward, the
    # SSM's training walk and backward in time chunks.
    xt = torch.randn(1, LONG_TRAIN_T, DM, generator=g, device="cuda").to(torch.bfloat16)
    wt = bm.bc_slice_width(1, LONG_TRAIN_T, DI, DS, 2)

    def train_step():
        blk.zero_grad(set_to_none=True)
        blk(xt.clone().requires_grad_()).float().pow(2).mean().backward()

    train_step()
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    base_mem = torch.cuda.memory_allocated()
    t0 = time.perf_counter()
    for _ in range(2):
        train_step()
    torch.cuda.synchronize()
    tms = (time.perf_counter() - t0) * 1e3 / 2
    tpeak = torch.cuda.max_memory_allocated() - base_mem
    blk.zero_grad(set_to_none=True)
    log(f"long context training: B1 T{LONG_TRAIN_T} forward+backward {tms:.1f} ms "
        f"({LONG_TRAIN_T / tms * 1e3:.0f} tokens/s), {wt} d's per slice, peak {tpeak / 2**30:.1f} GiB")
    del xt
    torch.cuda.empty_cache()
    return {"workload": f"QuaternionMamba2Block forward (config-3 width, bf16), batch 1, "
                        f"seq_len {LONG_T}, B/C projections fused into the SSM kernel "
                        f"(split halves)",
            "ms_per_step": round(ms, 2), "tokens_per_s": round(LONG_T / ms * 1e3, 1),
            "whole_bc_bytes": 2 * LONG_T * DI * DS * 4 * 2,
            "peak_alloc_GiB": round(peak, 2),
            "sliced": {"workload": "fuse_bc off: B/C projections in d-slices, chunked walks",
                       "ms_per_step": round(sliced_ms, 2),
                       "tokens_per_s": round(LONG_T / sliced_ms * 1e3, 1),
                       "bc_slice_d": width, "peak_alloc_GiB": round(sliced_peak, 2)},
            "train": {"workload": f"forward + backward, bf16, batch 1, seq_len {LONG_TRAIN_T}, "
                                  f"B/C in d-slices recomputed in the backward, chunked SSM "
                                  f"training walk and backward",
                      "ms_per_step": round(tms, 2),
                      "tokens_per_s": round(LONG_TRAIN_T / tms * 1e3, 1),
                      "bc_slice_d": wt, "peak_alloc_GiB": round(tpeak / 2**30, 2)}}


def train_timings(args):
    """Config 4: block forward + backward under fp16 autocast (loss scaled as
    GradScaler does), and the SSM's training forward and backward kernels alone
    at the same shape (bf16 storage)."""
    import torch
    from mambaqc_amd.kernels.ssm_fused import ssm_fused_dl_backward, ssm_fused_dl_train_forward

    torch.manual_seed(0)
    blk = make_block(torch.float32)
    g = torch.Generator(device="cuda").manual_seed(1)
    x = torch.randn(B, T, DM, generator=g, device="cuda")

    def step():
        # As the reference's training step (train.py:206): gradients set to None,
        # so each backward writes them fresh instead of accumulating.
        blk.zero_grad(set_to_none=True)
        with torch.autocast("cuda", dtype=torch.float16):
            loss = blk(x).float().pow(2).mean()
        (loss * 2.0 ** 16).backward()

    for _ in range(2):
        step()
    torch.cuda.synchronize()
    reps = max(3, min(args.steps, 10))
    t0 = time.perf_counter()
    for _ in range(reps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / reps
    log(f"config 4 block fwd+bwd (fp16 autocast): {ms:.2f} ms/step, {B * T / ms * 1e3:.0f} tokens/s")
    del blk
    torch.cuda.empty_cache()

    bf = torch.bfloat16
    delta = torch.nn.functional.softplus(torch.randn(B, T, DI, generator=g, device="cuda") - 2).to(bf)
    s = torch.randn(B, T, DI, generator=g, device="cuda").to(bf)
    Bq = torch.randn(B, T, DI, DS, 4, generator=g, device="cuda", dtype=bf) * 0.02
    Cq = torch.randn(B, T, DI, DS, 4, generator=g, device="cuda", dtype=bf) * 0.02
    la = torch.randn(DI, DS, generator=g, device="cuda") * 0.5 + 1
    li = torch.randn(DI, DS, 3, generator=g, device="cuda") * 0.1
    Dv = torch.ones(DI, device="cuda")
    gy = torch.randn(B, T, DI, 4, generator=g, device="cuda").to(bf)
    with torch.no_grad():
        _, _, saved = ssm_fused_dl_train_forward(delta, s, Bq, Cq, la, li, Dv)
        fwd_ms = event_time_ms(lambda: ssm_fused_dl_train_forward(delta, s, Bq, Cq, la, li, Dv), 5)
        ssm_fused_dl_backward(saved, gy)
        bwd_ms = event_time_ms(lambda: ssm_fused_dl_backward(saved, gy), 5)
    n_ckpt = -(-T // 8)
    fwd_bytes = ssm_bytes(B, T, DI, DS) + B * n_ckpt * DI * DS * 16
    bwd_bytes = ssm_bwd_bytes(B, T, DI, DS)
    log(f"ssm train fwd {fwd_ms:.3f} ms ({fwd_bytes / fwd_ms / 1e6:.0f} GB/s), "
        f"bwd {bwd_ms:.3f} ms ({bwd_bytes / bwd_ms / 1e6:.0f} GB/s)")
    return {
        "workload": "QuaternionMamba2Block forward+backward, fp16 autocast, B4 T2048 d768 s64",
        "ms_per_step": round(ms, 3),
        "tokens_per_s": round(B * T / ms * 1e3, 1),
        "ssm_train_fwd_ms": round(fwd_ms, 4),
        "ssm_train_fwd_GBs": round(fwd_bytes / fwd_ms / 1e6, 1),
        "ssm_bwd_ms": round(bwd_ms, 4),
        "ssm_bwd_GBs": round(bwd_bytes / bwd_ms / 1e6, 1),
        "ssm_bwd_algorithmic_bytes": bwd_bytes,
    }


def lm_timing(args):
    """Config 5: the 12-layer base preset (14.66 B parameters) forward in bf16 at
    B4 T2048, vocab 10000, input ids uniform in [0, 10000), random-init weights."""
    import torch
    import mambaqc_amd

    torch.manual_seed(0)
    with torch.device("cuda"):
        lm = mambaqc_amd.quaternion_mamba2_base(10000)
    lm = lm.to(torch.bfloat16).eval()
    g = torch.Generator(device="cuda").manual_seed(0)
    ids = torch.randint(0, 10000, (B, T), generator=g, device="cuda")
    reps = max(2, min(args.steps, 5))
    with torch.inference_mode():
        lm(ids)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            lm(ids)
        torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / reps
    n_params = sum(p.numel() for p in lm.parameters())
    log(f"config 5 LM forward ({n_params / 1e9:.2f} B params, bf16): {ms:.1f} ms, "
        f"{B * T / ms * 1e3:.0f} tokens/s")
    # Recurrent decoding after the 2048-token prompt: one step per new token
    # (the reference re-runs the whole sequence instead).
    # The decode step as generate() runs it: fed back tokens are sampled in
    # range, so the step skips the id check (a host round trip per step), and it
    # updates generate()'s own copies of the states in place.
    with torch.inference_mode():
        _, states = lm.forward_with_state(ids)
        tok = ids[:, -1:]
        st = [(tail.contiguous(), h.clone()) for tail, h in states]
        lm._step_state_(tok, st)
        dec_ms = event_time_ms(lambda: lm._step_state_(tok, st), 20)
    log(f"config 5 recurrent decode: {dec_ms:.2f} ms per step of {B} tokens")
    from mambaqc_amd.lm import DecodeGraph
    with torch.no_grad():
        graph = DecodeGraph(lm, states)
        graph.step(tok)
        dec_graph_ms = event_time_ms(lambda: graph.step(tok), 20)
    log(f"config 5 recurrent decode as a HIP graph: {dec_graph_ms:.2f} ms per step")
    del lm, states, graph
    torch.cuda.empty_cache()
    return {"workload": "QuaternionMamba2 base (12 layers) forward, bf16, B4 T2048, vocab 10000",
            "params": n_params, "ms_per_step": round(ms, 2),
            "tokens_per_s": round(B * T / ms * 1e3, 1),
            "decode_ms_per_token_step": round(dec_ms, 3),
            "decode_tokens_per_s": round(B / dec_ms * 1e3, 1),
            "decode_graph_ms_per_token_step": round(dec_graph_ms, 3)}


def run_kernel_loop(args):
    """One kernel in a loop (for rocprofv3 kernel traces and PMC passes)."""
    import torch
    from mambaqc_amd import kernels as K

    g = torch.Generator(device="cuda").manual_seed(0)
    reps = args.steps
    with torch.inference_mode():
        if args.mode in ("ssm", "ssm_b1", "ssm_b1_whole"):
            # ssm: config 3 (B4). ssm_b1: batch 1 with the library's choice of
            # time chunks; ssm_b1_whole: batch 1 as one whole walk.
            bb = B if args.mode == "ssm" else 1
            bf = torch.bfloat16
            delta = torch.nn.functional.softplus(torch.randn(bb, T, DI, generator=g, device="cuda") - 2).to(bf)
            s = torch.randn(bb, T, DI, generator=g, device="cuda").to(bf)
            Bq = torch.randn(bb, T, DI, DS, 4, generator=g, device="cuda", dtype=bf) * 0.02
            Cq = torch.randn(bb, T, DI, DS, 4, generator=g, device="cuda", dtype=bf) * 0.02
            la = torch.randn(DI, DS, generator=g, device="cuda") * 0.5 + 1
            li = torch.randn(DI, DS, 3, generator=g, device="cuda") * 0.1
            Dv = torch.ones(DI, device="cuda")
            L = T if args.mode == "ssm_b1_whole" else None
            fn = lambda: K.ssm_forward_fused_dl(delta, s, Bq, Cq, la, li, Dv, chunk_len=L)
            nbytes = ssm_bytes(bb, T, DI, DS)
        elif args.mode == "ssm_train":
            # The SSM's training forward (walk + fp32 state checkpoints) at config 3.
            from mambaqc_amd.kernels.ssm_fused import ssm_fused_dl_train_forward
            bf = torch.bfloat16
            delta = torch.nn.functional.softplus(torch.randn(B, T, DI, generator=g, device="cuda") - 2).to(bf)
            s = torch.randn(B, T, DI, generator=g, device="cuda").to(bf)
            Bq = torch.randn(B, T, DI, DS, 4, generator=g, device="cuda", dtype=bf) * 0.02
            Cq = torch.randn(B, T, DI, DS, 4, generator=g, device="cuda", dtype=bf) * 0.02
            la = torch.randn(DI, DS, generator=g, device="cuda") * 0.5 + 1
            li = torch.randn(DI, DS, 3, generator=g, device="cuda") * 0.1
            Dv = torch.ones(DI, device="cuda")
            fn = lambda: ssm_fused_dl_train_forward(delta, s, Bq, Cq, la, li, Dv)
            nbytes = ssm_bytes(B, T, DI, DS) + B * ((T + 7) // 8) * DI * DS * 16
        elif args.mode == "ssm_bwd":
            from mambaqc_amd.kernels.ssm_fused import (ssm_fused_dl_backward,
                                                       ssm_fused_dl_train_forward)
            bf = torch.bfloat16
            delta = torch.nn.functional.softplus(torch.randn(B, T, DI, generator=g, device="cuda") - 2).to(bf)
            s = torch.randn(B, T, DI, generator=g, device="cuda").to(bf)
            Bq = torch.randn(B, T, DI, DS, 4, generator=g, device="cuda", dtype=bf) * 0.02
            Cq = torch.randn(B, T, DI, DS, 4, generator=g, device="cuda", dtype=bf) * 0.02
            la = torch.randn(DI, DS, generator=g, device="cuda") * 0.5 + 1
            li = torch.randn(DI, DS, 3, generator=g, device="cuda") * 0.1
            Dv = torch.ones(DI, device="cuda")
            gy = torch.randn(B, T, DI, 4, generator=g, device="cuda").to(bf)
            _, _, saved = ssm_fused_dl_train_forward(delta, s, Bq, Cq, la, li, Dv)
            fn = lambda: ssm_fused_dl_backward(saved, gy)
            nbytes = ssm_bwd_bytes(B, T, DI, DS)
        elif args.mode in ("cumprod", "cayley"):
            q = torch.randn(2, 256, 768, 64, 4, generator=g, device="cuda")
            q = q / q.norm(dim=-1, keepdim=True)
            fn = ((lambda: K.parallel_scan_quaternion(q)) if args.mode == "cumprod"
                  else (lambda: K.cayley_discretization_fused(q)))
            nbytes = 2 * q.numel() * 4
        elif args.mode == "qln":
            y = torch.randn(B, T, DI, 4, generator=g, device="cuda").to(torch.bfloat16)
            gm = torch.ones(DI, device="cuda")
            bt = torch.zeros(DI, 4, device="cuda")
            fn = lambda: K.quaternion_layer_norm_fused(y, gm, bt)
            nbytes = qln_bytes(B * T, DI)
        elif args.mode in ("decode", "decode_graph"):
            # Recurrent decoding with a preset (--preset, base by default):
            # prompt of 64 tokens, then one step per token through every block
            # (bf16, batch 4); decode_graph replays the step as a HIP graph.
            import mambaqc_amd
            from mambaqc_amd.lm import DecodeGraph
            torch.manual_seed(0)
            build = getattr(mambaqc_amd, f"quaternion_mamba2_{args.preset}")
            # Parameters built outside inference mode, as in lm_timing.
            with torch.inference_mode(False), torch.device("cuda"):
                lm = build(10000).to(torch.bfloat16).eval()
            ids = torch.randint(0, 10000, (B, 64), generator=g, device="cuda")
            _, states = lm.forward_with_state(ids)
            tok = ids[:, -1:]
            if args.mode == "decode":
                st = [(tail.contiguous(), h.clone()) for tail, h in states]
                fn = lambda: lm._step_state_(tok, st)
            else:
                with torch.inference_mode(False), torch.no_grad():
                    graph = DecodeGraph(lm, states)
                fn = lambda: graph.step(tok)
            nbytes = sum(p.numel() * p.element_size() for p in lm.parameters())
        elif args.mode in ("block_long", "block_long_sliced"):
            # The long-context line: the benchmark's block on one sequence of
            # LONG_T tokens, on its default path (the split fused B/C kernel) or,
            # block_long_sliced, with fuse_bc off (B/C projections in d-slices).
            torch.manual_seed(0)
            with torch.inference_mode(False):
                blk = make_block(torch.bfloat16)
            if args.mode == "block_long_sliced":
                blk.fuse_bc = False
            x = torch.randn(1, LONG_T, DM, generator=g, device="cuda").to(torch.bfloat16)
            fn = lambda: blk(x)
            nbytes = 0
        elif args.mode == "train":
            # Config 4: block forward + backward under fp16 autocast, loss
            # scaled as in train_timings (kernel traces of the training step).
            torch.manual_seed(0)
            with torch.inference_mode(False):
                blk = make_block(torch.float32)
                x = torch.randn(B, T, DM, generator=g, device="cuda")

            def fn():
                with torch.inference_mode(False):
                    blk.zero_grad(set_to_none=True)
                    with torch.autocast("cuda", dtype=torch.float16):
                        loss = blk(x).float().pow(2).mean()
                    (loss * 2.0 ** 16).backward()
            nbytes = 0
        elif args.mode == "gemm":
            # The config-3 B projection through the library's MFMA GEMM.
            bf = torch.bfloat16
            x = torch.randn(B * T, DI, generator=g, device="cuda").to(bf)
            w = (torch.randn(DI * DS * 4, DI, generator=g, device="cuda") * 0.02).to(bf)
            out = torch.empty(B * T, DI * DS * 4, device="cuda", dtype=bf)
            fn = lambda: mqc_gemm(x, w, out)
            nbytes = 0
        elif args.mode == "gemm_hipblaslt":
            from mambaqc_amd.layers.quaternion_linear import wide_linear
            bf = torch.bfloat16
            x = torch.randn(B * T, DI, generator=g, device="cuda").to(bf)
            w = (torch.randn(DI * DS * 4, DI, generator=g, device="cuda") * 0.02).to(bf)
            fn = lambda: wide_linear(x, w)
            nbytes = 0
        elif args.mode in ("fused_bc", "bc_unfused"):
            # Config 3's B/C projections and SSM: fused in one launch
            # (mqc_ssm_fused_bc_fwd), or the block's unfused path (hipBLASLt GEMMs
            # in column blocks, then mqc_ssm_fused_fwd), on the same operands.
            from mambaqc_amd.layers.quaternion_linear import wide_linear
            bf = torch.bfloat16
            x = torch.randn(B, T, DI, generator=g, device="cuda").to(bf)
            wb = (torch.randn(DI * DS * 4, DI, generator=g, device="cuda") * 0.02).to(bf)
            wc = (torch.randn(DI * DS * 4, DI, generator=g, device="cuda") * 0.02).to(bf)
            delta = torch.nn.functional.softplus(torch.randn(B, T, DI, generator=g, device="cuda") - 2).to(bf)
            s = torch.randn(B, T, DI, generator=g, device="cuda").to(bf)
            la = torch.randn(DI, DS, generator=g, device="cuda") * 0.5 + 1
            li = torch.randn(DI, DS, 3, generator=g, device="cuda") * 0.1
            Dv = torch.ones(DI, device="cuda")
            if args.mode == "fused_bc":
                fn = lambda: K.ssm_forward_fused_bc(x, wb, wc, delta, s, la, li, Dv)
            else:
                def fn():
                    Bq = wide_linear(x, wb).view(B, T, DI, DS, 4)
                    Cq = wide_linear(x, wc).view(B, T, DI, DS, 4)
                    return K.ssm_forward_fused_dl(delta, s, Bq, Cq, la, li, Dv)
            nbytes = 0
        elif args.mode in ("out_step", "out_step_unfused"):
            # Config 3's output step: out_proj ([8192, 6144] x [6144, 768]) with the gate
            # and residual, as one kernel (mqc_out_proj_gate_fwd) or unfused (F.linear,
            # then mqc_out_gate_fwd), on the same operands.
            from mambaqc_amd.block import out_gate, out_proj_gate
            bf = torch.bfloat16
            xo = torch.randn(B * T, DM, generator=g, device="cuda").to(bf)
            xz = torch.randn(B * T, 2 * DI, generator=g, device="cuda").to(bf)
            zo = xz[:, DI:]
            yo = torch.randn(B * T, DI, 4, generator=g, device="cuda").to(bf)
            wo = (torch.randn(DM, 4 * DI, generator=g, device="cuda") * 0.02).to(bf)
            if args.mode == "out_step":
                fn = lambda: out_proj_gate(xo, zo, yo, wo)
            else:
                fn = lambda: out_gate(xo, zo, torch.nn.functional.linear(yo.view(B * T, -1), wo))
            nbytes = 0
        elif args.mode == "out_step_block":
            # The output step inside the block, for a kernel trace: per step, four
            # config-3 block forwards with the fused output step, then four unfused.
            torch.manual_seed(0)
            with torch.inference_mode(False):
                blk = make_block(torch.bfloat16)
            x = torch.randn(B, T, DM, generator=g, device="cuda").to(torch.bfloat16)

            def fn():
                for fo in (True, False):
                    blk.fuse_out = fo
                    for _ in range(4):
                        blk(x)
                blk.fuse_out = None
            nbytes = 0
        elif args.mode == "copy":
            src = torch.empty(1 << 28, device="cuda")  # 1 GiB
            dst = torch.empty_like(src)
            fn = lambda: dst.copy_(src)
            nbytes = 2 * src.numel() * 4
        else:
            raise SystemExit(f"unknown mode {args.mode}")
        for _ in range(args.warmup):
            fn()
        ms = event_time_ms(fn, reps)
    print(json.dumps({"mode": args.mode, "mean_ms": round(ms, 4), "bytes": nbytes,
                      "GBs": round(nbytes / (ms * 1e-3) / 1e9, 1)}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--mode", default="full")
    ap.add_argument("--preset", default="base", choices=["small", "base", "large"],
                    help="LM preset of the decode modes")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--block-only", action="store_true",
                    help="skip the config-4 and config-5 legs (for a kernel trace of the block)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build's hot path runs on a single MI355X "
              "(multi-GPU sharding is a design note, not implemented); use --gpus 1",
              file=sys.stderr)
        raise SystemExit(2)
    import torch

    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs a ROCm GPU")
    if args.mode == "full":
        run_full(args)
    else:
        run_kernel_loop(args)


if __name__ == "__main__":
    main()
