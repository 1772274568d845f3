#!/usr/bin/env python3
"""Headline benchmark: Sdpa forward + SdpaGrad backward on one MI355X.

Workload (the config the metric is quoted on):
fp16, batch = B*H = 128, S_q = S_kv = 4096, D_qk = D_v = 128, causal,
dropout 0.1 (seed 7, offset 0), scale 1/sqrt(128), q/k/v/dO ~ N(0,1)
(synthetic, seeded).  A "step" is one forward (1 kernel) plus one backward
over that batch, inputs resident in HBM.  The backward takes its dS path
(fp16 with a feature size over 64, given the workspace of
sdpa_hip_bwd_workspace_bytes_ds): the row kernel (stats2, delta), the dK/dV
kernel that also stores dS, and dQ as one product with the stored dS;
--bwd-path recompute times the path that forms dS in both kernels (dQ
kernel, then dK/dV kernel) instead.

FLOPs follow the FlashAttention convention (causal x1/2, dropout RNG not
counted):  fwd = 2*B*S_q*S_kv*(D_qk+D_v)/2,  bwd = 2*B*S_q*S_kv*(3*D_qk+2*D_v)/2.
`value` is (fwd + bwd FLOPs) / (median step time over the timed steps), the
median of >= 20 runs that BASELINE.md asks for; `ms_per_step` is the mean
(the whole timed region / steps).  fwd_ms / bwd_ms are per-kernel medians;
the roofline uses the dominant kernel's mean launch duration.

Prints ONE JSON line (rank 0).  --gpus N > 1 exits: this build runs on one GPU.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import platform
import re
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "fwd/bwd attention TFLOP/s + % fp16 MFMA peak, B·H=128 S=4096 D=128 causal"
PEAK_F16_TFLOPS = 2500.0  # MI355X dense fp16 MFMA, published
PEAK_F32_TFLOPS = 157.3   # MI355X fp32 MFMA, published

CONFIGS = {
    # name: (dtype, B, S_q, S_kv, D_qk, D_v, causal, dropout, seed, offset)
    "c4": ("f16", 128, 4096, 4096, 128, 128, True, 0.1, 7, 0),
    "c3": ("f16", 256, 2048, 2048, 64, 64, True, 0.0, 0, 0),
    "c5": ("f32", 64, 512, 16384, 128, 64, False, 0.0, 0, 0),
}


def flops(cfg):
    _, B, S_q, S_kv, D_qk, D_v, causal, *_ = cfg
    f = 0.5 if causal else 1.0
    fwd = 2.0 * B * S_q * S_kv * (D_qk + D_v) * f
    bwd_dkdv = 2.0 * B * S_q * S_kv * (2 * D_qk + 2 * D_v) * f  # S, dP, dV, dK
    bwd_dq = 2.0 * B * S_q * S_kv * D_qk * f                    # dQ (S, dP recomputed: not counted)
    return fwd, bwd_dq, bwd_dkdv


def read_traffic(kernel: str, workload: str):
    """HBM bytes per launch for `kernel` from the committed PMC summary, or None."""
    path = os.path.join(ROOT, "profiles", f"hbm_traffic_{workload}.md")
    if not os.path.exists(path):
        return None
    pat = re.compile(r"^\|\s*" + re.escape(kernel) + r"\s*\|.*\|\s*([0-9.eE+]+)\s*\|\s*$")
    for line in open(path):
        m = pat.match(line.strip())
        if m:
            return float(m.group(1))
    return None


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_baseline(cfg, rows: int, threads: int):
    """The CPU oracle (restatement of sdpa/sdpa_cpu.cc, fp16 instantiation with
    Eigen::half semantics, -O2 as reference build.sh:46) on a bounded sample of
    the same workload: `threads` batches of the real shape, one per thread as
    the reference's parallelFor over B, each computing the last `rows` query
    rows (the causal rows that see the most keys, i.e. a representative-or-
    heavier slice).  Returns TFLOP/s under the same FLOP convention."""
    import numpy as np
    from oracle import oracle as O  # checker/baseline only, never the product path

    dt, B, S_q, S_kv, D_qk, D_v, causal, p, seed, off = cfg
    nb = threads
    rng = np.random.default_rng(12345)
    npdt = np.float16 if dt == "f16" else np.float32
    q = rng.standard_normal((nb, S_q, D_qk), dtype=np.float32).astype(npdt)
    k = rng.standard_normal((nb, S_kv, D_qk), dtype=np.float32).astype(npdt)
    v = rng.standard_normal((nb, S_kv, D_v), dtype=np.float32).astype(npdt)
    d_o = rng.standard_normal((nb, S_q, D_v), dtype=np.float32).astype(npdt)
    r0, r1 = S_q - rows, S_q
    kw = dict(scale=1.0 / math.sqrt(D_qk), dropout=p, causal_mask=causal, seed=seed, offset=off,
              nthreads=threads, rows=(r0, r1), gpu_gates=False)
    t0 = time.perf_counter()
    o, s = O.sdpa_fwd(q, k, v, **kw)
    t1 = time.perf_counter()
    O.sdpa_bwd(q, k, v, o, s, d_o, accumulate_kv_in_t=True, **kw)
    t2 = time.perf_counter()
    keys = sum((i + 1) if causal else S_kv for i in range(r0, r1))  # visible (i, j) pairs per batch
    f_fwd = 2.0 * nb * keys * (D_qk + D_v)
    f_bwd = 2.0 * nb * keys * (3 * D_qk + 2 * D_v)
    return {
        "value": round((f_fwd + f_bwd) / (t2 - t0) / 1e12, 6),
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"{nb} batches x query rows [{r0},{r1}) of the {dt} workload shape "
                   f"(S={S_q}x{S_kv}, D={D_qk}/{D_v}, causal={causal}, p={p}); "
                   f"fwd {t1 - t0:.2f} s, bwd {t2 - t1:.2f} s wall on {threads} threads "
                   f"({cpu_model()}, nproc {os.cpu_count()})"),
        "fwd_tflops": round(f_fwd / (t1 - t0) / 1e12, 6),
        "bwd_tflops": round(f_bwd / (t2 - t1) / 1e12, 6),
    }


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="c4", choices=sorted(CONFIGS))
    ap.add_argument("--cpu-rows", type=int, default=512,
                    help="query rows per batch in the CPU baseline sample (0: skip it)")
    ap.add_argument("--cpu-threads", type=int, default=0, help="CPU baseline threads (0: auto)")
    ap.add_argument("--cold-steps", type=int, default=5,
                    help="extra steps timed with the caches flushed before every kernel (0: skip)")
    ap.add_argument("--bwd-path", default="ds", choices=["ds", "recompute"],
                    help="backward path: ds (where the shape allows) or recompute")
    ap.add_argument("--calibrate-copy-mib", type=int, default=0,
                    help="also run one plain device copy of this many MiB (PMC calibration)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one MI355X only; multi-GPU runs are not part of "
              "it (the op shards over the batch with offset += b0*S_q*S_kv)",
              file=sys.stderr)
        sys.exit(2)

    import torch
    import __graft_entry__

    pkg = __graft_entry__.package()
    L = pkg.library()
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    cfg = CONFIGS[args.config]
    dt, B, S_q, S_kv, D_qk, D_v, causal, p, seed, off = cfg
    tdt = torch.float16 if dt == "f16" else torch.float32
    dcode = pkg.DTYPE_F16 if dt == "f16" else pkg.DTYPE_F32
    scale = 1.0 / math.sqrt(D_qk)

    g = torch.Generator(device=dev)
    def randn(*shape, seed_):
        g.manual_seed(seed_)
        return torch.randn(shape, generator=g, device=dev, dtype=torch.float32).to(tdt)
    q = randn(B, S_q, D_qk, seed_=1024)
    k = randn(B, S_kv, D_qk, seed_=124)
    v = randn(B, S_kv, D_v, seed_=24)
    d_o = randn(B, S_q, D_v, seed_=4)
    o = torch.empty((B, S_q, D_v), dtype=tdt, device=dev)
    st = torch.empty((B, S_q), dtype=torch.float32, device=dev)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    rows_bytes = int(L.sdpa_hip_bwd_workspace_bytes(B, S_q))
    ds_bytes = int(L.sdpa_hip_bwd_workspace_bytes_ds(dcode, B, S_q, S_kv, D_qk, D_v, int(causal)))
    use_ds = args.bwd_path == "ds" and ds_bytes > rows_bytes
    ws_bytes = ds_bytes if use_ds else rows_bytes
    ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream(dev)
    h = stream.cuda_stream  # every launch below goes to this stream

    def check(rc):
        if rc != 0:
            raise RuntimeError(pkg.status_string(rc))

    def fwd():
        check(L.sdpa_hip_fwd(dcode, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                             st.data_ptr(), B, S_q, S_kv, D_qk, D_v, scale, p, int(causal), seed,
                             off, h))

    def bwd_dq():
        check(L.sdpa_hip_bwd_dq(dcode, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                st.data_ptr(), d_o.data_ptr(), dq.data_ptr(), ws.data_ptr(),
                                ws_bytes, B, S_q, S_kv, D_qk, D_v, scale, p, int(causal), seed,
                                off, h))

    def bwd_dkdv():
        check(L.sdpa_hip_bwd_dkdv(dcode, q.data_ptr(), k.data_ptr(), v.data_ptr(), st.data_ptr(),
                                  d_o.data_ptr(), dk.data_ptr(), dv.data_ptr(), ws.data_ptr(),
                                  ws_bytes, B, S_q, S_kv, D_qk, D_v, scale, p, int(causal), seed,
                                  off, h))

    def ds_phase(i):
        def run():
            check(L.sdpa_hip_bwd_ds_phase(i, dcode, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                          st.data_ptr(), d_o.data_ptr(), dq.data_ptr(), dk.data_ptr(),
                                          dv.data_ptr(), ws.data_ptr(), ws_bytes, B, S_q, S_kv, D_qk, D_v,
                                          scale, p, int(causal), seed, off, h))
        return run

    if use_ds:
        phases = [("sdpa_fwd", fwd), ("sdpa_bwd_rows", ds_phase(0)), ("sdpa_bwd_dkdv", ds_phase(1)),
                  ("sdpa_bwd_dq", ds_phase(2))]
    else:
        phases = [("sdpa_fwd", fwd), ("sdpa_bwd_dq", bwd_dq), ("sdpa_bwd_dkdv", bwd_dkdv)]
    for _ in range(args.warmup):
        for _, fn in phases:
            fn()
    torch.cuda.synchronize()

    K = args.steps
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(len(phases) + 1)] for _ in range(K)]
    t_begin = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    t_begin.record(stream)
    for i in range(K):
        ev[i][0].record(stream)
        for j, (_, fn) in enumerate(phases):
            fn()
            ev[i][j + 1].record(stream)
    t_end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    total_ms = t_begin.elapsed_time(t_end)
    ms_per_step = total_ms / K
    per = {name: sum(ev[i][j].elapsed_time(ev[i][j + 1]) for i in range(K)) / K
           for j, (name, _) in enumerate(phases)}
    med = {name: statistics.median(ev[i][j].elapsed_time(ev[i][j + 1]) for i in range(K))
           for j, (name, _) in enumerate(phases)}
    step_med = statistics.median(ev[i][0].elapsed_time(ev[i][len(phases)]) for i in range(K))

    # Cache-cold timing (reported beside the warm, back-to-back figures): before
    # every kernel a 512 MiB buffer is overwritten, which evicts the operands
    # from the L2s and from the 256 MB Infinity Cache; only the kernel itself
    # sits between its events.
    cold = None
    if args.cold_steps > 0:
        flush = torch.empty((512 << 20,), dtype=torch.uint8, device=dev)
        cev = [[torch.cuda.Event(enable_timing=True) for _ in range(2 * len(phases))]
               for _ in range(args.cold_steps)]
        for i in range(args.cold_steps):
            for j, (_, fn) in enumerate(phases):
                flush.fill_(i + j)
                cev[i][2 * j].record(stream)
                fn()
                cev[i][2 * j + 1].record(stream)
        torch.cuda.synchronize()
        cold = {name: round(statistics.median(cev[i][2 * j].elapsed_time(cev[i][2 * j + 1])
                                              for i in range(args.cold_steps)), 4)
                for j, (name, _) in enumerate(phases)}
        del flush

    f_fwd, f_dq, f_dkdv = flops(cfg)
    f_bwd = f_dq + f_dkdv
    fwd_ms, bwd_ms = med["sdpa_fwd"], sum(t for n_, t in med.items() if n_ != "sdpa_fwd")
    peak = PEAK_F16_TFLOPS if dt == "f16" else PEAK_F32_TFLOPS
    value = (f_fwd + f_bwd) / (step_med * 1e-3) / 1e12
    kflops = {"sdpa_fwd": f_fwd, "sdpa_bwd_dq": f_dq, "sdpa_bwd_dkdv": f_dkdv, "sdpa_bwd_rows": 0.0}
    dom = max(per, key=per.get)
    achieved = kflops[dom] / (per[dom] * 1e-3) / 1e12
    # fp16 shapes with D % 8 == 0 run the DMA-fed kernels (sdpa_f16_fwd/dq/dkdv.hip)
    sfx = "f16_dma" if (dt == "f16" and D_qk % 8 == 0 and D_v % 8 == 0) else dt
    # (dK/dV of a feature width above 64 runs the split-role variant, fp16
    # with the DMA-fed kernels and fp32 alike)
    split = max(D_qk, D_v) > 64 and (sfx == "f16_dma" or dt == "f32")
    kv_sfx = ("f16_split" if dt == "f16" else "f32_split") if split else sfx
    dq_sym = "sdpa_bwd_dq_ds_%s_kernel" % dt if use_ds else "sdpa_bwd_dq_%s_kernel" % sfx
    kernel_symbol = {"sdpa_fwd": "sdpa_fwd_%s_kernel" % sfx, "sdpa_bwd_dq": dq_sym,
                     "sdpa_bwd_dkdv": "sdpa_bwd_dkdv_%s_kernel" % kv_sfx,
                     "sdpa_bwd_rows": "sdpa_bwd_rows_%s_kernel" % dt}[dom]

    if args.calibrate_copy_mib:
        n = args.calibrate_copy_mib * (1 << 20)
        src = torch.ones((n,), dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()

    cpu = None
    if args.cpu_rows > 0:
        threads = args.cpu_threads or max(1, min(16, os.cpu_count() or 1))
        cpu = cpu_baseline(cfg, args.cpu_rows, threads)

    out = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "ms_per_step_median": round(step_med, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dt,
        "data": "synthetic (seeded N(0,1) q/k/v/dO generated on the device)",
        "config": {"workload": f"{args.config}: Sdpa fwd + SdpaGrad bwd, {dt}, B*H={B}, "
                               f"S_q={S_q}, S_kv={S_kv}, D_qk={D_qk}, D_v={D_v}, causal={causal}, "
                               f"dropout={p} (seed {seed}, offset {off})",
                   "global_batch": B, "seq_len": S_q, "parallelism": "none (1 GPU)"},
        "fwd_ms": round(fwd_ms, 4),
        "bwd_ms": round(bwd_ms, 4),
        "fwd_tflops": round(f_fwd / (fwd_ms * 1e-3) / 1e12, 3),
        "bwd_tflops": round(f_bwd / (bwd_ms * 1e-3) / 1e12, 3),
        "fwd_pct_peak": round(100.0 * f_fwd / (fwd_ms * 1e-3) / 1e12 / peak, 2),
        "bwd_pct_peak": round(100.0 * f_bwd / (bwd_ms * 1e-3) / 1e12 / peak, 2),
        "bwd_path": "ds" if use_ds else "recompute",
        "workspace_bytes": ws_bytes,
        "kernel_ms": {k_: round(v_, 4) for k_, v_ in per.items()},
        "kernel_ms_median": {k_: round(v_, 4) for k_, v_ in med.items()},
        "kernel_ms_cache_cold": cold,
        "wall_s": round(wall, 3),
        "roofline": {
            "kernel": kernel_symbol,
            "bound": "mfma",
            "achieved": round(achieved, 3),
            "peak": peak,
            "unit": "TFLOP/s",
            "frac": round(achieved / peak, 4),
            "traffic": read_traffic(kernel_symbol, args.config),
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
