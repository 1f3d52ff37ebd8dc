"""Benchmark of the KTIR gfx950 backend on BASELINE.json's configurations.

`python bench.py [--config NAME] [--steps K] [--warmup W]` prints ONE JSON
line.  A step is one replay of the recorded launch plan of the config's KTIR
kernel over inputs already resident in HBM (the host IR walk and the
host<->device copies are outside the timed region).  Timing uses HIP events
on the library's stream.  The CPU baseline times the NumPy oracle (a
restatement of the reference interpreter) on the host on a bounded sample of
the same workload and extrapolates by core count.
"""

import argparse
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MFMA_F16_TFLOPS = 2500.0


def _vector_add():
    from ktir_cpu_amd import configs
    n, block, cores = 64 * 1024 * 1024, 32768, 2048
    rng = np.random.default_rng(42)
    x = rng.standard_normal(n, dtype=np.float32).astype(np.float16)
    y = rng.standard_normal(n, dtype=np.float32).astype(np.float16)
    kw = dict(x_ptr=x, y_ptr=y, output_ptr=np.zeros(n, np.float16), BLOCK_SIZE=block)
    return dict(src=configs.vector_add(n, block, cores), fn="add_kernel", kw=kw, cores=cores,
                bytes=6 * n, flops=n, bound="hbm", dtype="f16",
                workload=f"vector_add n={n} f16 grid={cores} BLOCK={block}")


def _copy():
    from ktir_cpu_amd import configs
    n, block, cores = 64 * 1024 * 1024, 32768, 2048
    x = np.random.default_rng(42).standard_normal(n, dtype=np.float32)
    kw = dict(x_ptr=x, output_ptr=np.zeros(n, np.float32))
    return dict(src=configs.vector_copy(n, block, cores, "f32"), fn="copy_kernel", kw=kw, cores=cores,
                bytes=8 * n, flops=0, bound="hbm", dtype="f32",
                workload=f"copy n={n} f32 grid={cores} BLOCK={block} (HBM traffic calibration)")


def _gather():
    from ktir_cpu_amd import configs
    rows, dim, n_idx, cores, chunk = 1 << 20, 128, 262144, 64, 128
    rng = np.random.default_rng(42)
    table = rng.standard_normal((rows, dim), dtype=np.float32).astype(np.float16)
    uniq = rng.choice(rows, 235930, replace=False)
    dup = rng.choice(uniq, n_idx - 235930)
    idx = rng.permutation(np.concatenate([uniq, dup])).astype(np.int32)
    n_uniq = len(np.unique(idx))
    kw = dict(table_ptr=table, idx_ptr=idx, out_ptr=np.zeros((rows, dim), np.float32))
    alg = 4 * n_idx + n_idx * dim * 2 + 2 * dim * 4 * n_uniq
    return dict(src=configs.gather_scatter_add(rows, dim, n_idx, cores, chunk), fn="gather_scatter_add", kw=kw,
                cores=cores, bytes=alg, flops=n_idx * dim, bound="hbm", dtype="f16->f32",
                workload=f"gather_scatter_add table={rows}x{dim} f16 idx={n_idx} i32 (10% dup) out f32 "
                         f"grid={cores} chunk={chunk}")


def _softmax():
    from ktir_cpu_amd import configs
    rows, cols, cores, rblk = 32768, 4096, 512, 8
    rng = np.random.default_rng(42)
    x = (rng.standard_normal((rows, cols), dtype=np.float32) * 2).astype(np.float16)
    kw = dict(x_ptr=x, y_ptr=np.zeros_like(x))
    return dict(src=configs.softmax(rows, cols, cores, rblk), fn="softmax_kernel", kw=kw, cores=cores,
                bytes=4 * rows * cols, flops=5 * rows * cols, bound="hbm", dtype="f16/f32",
                workload=f"softmax {rows}x{cols} f16 grid={cores} rows/step={rblk}")


def _rmsnorm():
    from ktir_cpu_amd import configs
    rows, cols, cores, rblk = 32768, 4096, 512, 8
    rng = np.random.default_rng(42)
    x = (rng.standard_normal((rows, cols), dtype=np.float32) * 2).astype(np.float16)
    w = rng.uniform(0.5, 1.5, cols).astype(np.float16)
    kw = dict(x_ptr=x, w_ptr=w, y_ptr=np.zeros_like(x), eps=1e-6)
    return dict(src=configs.rmsnorm(rows, cols, cores, rblk), fn="rmsnorm_kernel", kw=kw, cores=cores,
                bytes=4 * rows * cols + 2 * cols, flops=4 * rows * cols, bound="hbm", dtype="f16/f32",
                workload=f"rmsnorm {rows}x{cols} f16 grid={cores} rows/step={rblk}")


def _gemm():
    from ktir_cpu_amd import configs
    M = N = K = 8192
    rng = np.random.default_rng(42)
    a = (rng.standard_normal((M, K), dtype=np.float32) * K ** -0.5).astype(np.float16)
    b = (rng.standard_normal((K, N), dtype=np.float32) * K ** -0.5).astype(np.float16)
    kw = dict(a_ptr=a, b_ptr=b, c_ptr=np.zeros((M, N), np.float16))
    return dict(src=configs.gemm(M, N, K, 128, 128, 64, 8, 8), fn="gemm_kernel", kw=kw, cores=64,
                bytes=3 * M * N * 2, flops=2 * M * N * K, bound="mfma", dtype="f16 (f32 acc)",
                workload=f"gemm {M}x{N}x{K} f16 tiles 128x128x64 grid=8x8")


def _attention():
    from ktir_cpu_amd import configs
    from oracle.interp import bf16_bits
    B, H, S, D = 4, 32, 8192, 128
    rng = np.random.default_rng(42)
    q, k, v = (bf16_bits(rng.standard_normal((B, H, S, D), dtype=np.float32)) for _ in range(3))
    kw = dict(q_ptr=q, k_ptr=k, v_ptr=v, o_ptr=np.zeros_like(q), scale=1.0 / math.sqrt(D))
    return dict(src=configs.flash_attention(B, H, S, D, 128), fn="flash_attention", kw=kw, cores=B * H * S // 128,
                bytes=4 * B * H * S * D * 2, flops=4 * B * H * S * S * D // 2, bound="mfma", dtype="bf16 (f32 acc)",
                workload=f"flash_attention causal B={B} H={H} S={S} D={D} kv_tile=128")


CONFIGS = {"vector_add": _vector_add, "copy": _copy, "gather": _gather, "softmax": _softmax, "rmsnorm": _rmsnorm,
           "gemm": _gemm, "attention": _attention}


# kernels that make up each kind of launch (the HIP kernel names)
_LAUNCH_KERNELS = {"mm": ("mm_mfma", "mm_generic"), "attn": ("attn_kernel", "attn_pp", "attn_v16"), "rmw": ("rmw_",),
                   "prog": ("prog_",)}


def _traffic(config, kind):
    """HBM bytes per launch of the config's dominant launch (of kind `kind`):
    the summed rocprofv3 FETCH_SIZE / WRITE_SIZE bytes of that launch's
    kernels, committed in profiles/traffic.json (scaled by a copy kernel of
    known size), or None when not measured."""
    try:
        with open(os.path.join(ROOT, "profiles", "traffic.json")) as f:
            t = json.load(f)["configs"].get(config)
    except (OSError, ValueError, KeyError):
        return None
    if not t:
        return None
    pats = _LAUNCH_KERNELS.get(kind, ())
    b = [v["bytes"] for k, v in t.get("kernels", {}).items() if any(p in k for p in pats)]
    return round(sum(b)) if b else None


def cpu_baseline(cfg, budget_s=15.0):
    """Time the oracle on k evenly spaced cores for growing k (1, 2, 4, ...)
    until about `budget_s` of CPU work, then extrapolate the per-core slope
    to all cores.  Even spacing keeps the sample representative where the
    work per core differs (causal attention: core qb visits qb + 1 KV tiles)."""
    from oracle.interp import OracleInterpreter
    o = OracleInterpreter(lx_size_mb=64)
    o.load(cfg["src"])
    cores = cfg["cores"]
    kw = cfg["kw"]
    samples = []
    k = 1
    t_all = time.perf_counter()
    while True:
        kk = min(k, cores)
        o.cores_to_run = sorted(set(int(c) for c in np.linspace(0, cores - 1, kk + 2)[1:-1].round()))
        kk = len(o.cores_to_run)
        t0 = time.perf_counter()
        o.execute_function(cfg["fn"], **kw)
        samples.append((kk, time.perf_counter() - t0))
        if k >= cores or time.perf_counter() - t_all > budget_s:
            break
        k *= 2
    if len(samples) >= 2:
        (k1, t1), (k2, t2) = samples[-2], samples[-1]
        per_core = max((t2 - t1) / max(k2 - k1, 1), 1e-9)
        setup = max(t1 - per_core * k1, 0.0)
    else:
        k2, t2 = samples[-1]
        per_core, setup = t2 / k2, 0.0
    t_full = setup + per_core * cores
    return t_full, samples


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="gather", choices=sorted(CONFIGS))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this backend runs on one GPU; multi-GPU runs are not part of this build",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    from ktir_cpu_amd import runtime as rt
    from ktir_cpu_amd.interpreter import KTIRInterpreter
    cfg = CONFIGS[args.config]()
    interp = KTIRInterpreter()
    interp.load(cfg["src"])
    t0 = time.perf_counter()
    prep = interp.prepare(cfg["fn"], **cfg["kw"])          # host walk + first launch
    walk_s = time.perf_counter() - t0
    plan = prep.plan
    for _ in range(args.warmup):
        prep.run()
    rt.sync()
    # Timed region: K replays of the plan on the library's stream, with a HIP
    # event after every launch so each launch's duration comes from the same
    # run that gives ms_per_step.
    from ktir_cpu_amd.executor import _launch
    L = rt.lib()
    n = len(plan.launches)
    instrument = 0 < n <= 64
    evs = [[rt.Event() for _ in range(n)] for _ in range(args.steps)] if instrument else None
    e0, e1 = rt.Event(), rt.Event()
    e0.record()
    for s_ in range(args.steps):
        if instrument:
            for i, (kind, desc, _) in enumerate(plan.launches):
                _launch(L, kind, desc)
                evs[s_][i].record()
        else:
            prep.run()
    e1.record()
    rt.sync()
    ms = e0.elapsed_ms(e1) / args.steps
    durs = np.zeros(n)
    if instrument:
        for s_ in range(args.steps):
            prev = e0 if s_ == 0 else evs[s_ - 1][-1]
            for i in range(n):
                durs[i] += prev.elapsed_ms(evs[s_][i])
                prev = evs[s_][i]
        durs /= args.steps
    dom = int(np.argmax(durs)) if n else 0
    dom_ms = float(durs[dom]) if instrument else ms
    # every bench workload's dominant launch processes all of the workload's
    # algorithmic units (all bytes moved / all flops), so per-launch units are
    # the workload's
    if cfg["bound"] == "hbm":
        value = cfg["bytes"] / (ms * 1e-3) / 1e9
        unit, peak = "GB/s", HBM_PEAK_GBS
        achieved = cfg["bytes"] / (dom_ms * 1e-3) / 1e9
    else:
        value = cfg["flops"] / (ms * 1e-3) / 1e12
        unit, peak = "TFLOP/s", MFMA_F16_TFLOPS
        achieved = cfg["flops"] / (dom_ms * 1e-3) / 1e12
    out = {
        "metric": "achieved HBM GB/s & MFMA TFLOP/s per KTIR kernel (% of roofline) vs NumPy",
        "value": round(value, 3), "unit": unit, "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 6), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": cfg["dtype"], "data": "synthetic (seed 42)",
        "config": {"workload": cfg["workload"], "launches_per_step": len(plan.launches),
                   "plan_mode": plan.mode, "host_walk_s": round(walk_s, 3)},
        "roofline": {"bound": cfg["bound"], "achieved": round(achieved, 3), "peak": peak, "unit": unit,
                     "frac": round(achieved / peak, 4), "traffic": _traffic(args.config, plan.launches[dom][0] if plan.launches else None),
                     "dominant_launch": plan.launches[dom][0] if plan.launches else None,
                     "dominant_ms": round(dom_ms, 6)},
    }
    if not args.no_cpu:
        t_full, samples = cpu_baseline(cfg)
        cpu_val = (cfg["bytes"] / t_full / 1e9) if cfg["bound"] == "hbm" else (cfg["flops"] / t_full / 1e12)
        out["cpu_baseline"] = {"value": cpu_val, "unit": unit, "cores": 1, "kind": "port",
                               "sample": f"oracle on {samples[-1][0]} evenly spaced of {cfg['cores']} simulated cores "
                                         f"({samples[-1][1]:.1f} s), extrapolated linearly by core count to "
                                         f"{t_full:.1f} s for the full run"}
    print(json.dumps(out))


if __name__ == "__main__":
    main()
