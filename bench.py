"""Benchmark of the KTIR gfx950 backend on BASELINE.json's configurations.

`python bench.py [--config NAME|all] [--steps K] [--warmup W] [--no-cpu]`
prints ONE JSON line.  A step is one replay of the recorded launch plan of a
config's KTIR kernel over inputs already resident in HBM (the host IR walk
and the host<->device copies are outside the timed region).  Untimed
warm-up replays (at least W, and at least 0.5 s of them unless W is 0) come
first, so the GPU's clocks have settled when timing starts.  Timing uses HIP
events on the library's stream, with an event after every launch, so the
dominant launch's own time gives `roofline.achieved`.  Every timed
attention replay converts V to f16 again, as a call with a new V does; the
figure for replays that reuse the f16 copy of an unchanged V (the plan
tracks writes to V) is reported beside it as `v16_reuse`.  For the
memory-bound configs `cold` times replays that each follow a 1 GiB read, so
that no input is left in L2 or the Infinity Cache.  By default the line's
top-level fields are the gather + scatter-add config
and `per_config` holds the same measurement for every config; each entry also
reports the host side of a real call (copies in and out, one end-to-end
execute_function).  The CPU baseline times the NumPy oracle (a restatement of
the reference interpreter, one core) on a bounded sample of the same
workload, median of 3, and extrapolates by simulated-core count.
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


def _vector_add_4096():
    from ktir_cpu_amd import configs
    n, block, cores = 4096, 128, 32
    rng = np.random.default_rng(42)
    x = rng.standard_normal(n).astype(np.float16)
    y = rng.standard_normal(n).astype(np.float16)
    kw = dict(x_ptr=x, y_ptr=y, output_ptr=np.zeros(n, np.float16), BLOCK_SIZE=block)
    return dict(src=configs.vector_add(n, block, cores), fn="add_kernel", kw=kw, cores=cores,
                bytes=6 * n, flops=n, bound="hbm", dtype="f16",
                workload=f"vector_add n={n} f16 grid={cores} BLOCK={block} (launch-bound: reported only)")


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
                cores=cores, bytes=alg, flops=n_idx * dim, bound="hbm", dtype="f16 table, f32 out (f32 adds)",
                workload=f"gather_scatter_add table={rows}x{dim} f16 idx={n_idx} i32 (10% dup) out f32 "
                         f"grid={cores} chunk={chunk}")


def _softmax():
    from ktir_cpu_amd import configs
    rows, cols, cores, rblk = 32768, 4096, 512, 8
    rng = np.random.default_rng(42)
    x = (rng.standard_normal((rows, cols), dtype=np.float32) * 2).astype(np.float16)
    kw = dict(x_ptr=x, y_ptr=np.zeros_like(x))
    return dict(src=configs.softmax(rows, cols, cores, rblk), fn="softmax_kernel", kw=kw, cores=cores,
                bytes=4 * rows * cols, flops=5 * rows * cols, bound="hbm",
                dtype="f16 in/out; f32 max, sum and 1/sum; exp(x - max) held in f16",
                workload=f"softmax {rows}x{cols} f16 grid={cores} rows/step={rblk}")


def _rmsnorm():
    from ktir_cpu_amd import configs
    rows, cols, cores, rblk = 32768, 4096, 512, 8
    rng = np.random.default_rng(42)
    x = (rng.standard_normal((rows, cols), dtype=np.float32) * 2).astype(np.float16)
    w = rng.uniform(0.5, 1.5, cols).astype(np.float16)
    kw = dict(x_ptr=x, w_ptr=w, y_ptr=np.zeros_like(x), eps=1e-6)
    return dict(src=configs.rmsnorm(rows, cols, cores, rblk), fn="rmsnorm_kernel", kw=kw, cores=cores,
                bytes=4 * rows * cols + 2 * cols, flops=4 * rows * cols, bound="hbm",
                dtype="f16 in/out; f32 squares, sum, rsqrt and scaling",
                workload=f"rmsnorm {rows}x{cols} f16 grid={cores} rows/step={rblk}")


def _softmax_extract():
    from ktir_cpu_amd import configs
    rows, cols, cores = 32768, 4096, 512
    rng = np.random.default_rng(42)
    x = (rng.standard_normal((rows, cols), dtype=np.float32) * 2).astype(np.float16)
    kw = dict(x_ptr=x, y_ptr=np.zeros_like(x), n_rows=rows)
    return dict(src=configs.softmax_extract(rows, cols, cores), fn="softmax_fwd", kw=kw, cores=cores,
                bytes=4 * rows * cols, flops=5 * rows * cols, bound="hbm",
                dtype="f16 (the reference example's f16 max, exp, sum and divide)",
                workload=f"softmax {rows}x{cols} f16 grid={cores}, one row per loop step, row max and sum "
                         f"read by tensor.extract (the reference's triton-ktir softmax_fwd form)")


def _rmsnorm_extract():
    from ktir_cpu_amd import configs
    rows, cols, cores = 32768, 4096, 512
    rng = np.random.default_rng(42)
    x = rng.standard_normal((rows, cols), dtype=np.float32).astype(np.float16)
    w = rng.uniform(0.5, 1.5, (1, cols)).astype(np.float16)
    kw = dict(x_ptr=x, w_ptr=w, y_ptr=np.zeros_like(x), n_rows=rows, eps=1e-3)
    return dict(src=configs.rmsnorm_extract(rows, cols, cores), fn="rmsnorm_fwd", kw=kw, cores=cores,
                bytes=4 * rows * cols + 2 * cols, flops=4 * rows * cols, bound="hbm",
                dtype="f16 (the reference example's f16 squares, sum and scalar math)",
                workload=f"rmsnorm {rows}x{cols} f16 grid={cores}, one row per loop step, sum of squares read "
                         f"by tensor.extract, then scalar divf / addf / rsqrt (the reference's latency-example form)")


def _gemm():
    from ktir_cpu_amd import configs
    M = N = K = 8192
    rng = np.random.default_rng(42)
    a = (rng.standard_normal((M, K), dtype=np.float32) * K ** -0.5).astype(np.float16)
    b = (rng.standard_normal((K, N), dtype=np.float32) * K ** -0.5).astype(np.float16)
    kw = dict(a_ptr=a, b_ptr=b, c_ptr=np.zeros((M, N), np.float16))
    return dict(src=configs.gemm(M, N, K, 128, 128, 64, 8, 8), fn="gemm_kernel", kw=kw, cores=64,
                bytes=3 * M * N * 2, flops=2 * M * N * K, bound="mfma", dtype="f16 MFMA, f32 accumulate, f16 out",
                workload=f"gemm {M}x{N}x{K} f16 tiles 128x128x64 grid=8x8")


def _bf16_bits(x):
    """bf16 bit patterns of finite float32 values, rounded to nearest even."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    r = u + np.uint32(0x7FFF)
    r += (u >> np.uint32(16)) & np.uint32(1)
    return (r >> np.uint32(16)).astype(np.uint16)


def _attention():
    from ktir_cpu_amd import configs
    B, H, S, D = 4, 32, 8192, 128
    rng = np.random.default_rng(42)
    q, k, v = (_bf16_bits(rng.standard_normal((B, H, S, D), dtype=np.float32)) for _ in range(3))
    kw = dict(q_ptr=q, k_ptr=k, v_ptr=v, o_ptr=np.zeros_like(q), scale=1.0 / math.sqrt(D))
    return dict(src=configs.flash_attention(B, H, S, D, 128), fn="flash_attention", kw=kw, cores=B * H * S // 128,
                bytes=4 * B * H * S * D * 2, flops=4 * B * H * S * S * D // 2, bound="mfma",
                dtype="bf16 Q K^T MFMA, f32 scores / m / l / acc; P and V rounded to f16 for the f16 P V MFMA; bf16 out",
                f32_blas=True,
                workload=f"flash_attention causal B={B} H={H} S={S} D={D} kv_tile=128")


def _rope():
    from ktir_cpu_amd import configs
    H, S, D = 40, 4096, 128
    rng = np.random.default_rng(42)
    x = rng.standard_normal((H * S, D), dtype=np.float32).astype(np.float16)
    freq = 10000.0 ** (-np.arange(D // 2, dtype=np.float64) * 2.0 / D)
    ang = np.outer(np.arange(S, dtype=np.float64), freq)
    kw = dict(x_ptr=x, cos_ptr=np.cos(ang).astype(np.float16), sin_ptr=np.sin(ang).astype(np.float16),
              out_ptr=np.zeros_like(x))
    return dict(src=configs.rope(H, S, D, 4, 2, 256), fn="rope_fwd_kernel", kw=kw, cores=8,
                bytes=2 * H * S * D * 2 + 2 * S * (D // 2) * 2, flops=6 * H * S * D // 2, bound="hbm",
                # two launches, one per half of the rotated rows: each does half of the work
                dominant_share=0.5,
                dtype="f16 (products, sum and difference each rounded to f16)",
                workload=f"rope H={H} S={S} D={D} f16 grid=4x2 seq tile 256 (the reference's "
                         f"latency/rope_fwd_4x2 form)")


def _paged_attention():
    from ktir_cpu_amd import configs
    T, HQ, HK, D, P, BQ, ctx = 256, 32, 8, 128, 16, 2, 1024
    nt = (ctx + T + P - 1) // P
    blocks, max_pages = 2 * nt, nt
    rng = np.random.default_rng(42)
    kw = dict(output_ptr=np.zeros((T, HQ, D), np.float16),
              query_ptr=rng.standard_normal((T, HQ, D), dtype=np.float32).astype(np.float16),
              key_cache_ptr=rng.standard_normal((blocks, P, HK, D), dtype=np.float32).astype(np.float16),
              value_cache_ptr=rng.standard_normal((blocks, P, HK, D), dtype=np.float32).astype(np.float16),
              block_tables_ptr=rng.permutation(blocks)[:max_pages].astype(np.int32).reshape(1, max_pages),
              cur_batch_start_index=0, block_table_offset=0, num_tiles=nt, context_len=ctx,
              scale=1.0 / math.sqrt(D))
    # causal keys per token: ctx + t + 1; executed keys: all nt pages
    keys = sum(ctx + t + 1 for t in range(T))
    return dict(src=configs.paged_attention(T, HQ, HK, D, P, blocks, max_pages, BQ), fn="kernel_unified_attention_spyre_2d",
                kw=kw, cores=(T // BQ) * HK, bytes=2 * HQ * T * D * 2 + 2 * blocks * P * HK * D * 2,
                flops=4 * HQ * keys * D, bound="mfma",
                dtype="f16 in/out; Q K^T and P V on f16 MFMA (exact f16 products, f32 accumulation, P rounded "
                      "once to f16), f32 scores and online-softmax state",
                workload=f"paged attention {T} tokens after a {ctx}-token context, {HQ} query / {HK} KV heads, "
                         f"D={D}, page {P}, {BQ} tokens per core (the reference's triton-ktir paged_attention form)")


CONFIGS = {"vector_add": _vector_add, "vector_add_4096": _vector_add_4096, "copy": _copy, "gather": _gather, "softmax": _softmax, "rmsnorm": _rmsnorm,
           "gemm": _gemm, "attention": _attention, "softmax_extract": _softmax_extract,
           "rmsnorm_extract": _rmsnorm_extract, "rope": _rope,
           "paged_attention": _paged_attention}


# kernels that make up each kind of launch (the HIP kernel names)
_LAUNCH_KERNELS = {"mm": ("mm_mfma", "mm_generic"), "attn": ("attn_kernel", "attn_pp", "attn_v16"), "rmw": ("rmw_",),
                   "prog": ("prog_",), "pattn": ("pattn_kernel",)}


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
    # the kernels of that launch that run on every timed replay: the
    # attention launch's f16 copy of V included, since every timed replay
    # converts V as a call with a new V does
    b = [v["bytes"] for k, v in t.get("kernels", {}).items()
         if any(p in k for p in pats) and (v.get("every_run", True) or kind in ("attn", "pattn"))]
    return round(sum(b)) if b else None


def _cpu_env():
    """Host cores and BLAS thread settings the CPU baseline ran under."""
    try:
        aff = len(os.sched_getaffinity(0))
    except AttributeError:
        aff = os.cpu_count()
    blas = {k: os.environ.get(k) for k in ("OMP_NUM_THREADS", "OPENBLAS_NUM_THREADS", "MKL_NUM_THREADS")}
    return {"os_cpu_count": os.cpu_count(), "sched_affinity": aff, "blas_threads": blas}


def cpu_baseline(cfg, budget_s=2.5, repeats=3):
    """The oracle (a NumPy restatement of the reference interpreter, one core)
    timed on the host: the fixed part of a run (placing and reading back the
    arrays, no simulated core) and a run of k evenly spaced simulated cores,
    k doubling until the cores' part takes about `budget_s`; each the median
    of `repeats` runs.  The time per simulated core is extrapolated to all
    cores.  Even spacing keeps the sample representative where the work per
    core differs (causal attention: core qb visits qb + 1 KV tiles)."""
    from oracle.interp import OracleInterpreter
    o = OracleInterpreter(lx_size_mb=64)
    o.load(cfg["src"])
    cores = cfg["cores"]
    kw = cfg["kw"]

    def sample(k):
        o.cores_to_run = sorted(set(int(c) for c in np.linspace(0, cores - 1, k + 2)[1:-1].round())) if k else []
        t0 = time.perf_counter()
        o.execute_function(cfg["fn"], **kw)
        return len(o.cores_to_run), time.perf_counter() - t0

    t_fixed = float(np.median([sample(0)[1] for _ in range(repeats)]))
    k = 1
    while True:
        kk, t = sample(min(k, cores))
        if k >= cores or t - t_fixed > budget_s:
            break
        k *= 2
    t_k = float(np.median([t] + [sample(kk)[1] for _ in range(repeats - 1)]))
    per_core = max(t_k - t_fixed, 1e-9) / kk
    t_full = t_fixed + per_core * cores
    return t_full, {"k": kk, "t_k": t_k, "t_fixed": t_fixed}


def _instrumented_steps(prep, steps, reuse_v16=True):
    """K replays of the plan with a HIP event after every launch (library
    stream): returns (ms per step, mean ms of each launch)."""
    from ktir_cpu_amd import runtime as rt
    plan = prep.plan
    n = len(plan.launches)
    instrument = 0 < n <= 64
    evs = [[rt.Event() for _ in range(n)] for _ in range(steps)] if instrument else None
    e0, e1 = rt.Event(), rt.Event()
    # one untimed replay ahead of the start event keeps the GPU busy while
    # the host queues the timed ones, so the region does not open with the
    # GPU idle, waiting for the first launch to be submitted
    plan.run(reuse_v16=reuse_v16)
    e0.record()
    for s_ in range(steps):
        if instrument:
            plan.run(after=lambda i, row=evs[s_]: row[i].record(), reuse_v16=reuse_v16)
        else:
            plan.run(reuse_v16=reuse_v16)
    e1.record()
    rt.sync()
    ms = e0.elapsed_ms(e1) / steps
    durs = np.zeros(n)
    if instrument:
        for s_ in range(steps):
            prev = e0 if s_ == 0 else evs[s_ - 1][-1]
            for i in range(n):
                durs[i] += prev.elapsed_ms(evs[s_][i])
                prev = evs[s_][i]
        durs /= steps
    return ms, durs


FLUSH_ROWS, FLUSH_COLS = 65536, 4096      # 1 GiB of f32 read by the flush
WARMUP_S = 0.5                            # least warm-up time per workload


def _flush_plan():
    """A KTIR row sum over a 1 GiB f32 array (1024 cores x 64 rows of 4096):
    replayed on the library stream it reads 1 GiB and writes 256 KB, which
    evicts the L2 caches and MI355X's 256 MB Infinity Cache and leaves them
    holding clean lines (a fill would leave dirty lines, whose write-back
    the timed launch would then pay)."""
    from ktir_cpu_amd import configs
    from ktir_cpu_amd.interpreter import KTIRInterpreter
    rows, cols, cores = FLUSH_ROWS, FLUSH_COLS, 1024      # 1 MiB of LX per core
    blk = rows // cores
    T, V = configs._t([blk, cols], "f32"), configs._t([blk], "f32")
    src = f"""module {{
  func.func @flush(%x_ptr: index, %y_ptr: index) attributes {{grid = [{cores}, 1]}} {{
    %core_id = ktdp.get_compute_tile_id : index
    %c0 = arith.constant 0 : index
    %B = arith.constant {blk} : index
    %r0 = arith.muli %core_id, %B : index
    %zero = arith.constant 0.0 : f32
{configs._view("x_view", "x_ptr", [rows, cols], [cols, 1], "f32")}
{configs._view("y_view", "y_ptr", [rows], [1], "f32")}
{configs._tile("xt", "x_view", ["%r0", "%c0"], [blk, cols], [rows, cols], "f32")}
{configs._tile("yt", "y_view", ["%r0"], [blk], [rows], "f32")}
    %x = ktdp.load %xt : !ktdp.access_tile<{blk}x{cols}xindex> -> {T}
    %init = tensor.splat %zero : {V}
    %s = linalg.reduce {{ arith.addf }} ins(%x : {T}) outs(%init : {V}) dimensions = [1]
    ktdp.store %s, %yt : {V}, !ktdp.access_tile<{blk}xindex>
    return
  }}
}}
"""
    it = KTIRInterpreter()
    it.load(src)
    prep = it.prepare("flush", x_ptr=np.ones((rows, cols), np.float32), y_ptr=np.zeros(rows, np.float32))
    return it, prep


def _cold_steps(prep, steps):
    """K replays, each preceded (outside its own events, on the same stream)
    by the flush plan: the mean ms of one replay whose inputs come from HBM
    only."""
    from ktir_cpu_amd import runtime as rt
    _it, flush = _flush_plan()
    plan = prep.plan
    evs = [(rt.Event(), rt.Event()) for _ in range(steps)]
    for a, b in evs:
        flush.plan.run()
        a.record()
        plan.run()
        b.record()
    rt.sync()
    ms = float(np.mean([a.elapsed_ms(b) for a, b in evs]))
    del flush, _it
    return ms


def measure(name, steps, warmup, with_cpu):
    """One config: whole-step throughput on resident inputs, the dominant
    launch against its roofline, host<->device copy times, one end-to-end
    execute_function, and (optionally) the CPU baseline."""
    from ktir_cpu_amd import runtime as rt
    from ktir_cpu_amd.interpreter import KTIRInterpreter
    cfg = CONFIGS[name]()
    interp = KTIRInterpreter()
    interp.load(cfg["src"])
    t0 = time.perf_counter()
    prep = interp.prepare(cfg["fn"], **cfg["kw"])          # copies in, host walk, first launch
    prepare_s = time.perf_counter() - t0
    plan = prep.plan
    # at least W replays and at least WARMUP_S seconds of them (none for
    # W = 0, as the counter runs ask): the GPU's clocks take tens of
    # milliseconds of load to settle, and a few replays of a
    # millisecond-scale launch end before they do
    t0, k = time.perf_counter(), 0
    while k < warmup or (warmup and time.perf_counter() - t0 < WARMUP_S):
        prep.run()
        k += 1
        if k % 4 == 0:
            rt.sync()
    rt.sync()
    # attention converts V to f16 on every timed replay, as a call whose V is
    # new does; the replays that reuse the copy of an unchanged V are
    # reported beside the value
    ms, durs = _instrumented_steps(prep, steps, reuse_v16=False)
    reuse_ms = None
    if plan.v16:
        reuse_ms, _ = _instrumented_steps(prep, steps, reuse_v16=True)
    cold_ms = _cold_steps(prep, steps) if cfg["bound"] == "hbm" else None
    n = len(plan.launches)
    dom = int(np.argmax(durs)) if n else 0
    dom_ms = float(durs[dom]) if n and durs.any() else ms
    kind = plan.launches[dom][0] if n else None
    # the dominant launch processes all of the workload's algorithmic units
    # (all bytes moved / all flops), or the share the config states
    if cfg["bound"] == "hbm":
        units, unit, peak, scale = cfg["bytes"], "GB/s", HBM_PEAK_GBS, 1e9
    else:
        units, unit, peak, scale = cfg["flops"], "TFLOP/s", MFMA_F16_TFLOPS, 1e12
    value = units / (ms * 1e-3) / scale
    achieved = units * cfg.get("dominant_share", 1.0) / (dom_ms * 1e-3) / scale
    # host <-> device copies of all array arguments, and one whole call
    t0 = time.perf_counter()
    prep.reset_inputs()
    rt.sync()
    h2d_s = time.perf_counter() - t0
    t0 = time.perf_counter()
    prep.outputs()
    d2h_s = time.perf_counter() - t0
    del prep
    t0 = time.perf_counter()
    interp.execute_function(cfg["fn"], **cfg["kw"])
    e2e_s = time.perf_counter() - t0
    out = {"config": name, "workload": cfg["workload"], "value": round(value, 3), "unit": unit,
           "ms_per_step": round(ms, 6), "dtype": cfg["dtype"], "launches_per_step": n, "plan_mode": plan.mode,
           "roofline": {"bound": cfg["bound"], "achieved": round(achieved, 3), "peak": peak, "unit": unit,
                        "frac": round(achieved / peak, 4), "traffic": _traffic(name, kind),
                        "dominant_launch": kind, "dominant_ms": round(dom_ms, 6)},
           **({"v16_reuse": {"ms_per_step": round(reuse_ms, 6),
                             "value": round(units / (reuse_ms * 1e-3) / scale, 3)}} if reuse_ms else {}),
           **({"cold": {"ms_per_step": round(cold_ms, 6), "value": round(units / (cold_ms * 1e-3) / scale, 3),
                        "frac": round(units / (cold_ms * 1e-3) / scale / peak, 4),
                        "how": f"each replay after a row sum that reads {FLUSH_ROWS * FLUSH_COLS * 4 >> 20} MiB "
                               "(outside the timed region, same stream), which evicts L2 and the 256 MB "
                               "Infinity Cache"}} if cold_ms else {}),
           "host": {"prepare_s": round(prepare_s, 3), "h2d_s": round(h2d_s, 4), "d2h_s": round(d2h_s, 4),
                    "execute_function_s": round(e2e_s, 3),
                    "execute_function_rate": round(units / e2e_s / scale, 4)}}
    if with_cpu:
        t_full, smp = cpu_baseline(cfg)
        env = _cpu_env()
        # the oracle is single-threaded NumPy except f32 matmuls, which go
        # through BLAS (attention's S = Q K^T and P V are f32 products)
        blas_n = int(env["blas_threads"].get("OPENBLAS_NUM_THREADS") or env["blas_threads"].get("OMP_NUM_THREADS")
                     or env["sched_affinity"] or 1)
        cores = blas_n if cfg.get("f32_blas") else 1
        out["cpu_baseline"] = {"value": units / t_full / scale, "unit": unit, "cores": cores, "kind": "port",
                               "sample": f"oracle on {smp['k']} evenly spaced of {cfg['cores']} simulated cores "
                                         f"({smp['t_k']:.2f} s, of which {smp['t_fixed']:.2f} s is the run's "
                                         f"fixed part, timed without cores; medians of 3), extrapolated by "
                                         f"core count to {t_full:.1f} s for the full run"
                                         + ("; f32 matmuls on BLAS threads, the rest on one core"
                                            if cfg.get("f32_blas") else "; one core"),
                               **env}
    print(f"[bench] {name}: {out['value']} {unit}, frac {out['roofline']['frac']}", file=sys.stderr, flush=True)
    return out


HEADLINE = "gather"
PER_CONFIG = ["vector_add", "gather", "softmax", "rmsnorm", "gemm", "attention", "softmax_extract", "rmsnorm_extract",
              "paged_attention", "rope", "vector_add_4096"]


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="all", choices=["all"] + sorted(CONFIGS),
                    help="one config, or all (the gather headline plus every config in per_config)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    ap.add_argument("--collect-traffic", metavar="DIR",
                    help="build profiles/traffic.json from rocprofv3 FETCH_SIZE/WRITE_SIZE runs under DIR")
    ap.add_argument("--collect-counters", metavar="DIR",
                    help="build profiles/counters.json from rocprofv3 --pmc runs (COUNTER_PASSES) under DIR")
    args = ap.parse_args()
    if args.collect_traffic:
        collect_traffic(args.collect_traffic)
        return
    if args.collect_counters:
        for r in collect_counters(args.collect_counters):
            print(json.dumps(r))
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this backend runs on one GPU; multi-GPU runs are not part of this build",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    names = PER_CONFIG if args.config == "all" else [args.config]
    head = HEADLINE if args.config == "all" else args.config
    results = [measure(n, args.steps, args.warmup, not args.no_cpu) for n in names]
    h = next(r for r in results if r["config"] == head)
    out = {
        "metric": "achieved HBM GB/s & MFMA TFLOP/s per KTIR kernel (% of roofline) vs NumPy",
        "value": h["value"], "unit": h["unit"], "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "warmup_min_s": WARMUP_S,
        "ms_per_step": h["ms_per_step"], "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": h["dtype"], "data": "synthetic (seed 42)",
        "config": {"workload": h["workload"], "launches_per_step": h["launches_per_step"],
                   "plan_mode": h["plan_mode"]},
        "roofline": h["roofline"],
    }
    for k in ("cold", "v16_reuse"):
        if k in h:
            out[k] = h[k]
    if "cpu_baseline" in h:
        out["cpu_baseline"] = h["cpu_baseline"]
    out["host"] = h["host"]
    if args.config == "all":
        out["per_config"] = results
    print(json.dumps(out))


COUNTER_PASSES = {
    "mfma": ["SQ_WAVE_CYCLES", "SQ_BUSY_CYCLES", "SQ_VALU_MFMA_BUSY_CYCLES", "SQ_VALU_MFMA_COEXEC_CYCLES",
             "SQ_INSTS_MFMA", "SQ_INSTS_VALU", "SQ_INSTS_VALU_TRANS_F32", "GRBM_GUI_ACTIVE"],
    "lds": ["SQ_LDS_BANK_CONFLICT", "SQ_LDS_IDX_ACTIVE", "SQ_INSTS_LDS", "SQ_WAIT_INST_LDS", "SQ_ACTIVE_INST_LDS",
            "GRBM_GUI_ACTIVE"],
}
SIMDS, XCDS, PEAK_GHZ = 1024, 8, 2.4


def collect_counters(root):
    """profiles/counters.md from rocprofv3 --pmc runs under
    ROOT/counters_<config>_<pass>/ (passes in COUNTER_PASSES), for the MFMA
    kernels of the gemm and attention configs: MFMA busy (the MfmaUtil
    expression: SQ_VALU_MFMA_BUSY_CYCLES over GRBM_GUI_ACTIVE x SIMDs), VALU
    co-executing with MFMA, instruction counts, LDS bank conflicts per active
    LDS cycle, and the shader clock (GRBM_GUI_ACTIVE per XCD over the
    dispatch's duration), beside the MFMA fraction of 2.5 PF scaled to that
    clock."""
    import csv
    import glob
    rows = []
    for config, kern, flops in (("gemm", "mm_mfma_256", 2 * 8192 ** 3),
                                ("attention", "attn_pp", 4 * 4 * 32 * 8192 * 8192 * 128 // 2)):
        vals, durs = {}, {}
        for pas in COUNTER_PASSES:
            for fn in glob.glob(os.path.join(root, f"counters_{config}_{pas}", "**", "*counter_collection.csv"),
                                recursive=True):
                with open(fn) as f:
                    for r in csv.DictReader(f):
                        if kern not in r.get("Kernel_Name", ""):
                            continue
                        name = r["Kernel_Name"]
                        vals.setdefault((name, r["Counter_Name"]), []).append(float(r["Counter_Value"]))
                        if r["Counter_Name"] == "GRBM_GUI_ACTIVE":
                            durs.setdefault(name, []).append(
                                (float(r["End_Timestamp"]) - float(r["Start_Timestamp"])) * 1e-9)
        for name in sorted(durs):
            v = {c: float(np.median(x)) for (n, c), x in vals.items() if n == name}
            # the MFMA pass and the LDS pass each give GRBM_GUI_ACTIVE; both
            # runs' dispatches are pooled for the clock
            t = float(np.median(durs[name]))
            ghz = v["GRBM_GUI_ACTIVE"] / XCDS / t / 1e9
            tf = flops / t / 1e12
            rows.append({
                "config": config, "kernel": name, "dispatches": len(durs[name]), "duration_us": t * 1e6,
                "clock_ghz": ghz, "tflops": tf, "frac_2_5pf": tf / MFMA_F16_TFLOPS,
                "frac_at_clock": tf / (MFMA_F16_TFLOPS * ghz / PEAK_GHZ),
                "mfma_busy": v.get("SQ_VALU_MFMA_BUSY_CYCLES", 0) / (v["GRBM_GUI_ACTIVE"] / XCDS * SIMDS),
                "coexec_of_busy": v.get("SQ_VALU_MFMA_COEXEC_CYCLES", 0) / max(v.get("SQ_VALU_MFMA_BUSY_CYCLES", 1), 1),
                "mfma_insts": v.get("SQ_INSTS_MFMA"), "valu_insts": v.get("SQ_INSTS_VALU"),
                "trans_insts": v.get("SQ_INSTS_VALU_TRANS_F32"),
                "lds_conflict_rate": v.get("SQ_LDS_BANK_CONFLICT", 0) / max(v.get("SQ_LDS_IDX_ACTIVE", 1), 1),
                "lds_bank_conflict": v.get("SQ_LDS_BANK_CONFLICT"), "lds_insts": v.get("SQ_INSTS_LDS")})
    path = os.path.join(ROOT, "profiles", "counters.json")
    with open(path, "w") as fh:
        json.dump(rows, fh, indent=1)
    return rows


def collect_traffic(root):
    """profiles/traffic.json from two rocprofv3 --pmc runs per config
    (FETCH_SIZE, then WRITE_SIZE; KiB per dispatch) under ROOT/traffic_<config>_<counter>/,
    each scaled by what the counter reads for the `copy` config (256 MiB in,
    256 MiB out per dispatch)."""
    import csv
    import glob

    def per_kernel(config, counter):
        files = glob.glob(os.path.join(root, f"traffic_{config}_{counter}", "**", "*counter_collection.csv"),
                          recursive=True)
        vals = {}
        for fn in files:
            with open(fn) as f:
                for row in csv.DictReader(f):
                    name = row.get("Kernel_Name", "")
                    # set-up work outside the timed launch: the runtime's copies and
                    # fills, and the library's one-time fill of its own scratch array
                    if name.startswith("__amd_rocclr") or name.startswith("rmw_fill"):
                        continue
                    if row.get("Counter_Name") == counter:
                        vals.setdefault(name, []).append(float(row["Counter_Value"]))
        return {k: float(np.median(v)) for k, v in vals.items()}, {k: len(v) for k, v in vals.items()}

    (cf, _), (cw, _) = per_kernel("copy", "FETCH_SIZE"), per_kernel("copy", "WRITE_SIZE")
    ck = max(cf, key=cf.get)
    each = 256 * 1024 * 1024
    fscale, wscale = each / (cf[ck] * 1024), each / (cw[ck] * 1024)
    out = {"calibration": {"kernel": ck, "bytes_each_way": each, "fetch_kib": cf[ck], "write_kib": cw[ck],
                           "fetch_scale": fscale, "write_scale": wscale}, "configs": {}}
    for config in sorted(CONFIGS):
        (f, nf), (w, _) = per_kernel(config, "FETCH_SIZE"), per_kernel(config, "WRITE_SIZE")
        if not f:
            continue
        # the launch of a timed replay: the kernels dispatched on every run
        # of the plan, plus the attention launch's f16 copy of V (made by a
        # run whose V is new and skipped by a replay that reuses it; every
        # timed replay converts V, as a call with a new V does)
        top = max(nf.values())
        ks = {k: {"fetch_kib": f[k], "write_kib": w.get(k, 0.0), "dispatches": nf[k], "every_run": nf[k] == top,
                  "bytes": f[k] * 1024 * fscale + w.get(k, 0.0) * 1024 * wscale} for k in f}
        out["configs"][config] = {"traffic_bytes": sum(v["bytes"] for k, v in ks.items()
                                                       if v["every_run"] or "attn_v16" in k),
                                  "kernels": ks}
    path = os.path.join(ROOT, "profiles", "traffic.json")
    with open(path, "w") as fh:
        json.dump(out, fh, indent=1)
    print(path)


if __name__ == "__main__":
    main()
