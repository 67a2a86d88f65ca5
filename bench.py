"""op1 benchmark on one MI355X: Mixtral-8x7B MoE layer over a 64-node tree.

One step = one ``tree_moe_forward`` call (router, budget routing/bucketing,
gate/up GEMM + SwiGLU, down GEMM, fixed-order combine) at config 2 of the
baseline: T=64, H=4096, I=14336, E=8, top-2, B=8, bf16, inputs resident in
HBM.  ``value`` is algorithmic HBM throughput (compulsory bytes / step time).

Prints ONE JSON line.  Also reports, in the same line, the dominant kernel's
roofline (HIP events on the launch stream), the CPU baseline (torch
restatement of treemoe/ref on the host cores), and secondary configurations.
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

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
METRIC = "op1 MoE layer µs + HBM GB/s (% peak), Mixtral shape, 64-node tree, 1 MI355X"


def parse_args():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--cpu-seconds", type=float, default=15.0,
                   help="time budget of the CPU-baseline sample (0 disables it)")
    p.add_argument("--no-secondary", action="store_true")
    p.add_argument("--copy-probe-mb", type=int, default=0,
                   help="run one plain device copy of this many MiB first (a known-size "
                        "reference for rocprofv3 FETCH_SIZE / WRITE_SIZE scaling)")
    return p.parse_args()


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def step_times_ms(fn, reps: int) -> list[float]:
    """Per-call device time of fn() for `reps` back-to-back calls: one HIP
    event pair per call on the current stream (the stream the library
    launches on)."""
    import torch

    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(reps)]
    for s, e in ev:
        s.record()
        fn()
        e.record()
    ev[-1][1].synchronize()
    return [s.elapsed_time(e) for s, e in ev]


def median(xs: list[float]) -> float:
    ys = sorted(xs)
    n = len(ys)
    return ys[n // 2] if n % 2 else 0.5 * (ys[n // 2 - 1] + ys[n // 2])


def events_time_ms(fn, reps: int) -> float:
    """Median per-call device time of fn() over `reps` calls (HIP events)."""
    return median(step_times_ms(fn, reps))


def device_time_ms(fn, reps: int, spin_cycles: int = 200_000) -> float:
    """Median device time of fn() over `reps` calls, each queued behind a GPU
    spin (torch.cuda._sleep) long enough for the host to issue all of the
    call's launches first: host-side launch cost then opens no gaps between
    its kernels.  One HIP event pair per call on the current stream."""
    import torch

    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(reps)]
    for s, e in ev:
        torch.cuda._sleep(spin_cycles)
        s.record()
        fn()
        e.record()
    ev[-1][1].synchronize()
    return median([s.elapsed_time(e) for s, e in ev])


def host_cpu() -> dict:
    """What the host says about its CPU: /proc/cpuinfo's model name, family,
    model and stepping numbers (some hosts give no model number in the
    name), the logical CPUs and the ones this process may run on."""
    info = {"model_name": platform.processor() or platform.machine()}
    fields = {"model name": "model_name", "cpu family": "family", "model": "model",
              "stepping": "stepping", "cpu MHz": "mhz"}
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if not line.strip():
                break  # the first processor's block is enough
            key, _, val = line.partition(":")
            key = key.strip()
            if key in fields:
                info[fields[key]] = val.strip()
    except OSError:
        pass
    info["logical_cpus"] = os.cpu_count()
    try:
        info["usable_cpus"] = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        info["usable_cpus"] = os.cpu_count()
    return info


def cpu_model() -> str:
    c = host_cpu()
    desc = c.get("model_name", "unknown")
    if "family" in c:
        desc += f" (family {c['family']}, model {c.get('model', '?')}, stepping " \
                f"{c.get('stepping', '?')})"
    return desc


def _median_cpu_ms(fn, reps: int = 10, warmup: int = 2) -> tuple[float, int]:
    for _ in range(warmup):
        fn()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return median(times) * 1e3, reps


def cpu_path_timings() -> dict:
    """The reference's CPU path at the two other shapes the baseline plan
    names, through the torch restatement in oracle/ (same torch calls in the
    same order as treemoe/ref): op1 at config 1 (T=64, H=1024, I=3584, E=8,
    B=8; tree_moe_ref.py:102-130) and op4 at config 4 (greedy tree_verify,
    verify_ref.py:35-103, then commit_tree at page 16, kv_cache.py:88-106:
    N=64, V=32000 fp32 logits as the engine passes them, 32 layers x 8 KV
    heads x 128, 4096 committed positions).  Median of 10 after 2 warm-ups."""
    import torch

    from oracle import op1_ref, op4_ref
    from treemoe_spec_amd.workloads import op1_workload, op4_workload

    inp = op1_workload("config1_cpu_small", device="cpu")
    args = (inp.x, inp.w1, inp.w2, inp.w3, inp.router, inp.accept, inp.budget)
    c1_ms, c1_reps = _median_cpu_ms(lambda: op1_ref.tree_moe_forward(*args))
    del inp, args

    w = op4_workload(n=64, vocab=32000, max_depth=8, seed=3)
    logits = w.logits.float()
    layers, kvh, hd, page, seq = 32, 8, 128, 16, 4096
    n_scratch = (64 + page - 1) // page
    pages = n_scratch + seq // page + 1
    g = torch.Generator().manual_seed(3)
    k = torch.randn(layers, pages, page, kvh, hd, generator=g).to(torch.bfloat16)
    v = torch.randn(layers, pages, page, kvh, hd, generator=g).to(torch.bfloat16)
    scratch = list(range(n_scratch))
    table = (torch.randperm(pages - n_scratch, generator=g) + n_scratch).tolist()

    def op4_step():
        slots, _, _, num = op4_ref.tree_verify(logits, None, w.tokens, w.children)
        commit = torch.cat([torch.zeros(1, dtype=torch.long), slots[:num]])
        op4_ref.commit_tree(k, v, commit, scratch, table, seq)
        return num

    accepted = op4_step()
    op4_ms, op4_reps = _median_cpu_ms(op4_step)
    return {"config1_ms": round(c1_ms, 3), "config1_reps": c1_reps,
            "op4_config4_ms": round(op4_ms, 3), "op4_config4_reps": op4_reps,
            "op4_config4_accepted": accepted}


def kernel_breakdown(m, inp, reps: int) -> dict:
    """Median duration (ms) of each phase of one op1 step over `reps` steps:
    tree_moe_forward's own launches (op1_tree_moe._forward), with an event
    recorded after each phase on the stream the library launches on (torch's
    current stream).  "route" is the router and, unless the gate/up launch
    routes its own jobs, the bucketing; "gemm1" the gate/up launch."""
    import torch

    x, w1, w2, w3, router, accept, budget = (inp.x, inp.w1, inp.w2, inp.w3, inp.router,
                                             inp.accept, inp.budget)
    n, hidden = x.shape
    e, inter, _ = w1.shape
    names = ["route", "gemm1", "gemm2", "combine"]
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(5)] for _ in range(reps)]
    out = torch.empty_like(x)
    for r in range(reps):
        marks = iter(ev[r][1:])
        ev[r][0].record()
        m._forward(x, w1, w2, w3, router, accept, budget, out, None, "mass",
                   on_phase=lambda name, marks=marks: next(marks).record())
    torch.cuda.synchronize()
    res = {}
    for k, name in enumerate(names):
        res[name] = median([ev[r][k].elapsed_time(ev[r][k + 1]) for r in range(reps)])
    res["tiled"] = m.uses_tiled_gemms(n, budget, e, inter)
    res["self_routed"] = m.self_routed(n, budget, e, inter)
    res["max_tiles"] = m.compact_block_limit(2 * n, budget, m.TILE_M)
    return res


def measured_traffic(profile: Path) -> float | None:
    """HBM bytes per gemm1 launch from the committed rocprofv3 --pmc summary
    (line 'gemm1_hbm_bytes_per_launch: <bytes>'), None if absent."""
    if not profile.exists():
        return None
    for line in profile.read_text().splitlines():
        if line.startswith("gemm1_hbm_bytes_per_launch:"):
            return float(line.split(":", 1)[1])
    return None


def cpu_baseline(inp, budget_s: float, bytes_alg: int) -> dict:
    import torch

    from oracle import op1_ref

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    cpu = [t.detach().cpu() for t in (inp.x, inp.w1, inp.w2, inp.w3, inp.router, inp.accept)]
    op1_ref.tree_moe_forward(*cpu, inp.budget)  # warm-up
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or not times:
        t0 = time.perf_counter()
        op1_ref.tree_moe_forward(*cpu, inp.budget)
        times.append(time.perf_counter() - t0)
        if len(times) >= 200:
            break
    times.sort()
    med = times[len(times) // 2]
    line = {
        "value": round(bytes_alg / med / 1e9, 3),
        "unit": "GB/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"{len(times)} full config-2 layers (T=64, H=4096, I=14336, E=8, B=8) "
                   f"through the torch CPU restatement of treemoe/ref/tree_moe_ref.py; "
                   f"median {med * 1e3:.1f} ms/layer; host CPU {cpu_model()}, "
                   f"os.cpu_count()={threads}, torch threads {torch.get_num_threads()}; "
                   "config1_ms / op4_config4_ms: the same restatement at config 1 and "
                   "op4 (tree_verify + commit_tree, page 16) at config 4, median of 10 "
                   "after 2 warm-ups"),
        "ms_per_layer": round(med * 1e3, 3),
        "host_cpu": host_cpu(),
        "torch_threads": torch.get_num_threads(),
    }
    line.update(cpu_path_timings())
    return line


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(the op1/op4 path is built and measured on a single MI355X)", file=sys.stderr)
        sys.exit(2)
    import torch

    from treemoe_spec_amd.kernels import op1_tree_moe as m
    from treemoe_spec_amd.workloads import (op1_algorithmic_bytes, op1_flops, op1_workload)

    torch.cuda.set_device(0)
    if args.copy_probe_mb > 0:
        src = torch.ones(args.copy_probe_mb << 20, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copy probe: {args.copy_probe_mb} MiB device-to-device")
        del src, dst
    log("drawing config 2 inputs")
    inp = op1_workload("config2_mixtral_t64_b8", device="cuda")
    t, h, i, e = inp.shape
    fwd = lambda: m.tree_moe_forward(inp.x, inp.w1, inp.w2, inp.w3, inp.router, inp.accept,
                                     inp.budget)
    for _ in range(args.warmup):
        fwd()
    torch.cuda.synchronize()
    routing = m.route_experts(inp.x, inp.router, inp.accept, inp.budget, i)
    n_active = len(routing.expert_ids())
    bytes_alg = op1_algorithmic_bytes(t, h, i, e, n_active)
    flops = op1_flops(t, h, i, e)

    log(f"timing {args.steps} steps")
    torch.cuda.synchronize()
    w0 = time.perf_counter()
    times = step_times_ms(fwd, args.steps)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - w0) * 1e3 / args.steps
    ms = median(times)
    mean_ms = sum(times) / len(times)

    # per-launch breakdown: median over at least 50 steps after 10 more warm-ups
    reps = max(args.steps, 50)
    for _ in range(10):
        fwd()
    bd = kernel_breakdown(m, inp, reps)
    tiled = bd.pop("tiled")
    routed = bd.pop("self_routed")
    max_tiles = bd.pop("max_tiles")
    gemm1_kernel = (f"tm_prefill_gemm1{'_routed' if routed else ''}_kernel"
                    f"<{m.tiled_gate_up_tile(t, e, max_tiles)}>" if tiled else "tm_gemm1_kernel")
    # algorithmic bytes per launch: one read of the active experts' weights
    # (w1 + w3 for gemm1, w2 for gemm2) plus the activation rows in (x); the
    # h and fp32-partial workspaces are not counted
    gemm1_bytes = n_active * 2 * h * i * 2 + t * h * 2
    gemm1_gbs = gemm1_bytes / (bd["gemm1"] * 1e-3) / 1e9
    gemm2_bytes = n_active * h * i * 2
    gemm2_gbs = gemm2_bytes / (bd["gemm2"] * 1e-3) / 1e9
    traffic = measured_traffic(ROOT / "profiles" / "op1_gemm1_config2_pmc.txt")
    value = bytes_alg / (ms * 1e-3) / 1e9

    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "us_per_layer": round(ms * 1e3, 2),
        "timing": {"statistic": "median of the timed steps (one HIP event pair per step)",
                   "mean_us": round(mean_ms * 1e3, 2), "min_us": round(min(times) * 1e3, 2),
                   "max_us": round(max(times) * 1e3, 2),
                   "breakdown_steps": reps},
        "pct_hbm_peak": round(100.0 * value / HBM_PEAK_GBS, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "op1 Mixtral-8x7B MoE layer, T=64 tree tokens, top-2, B=8 (config 2)",
                   "tokens": t, "hidden": h, "ffn": i, "experts": e, "budget": inp.budget,
                   "active_experts": n_active, "bytes_alg": bytes_alg, "flops_alg": flops},
        "roofline": {"bound": "hbm", "kernel": gemm1_kernel,
                     "achieved": round(gemm1_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gemm1_gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "bytes_alg_per_launch": gemm1_bytes,
                     "bytes_alg_unit": "w1 + w3 row pair (2 x H x 2 B = 16 KiB) x I x "
                                       "active experts, plus x (T x H x 2 B)",
                     "median_launch_us": round(bd["gemm1"] * 1e3, 2)},
        "kernels_us": {k: round(v * 1e3, 2) for k, v in bd.items()},
        "gemm2_gbs": round(gemm2_gbs, 1),
        "wall_ms_per_step": round(wall_ms, 4),
        "tflops": round(flops / (ms * 1e-3) / 1e12, 2),
    }

    if not args.no_secondary:
        line["secondary"] = secondary(m, inp, args)
    if args.cpu_seconds > 0:
        log("CPU baseline")
        line["cpu_baseline"] = cpu_baseline(inp, args.cpu_seconds, bytes_alg)
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line), flush=True)


def secondary(m, inp2, args) -> dict:
    """Config 3 (B=4 skew), config 5 (T=2048 Zipf) and op4 (config 4), reusing
    config 2's expert weights (weights do not affect timing; routing inputs
    follow each config's own seed)."""
    import torch

    from treemoe_spec_amd.kernels import op4_commit
    from treemoe_spec_amd.kv_cache import MixtralConfig, PagedKVCache
    from treemoe_spec_amd.workloads import (op1_algorithmic_bytes, op1_flops, op1_workload,
                                            op4_algorithmic_bytes, op4_workload)

    out = {}
    weights = (inp2.w1, inp2.w2, inp2.w3)
    reps = max(10, args.steps // 2)
    for name in ("config3_mixtral_t64_b4_skew", "config5_mixtral_t2048_zipf"):
        log(f"secondary {name}")
        inp = op1_workload(name, device="cuda", weights=weights)
        t, h, i, e = inp.shape
        fwd = lambda: m.tree_moe_forward(inp.x, inp.w1, inp.w2, inp.w3, inp.router,
                                         inp.accept, inp.budget)
        for _ in range(3):
            fwd()
        ms = events_time_ms(fwd, reps)
        r = m.route_experts(inp.x, inp.router, inp.accept, inp.budget, i)
        n_active = len(r.expert_ids())
        b = op1_algorithmic_bytes(t, h, i, e, n_active)
        fl = op1_flops(t, h, i, e)
        out[name] = {"us": round(ms * 1e3, 2), "gbs": round(b / (ms * 1e-3) / 1e9, 1),
                     "pct_hbm_peak": round(100 * b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 2),
                     "tflops": round(fl / (ms * 1e-3) / 1e12, 2),
                     "pct_mfma_peak": round(100 * fl / (ms * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 2),
                     "active_experts": n_active}
    # one GPU's share of a G-way tensor-parallel config-2 layer: I / G columns
    # of w1/w3 and of w2 for all 8 experts (routing replicated; the rank-order
    # reduce of the fp32 partials across GPUs is not part of this)
    log("secondary tensor-parallel shares")
    t, h, i, e = inp2.shape
    shares = {}
    for g in (2, 4, 8):
        ig = i // g
        w1 = inp2.w1[:, :ig, :].contiguous()
        w3 = inp2.w3[:, :ig, :].contiguous()
        w2 = inp2.w2[:, :, :ig].contiguous()
        fwd = lambda: m.tree_moe_forward(inp2.x, w1, w2, w3, inp2.router, inp2.accept,
                                         inp2.budget)
        for _ in range(3):
            fwd()
        ms = events_time_ms(fwd, reps)
        b = op1_algorithmic_bytes(t, h, ig, e, e)
        shares[f"tp{g}_i{ig}"] = {"us": round(ms * 1e3, 2), "gbs": round(b / (ms * 1e-3) / 1e9, 1),
                                  "pct_hbm_peak": round(100 * b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 2)}
        del w1, w2, w3
    out["config2_tensor_parallel_share"] = shares
    out["config2_torch_composition"] = torch_composition_op1(m, inp2, reps)
    log("secondary op4 config 4")
    w = op4_workload(n=64, vocab=32000, max_depth=8, seed=3)
    cfg = MixtralConfig()
    page = 16
    kv = PagedKVCache(cfg, 4096 // page + 4 + 16, device="cuda", page_size=page, tree_size=64)
    kv._ensure_capacity(4096)
    logits = w.logits.cuda()
    tokens = w.tokens.cuda()
    parent = w.parent.cuda()

    def step():
        kv.seq_len = 4096
        return op4_commit.fused_verify_commit(logits, None, tokens, parent, w.children, kv=kv,
                                              max_depth=8)

    for _ in range(3):
        res = step()
    num = int(res.num_accepted)
    ms = events_time_ms(step, reps)
    # device side alone: the two C-ABI calls with the CSR, tables and outputs
    # already resident (the host glue above builds the CSR and reads back
    # num_accepted, as the reference does), each call queued behind a GPU spin
    # so that the host's launch cost is not timed
    from treemoe_spec_amd import _capi

    dev = logits.device
    n, v = logits.shape
    csr, num_edges = op4_commit._children_csr(w.children, n, dev)
    am = torch.empty(n, dtype=torch.int32, device=dev)
    slots = torch.empty(n, dtype=torch.int64, device=dev)
    toks = torch.empty(n, dtype=torch.int64, device=dev)
    result = torch.empty(3, dtype=torch.int64, device=dev)
    wsp = op4_commit.argmax_workspace(n, dev)
    table, scratch = kv.device_tables(dev)
    k = kv.k
    stream = _capi.stream_of(dev)

    def device_step():
        _capi.call("tm_op4_argmax_walk", logits.data_ptr(), _capi.TM_DTYPE_BF16, n, v,
                   logits.stride(0), tokens.data_ptr(), csr.data_ptr(), csr.data_ptr() + 4 * n,
                   csr.data_ptr() + 8 * n, num_edges, 8, 0, am.data_ptr(), slots.data_ptr(),
                   toks.data_ptr(),
                   result.data_ptr(), wsp.data_ptr(), stream)
        _capi.call("tm_op4_kv_commit", k.data_ptr(), kv.v.data_ptr(), k.element_size(),
                   k.shape[0], k.shape[3] * k.shape[4], k.stride(0), k.stride(1), k.stride(2),
                   kv.block_size, slots.data_ptr(), result.data_ptr(), scratch.data_ptr(),
                   len(kv.tree_pages), table.data_ptr(), len(kv.block_table), 4096, 8, 0, stream)

    for _ in range(3):
        device_step()
    dev_ms = device_time_ms(device_step, max(reps, 50))
    # cold: a 512 MB write before each timed call evicts the 256 MB Infinity
    # Cache and the L2s, so the logits and KV rows come from HBM
    flush = torch.empty(512 << 20, dtype=torch.uint8, device=dev)
    cold = []
    for _ in range(20):
        flush.fill_(1)
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        device_step()
        e1.record()
        e1.synchronize()
        cold.append(e0.elapsed_time(e1))
    del flush
    cold_ms = sorted(cold)[len(cold) // 2]
    b = op4_algorithmic_bytes(64, 32000, 2, num + 1, cfg.num_layers,
                              cfg.num_kv_heads * cfg.head_dim * 2)
    out["config4_op4_verify_commit"] = {"us_incl_host_glue": round(ms * 1e3, 2),
                                        "us_device": round(dev_ms * 1e3, 2),
                                        "us_device_cold": round(cold_ms * 1e3, 2),
                                        "gbs_device": round(b / (dev_ms * 1e-3) / 1e9, 1),
                                        "accepted": num, "bytes_alg": b}
    # sampling mode (temperature 1) and the repetition penalty at the same shape:
    # device time of one C-ABI call each, inputs resident
    g = torch.Generator().manual_seed(5)
    q = torch.softmax(torch.randn(n, v, generator=g), -1).cuda()
    uni = torch.rand(n, generator=g).cuda()
    bonus_exp = torch.empty(v).exponential_(1.0, generator=g).cuda()
    resid = torch.empty(v, dtype=torch.float32, device=dev)

    def sample_step():
        _capi.call("tm_op4_sample_walk", logits.data_ptr(), _capi.TM_DTYPE_BF16, n, v,
                   logits.stride(0), q.data_ptr(), q.stride(0), tokens.data_ptr(), csr.data_ptr(),
                   csr.data_ptr() + 4 * n, csr.data_ptr() + 8 * n, num_edges, uni.data_ptr(),
                   bonus_exp.data_ptr(),
                   1.0, resid.data_ptr(), slots.data_ptr(), toks.data_ptr(), result.data_ptr(),
                   stream)

    for _ in range(3):
        sample_step()
    sample_ms = device_time_ms(sample_step, max(reps, 50))
    nodes_visited = int(result[1]) + 1
    pen_logits = logits.clone()
    prev = torch.randint(0, v, (512,), generator=g).cuda()
    size = op4_commit._penalty_table_size(prev.numel())
    table_ws = torch.empty(2 * size, dtype=torch.int32, device=dev)

    def penalty_step():
        _capi.call("tm_op4_rep_penalty", pen_logits.data_ptr(), _capi.TM_DTYPE_BF16, n, v,
                   pen_logits.stride(0), prev.data_ptr(), prev.numel(), 1.1,
                   table_ws.data_ptr(), size, stream)

    for _ in range(3):
        penalty_step()
    pen_ms = device_time_ms(penalty_step, max(reps, 50))
    out["config4_op4_sampling"] = {
        "us_sample_walk": round(sample_ms * 1e3, 2), "nodes_visited": nodes_visited,
        # per visited node: the row's softmax (3 logit passes) and the residual
        # written once; per rejected child: q row read, residual read/written
        "us_rep_penalty_512_prev_tokens": round(pen_ms * 1e3, 2)}
    out["config4_tree_attention"] = tree_attention_secondary(reps)
    return out


def torch_composition_op1(m, inp, reps: int) -> dict:
    """Config 2's expert FFN and combine as plain torch ops on this GPU (one
    F.linear per expert and projection, i.e. hipBLASLt, SiLU, the gate
    weights and an index_add), with this build's routing computed and the
    per-expert row lists built before the timed region: a vendor-library
    point of comparison for tree_moe_forward, not the reference's kernels."""
    import torch
    import torch.nn.functional as F

    x, w1, w2, w3 = inp.x, inp.w1, inp.w2, inp.w3
    t, h = x.shape
    e = w1.shape[0]
    r = m.route_experts(x, inp.router, inp.accept, inp.budget, w1.shape[1])
    ids = r.topk_ids.reshape(-1)
    gates = r.gates_flat.reshape(-1)
    groups = []
    for k in range(e):
        slots = torch.nonzero(ids == k).flatten()
        if slots.numel():
            groups.append((k, slots // 2, gates[slots].unsqueeze(1)))

    def step():
        y = torch.zeros(t, h, dtype=torch.float32, device=x.device)
        for k, tok, g in groups:
            xe = x[tok]
            he = F.silu(F.linear(xe, w1[k])) * F.linear(xe, w3[k])
            y.index_add_(0, tok, F.linear(he, w2[k]).float() * g)
        return y.to(x.dtype)

    ref = step().float()
    ours = m.tree_moe_forward(x, w1, w2, w3, inp.router, inp.accept, inp.budget).float()
    for _ in range(3):
        step()
    ms = events_time_ms(step, reps)
    return {"us": round(ms * 1e3, 2),
            "rel_l2_vs_tree_moe_forward": round(float((ref - ours).norm() / ref.norm()), 5)}


def tree_attention_secondary(reps: int) -> dict:
    """The verification forward's attention at the config-4 cache shape: a
    64-node tree (random parents, depth <= 8), 32 query heads over 8 KV heads,
    head dim 128, page 16, 4096 committed positions, one layer.  Device time
    of the C-ABI call (mask packed and tables resident), the reference's torch
    composition of the same step on this GPU, and the CPU oracle on a bounded
    sample beside them."""
    import ctypes

    import torch

    from oracle import attn_ref
    from treemoe_spec_amd import _capi
    from treemoe_spec_amd.kernels import tree_attention as ta
    from treemoe_spec_amd.kv_cache import MixtralConfig, PagedKVCache
    from treemoe_spec_amd.workloads import random_tree

    log("secondary tree attention config 4")
    n, hq, kvh, hd, seq, page = 64, 32, 8, 128, 4096, 16
    g = torch.Generator().manual_seed(4)
    cfg = MixtralConfig(num_layers=1)
    kv = PagedKVCache(cfg, seq // page + 4 + 8, device="cuda", page_size=page, tree_size=n)
    gd = torch.Generator(device="cuda").manual_seed(4)
    kv.k.normal_(generator=gd)
    kv.v.normal_(generator=gd)
    kv._ensure_capacity(seq)
    kv.seq_len = seq
    q = torch.randn(n, hq, hd, generator=g).to(torch.bfloat16).cuda()
    k = torch.randn(n, kvh, hd, generator=g).to(torch.bfloat16).cuda()
    v = torch.randn(n, kvh, hd, generator=g).to(torch.bfloat16).cuda()
    parent, _, _, _ = random_tree(g, n, 8, 32000)
    mask = attn_ref.ancestor_mask(parent).cuda()
    out = ta.tree_attention(q, k, v, kv, 0, mask)
    bits = ta.pack_tree_mask(mask)
    table, scratch = kv.device_tables(q.device)
    chunks, wbytes = ctypes.c_int64(), ctypes.c_int64()
    _capi.call("tm_tree_attention_plan", n, hq, kvh, hd, seq, page, 0, ctypes.byref(chunks),
               ctypes.byref(wbytes))
    ws = torch.empty(max(wbytes.value, 16), dtype=torch.uint8, device="cuda")
    kc, vc = kv.k[0], kv.v[0]
    stream = _capi.stream_of(q.device)
    args = (q.data_ptr(), hq * hd, k.data_ptr(), v.data_ptr(), kvh * hd, kc.data_ptr(),
            vc.data_ptr(), kc.stride(0), kc.stride(1), page, table.data_ptr(),
            len(kv.block_table), seq, scratch.data_ptr(), len(kv.tree_pages), 1,
            bits.data_ptr(), n, hq, kvh, hd, hd ** -0.5, out.data_ptr(), hq * hd, 0,
            ws.data_ptr(), wbytes.value, stream)
    fn = _capi.lib().tm_tree_attention

    def step():
        rc = fn(*args)
        if rc:
            raise RuntimeError(f"tm_tree_attention status {rc}")

    for _ in range(5):
        step()
    dev_ms = events_time_ms(step, max(reps, 50))
    bytes_alg = (2 * seq * kvh * hd * 2          # prefix K and V, read once
                 + 2 * 2 * n * kvh * hd * 2      # tree K and V read, and stored to scratch
                 + 2 * n * hq * hd * 2)          # q in, context out
    flops = 4 * n * hq * (seq + n) * hd          # QK^T and PV over every key, masked or not
    # the reference's own torch composition on this GPU (mixtral.py:208-250):
    # write_tree, gather_with_tail, the boolean mask, SDPA with enable_gqa
    import torch.nn.functional as F

    def torch_composition():
        kv.write_tree(0, k, v)
        fk, fv = kv.gather_with_tail(0, k, v)
        pre = fk.shape[0] - n
        full = torch.zeros(n, pre + n, dtype=torch.bool, device="cuda")
        full[:, :pre] = True
        full[:, pre:] = mask
        o = F.scaled_dot_product_attention(
            q.transpose(0, 1).unsqueeze(0), fk.transpose(0, 1).unsqueeze(0),
            fv.transpose(0, 1).unsqueeze(0), attn_mask=full[None, None], scale=hd ** -0.5,
            enable_gqa=True)
        return o.transpose(1, 2).contiguous().reshape(n, hq * hd)

    for _ in range(3):
        torch_composition()
    torch_ms = events_time_ms(torch_composition, 20)
    # CPU: the oracle (float32 restatement of gather + mask + SDPA) on the host
    kc_cpu, vc_cpu = kv.k.cpu(), kv.v.cpu()
    qc, kt, vt, mc = q.cpu(), k.cpu(), v.cpu(), mask.cpu()
    t0 = time.perf_counter()
    attn_ref.tree_attention(qc, kt, vt, kc_cpu, vc_cpu, 0, kv.block_table, seq, page, mc)
    cpu_ms = (time.perf_counter() - t0) * 1e3
    return {"us_device": round(dev_ms * 1e3, 2), "chunks": chunks.value,
            "gbs": round(bytes_alg / (dev_ms * 1e-3) / 1e9, 1),
            "pct_hbm_peak": round(100 * bytes_alg / (dev_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 2),
            "tflops": round(flops / (dev_ms * 1e-3) / 1e12, 2),
            "pct_mfma_peak": round(100 * flops / (dev_ms * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS,
                                   2),
            "bytes_alg": bytes_alg, "flops": flops,
            "us_torch_reference_composition": round(torch_ms * 1e3, 2),
            "cpu_oracle_ms": round(cpu_ms, 2), "cpu_threads": torch.get_num_threads()}


if __name__ == "__main__":
    main()
