#!/usr/bin/env python3
"""Prefill throughput of exact-max shared-selection thresholded attention on one MI355X.

A step is one pass of the whole prefill path over one attention layer of synthetic input
(config 1 of the benchmark table: 32 heads x d128 x 12288 tokens bf16, PI 4096 -> 12288,
tau 5, tile 64, top-30% with the 25/20% fallback under the 2048-key cap): RoPE pre-kernels,
pass 1 (exact row max), pass 2 (threshold + votes), LDS selection and the sparse
gather-attention, all through the C ABI with inputs already resident in HBM and outputs /
workspace allocated before the timed region.

Prints one JSON line (rank 0).  Only one GPU is supported: --gpus above 1 exits with a message.
Besides the throughput it reports per-stage times measured with HIP events recorded on the
launch stream inside the timed region, the roofline fraction of the dominant kernel, and the
CPU oracle timed on a bounded sample of the same workload.
"""
import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "sparse-thresholded-attention_amd")
for _p in (ROOT, PKG):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "prefill tokens/sec @32h x d128 x 12k bf16; % MFMA peak (score) / % HBM peak (gather)"
PEAK_BF16_TFLOPS = 2500.0      # MI355X dense bf16 MFMA
PEAK_FP32_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0          # MI355X HBM3E
STAGES = ["rope", "score", "select", "gather"]
STREAM_STAGES = ["rope", "score", "attend_rope", "stream"]
DCA_STAGES = ["rope", "attention"]
DECODE_STAGES = ["scores", "select", "attend"]
DECODE_METRIC = "decode tokens/sec (one attention layer, one new query per head over the KV cache)"


def parse():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="c1")
    ap.add_argument("--cpu-baseline-seconds", type=float, default=15.0,
                    help="target CPU time of the oracle sample (0 disables it)")
    ap.add_argument("--traffic-file", default=None,
                    help="summary of the rocprofv3 FETCH_SIZE/WRITE_SIZE runs, with one "
                         "'<kernel> traffic_bytes: <bytes per launch>' line per kernel "
                         "(default: profiles/prefill_<config>_hbm_traffic.md)")
    ap.add_argument("--stream-mode", default="auto", choices=["auto", "fused", "unfused"],
                    help="PQ Stream configs: the keep bits from a separate pass ('unfused'), "
                         "computed inside the sweep ('fused'), or chosen by the bit buffer's size")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only run a plain device-to-device copy of MIB MiB (3 times) and exit: "
                         "the known-size reference for the HBM byte counters")
    return ap.parse_args()


def calibrate_copy(mib):
    import torch
    n = mib * 1024 * 1024
    src = torch.ones(n, dtype=torch.uint8, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calibration_copy_bytes": n, "launches": 3}), flush=True)
    return 0


def gather_bytes(kept, k_max, D, esz, H, N):
    """Algorithmic bytes of the gather: every kept (tile, head) slot requests one K row and one V
    row plus its idx/newpos entries; Q is read and O written once."""
    slots = kept.clamp(max=k_max).to(torch.int64).sum().item()
    return slots * 2 * D * esz + slots * 8 + 2 * H * N * D * esz


def read_traffic(path, kernel):
    """HBM bytes per launch of `kernel` from the counter summary (None when not measured)."""
    if not path or not os.path.exists(path):
        return None
    key = f"{kernel} traffic_bytes:"
    for line in open(path):
        line = line.strip().strip("`")
        if line.startswith(key):
            return float(line[len(key):].split()[0])
    return None


def cpu_model():
    """The host CPU's model name (first /proc/cpuinfo entry), or the platform string."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or platform.machine()


def with_traffic(roof, stage_ms):
    """Add the measured-traffic rate beside the algorithmic one: the counter bytes of one launch
    (rocprofv3 FETCH_SIZE + WRITE_SIZE, from the traffic file) over the stage time."""
    if roof.get("traffic"):
        gbs = roof["traffic"] / (stage_ms * 1e-3) / 1e9
        roof["traffic_gbs"] = round(gbs, 1)
        roof["traffic_frac_of_hbm"] = round(gbs / PEAK_HBM_GBS, 4)
    return roof


def cpu_baseline(cfg, q, k, v, invf, ps, rs, budget_s):
    """The oracle (C port of the reference's three stages) on whole heads of the same workload."""
    import numpy as np
    from oracle import sta_oracle as orc
    sm = 1.0 / math.sqrt(cfg.D)
    threads = orc.num_threads()
    stage_s = {}

    def timed(name, fn, *args, **kw):
        t1 = time.perf_counter()
        out = fn(*args, **kw)
        stage_s[name] = stage_s.get(name, 0.0) + time.perf_counter() - t1
        return out

    def one(h):
        qn, dt = orc.from_torch(q[0, h:h + 1])
        kn, _ = orc.from_torch(k[0, h // (cfg.H // cfg.Hkv):h // (cfg.H // cfg.Hkv) + 1])
        vn, _ = orc.from_torch(v[0, h // (cfg.H // cfg.Hkv):h // (cfg.H // cfg.Hkv) + 1])
        tau = np.full(1, cfg.tau, np.float32)
        t0 = time.perf_counter()
        if cfg.variant == "dca":
            # per-row cost from two evenly spaced row samples (64 and 128 rows); the key rotation
            # both pay is counted once
            t = []
            for n in (64, 128):
                rows = np.linspace(0, cfg.N - 1, n).astype(np.int32)
                t1 = time.perf_counter()
                orc.dca_attention(qn, kn, vn, dt, invf.numpy(), cfg.dca[0], cfg.dca[1], cfg.dca[2], rows=rows)
                t.append(time.perf_counter() - t1)
            per_row = max(t[1] - t[0], 1e-9) / 64
            return max(t[0] - 64 * per_row, 0.0) + per_row * cfg.N
        if cfg.variant == "pqstream":
            orc.pqstream(qn, kn, vn, dt, tau, invf.numpy(), invf.numpy(), ps, rs, sm, cfg.n_global,
                         cfg.n_local, cfg.tile, 32, "max", True, want_band=False)
        elif cfg.variant == "pq":
            wm = orc.WMODES[cfg.select_score]
            a = timed("kernel_a", orc.select_bits, qn, kn, dt, tau, invf.numpy(), ps, rs, sm, cfg.tile, 0, wm)
            s = timed("build_sets", orc.build_sets_pq, a["votes"], a["bits"], a["wvotes"], cfg.n_global, cfg.n_local,
                      cfg.tile, cfg.k_max, 0, wm)
            timed("kernel_c", orc.gather_attn_mask, qn, kn, vn, dt, s[0], s[1], s[2], s[3], invf.numpy(), 1.0, sm,
                  cfg.tile, cfg.k_max)
        else:
            a = timed("kernel_a", orc.select_vote, qn, kn, dt, tau, invf.numpy(), ps, rs, sm, cfg.tile,
                      wmode=orc.WMODES[cfg.select_score])
            s = timed("build_sets", orc.build_sets, a["votes"], ps, cfg.n_global, cfg.n_local, cfg.pct, cfg.tile,
                      cfg.k_max, wvotes=a.get("wvotes"))
            timed("kernel_c", orc.gather_attn, qn, kn, vn, dt, s[0], s[1], s[2], invf.numpy(), rs, sm, cfg.tile,
                  cfg.k_max)
        return time.perf_counter() - t0

    t_first = one(0)
    heads = max(1, min(cfg.H, int(budget_s / max(t_first, 1e-3))))
    total = t_first + sum(one(h) for h in range(1, heads))
    per_head = total / heads
    stages = {"pq": "Kernel A + _build_sets_pq + masked Kernel C",
              "pqstream": "the fused PQ Stream kernel",
              "dca": "the DCA prefill on 64 and 128 evenly spaced query rows, scaled to all rows"}.get(
                  cfg.variant, "Kernel A + _build_sets + Kernel C")
    out = {"value": round(cfg.N / (per_head * cfg.H), 3), "unit": "tokens/s", "cores": threads,
           "kind": "port",
           "sample": f"{heads} of {cfg.H} heads of the same workload through the CPU oracle "
                     f"({stages}, {threads} OpenMP threads), scaled x{cfg.H / heads:g}",
           "cpu_model": cpu_model()}
    if stage_s:
        # seconds per step (all heads) of each reference stage, from the sampled heads
        out["stage_seconds_per_step"] = {n: round(t / heads * cfg.H, 3) for n, t in stage_s.items()}
    return out


def bench_decode(args, cfg, q, k, v, q_cpu, k_cpu, v_cpu, invf, ps, rs, tau):
    """Decode steps: the last decode_q positions query the cache of N keys (scores, selection,
    attend).  ms_per_step is the wall clock per step, launches included."""
    import _sta_native as native
    Q, N = cfg.decode_q, cfg.N
    dev = q.device
    qd = q[0, :, N - Q:, :].contiguous()
    plan = native.DecodePlan(qd, k, v, tau, invf, N - Q, ps, rs, None, cfg.n_global, cfg.n_local, cfg.k_max,
                             cfg.pct_decode)
    stream = torch.cuda.current_stream(dev)
    for _ in range(args.warmup):
        plan.run()
    torch.cuda.synchronize()
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(len(DECODE_STAGES) + 1)] for _ in range(args.steps)]
    for row in evs:
        for e in row:
            e.record(stream)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        plan.run(evs[i])
    torch.cuda.synchronize()
    ms_per_step = (time.perf_counter() - t0) * 1000.0 / args.steps
    stage_ms = {s: sum(evs[i][j].elapsed_time(evs[i][j + 1]) for i in range(args.steps)) / args.steps
                for j, s in enumerate(DECODE_STAGES)}
    r = plan.out
    esz = q.element_size()
    # scores: the cache's keys once per kv head, the scores written once
    sbytes = cfg.Hkv * N * cfg.D * esz + cfg.H * Q * N * 4
    kept = r["set_size"].clamp(max=cfg.k_max)
    abytes = int(kept.sum().item()) * (2 * cfg.D * esz + 8) + 2 * cfg.H * Q * cfg.D * esz
    roof = {}
    for name, kern, b in (("scores", "decode_score_kernel", sbytes), ("attend", "decode_attend_kernel", abytes)):
        gbs = b / (stage_ms[name] * 1e-3) / 1e9
        roof[name] = {"kernel": kern, "bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS,
                      "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4), "algorithmic_per_launch": int(b),
                      "traffic": read_traffic(args.traffic_file, kern)}
    dominant = roof["scores"] if stage_ms["scores"] >= stage_ms["attend"] else roof["attend"]
    print(f"[bench] {ms_per_step:.4f} ms/step; stages {stage_ms}", file=sys.stderr, flush=True)
    cpu = None
    if args.cpu_baseline_seconds > 0:
        cpu = cpu_baseline_decode(cfg, q_cpu, k_cpu, v_cpu, invf, ps, rs, args.cpu_baseline_seconds)
    line = {
        "metric": DECODE_METRIC,
        "value": round(Q / (ms_per_step * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {torch.bfloat16: "bf16", torch.float16: "fp16", torch.float32: "fp32"}[q.dtype],
        "data": "synthetic (seeded Gaussian Q/K/V with planted keys)",
        "config": {"workload": cfg.name, "variant": "decode", "heads": cfg.H, "kv_heads": cfg.Hkv,
                   "cache_len": N, "queries": Q, "head_dim": cfg.D, "tau": cfg.tau, "k_max": cfg.k_max,
                   "pct_decode": cfg.pct_decode, "pos_scale": ps, "rope_scale": rs,
                   "parallelism": "none (1 GPU)"},
        "stages_ms": {s: round(t, 5) for s, t in stage_ms.items()},
        "gpu_ms_per_step": round(sum(stage_ms.values()), 5),
        "roofline": dominant,
        "rooflines": roof,
        "selection": {"set_size_mean": round(r["set_size"].float().mean().item(), 1),
                      "capped": int((r["set_size"] > cfg.k_max).sum().item()), "queries": int(kept.numel())},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


def bench_perquery(args, cfg, q, k, v, q_cpu, k_cpu, v_cpu, invf, ps, rs, tau):
    """Config 3 as written: every prompt position selects its own keys (threshold passers plus the
    forced keys, capped at k_max by score, dense-rank positions) and attends them -- the per-query
    rule of perquery.py:651-720 at every position (prefill_mode="perquery", :905-924).  Stages are
    summed over the head groups of the plan."""
    import _sta_native as native
    plan = native.PerQueryPrefillPlan(q, k, v, tau, invf.to(q.device), invf.to(q.device), ps, rs,
                                      n_global=cfg.n_global, n_local=cfg.n_local, k_max=cfg.k_max)
    stream = torch.cuda.current_stream(q.device)
    for _ in range(args.warmup):
        plan.run()
    torch.cuda.synchronize()
    print(f"[bench] warmup done ({args.warmup} steps, {len(plan.plans)} head groups), timing {args.steps} steps",
          file=sys.stderr, flush=True)
    ng = len(plan.plans)
    evs = [[[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(ng)] for _ in range(args.steps)]
    for step in evs:
        for grp in step:
            for e in grp:
                e.record(stream)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        plan.run(evs[i])
    torch.cuda.synchronize()
    ms_per_step = (time.perf_counter() - t0) * 1000.0 / args.steps
    stage_ms = {s: sum(evs[i][g][j].elapsed_time(evs[i][g][j + 1]) for i in range(args.steps) for g in range(ng))
                / args.steps for j, s in enumerate(DECODE_STAGES)}
    r = plan.out
    esz = q.element_size()
    # scores: the fp32 score rows written (4 B per causal (query, key) pair); select: those rows
    # read and the k_max index slots of every query written; attend: each query's kept K and V
    # rows plus its index per slot, the query read and the output written.  The attend's rows
    # come mostly from L2 (neighbouring queries of a head share the cache rows), so its roofline
    # is the HBM traffic the counters measure (the traffic file holds each kernel's bytes per
    # step, summed over the plan's launches), not the algorithmic bytes, which exceed what HBM
    # could deliver.
    sbytes = 4 * cfg.H * cfg.N * (cfg.N + 1) // 2
    selbytes = sbytes + 4 * cfg.k_max * cfg.H * cfg.N
    kept = r["set_size"].clamp(max=cfg.k_max).to(torch.int64)
    abytes = int(kept.sum().item()) * (2 * cfg.D * esz + 4) + 2 * cfg.H * cfg.N * cfg.D * esz

    def hbm_roof(kernel, algo, ms, note):
        traffic = read_traffic(args.traffic_file, kernel)
        d = {"kernel": kernel, "bound": "hbm", "peak": PEAK_HBM_GBS, "unit": "GB/s",
             "algorithmic_per_step": algo, "algorithmic_gbs": round(algo / (ms * 1e-3) / 1e9, 1),
             "traffic": traffic, "note": note}
        if traffic:
            gbs = traffic / (ms * 1e-3) / 1e9
            d.update({"achieved": round(gbs, 1), "frac": round(gbs / PEAK_HBM_GBS, 4), "basis": "counter traffic"})
        else:
            gbs = algo / (ms * 1e-3) / 1e9
            d.update({"achieved": round(gbs, 1), "frac": round(gbs / PEAK_HBM_GBS, 4), "basis": "algorithmic"})
        return d

    roof = {
        "scores": hbm_roof("score_rows_kernel", sbytes, stage_ms["scores"],
                           "the fp32 score rows of every (query, key) pair are written once, in 64-row tiles, "
                           "and read by the selection"),
        "select": hbm_roof("decode_select_pq_reg_kernel", selbytes, stage_ms["select"],
                           "one pass over each score row held in registers; the vector ALU (68% busy) "
                           "bounds it, not HBM"),
        "attend": hbm_roof("decode_attend_grouped_kernel", abytes, stage_ms["attend"],
                           "each query gathers its own K / V rows, served mostly from L2; the counters put the "
                           "vector memory data path at 92% busy, which bounds it, and the vector ALU at 79%"),
    }
    dominant = max(("scores", "select", "attend"), key=lambda n: stage_ms[n])
    print(f"[bench] {ms_per_step:.3f} ms/step; stages {stage_ms}", file=sys.stderr, flush=True)
    cpu = None
    if args.cpu_baseline_seconds > 0:
        print("[bench] timing the CPU oracle sample", file=sys.stderr, flush=True)
        cpu = cpu_baseline_perquery(cfg, q_cpu, k_cpu, v_cpu, invf, ps, rs, args.cpu_baseline_seconds)
    line = {
        "metric": METRIC,
        "value": round(cfg.N / (ms_per_step * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {torch.bfloat16: "bf16", torch.float16: "fp16", torch.float32: "fp32"}[q.dtype],
        "data": "synthetic (seeded Gaussian Q/K/V with planted keys)",
        "config": {"workload": cfg.name, "variant": cfg.variant, "heads": cfg.H, "kv_heads": cfg.Hkv,
                   "seq_len": cfg.N, "head_dim": cfg.D, "tau": cfg.tau, "k_max": cfg.k_max,
                   "rule": "per-query threshold + forced keys, capped at k_max by score, dense ranks",
                   "head_groups": ng, "pos_scale": ps, "rope_scale": rs, "parallelism": "none (1 GPU)"},
        "stages_ms": {s: round(t, 4) for s, t in stage_ms.items()},
        "roofline": roof[dominant],
        "rooflines": roof,
        "selection": {"set_size_mean": round(r["set_size"].float().mean().item(), 1),
                      "capped_queries": int(r["overflow"].sum().item()), "queries": int(r["overflow"].numel()),
                      "usize_mean": round(r["usize"].float().mean().item(), 1)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


DCA_SELECT_STAGES = ["rope", "votes", "select", "attention"]


def bench_dca_select(args, cfg, q, k, v, q_cpu, k_cpu, v_cpu, invf, tau):
    """Config 4: DCA positions with exact-max selection over each 64-query tile's inter-chunk keys
    (two score passes of one product per pair), the tile selection, then the attention over the
    selected inter keys plus the dense local keys."""
    import _sta_native as native
    s, c, w = cfg.dca
    plan = native.DcaPlan(q, k, v, invf, s, c, w, None, tau, cfg.pct, cfg.k_max, cfg.n_global)
    stream = torch.cuda.current_stream(q.device)
    for _ in range(args.warmup):
        plan.run()
    torch.cuda.synchronize()
    print(f"[bench] warmup done ({args.warmup} steps), timing {args.steps} steps", file=sys.stderr, flush=True)
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(5)] for _ in range(args.steps)]
    for row in evs:
        for e in row:
            e.record(stream)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        plan.run(evs[i])
    torch.cuda.synchronize()
    ms_per_step = (time.perf_counter() - t0) * 1000.0 / args.steps
    stage_ms = {st: sum(evs[i][j].elapsed_time(evs[i][j + 1]) for i in range(args.steps)) / args.steps
                for j, st in enumerate(DCA_SELECT_STAGES)}
    r = plan.out
    L = s - w
    N, D, H = cfg.N, cfg.D, cfg.H
    rows = torch.arange(N, dtype=torch.int64)
    chunk = rows // L
    ext = torch.where(chunk >= 2, (chunk - 1) * L, torch.zeros_like(chunk))   # inter keys per row
    local = rows + 1 - ext                                                     # dense local keys per row
    inter_pairs = int(ext.sum().item()) * H
    # votes: pass 1 (row max) and pass 2 (threshold) over the inter pairs, one product each
    vflops = 2 * 2 * D * inter_pairs
    nsel = r["kept_size"].clamp(max=cfg.k_max).to(torch.int64).cpu()          # (H, nt)
    sel_rows = nsel.repeat_interleave(64, dim=1)[:, :N].sum().item()
    aflops = 2 * 2 * D * (int(sel_rows) + H * int(local.sum().item()))       # QK^T and PV
    peak = PEAK_FP32_TFLOPS if q.dtype == torch.float32 else PEAK_BF16_TFLOPS
    v_tf = vflops / (stage_ms["votes"] * 1e-3) / 1e12
    a_tf = aflops / (stage_ms["attention"] * 1e-3) / 1e12
    roof = {
        "votes": {"kernel": "dca_vote_kernel", "bound": "mfma", "achieved": round(v_tf, 2), "peak": peak,
                  "unit": "TFLOP/s", "frac": round(v_tf / peak, 4), "algorithmic_per_launch": vflops,
                  "traffic": read_traffic(args.traffic_file, "dca_vote_kernel")},
        "attention": {"kernel": "dca_attn_kernel", "bound": "mfma", "achieved": round(a_tf, 2), "peak": peak,
                      "unit": "TFLOP/s", "frac": round(a_tf / peak, 4), "algorithmic_per_launch": aflops,
                      "traffic": read_traffic(args.traffic_file, "dca_attn_kernel")},
    }
    dominant = roof["votes"] if stage_ms["votes"] >= stage_ms["attention"] else roof["attention"]
    print(f"[bench] {ms_per_step:.3f} ms/step; stages {stage_ms}", file=sys.stderr, flush=True)
    cpu = None
    if args.cpu_baseline_seconds > 0:
        print("[bench] timing the CPU oracle sample", file=sys.stderr, flush=True)
        cpu = cpu_baseline_dca_select(cfg, q_cpu, k_cpu, v_cpu, invf, args.cpu_baseline_seconds)
    line = {
        "metric": METRIC,
        "value": round(N / (ms_per_step * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {torch.bfloat16: "bf16", torch.float16: "fp16", torch.float32: "fp32"}[q.dtype],
        "data": "synthetic (seeded Gaussian Q/K/V with planted keys)",
        "config": {"workload": cfg.name, "variant": cfg.variant, "heads": H, "kv_heads": cfg.Hkv, "seq_len": N,
                   "head_dim": D, "tile": 64, "tau": cfg.tau, "pct": cfg.pct, "k_max": cfg.k_max,
                   "dca_chunk_pretrain_local": cfg.dca, "parallelism": "none (1 GPU)"},
        "stages_ms": {st: round(t, 4) for st, t in stage_ms.items()},
        "roofline": dominant,
        "rooflines": roof,
        "selection": {"kept_mean": round(r["kept_size"].float().mean().item(), 1),
                      "overflow20_tiles": int(r["overflow20"].sum().item()), "tiles": int(r["kept_size"].numel()),
                      "inter_pairs": inter_pairs},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


def cpu_baseline_dca_select(cfg, q, k, v, invf, budget_s):
    """The config-4 oracle on whole heads of a shorter prefix (votes, selection, attention), timed
    per head at two lengths and scaled quadratically to the full length."""
    import numpy as np
    from oracle import sta_oracle as orc
    s, c, w = cfg.dca
    threads = orc.num_threads()
    t = {}
    for n in (8192, 16384):
        qn, dt = orc.from_torch(q[0, :1, :n])
        kn, _ = orc.from_torch(k[0, :1, :n])
        vn, _ = orc.from_torch(v[0, :1, :n])
        t0 = time.perf_counter()
        orc.dca_select_attention(qn, kn, vn, dt, invf.numpy(), s, c, w, np.full(1, cfg.tau, np.float32), cfg.pct,
                                 cfg.k_max, cfg.n_global)
        t[n] = time.perf_counter() - t0
    # quadratic in the length: scale the longer sample
    per_head = t[16384] * (cfg.N / 16384) ** 2
    return {"value": round(cfg.N / (per_head * cfg.H), 3), "unit": "tokens/s", "cores": threads, "kind": "port",
            "cpu_model": cpu_model(),
            "sample": f"one head at 8192 and 16384 tokens through the CPU oracle (inter votes, selection, "
                      f"attention; {threads} OpenMP threads), the 16384-token time scaled by (N / 16384)^2 to "
                      f"{cfg.N} tokens and by {cfg.H} heads"}


def cpu_baseline_perquery(cfg, q, k, v, invf, ps, rs, budget_s):
    """The oracle's per-query rule (scores, _decode_build_sets_pq, attend) on evenly spaced query
    rows of one head at a time, scaled to every row of every head by the causal key count."""
    import numpy as np
    from oracle import sta_oracle as orc
    sm = 1.0 / math.sqrt(cfg.D)
    threads = orc.num_threads()
    N = cfg.N
    rows_done, keys_done, t_total, heads = 0, 0, 0.0, 0
    while t_total < budget_s and heads < cfg.H:
        h = heads
        hk = h // (cfg.H // cfg.Hkv)
        rows = np.linspace(0, N - 1, 64).astype(np.int64)
        kn, dt = orc.from_torch(k[0, hk:hk + 1])
        vn, _ = orc.from_torch(v[0, hk:hk + 1])
        t0 = time.perf_counter()
        for r in rows:
            qn, _ = orc.from_torch(q[0, h:h + 1, r:r + 1])
            s = orc.decode_scores(qn, kn[:, :r + 1], dt, invf.numpy(), ps, rs, sm, int(r))
            idx, npk, npq, *_ = orc.decode_build_sets_pq(s, np.full(1, cfg.tau, np.float32), int(r), cfg.n_global,
                                                         cfg.n_local, cfg.k_max)
            orc.decode_attend(qn, kn[:, :r + 1], vn[:, :r + 1], dt, invf.numpy(), 1.0, sm, int(r), idx, npk, npq)
        t_total += time.perf_counter() - t0
        rows_done += len(rows)
        keys_done += int((rows + 1).sum())
        heads += 1
    per_key = t_total / keys_done
    total = per_key * cfg.H * N * (N + 1) / 2
    return {"value": round(N / total, 3), "unit": "tokens/s", "cores": threads, "kind": "port",
            "cpu_model": cpu_model(),
            "sample": f"{rows_done} query rows ({heads} heads x 64 evenly spaced positions) through the CPU "
                      f"oracle's scores, per-query selection and attend ({threads} OpenMP threads), scaled "
                      f"to all {cfg.H} x {N} rows by their causal key counts"}


def cpu_baseline_decode(cfg, q, k, v, invf, ps, rs, budget_s):
    """The oracle's decode (scores, selection, attend) for one query per head, all heads."""
    import numpy as np
    from oracle import sta_oracle as orc
    sm = 1.0 / math.sqrt(cfg.D)
    Q, N = cfg.decode_q, cfg.N
    qn, dt = orc.from_torch(q[0, :, N - Q:, :])
    kn, _ = orc.from_torch(k[0])
    vn, _ = orc.from_torch(v[0])
    tau = np.full(cfg.H, cfg.tau, np.float32)
    steps, t0 = 0, time.perf_counter()
    while True:
        s = orc.decode_scores(qn, kn, dt, invf.numpy(), ps, rs, sm, N - Q)
        idx, npk, npq, _ = orc.decode_build_sets(s, tau, N - Q, ps, cfg.n_global, cfg.n_local, cfg.k_max,
                                                 cfg.pct_decode)
        orc.decode_attend(qn, kn, vn, dt, invf.numpy(), rs, sm, N - Q, idx, npk, npq)
        steps += 1
        el = time.perf_counter() - t0
        if el >= budget_s or steps >= 50:
            break
    threads = orc.num_threads()
    return {"value": round(Q * steps / el, 3), "unit": "tokens/s", "cores": threads, "kind": "port",
            "cpu_model": cpu_model(),
            "sample": f"{steps} decode steps of the same workload (all {cfg.H} heads) through the CPU "
                      f"oracle's scores, selection and attend ({threads} OpenMP threads)"}


def main():
    args = parse()
    if args.calibrate_copy:
        return calibrate_copy(args.calibrate_copy)
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE {world}); "
              "heads would shard across GPUs with no exchange, which is not built here.",
              file=sys.stderr)
        return 2
    global torch
    import torch
    import _sta_native as native
    from synthetic import CONFIGS

    cfg = CONFIGS[args.config]
    if args.traffic_file is None:
        args.traffic_file = os.path.join(ROOT, "profiles", f"prefill_{args.config}_hbm_traffic.md")
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    q_cpu, k_cpu, v_cpu = cfg.inputs("cpu")
    q, k, v = q_cpu.to(dev), k_cpu.to(dev), v_cpu.to(dev)
    invf, ps, rs = cfg.geometry()
    tau = torch.full((cfg.H,), cfg.tau)
    if cfg.variant == "decode":
        return bench_decode(args, cfg, q, k, v, q_cpu, k_cpu, v_cpu, invf, ps, rs, tau)
    if cfg.variant == "perquery":
        return bench_perquery(args, cfg, q, k, v, q_cpu, k_cpu, v_cpu, invf, ps, rs, tau)
    if cfg.variant == "dca_select":
        return bench_dca_select(args, cfg, q, k, v, q_cpu, k_cpu, v_cpu, invf, tau)
    if cfg.variant == "dca":
        plan = native.DcaPlan(q, k, v, invf, cfg.dca[0], cfg.dca[1], cfg.dca[2])
    elif cfg.variant == "pqstream":
        plan = native.StreamPlan(q, k, v, tau, invf, invf, ps, rs, tile=cfg.tile, block_n=32,
                                 n_global=cfg.n_global, n_local=cfg.n_local, fused=args.stream_mode)
    elif cfg.variant == "pq":
        plan = native.PqPlan(q, k, v, tau, invf, invf, ps, rs, tile=cfg.tile, k_max=cfg.k_max,
                             n_global=cfg.n_global, n_local=cfg.n_local, select_score=cfg.select_score)
    else:
        plan = native.SharedPlan(q, k, v, tau, invf, ps, rs, invf, ps, rs, pct=cfg.pct, tile=cfg.tile,
                                 k_max=cfg.k_max, n_global=cfg.n_global, n_local=cfg.n_local,
                                 select_score=cfg.select_score)
    stream = torch.cuda.current_stream(dev)
    for _ in range(args.warmup):
        plan.run()
    torch.cuda.synchronize()
    print(f"[bench] warmup done ({args.warmup} steps), timing {args.steps} steps", file=sys.stderr, flush=True)

    stages = {"pqstream": STREAM_STAGES, "dca": DCA_STAGES}.get(cfg.variant, STAGES)
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(len(stages) + 1)] for _ in range(args.steps)]
    for row in evs:                      # materialise the event handles outside the timed region
        for e in row:
            e.record(stream)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        plan.run(evs[i])
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_per_step = elapsed * 1000.0 / args.steps
    stage_ms = {s: sum(evs[i][j].elapsed_time(evs[i][j + 1]) for i in range(args.steps)) / args.steps
                for j, s in enumerate(stages)}
    r = plan.out
    esz = q.element_size()
    peak_tf = PEAK_FP32_TFLOPS if q.dtype == torch.float32 else PEAK_BF16_TFLOPS
    if cfg.variant != "dca":
        score_tf = cfg.score_flops() / (stage_ms["score"] * 1e-3) / 1e12
        roof_score = {"kernel": "score_kernel", "bound": "mfma", "achieved": round(score_tf, 2),
                      "peak": peak_tf, "unit": "TFLOP/s", "frac": round(score_tf / peak_tf, 4),
                      "algorithmic_per_launch": cfg.score_flops(),
                      "traffic": read_traffic(args.traffic_file, "score_kernel")}
    if cfg.variant == "dca":
        # dense: Q.K^T and P.V over the causal pairs; no selection passes
        sflops = 2 * 2 * cfg.D * cfg.H * cfg.N * (cfg.N + 1) // 2
        attn_tf = sflops / (stage_ms["attention"] * 1e-3) / 1e12
        roof_score = {"kernel": "dca_attn_kernel", "bound": "mfma", "achieved": round(attn_tf, 2),
                      "peak": peak_tf, "unit": "TFLOP/s", "frac": round(attn_tf / peak_tf, 4),
                      "algorithmic_per_launch": sflops,
                      "traffic": read_traffic(args.traffic_file, "dca_attn_kernel")}
        roof_second = None
        second = None
        selection = None
    elif cfg.variant == "pqstream":
        # the sweep's products: Q.K^T and P.V over the causal pairs
        sflops = 2 * 2 * cfg.D * cfg.H * cfg.N * (cfg.N + 1) // 2
        stream_tf = sflops / (stage_ms["stream"] * 1e-3) / 1e12
        roof_second = {"kernel": "stream_kernel", "bound": "mfma", "achieved": round(stream_tf, 2),
                       "peak": peak_tf, "unit": "TFLOP/s", "frac": round(stream_tf / peak_tf, 4),
                       "algorithmic_per_launch": sflops,
                       "traffic": read_traffic(args.traffic_file, "stream_kernel")}
        second = "stream"
        kept = r["kept"]
        selection = {"kept_per_query_mean": round(kept.float().mean().item(), 1),
                     "span_max": float(r["span"].max().item()),
                     "skipped_blocks": int(r["skipped"].sum().item()),
                     "blocks": int(r["blocks"].sum().item())}
    else:
        kept = r["kept_size"]
        gbytes = gather_bytes(kept, cfg.k_max, cfg.D, esz, cfg.H, cfg.N)
        gather_gbs = gbytes / (stage_ms["gather"] * 1e-3) / 1e9
        roof_second = {"kernel": "gather_kernel", "bound": "hbm", "achieved": round(gather_gbs, 1),
                       "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(gather_gbs / PEAK_HBM_GBS, 4),
                       "algorithmic_per_launch": int(gbytes),
                       "traffic": read_traffic(args.traffic_file, "gather_kernel")}
        second = "gather"
        if cfg.variant == "pq":
            selection = {"kept_mean": round(kept.float().mean().item(), 1),
                         "overflow_tiles": int(r["overflow"].sum().item()), "tiles": int(kept.numel())}
        else:
            selection = {"kept_mean": round(kept.float().mean().item(), 1),
                         "overflow20_tiles": int(r["overflow20"].sum().item()), "tiles": int(kept.numel())}
    if cfg.variant == "dca":
        with_traffic(roof_score, stage_ms["attention"])
    else:
        with_traffic(roof_score, stage_ms["score"])
    if second is not None:
        with_traffic(roof_second, stage_ms[second])
    if second is None:
        dominant = roof_score
    else:
        dominant = roof_score if stage_ms["score"] >= stage_ms[second] else roof_second
    print(f"[bench] {ms_per_step:.3f} ms/step; stages {stage_ms}", file=sys.stderr, flush=True)

    cpu = None
    if args.cpu_baseline_seconds > 0:
        print("[bench] timing the CPU oracle sample", file=sys.stderr, flush=True)
        cpu = cpu_baseline(cfg, q_cpu, k_cpu, v_cpu, invf, ps, rs, args.cpu_baseline_seconds)

    line = {
        "metric": METRIC,
        "value": round(cfg.N / (ms_per_step * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {torch.bfloat16: "bf16", torch.float16: "fp16", torch.float32: "fp32"}[q.dtype],
        "data": "synthetic (seeded Gaussian Q/K/V with planted keys)",
        "config": {"workload": cfg.name, "variant": cfg.variant, "heads": cfg.H, "kv_heads": cfg.Hkv,
                   "seq_len": cfg.N, "head_dim": cfg.D, "tile": cfg.tile, "tau": cfg.tau,
                   "pct": cfg.pct if cfg.variant == "shared" else None,
                   "select_score": cfg.select_score,
                   "k_max": cfg.k_max if cfg.variant in ("shared", "pq") else None,
                   "dca_chunk_pretrain_local": cfg.dca,
                   "stream_mode": args.stream_mode if cfg.variant == "pqstream" else None,
                   "pos_scale": ps, "rope_scale": rs, "parallelism": "none (1 GPU)"},
        "stages_ms": {s: round(t, 4) for s, t in stage_ms.items()},
        "roofline": dominant,
        "rooflines": ({"attention": roof_score} if second is None else {"score": roof_score, second: roof_second}),
        "selection": selection,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
