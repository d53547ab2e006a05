#!/usr/bin/env python3
"""Benchmark of the EXL3 quantized MoE expert path on one MI355X.

One step = one MoE layer forward (route, group, gate/up, SiLU * up, down, combine) over
one fresh batch of synthetic rows, inputs already resident in HBM.

Headline workload: 512-expert top-10 MoE layer, hidden 2048, expert
intermediate 512, one shared expert, all EXL3 4.0 bpw; 8 ragged sessions of 1..5 rows
per step (decode).  Weights are read cold: steps rotate over several seeded layers
(> 2 GiB together, far above the 256 MB Infinity Cache) and every step routes fresh
logits.  Secondary objects in the same line: the 2048-token Zipf-skewed prefill
(config 4), the ragged EXL3 linear GEMVs (config 2, rotating over 128 seeded weight pairs),
the 8192-token mixed-rate prefill and 6-bpw output head (config 5), and the measured HBM
stream rate of a 2 GiB device copy.

Prints ONE JSON line (rank 0).  `value` is decode tokens/s (rows/s through the layer).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "crucible-strix-halo_amd"))

HBM_PEAK_GBS = 8000.0     # MI355X HBM3E, published
MFMA_F16_PEAK_TFS = 2500.0  # MI355X dense fp16 MFMA, published (no sparsity)

E, H, IE, TOPK = 512, 2048, 512, 10


STAGE_KERNEL = "Exl3DecodeStageKernel<8, 8, 2>"  # gate/up + mid + down of a decode call in one launch (4.0 bpw, mul1)


def uses_stage(M):
    """Whether the library runs a config-3 decode call of M rows as one stage launch (gate/up,
    mid and down): M (topk + 1) above 128 (below, the down GEMM computes the mid in its
    prologue), M <= 64, and CX_STAGE not 0 (csrc/moe.hip PlanMoe)."""
    return os.environ.get("CX_STAGE", "1") != "0" and M * (TOPK + 1) > 128 and M <= 64
# The prefill GEMM instantiations this build launches: (profile entry, kernel) per stage.
PREFILL_KERNELS = {
    "config4": {"gate_up": ("config 4 gate/up + fused mid", "Exl3GemmPrefillKernel<8, 2, 4, 1, 4, true>"),
                "down": ("config 4 down", "Exl3GemmPrefillKernel<8, 2, 4, 1, 4, false>")},
    "config5": {"gate_up": ("config 5 gate/up (3 bpw)", "Exl3GemmTallKernel<6, 2, 3>"),
                "down": ("config 5 down (5 bpw)", "Exl3GemmTallKernel<10, 2, 3>")},
}


def prefill_traffic(config, stage_us):
    """HBM bytes per launch of a prefill workload's two GEMMs (FETCH_SIZE + WRITE_SIZE) from
    the committed counter profile of the same workload, each beside the rate it implies at
    this run's stage time; None for a stage whose profiled kernel is not the one this build
    launches (counter collection needs its own rocprofv3 run)."""
    f = ROOT / "profiles" / "traffic_prefill_gemms_config4_config5.json"
    try:
        prof = json.loads(f.read_text())
    except Exception:
        return None
    out = {}
    for stage, (entry, kernel) in PREFILL_KERNELS[config].items():
        k = prof.get("kernels", {}).get(entry, {})
        if k.get("kernel") != kernel:
            out[stage] = None
            continue
        b = int(k["hbm_fetch_bytes_per_launch"]) + int(k["hbm_write_bytes_per_launch"])
        out[stage] = {"kernel": kernel, "hbm_bytes_per_launch": b,
                      "GBps_at_stage_time": round(b / (stage_us[stage] * 1e-6) / 1e9, 1)}
    out["source"] = {"file": "profiles/traffic_prefill_gemms_config4_config5.json", "command": prof.get("command")}
    return out


def matrix_bytes(i, o, k2):
    return i * o * k2 // 16 + 2 * i + 2 * o


def expert_bytes(k2_gu, k2_d):
    return 2 * matrix_bytes(H, IE, k2_gu) + matrix_bytes(IE, H, k2_d)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--layers", type=int, default=3, help="seeded layers the steps rotate over (cold reads)")
    ap.add_argument("--prefill-steps", type=int, default=6)
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-linear", action="store_true", help="skip the config-2 ragged linear measurement")
    ap.add_argument("--no-long", action="store_true", help="skip the config-5 long prefill + output head")
    ap.add_argument("--no-r1", action="store_true", help="skip the R = 1 decode latency measurement")
    ap.add_argument("--no-router", action="store_true", help="skip the router GEMV measurement")
    ap.add_argument("--no-stream", action="store_true", help="skip the device-copy HBM stream measurement")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--min-warmup-s", type=float, default=0.5,
                    help="the untimed warmup also runs until this much wall time has passed (GPU clocks settle)")
    ap.add_argument("--seed", type=int, default=2024)
    ap.add_argument("--host-data", action="store_true",
                    help="generate the layers with numpy on the host (no torch kernels in the process)")
    ap.add_argument("--calibrate-copy-mib", type=int, default=0,
                    help="before the timed region, one device-to-device copy of this many MiB "
                         "(the reference kernel for scaling HBM byte counters)")
    return ap.parse_args()


def make_batches(n, seed, prefill=False):
    import numpy as np
    import torch
    from exl3moe import synth
    rng = np.random.default_rng(seed)
    out = []
    bias = synth.zipf_bias(rng, E) if prefill else None
    for _ in range(n):
        if prefill:
            offs = [0, 2048]
        else:
            offs = synth.sessions(rng, 8, 1, 5)
        M = offs[-1]
        x = torch.from_numpy(rng.standard_normal((M, H)).astype(np.float16)).cuda()
        lg = rng.standard_normal((M, E + 1)).astype(np.float32)
        if bias is not None:
            lg[:, :E] += bias
        out.append((offs, x, torch.from_numpy(lg).cuda()))
    return out


def run_workload(plans, batches, warmup, steps, mode, min_warm_s=0.0):
    """Times `steps` layer calls after `warmup` untimed calls (no instrumentation in the
    timed loop), then repeats the same calls with the library's stage events to get
    per-stage times.  The warmup also continues until `min_warm_s` seconds of calls have
    run: the GPU's clocks take a few hundred milliseconds of sustained load to settle, and
    a handful of 0.1 ms steps would time the ramp instead of the steady state."""
    import torch
    from exl3moe.trace import StageTrace
    maxM = max(b[0][-1] for b in batches)
    ws = torch.empty(max(p.workspace_size(maxM, mode) for p in plans), dtype=torch.uint8, device="cuda")
    ys = torch.empty(maxM, H, dtype=torch.float32, device="cuda")
    sels = [torch.empty(b[0][-1], TOPK, dtype=torch.int32, device="cuda") for b in batches]

    def call(i):
        b = i % len(batches)
        offs, x, lg = batches[b]
        plans[i % len(plans)](x, lg, row_offsets=offs, mode=mode, workspace=ws, y=ys[:offs[-1]], sel=sels[b])
        return b

    w0 = time.perf_counter()
    nwarm = 0
    while nwarm < warmup or time.perf_counter() - w0 < min_warm_s:
        call(nwarm)
        nwarm += 1
        if nwarm % 32 == 0:
            torch.cuda.synchronize()  # keep the host within a few steps of the GPU
    torch.cuda.synchronize()
    # The timed steps continue the same sequence as if exactly `warmup` steps had run.
    t0 = time.perf_counter()
    order = [call(warmup + s) for s in range(steps)]
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    # Same calls again with stage events: each plan's ring holds its own calls in order.
    traces = {id(p): StageTrace(p, steps) for p in plans}
    for s in range(steps):
        call(warmup + s)
    torch.cuda.synchronize()
    pis = [(warmup + s) % len(plans) for s in range(steps)]
    ncalls = {id(p): sum(1 for pi in pis if plans[pi] is p) for p in plans}
    per_plan = {id(p): traces[id(p)].stage_ms(ncalls[id(p)]) for p in plans}
    seen = {id(p): 0 for p in plans}
    stage_rows = []
    for pi in pis:
        pid = id(plans[pi])
        stage_rows.append(per_plan[pid][seen[pid]])
        seen[pid] += 1
    for t in traces.values():
        t.close()
    rows = sum(batches[b][0][-1] for b in order)
    used = [len(set(sels[b].cpu().numpy().ravel().tolist())) for b in order]
    return {"wall_s": wall, "rows": rows, "stages": stage_rows, "distinct": used,
            "M": [batches[b][0][-1] for b in order], "warmup_run": nwarm}


def graph_decode(plans, batches, warmup, steps, mode):
    """The same decode steps captured in one HIP graph (the layer records only kernel
    launches, no allocations or memsets) and replayed: the device time of the layer chain
    without the host launch cost, as a serving loop that captures one graph per batch
    shape sees it.  The graph holds at least 200 steps (a replay has a fixed start-up cost
    that shorter graphs do not amortize).  Returns (ms per step, best of 3 replays, steps in
    the graph) or None."""
    import numpy as np
    import torch
    from exl3moe.trace import EventTimer
    maxM = max(b[0][-1] for b in batches)
    ws = torch.empty(max(p.workspace_size(maxM, mode) for p in plans), dtype=torch.uint8, device="cuda")
    ys = torch.empty(maxM, H, dtype=torch.float32, device="cuda")
    sels = [torch.empty(b[0][-1], TOPK, dtype=torch.int32, device="cuda") for b in batches]

    def call(i):
        offs, x, lg = batches[i % len(batches)]
        plans[i % len(plans)](x, lg, row_offsets=offs, mode=mode, workspace=ws, y=ys[:offs[-1]],
                              sel=sels[i % len(batches)])
    steps = max(steps, 200)
    try:
        for i in range(warmup):
            call(i)
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            for s in range(steps):
                call(warmup + s)
        gr.replay()
        torch.cuda.synchronize()
        tg = EventTimer(3, torch.cuda.current_stream().cuda_stream)
        for _ in range(3):
            tg.mark()
            gr.replay()
        tg.mark()
        ms = float(np.min(tg.ms())) / steps
        tg.close()
        del gr
        return ms, steps
    except RuntimeError as e:  # capture unsupported: report eager numbers only
        print(f"bench.py: graph capture of the decode steps failed: {e}", file=sys.stderr)
        return None


def pct(v):
    import numpy as np
    v = np.asarray(v, dtype=np.float64)
    return {"p10": round(float(np.percentile(v, 10)), 2), "median": round(float(np.median(v)), 2),
            "p90": round(float(np.percentile(v, 90)), 2), "mean": round(float(v.mean()), 2)}


def stream_peak():
    """Measured HBM stream rate: device-to-device copies of 2 GiB (read + write bytes / time)."""
    import torch
    from exl3moe.trace import EventTimer
    n = 2 << 30
    a = torch.empty(n, dtype=torch.uint8, device="cuda")
    b = torch.empty(n, dtype=torch.uint8, device="cuda")
    a.fill_(1)
    b.copy_(a)
    t = EventTimer(5, torch.cuda.current_stream().cuda_stream)
    for _ in range(5):
        t.mark()
        b.copy_(a)
    t.mark()
    ms = t.ms()
    t.close()
    del a, b
    return round(2 * n / (min(ms) / 1000) / 1e9, 1)


def bench_linear(seed, copies=128, warmup=10):
    """Config 2: ragged decode GEMVs 2048->4096 and 4096->2048 at 4 bpw, 8 sessions of 1 + d
    rows (d ~ U{0..4}), rotating over `copies` seeded weight pairs (> 1 GiB, cold reads)."""
    import numpy as np
    import torch
    from exl3moe import synth
    from exl3moe.trace import EventTimer
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    pairs = [(synth.device_linear(gen, 2048, 4096, 4), synth.device_linear(gen, 4096, 2048, 4)) for _ in range(copies)]
    for a, b in pairs:  # only the repacked tiles are used here
        a.trellis = b.trellis = None
    rng = np.random.default_rng(seed)
    batches = []
    for _ in range(16):
        offs = synth.sessions(rng, 8, 1, 5)
        M = offs[-1]
        batches.append((offs, torch.from_numpy(rng.standard_normal((M, 2048)).astype(np.float16)).cuda(),
                        torch.from_numpy(rng.standard_normal((M, 4096)).astype(np.float16)).cuda()))
    ws = torch.empty(max(pairs[0][0].workspace_size(40), pairs[0][1].workspace_size(40)), dtype=torch.uint8,
                     device="cuda")
    y1 = torch.empty(40, 4096, dtype=torch.float32, device="cuda")
    y2 = torch.empty(40, 2048, dtype=torch.float32, device="cuda")

    def call(i, which):
        offs, x1, x2 = batches[i % len(batches)]
        a, b = pairs[i % copies]
        M = offs[-1]
        if which == 0:
            a.forward_into(x1, y1[:M], offs, ws)
        else:
            b.forward_into(x2, y2[:M], offs, ws)

    for i in range(warmup):
        call(i, 0)
        call(i, 1)
    torch.cuda.synchronize()
    t = EventTimer(2 * copies, torch.cuda.current_stream().cuda_stream)
    for i in range(copies):
        t.mark()
        call(warmup + i, 0)
        t.mark()
        call(warmup + i, 1)
    t.mark()
    ms = np.array(t.ms()).reshape(copies, 2)
    t.close()
    # The same calls captured in one HIP graph (the library records only kernel launches):
    # the device time without the per-call host launch cost of the eager loop above.
    graph_ms = None
    try:
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            for i in range(copies):
                call(warmup + i, 0)
                call(warmup + i, 1)
        gr.replay()
        torch.cuda.synchronize()
        tg = EventTimer(3, torch.cuda.current_stream().cuda_stream)
        for _ in range(3):
            tg.mark()
            gr.replay()
        tg.mark()
        graph_ms = float(np.min(tg.ms()))
        tg.close()
        del gr
    except RuntimeError as e:  # capture unsupported: report eager numbers only
        print(f"bench.py: graph capture of the linear calls failed: {e}", file=sys.stderr)
    out = {"workload": "config2: ragged decode GEMV, 8 sessions x (1 + U{0..4}) rows, EXL3 4.0 bpw, "
                       f"rotating over {copies} seeded weight pairs", "copies": copies}
    if graph_ms is not None:
        Ms = np.array([batches[(warmup + i) % len(batches)][0][-1] for i in range(copies)])
        by = sum(float((matrix_bytes(I, O, 8) + Ms * I * 2 + Ms * O * 4).sum()) for I, O in ((2048, 4096), (4096, 2048)))
        out["graph"] = {"us_per_call": round(graph_ms * 1000 / (2 * copies), 2),
                        "algorithmic_GBps": round(by / (graph_ms / 1000) / 1e9, 1)}
    for j, (I, O) in enumerate(((2048, 4096), (4096, 2048))):
        Ms = np.array([batches[(warmup + i) % len(batches)][0][-1] for i in range(copies)])
        by = matrix_bytes(I, O, 8) + Ms * I * 2 + Ms * O * 4
        gbs = float(by.sum() / (ms[:, j].sum() / 1000)) / 1e9
        out[f"{I}x{O}"] = {"us": pct(ms[:, j] * 1000), "algorithmic_GBps": round(gbs, 1),
                           "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
                           "rows_per_s": round(float(Ms.sum() / (ms[:, j].sum() / 1000)), 1)}
    # A group of linears over the same rows (cx_exl3_group, e.g. the q / k / v projections):
    # 2048 -> 4096 (the pairs' first matrices), 512 and 512, at 4 bpw; the three GEMMs of
    # one rate run as one launch.
    from exl3moe import ops
    kv = [(synth.device_linear(gen, 2048, 512, 4), synth.device_linear(gen, 2048, 512, 4)) for _ in range(copies)]
    for a, b in kv:
        a.trellis = b.trellis = None
    yk = torch.empty(40, 512, dtype=torch.float32, device="cuda")
    yv = torch.empty(40, 512, dtype=torch.float32, device="cuda")
    gws = torch.empty(int(ops.group_workspace_size([pairs[0][0], kv[0][0], kv[0][1]], 40)), dtype=torch.uint8,
                      device="cuda")

    def gcall(i):
        offs, x1, _ = batches[i % len(batches)]
        M = offs[-1]
        ops.linear_group([(pairs[i % copies][0], x1, y1[:M]), (kv[i % copies][0], x1, yk[:M]),
                          (kv[i % copies][1], x1, yv[:M])], row_offsets=offs, workspace=gws)

    for i in range(warmup):
        gcall(i)
    torch.cuda.synchronize()
    t = EventTimer(copies, torch.cuda.current_stream().cuda_stream)
    for i in range(copies):
        t.mark()
        gcall(warmup + i)
    t.mark()
    gms = np.array(t.ms())
    t.close()
    Ms = np.array([batches[(warmup + i) % len(batches)][0][-1] for i in range(copies)])
    by = sum(matrix_bytes(2048, O, 8) + Ms * 2048 * 2 + Ms * O * 4 for O in (4096, 512, 512))
    gbs = float(by.sum() / (gms.sum() / 1000)) / 1e9
    out["group_qkv"] = {"workload": "cx_exl3_group of 2048->4096, 2048->512, 2048->512 at 4 bpw over the same rows",
                        "us": pct(gms * 1000), "algorithmic_GBps": round(gbs, 1),
                        "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)}
    del pairs, kv
    torch.cuda.empty_cache()
    return out


def bench_router(seed, copies=512, calls=256, warmup=16):
    """The router GEMV with the shared-gate logit (cx_dense_linear, W [E + 1][H] fp16, the
    engine's fp32 x): decode-sized (24 rows, fp32 products) and config-4-sized (2048 rows,
    MFMA) calls, rotating over `copies` seeded weight copies (> 1 GiB, cold reads)."""
    import numpy as np
    import torch
    from exl3moe import ops
    from exl3moe.trace import EventTimer
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    Ws = [torch.randn(E + 1, H, generator=g, device="cuda").half() for _ in range(copies)]
    out = {"workload": f"router GEMV W [{E + 1}][{H}] fp16, fp32 x, rotating over {copies} weight copies",
           "copies": copies}
    for M in (4, 24, 2048):
        x = torch.randn(M, H, generator=g, device="cuda")
        y = torch.empty(M, E + 1, dtype=torch.float32, device="cuda")
        for i in range(warmup):
            ops.dense_linear(Ws[i % copies], x, y)
        torch.cuda.synchronize()
        t = EventTimer(calls, torch.cuda.current_stream().cuda_stream)
        for i in range(calls):
            t.mark()
            ops.dense_linear(Ws[(warmup + i) % copies], x, y)
        t.mark()
        us = np.array(t.ms()) * 1000
        t.close()
        by = (E + 1) * H * 2 + M * H * 4 + M * (E + 1) * 4
        med = float(np.median(us))
        r = {"us": pct(us), "algorithmic_GBps": round(by / (med * 1e-6) / 1e9, 1),
             "frac_hbm": round(by / (med * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
        if M > 8:
            tf = 2.0 * M * (E + 1) * H / (med * 1e-6) / 1e12
            r["TFLOPs"] = round(tf, 1)
            r["frac_mfma"] = round(tf / MFMA_F16_PEAK_TFS, 4)
        out[f"M{M}"] = r
    del Ws
    torch.cuda.empty_cache()
    return out


def bench_long(seed, steps=3, head_copies=5, head_calls=20):
    """Config 5: an 8192-token chunk through the layer with gate/up at 3 bpw and down at
    5 bpw, plus a 6-bpw output head 2048->151936 applied to 4 last-token rows (rotating
    over `head_copies` seeded heads, > 1 GiB)."""
    import numpy as np
    import torch
    from exl3moe import CX_MOE_PREFILL, synth
    from exl3moe.trace import EventTimer
    plan = synth.device_moe_layer(seed, E=E, H=H, Ie=IE, topk=TOPK, bits_gu=3, bits_d=5)
    rng = np.random.default_rng(seed)
    M = 8192
    batch = [([0, M], torch.from_numpy(rng.standard_normal((M, H)).astype(np.float16)).cuda(),
              torch.from_numpy(rng.standard_normal((M, E + 1)).astype(np.float32)).cuda())]
    r = run_workload([plan], batch, 1, steps, CX_MOE_PREFILL)
    del plan
    ms = r["wall_s"] * 1000 / steps
    st = np.array(r["stages"])
    flops = 2.0 * (TOPK + 1) * M * 3 * H * IE
    out = {"workload": "config5: 8192 tokens, gate/up 3 bpw, down 5 bpw, E=512 top-10 + shared",
           "tokens_per_s": round(M / (ms / 1000), 1), "ms_per_step": round(ms, 4),
           "mfma": {"achieved_TFLOPs_layer": round(flops / (ms / 1000) / 1e12, 1), "peak": MFMA_F16_PEAK_TFS,
                    "frac_layer": round(flops / (ms / 1000) / 1e12 / MFMA_F16_PEAK_TFS, 4)},
           "stage_us_mean": {n: round(float(st[:, i].mean() * 1000), 2) for i, n in enumerate(
               ["route", "group", "input", "gate_up", "mid", "down", "combine"])}}
    out["traffic"] = prefill_traffic("config5", out["stage_us_mean"])
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed + 1)
    heads = []
    for _ in range(head_copies):
        h = synth.device_linear(gen, 2048, 151936, 6)
        h.trellis = None
        heads.append(h)
    x = torch.from_numpy(rng.standard_normal((4, 2048)).astype(np.float16)).cuda()
    y = torch.empty(4, 151936, dtype=torch.float32, device="cuda")
    offs = [0, 1, 2, 3, 4]
    ws = torch.empty(heads[0].workspace_size(4), dtype=torch.uint8, device="cuda")
    for i in range(head_copies):
        heads[i].forward_into(x, y, offs, ws)
    torch.cuda.synchronize()
    t = EventTimer(head_calls, torch.cuda.current_stream().cuda_stream)
    for i in range(head_calls):
        t.mark()
        heads[i % head_copies].forward_into(x, y, offs, ws)
    t.mark()
    hm = np.array(t.ms())
    t.close()
    by = matrix_bytes(2048, 151936, 12) + 4 * 2048 * 2 + 4 * 151936 * 4
    gbs = by / (hm.mean() / 1000) / 1e9
    out["head"] = {"workload": "EXL3 6.0 bpw 2048->151936 GEMV, 4 rows (one per session)", "copies": head_copies,
                   "us": pct(hm * 1000), "algorithmic_GBps": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)}
    del heads
    torch.cuda.empty_cache()
    return out


def bench_r1(plans, seed, calls=200, warmup=50):
    """R = 1 decode (one row, the serial-decode case): per-layer latency, eager (events
    around each call) and replayed from one HIP graph, beside the launch-bound floor: the
    same number of dependent minimal kernels (torch's one-wave spin kernel, 0 cycles)
    timed the same two ways."""
    import numpy as np
    import torch
    from exl3moe import CX_MOE_DECODE
    from exl3moe.trace import EventTimer
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    xs = [torch.randn(1, H, generator=g, device="cuda").half() for _ in range(8)]
    lgs = [torch.randn(1, E + 1, generator=g, device="cuda") for _ in range(8)]
    ws = torch.empty(max(p.workspace_size(1, CX_MOE_DECODE) for p in plans), dtype=torch.uint8, device="cuda")
    y = torch.empty(1, H, dtype=torch.float32, device="cuda")
    # route + grouping + input transforms (one launch at M <= 16), gate/up, down (the mid in
    # its prologue at small M unless CX_DOWN_MID=0 makes it a launch of its own), combine
    n_launch = 5 if os.environ.get("CX_DOWN_MID") == "0" else 4

    def call(i):
        plans[i % len(plans)](xs[i % 8], lgs[i % 8], mode=CX_MOE_DECODE, workspace=ws, y=y)

    def floor_call(i):
        for _ in range(n_launch):
            torch.cuda._sleep(0)

    def eager(fn):
        for i in range(warmup):
            fn(i)
        torch.cuda.synchronize()
        t = EventTimer(calls, torch.cuda.current_stream().cuda_stream)
        for i in range(calls):
            t.mark()
            fn(i)
        t.mark()
        v = np.array(t.ms()) * 1000
        t.close()
        return v

    def graphed(fn, n=50):
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            for i in range(n):
                fn(i)
        gr.replay()
        torch.cuda.synchronize()
        tg = EventTimer(5, torch.cuda.current_stream().cuda_stream)
        for _ in range(5):
            tg.mark()
            gr.replay()
        tg.mark()
        us = float(np.min(tg.ms())) * 1000 / n
        tg.close()
        del gr
        return us

    out = {"workload": "config-3 layer at R = 1 (one row, E=512 top-10 + shared, 4.0 bpw), rotating over the "
                       "seeded layers", "launches": n_launch}
    out["eager_us"] = pct(eager(call))
    out["floor_eager_us"] = pct(eager(floor_call))
    try:
        out["graph_us"] = round(graphed(call), 2)
        out["floor_graph_us"] = round(graphed(floor_call), 2)
    except RuntimeError as e:
        print(f"bench.py: graph capture at R = 1 failed: {e}", file=sys.stderr)
    return out


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _oracle_step(plan, xh, sel, wts):
    """A callable running one whole layer call through the oracle on the host: decode of the
    distinct routed experts' weights + the shared expert's, then the layer math over every
    row.  The weights leave the GPU before; the callable returns its own duration."""
    import numpy as np
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle as O
    used = sorted(set(sel.ravel().tolist()))

    def host(t):
        return (t.cpu().numpy() if hasattr(t, "cpu") else t).view(np.uint16)

    raw = {e: {k: (host(plan._experts[e][k].trellis), plan._experts[e][k]) for k in ("gate", "up", "down")}
           for e in used}
    sh_raw = {k: (host(plan._shared[k].trellis), plan._shared[k]) for k in ("gate", "up", "down")}
    scales = {id(lin): (lin.suh.cpu().numpy(), lin.svh.cpu().numpy())
              for d in list(raw.values()) + [sh_raw] for _, lin in d.values()}

    def dec3(d):
        out = {}
        for n, key in (("g", "gate"), ("u", "up"), ("d", "down")):
            tr, lin = d[key]
            out["w" + n] = O.reconstruct_inner(tr, lin.k2 / 2, lin.codebook)
            out["s" + n], out["v" + n] = scales[id(lin)]
        return out

    def one_step():
        t1 = time.perf_counter()
        experts = {e: dec3(raw[e]) for e in used}
        shd = dec3(sh_raw)
        dummy = experts[used[0]]
        O.moe_layer([experts.get(e, dummy) for e in range(E)], shd, xh, sel, wts)
        return time.perf_counter() - t1

    return one_step, len(used)


def cpu_baseline_prefill(plan, batch, seconds):
    """The oracle over one whole config-4 prefill call (2048 rows, Zipf-skewed routing) on the
    host cores: decode of every routed expert's weights + the layer math over all rows, no
    subset and no scaling.  One untimed warm-up call, then timed calls while they fit in
    `seconds` (at least one); the median is reported."""
    import numpy as np
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle as O
    offs, x, lg = batch
    xh = x.cpu().numpy()
    sel, wts = O.route(lg.cpu().numpy(), E, TOPK)
    one_step, n_used = _oracle_step(plan, xh, sel, wts)
    threads = O.num_threads()
    t0 = time.perf_counter()
    one_step()
    runs = [one_step()]
    while time.perf_counter() - t0 + runs[-1] < seconds and len(runs) < 5:
        runs.append(one_step())
    med = float(np.median(runs))
    rows = xh.shape[0]
    return {"value": round(rows / med, 2), "unit": "tokens/s", "cores": threads, "kind": "port",
            "cpu_model": _cpu_model(), "omp_threads": threads, "runs": len(runs),
            "step_s": {"median": round(med, 4), "min": round(min(runs), 4), "max": round(max(runs), 4)},
            "sample": f"one whole config-4 prefill call of {rows} rows ({n_used} distinct routed experts + the "
                      f"shared one): host decode of their weights + the layer math over every row "
                      f"(oracle/exl3_oracle.c, OpenMP); median of {len(runs)} timed calls after one warm-up call"}


def cpu_baseline(plan, batch, seconds):
    """The oracle (C restatement, OpenMP) on the host cores over whole decode steps of the
    same workload: decode of the routed experts' weights + the layer math.  One untimed
    warm-up step, then >= 5 timed steps at the process's OpenMP thread count (median
    reported), then one step on a single thread; the sample is bounded by `seconds`."""
    import numpy as np
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle as O
    offs, x, lg = batch
    xh = x.cpu().numpy()
    lgh = lg.cpu().numpy()
    sel, wts = O.route(lgh, E, TOPK)
    # Weights leave the GPU before any clock starts; decode + math is timed.
    one_step, n_used = _oracle_step(plan, xh, sel, wts)

    threads = O.num_threads()
    t_start = time.perf_counter()
    one_step()  # warm-up (page faults, OpenMP pool)
    runs = []
    while len(runs) < 5 or (time.perf_counter() - t_start < seconds / 2 and len(runs) < 50):
        runs.append(one_step())
    O.set_num_threads(1)
    try:
        single = one_step()
    finally:
        O.set_num_threads(threads)
    med = float(np.median(runs))
    rows = xh.shape[0]
    return {"value": round(rows / med, 2), "unit": "tokens/s", "cores": threads, "kind": "port",
            "cpu_model": _cpu_model(), "nproc": os.cpu_count(),
            "affinity_cpus": len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else None,
            "omp_threads": threads, "runs": len(runs),
            "step_s": {"median": round(med, 4), "min": round(min(runs), 4), "max": round(max(runs), 4)},
            "single_thread": {"value": round(rows / single, 3), "unit": "tokens/s", "step_s": round(single, 3)},
            "sample": f"config-3 decode step of {rows} rows ({n_used} distinct routed experts + the shared one): "
                      f"host decode of their weights + the layer math (oracle/exl3_oracle.c, OpenMP); median of "
                      f"{len(runs)} timed steps after one warm-up step, then one step on 1 thread"}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); the expert-parallel "
              "multi-GPU design is described in DESIGN.md but not built.", file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch
    from exl3moe import CX_MOE_DECODE, CX_MOE_PREFILL, synth

    torch.cuda.init()
    make_layer = synth.host_moe_layer if args.host_data else synth.device_moe_layer
    plans = [make_layer(args.seed + i, E=E, H=H, Ie=IE, topk=TOPK) for i in range(args.layers)]
    if args.calibrate_copy_mib:
        n = args.calibrate_copy_mib << 20
        src = torch.from_numpy(np.ones(n, dtype=np.uint8)).cuda()
        dst = torch.from_numpy(np.zeros(n, dtype=np.uint8)).cuda()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    k2 = 8
    eb = expert_bytes(k2, k2)
    nb = max(args.steps, 8)
    batches = make_batches(nb, args.seed + 100)
    r = run_workload(plans, batches, args.warmup, args.steps, CX_MOE_DECODE, args.min_warmup_s)
    ms_step = r["wall_s"] * 1000 / args.steps
    tok_s = r["rows"] / r["wall_s"]
    st = np.array(r["stages"])  # [steps][7] ms
    # The dominant kernel: the decode stage launch (gate/up, mid and down in one kernel; its
    # trace interval is the gate/up stage, the mid and down intervals hold no kernel).
    # Algorithmic bytes per launch: the distinct routed experts' + the shared expert's gate,
    # up and down weights (tiles + scales), the gate/up inputs it reads (xg, xu fp16) and the
    # down output rows it writes (fp32); the gate/up sums and the mid rows it passes between
    # its workgroups inside one XCD's L2 are not counted.  Steps whose row count runs the
    # GEMMs as separate launches (few rows) are left out of it.
    sm = np.array([uses_stage(m) for m in r["M"]])
    P = np.array([m * TOPK + m for m in r["M"]])
    dist = np.array(r["distinct"])
    kb = (dist + 1) * eb + P * H * 2 * 2 + P * H * 4
    gu = st[:, 3]
    stage_achieved = float(kb[sm].sum() / (gu[sm].sum() / 1000)) / 1e9 if sm.any() else 0.0
    layer_bytes = np.array([(u + 1) * eb + m * H * 2 + m * H * 4 + m * (E + 1) * 4 for u, m in zip(r["distinct"], r["M"])])
    layer_gbs = float(layer_bytes.sum() / r["wall_s"]) / 1e9
    # HBM bytes per gate/up launch: not measurable inside this run (counter collection needs
    # rocprofv3); taken from the committed counter profile of the same kernel and workload,
    # with its provenance beside it (traffic_source), and dropped when the profile names
    # another kernel instantiation than the one this build launches.
    traffic, traffic_src = None, None
    tf = ROOT / "profiles" / "traffic_decode_stage.json"
    if tf.exists():
        try:
            tj = json.loads(tf.read_text())
            if tj.get("kernel") == STAGE_KERNEL:
                traffic = tj.get("hbm_bytes_per_launch")
                traffic_src = {"file": "profiles/traffic_decode_stage.json", "kernel": tj.get("kernel"),
                               "command": tj.get("command"), "note": "measured by rocprofv3 --pmc in a separate "
                               "run of this bench workload, FETCH_SIZE scaled by a device-copy calibration"}
        except Exception:
            traffic = None
    out = {
        "metric": "MoE-layer tokens/s (8-session ragged decode; 2048-tok prefill) + % roofline",
        "value": round(tok_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "warmup_steps_run": r["warmup_run"],
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic",
        "config": {"workload": "config3: MoE layer decode, E=512 top-10 + shared, H=2048, I=512, EXL3 4.0 bpw, "
                               "8 ragged sessions x 1..5 rows",
                   "layers_rotated": args.layers, "rows_per_step_mean": round(float(np.mean(r["M"])), 2),
                   "distinct_experts_mean": round(float(np.mean(r["distinct"])), 1)},
        "roofline": {"bound": "hbm", "kernel": "Exl3DecodeStageKernel (gate/up, mid, down)",
                     "achieved": round(stage_achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(stage_achieved / HBM_PEAK_GBS, 4), "traffic": traffic, "traffic_source": traffic_src,
                     "avg_us": round(float(gu[sm].mean() * 1000), 2) if sm.any() else None,
                     "algorithmic_bytes_per_launch": int(kb[sm].mean()) if sm.any() else None,
                     "launches": int(sm.sum())},
        "layer": {"algorithmic_GBps": round(layer_gbs, 1), "frac_hbm": round(layer_gbs / HBM_PEAK_GBS, 4),
                  "traced_step_us": pct(st.sum(1) * 1000),
                  "stage_us_mean": {n: round(float(st[:, i].mean() * 1000), 2) for i, n in enumerate(
                      ["route", "group", "input", "gate_up", "mid", "down", "combine"])}},
    }
    g = graph_decode(plans, batches, args.warmup, args.steps, CX_MOE_DECODE)
    if g is not None:
        gms, gsteps = g
        out["graph"] = {"tokens_per_s": round(r["rows"] / (gms * args.steps / 1000), 1), "ms_per_step": round(gms, 4),
                        "steps_in_graph": gsteps}
    if not args.no_prefill:
        pb = make_batches(2, args.seed + 200, prefill=True)
        rp = run_workload(plans, pb, 2, args.prefill_steps, CX_MOE_PREFILL, args.min_warmup_s)
        stp = np.array(rp["stages"])
        ms_p = rp["wall_s"] * 1000 / args.prefill_steps
        flops = 2.0 * (TOPK + 1) * 2048 * 3 * H * IE
        gemm_ms = float((stp[:, 3] + stp[:, 5]).mean())
        wbytes = np.mean([(u + 1) * eb for u in rp["distinct"]])
        out["prefill"] = {
            "workload": "config4: 2048 tokens, Zipf(1.1) router bias, same layer",
            "tokens_per_s": round(2048 / (ms_p / 1000), 1), "ms_per_step": round(ms_p, 4),
            "mfma": {"achieved_TFLOPs_layer": round(flops / (ms_p / 1000) / 1e12, 1),
                     "achieved_TFLOPs_gemms": round(flops / (gemm_ms / 1000) / 1e12, 1),
                     "peak": MFMA_F16_PEAK_TFS, "frac_layer": round(flops / (ms_p / 1000) / 1e12 / MFMA_F16_PEAK_TFS, 4)},
            "hbm": {"weight_GBps_layer": round(wbytes / (ms_p / 1000) / 1e9, 1),
                    "frac_layer": round(wbytes / (ms_p / 1000) / 1e9 / HBM_PEAK_GBS, 4)},
            "stage_us_mean": {n: round(float(stp[:, i].mean() * 1000), 2) for i, n in enumerate(
                ["route", "group", "input", "gate_up", "mid", "down", "combine"])},
        }
        out["prefill"]["traffic"] = prefill_traffic("config4", out["prefill"]["stage_us_mean"])
    if not args.no_r1:
        out["decode_r1"] = bench_r1(plans, args.seed + 500)
    if not args.no_linear:
        out["linear"] = bench_linear(args.seed + 300)
    if not args.no_router:
        out["router"] = bench_router(args.seed + 600)
    if not args.no_long:
        out["prefill_long"] = bench_long(args.seed + 400)
    if not args.no_stream:
        out["roofline"]["measured_stream_GBps"] = stream_peak()
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(plans[0], batches[0], args.cpu_seconds)
        if not args.no_prefill:
            out["prefill"]["cpu_baseline"] = cpu_baseline_prefill(plans[0], pb[0], args.cpu_seconds)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
