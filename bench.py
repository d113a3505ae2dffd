"""Benchmark of the decode hot path on one MI355X.

Headline (BASELINE.json metric, configuration C2 at B=32): one decode step =
store_kvcache of one new K/V row per sequence + paged decode attention at
Qwen3-4B geometry (32q / 8kv / 128, bf16, 256-token pages, contexts
U[512, 4096], 2048-page pool). ``value`` is the step's algorithmic HBM bytes
divided by its time (GB/s). Inputs are resident in HBM; each timed step is a
HIP-graph replay, and consecutive steps use disjoint page sets of the pool so
repeated reads cannot be served by the 256 MB MALL.

Also reported on the same JSON line:
  roofline      the dominant kernel (split-KV attention main kernel): its
                algorithmic bytes per launch / its average duration, measured
                with HIP events around each launch on the launching stream
  cpu_baseline  the reference's CPU path restated in torch fp32 (oracle/torch_cpu.py)
                on the host: the whole C2 B=32 step, median of 5 after 2 warm-ups
                (extra.cpu_baselines: C1, C3, the slot scatter, C4 at M 1 / 56)
  extra         C3 verify, C4 W8A16 (all shapes x M, cold weights), C5 draft
                chain (us per draft step, attention / GEMV shares) and the
                attention op split into main + combine

usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
       python bench.py --profile-pass   (few launches of each kernel + a copy of
                                         known size, for rocprofv3 counter runs)
       python bench.py --twin-pass      (the attention main kernel and its read-only
                                         floor twin, C2 B=32 then C3, for counter runs)
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "paged decode/verify attn + W8A16 GEMV: achieved HBM GB/s, % of MI355X peak"
PEAK_HBM_GBS = 8000.0
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic.json")


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--batch", type=int, default=32)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--no-draft-chain", action="store_true",
                    help="skip the C5 draft-chain extra (its thousands of launches swamp a trace)")
    ap.add_argument("--profile-pass", action="store_true")
    ap.add_argument("--twin-pass", action="store_true",
                    help="main kernel and floor twin, 3 launches each, C2 B=32 then C3")
    ap.add_argument("--draft-chain-only", type=int, default=0, metavar="B",
                    help="only the fused C5 draft chain at batch B, replayed a few times "
                         "(for a kernel trace); prints us per draft step")
    return ap.parse_args()


# --------------------------------------------------------------------------- helpers
def graph_of(fn, torch):
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    return g


def time_replays(graphs, steps, warmup, torch, per_launch=False):
    """Average ms per replay over ``steps`` replays (cycling through ``graphs``).
    per_launch: HIP events around every replay (kernel-duration view)."""
    settle(graphs[0], torch)  # untimed: the clocks settle (see settle)
    for i in range(warmup):
        graphs[i % len(graphs)].replay()
    torch.cuda.synchronize()
    if per_launch:
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(steps)]
        for i in range(steps):
            ev[i][0].record()
            graphs[i % len(graphs)].replay()
            ev[i][1].record()
        torch.cuda.synchronize()
        return sum(a.elapsed_time(b) for a, b in ev) / steps
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(steps):
        graphs[i % len(graphs)].replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


SETTLE_MS = 20.0


def settle(graph, torch, ms=SETTLE_MS):
    """Replay ``graph`` until about ``ms`` of GPU work has run, untimed. The
    GPU's clocks settle over milliseconds of continuous load: lm_head at M = 1
    measured 28.4 us per call after 2 replays of its chain, 27.2 after 50 and
    26.4 after 200 (same process, same graph); every figure here is the steady
    state a serving loop runs at."""
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    graph.replay()
    b.record()
    torch.cuda.synchronize()
    n = min(4000, math.ceil(ms / max(a.elapsed_time(b), 1e-3)))
    for _ in range(n):
        graph.replay()
    torch.cuda.synchronize()


# Launches per timed graph: each per-call leg repeats its cycle of page sets or
# weight copies until one graph holds at least this many. Replaying a graph costs
# about 4 us on the GPU between its last kernel and the next replay's first (one
# process, lm_head M = 1: 25.6 us per call with 4 calls per graph, 24.8 with 20,
# 24.6 with 40), a gap a serving step's graph, which holds hundreds of launches,
# amortizes; at 4-8 calls per graph it was charged to every call.
MIN_GRAPH_CALLS = 40


def cycle(fns, min_calls=MIN_GRAPH_CALLS):
    """(body, calls): one graph body calling ``fns`` in turn, the cycle repeated
    until it holds at least ``min_calls`` launches, and how many it holds."""
    reps = max(1, math.ceil(min_calls / len(fns)))
    return (lambda: [f() for _ in range(reps) for f in fns]), reps * len(fns)


def time_groups(graph, per_replay, torch, groups=5, min_launches=20, warmup=2):
    """Per-launch time of the launches one replay of ``graph`` holds
    (``per_replay`` of them): after ``settle`` and ``warmup`` replays, HIP
    events on the current stream around each of ``groups`` groups of
    back-to-back replays, each group at least ``min_launches`` launches;
    returns (median, min, max) in ms over the groups' per-launch means. The
    decision protocol for the roofline legs and the per-shape rows: a median
    of groups, not one mean, with the spread."""
    import statistics
    reps = max(1, math.ceil(min_launches / per_replay))
    settle(graph, torch)
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    ts = []
    for _ in range(groups):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(reps):
            graph.replay()
        b.record()
        torch.cuda.synchronize()
        ts.append(a.elapsed_time(b) / (reps * per_replay))
    return statistics.median(ts), min(ts), max(ts)


def us3(t):
    """(median, min, max) ms -> {"us", "min_us", "max_us"}."""
    return {"us": round(t[0] * 1e3, 2), "min_us": round(t[1] * 1e3, 2),
            "max_us": round(t[2] * 1e3, 2)}


def read_ceiling(ops, torch):
    """The box's streaming-read ceiling (sd_stream_read over a 1 GiB buffer,
    4 / 6 / 8 workgroups per CU, the best median kept) and, as the reference
    measured its own (nanovllm/kernels/README.md:27-35), a plain 512 MiB
    device copy counted as read + write bytes."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    buf = torch.empty(1 << 30, dtype=torch.uint8, device="cuda").fill_(3)
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")
    best = None
    sweep = {}
    for per_cu in (4, 6, 8):
        g = graph_of(lambda: [ops.stream_read(buf, sink, per_cu * cus) for _ in range(4)], torch)
        t = time_groups(g, 4, torch, groups=5, min_launches=8)
        del g
        gbs = (1 << 30) / (t[0] * 1e-3) / 1e9
        sweep[f"{per_cu}_per_cu"] = round(gbs, 1)
        if best is None or gbs > best[0]:
            best = (gbs, per_cu, t)
    del buf
    src = torch.empty(512 << 20, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    g = graph_of(lambda: [dst.copy_(src) for _ in range(4)], torch)
    tc = time_groups(g, 4, torch, groups=5, min_launches=8)
    del g, src, dst
    torch.cuda.empty_cache()
    return {"read_GBps": round(best[0], 1), "read_workgroups_per_cu": best[1],
            "read_bytes": 1 << 30, "read_us": round(best[2][0] * 1e3, 2),
            "read_sweep_GBps": sweep,
            "copy_GBps": round(2 * (512 << 20) / (tc[0] * 1e-3) / 1e9, 1),
            "copy_bytes_each_way": 512 << 20,
            "note": "sd_stream_read: grid-stride 16-byte nontemporal loads, median of 5 "
                    "groups; copy: torch copy_ of 512 MiB, read + write bytes"}


def chain_len(steps, sets, cap=60):
    """Steps per graph of the timed decode chain: ``steps`` itself when it is at
    most ``cap``, else its largest divisor up to ``cap`` that is at least ``sets``
    (so that exactly ``steps`` steps are whole replays), else ``sets``."""
    if steps <= cap:
        return max(steps, 1)
    for n in range(cap, sets - 1, -1):
        if steps % n == 0:
            return n
    return sets


def time_steps(chain_graph, step_graphs, steps, warmup, torch):
    """ms per decode step over exactly ``steps`` steps: steps // n replays of
    ``chain_graph`` (n consecutive steps in one graph, cycling over the page
    sets, as a model forward holds every layer's attention call in one graph),
    then any remainder as single-step graphs."""
    n = chain_graph.steps
    settle(chain_graph, torch)  # untimed: the clocks settle (see settle)
    for _ in range(max(1, -(-warmup // n))):
        chain_graph.replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps // n):
        chain_graph.replay()
    for i in range(steps % n):
        step_graphs[i % len(step_graphs)].replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def decode_bytes(lens, hq, hkv, d, eb, store_rows):
    """Algorithmic bytes of one decode step: every visible K and V row once,
    q read + o written, the new K/V rows read and written, tables/lengths/slots."""
    kv = sum(int(L) for L in lens) * hkv * d * eb * 2
    qo = 2 * len(lens) * hq * d * eb
    store = store_rows * hkv * d * eb * 2 * 2
    idx = sum(math.ceil(int(L) / 256) for L in lens) * 4 + 4 * len(lens) * 2
    return kv + qo + store + idx


def attn_bytes(lens, hq, hkv, d, eb, q_rows=1):
    return sum(int(L) for L in lens) * hkv * d * eb * 2 + 2 * len(lens) * q_rows * hq * d * eb


def load_traffic(kernel_key):
    """Measured HBM bytes per launch from the committed rocprofv3 counter runs
    (profiles/traffic.json, written from FETCH_SIZE / WRITE_SIZE passes)."""
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
        return t.get(kernel_key, {}).get("bytes_per_launch")
    except (OSError, ValueError):
        return None


# ------------------------------------------------------------------------ CPU baseline
# The reference's CPU path (nanovllm/kernels/paged_decode_attn.py:472-495: page
# gather + fp32 softmax attention; quant.py:151-159: fp32 dequantize then
# matmul; the slot scatter of attention.py:21-30) restated in torch fp32 on the
# host (oracle/torch_cpu.py), timed under inference_mode: 2 warm-ups, then the
# median of 5, GB/s on the same algorithmic bytes as the GPU rows. The thread
# count is torch's (OMP_NUM_THREADS: the CPU share the box gives one GPU).
def _cpu_info(torch):
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": model, "torch_threads": torch.get_num_threads(),
            "os_cpu_count": os.cpu_count()}


def _time_cpu(fn, torch, warm=2, reps=5):
    import statistics
    with torch.inference_mode():
        for _ in range(warm):
            fn()
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
    return statistics.median(ts)


def _host_pages(k_cache, v_cache, tables):
    """The pages the tables use, copied to the host as fp32 (outside any
    timing), and the tables remapped onto them."""
    import torch
    used = sorted({int(x) for t in tables for x in t.flatten().tolist() if x >= 0})
    remap = torch.full((k_cache.shape[0],), -1, dtype=torch.int64)
    remap[torch.tensor(used)] = torch.arange(len(used))
    idx = torch.tensor(used, device=k_cache.device)
    kc, vc = k_cache[idx].float().cpu(), v_cache[idx].float().cpu()
    out = [torch.where(t >= 0, remap[t.clamp(min=0).long()], -1) for t in tables]
    return kc, vc, out


def cpu_baseline_decode(case, torch):
    """The whole C2 decode step on the host: the slot scatter of the new rows,
    then attention of every sequence over its pages (the headline line's
    cpu_baseline)."""
    from oracle import torch_cpu as otc
    bt = case["tables"][0]
    kc, vc, (tbl,) = _host_pages(case["k_cache"], case["v_cache"], [bt])
    lens = case["lens"]
    q = case["q"].float().cpu()
    kn, vn = case["k_new"].float().cpu(), case["v_new"].float().cpu()
    bs = case["block_size"]
    slots = torch.tensor([int(tbl[b, (int(L) - 1) // bs]) * bs + (int(L) - 1) % bs
                          for b, L in enumerate(lens)], dtype=torch.int64)

    def step():
        otc.store_kvcache(kn, vn, kc, vc, slots)
        otc.paged_attention(q, kc, vc, tbl, lens, case["scale"])
    sec = _time_cpu(step, torch)
    info = _cpu_info(torch)
    nbytes = decode_bytes(lens.tolist(), case["num_q_heads"], case["num_kv_heads"],
                          case["head_dim"], 2, len(lens))
    return {"value": round(nbytes / sec / 1e9, 3), "unit": "GB/s", "cores": info["torch_threads"],
            "kind": "port", "us": round(sec * 1e6, 1),
            "sample": f"the whole C2 B={len(lens)} decode step (store + attention of every "
                      f"sequence), torch fp32 on the host (oracle/torch_cpu.py), inference_mode, "
                      f"median of 5 after 2 warm-ups; {info['cpu_model']}, "
                      f"{info['torch_threads']} threads (os.cpu_count()={info['os_cpu_count']})"}


def cpu_baselines_extra(torch, workloads, verify_case):
    """The other rows of the CPU-baseline plan: C1 (the fp32 CPU configuration
    itself), C3 verify, the C2 B=32 slot scatter alone, and C4 dequantize then
    matmul at every shape for M in {1, 56}."""
    import math as _m
    from oracle import torch_cpu as otc
    info = _cpu_info(torch)
    rows = {"protocol": "torch fp32 on the host (oracle/torch_cpu.py), inference_mode, median "
                        "of 5 after 2 warm-ups; GB/s on the GPU rows' algorithmic bytes",
            **info}
    # C1: Qwen3-0.6B attention geometry, B=1, L=1000, 64-page pool, 4 permuted pages
    g = torch.Generator().manual_seed(0)
    kc = torch.randn((64, 256, 8, 128), generator=g)
    vc = torch.randn((64, 256, 8, 128), generator=g)
    q = torch.randn((1, 16, 128), generator=g)
    bt = torch.randperm(64, generator=g)[:4].view(1, 4)
    sec = _time_cpu(lambda: otc.paged_attention(q, kc, vc, bt, [1000], 128 ** -0.5), torch)
    nb = 1000 * 8 * 128 * 4 * 2 + 2 * 16 * 128 * 4
    rows["C1_decode_fp32"] = {"us": round(sec * 1e6, 1), "GBps": round(nb / sec / 1e9, 3)}
    # C3 verify: 8 sequences x 7 bottom-right causal rows
    v = verify_case
    kcv, vcv, (tv,) = _host_pages(v["k_cache"], v["v_cache"], [v["table"]])
    qv = v["q"].float().cpu()
    sec = _time_cpu(lambda: otc.paged_attention(qv, kcv, vcv, tv, v["keys"].tolist(),
                                                v["scale"], v["cu_q"]), torch)
    nb = attn_bytes(v["keys"].tolist(), 32, 8, 128, 2, q_rows=v["k"] + 1)
    rows["C3_verify"] = {"us": round(sec * 1e6, 1), "GBps": round(nb / sec / 1e9, 3)}
    del kcv, vcv
    # the slot scatter of C2 B=32 alone (32 new rows into a 2048-page pool slice)
    pool_k = torch.zeros((300, 256, 8, 128))
    pool_v = torch.zeros_like(pool_k)
    kn, vn = torch.randn((32, 8, 128), generator=g), torch.randn((32, 8, 128), generator=g)
    sl = torch.randperm(300 * 256, generator=g)[:32]
    sec = _time_cpu(lambda: otc.store_kvcache(kn, vn, pool_k, pool_v, sl), torch)
    nb = 32 * 8 * 128 * 2 * 2 * 2
    rows["store_kvcache_C2_B32"] = {"us": round(sec * 1e6, 1), "GBps": round(nb / sec / 1e9, 3)}
    del pool_k, pool_v
    # C4: every shape, M in {1, 56}
    c4 = []
    for name, N, K in workloads.W8A16_SHAPES:
        w = torch.clamp(torch.round(torch.randn((N, K), generator=g) * 40), -127, 127) \
            .to(torch.int8)
        s = torch.rand((N,), generator=g) * 3e-3 + 1e-3
        for M in (1, 56):
            x = torch.randn((M, K), generator=g)
            sec = _time_cpu(lambda: otc.dequant_linear(x, w, s), torch)
            nb = N * K + 2 * N + 2 * M * K + 2 * M * N
            c4.append({"shape": name, "M": M, "us": round(sec * 1e6, 1),
                       "GBps": round(nb / sec / 1e9, 3)})
        del w
    rows["C4_w8a16"] = c4
    return rows


# ----------------------------------------------------------------------------- extras
def bench_verify(ops, workloads, torch, steps):
    """C3 verify step (fused store + attention) over 8 disjoint page sets (537 MB
    of K/V in all, more than the 256 MB MALL), the 8 calls back to back in one
    graph so the GPU, not the host's graph launches, sets the time; plus the
    plain call, its main kernel and read-only floor over the same sets."""
    sets = 8
    case = workloads.verify_case(seed=0, sets=sets)
    dev = "cuda"
    tables = [t.to(dev) for t in case["tables"]]
    slot_sets = [x.to(dev) for x in case["slot_sets"]]
    cuq, cuk = case["cu_q"].to(dev), case["cu_k"].to(dev)
    out = torch.empty_like(case["q"])
    ws_bytes = ops.paged_attention_workspace_bytes(8, case["k"] + 1, 32, 8,
                                                   tables[0].shape[1] * 256, device=dev)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)

    def chain(store, twin=None):
        def one(i):
            kw = (dict(key=case["k_new"], value=case["v_new"], slot_mapping=slot_sets[i])
                  if store else dict(twin=twin, workspace=ws))
            return lambda: ops.paged_attention(case["q"], case["k_cache"], case["v_cache"],
                                               tables[i], case["scale"], cu_seqlens_k=cuk,
                                               cu_seqlens_q=cuq, max_seqlen_q=case["k"] + 1,
                                               out=out, **kw)
        return cycle([one(i) for i in range(sets)])
    del steps
    body, calls = chain(True)
    t = time_groups(graph_of(body, torch), calls, torch)
    ms = t[0]
    nbytes = (attn_bytes(case["keys"].tolist(), 32, 8, 128, 2, q_rows=case["k"] + 1)
              + case["slots"].numel() * 8 * 128 * 2 * 2 * 2)
    flops = sum(4 * 32 * 128 * (case["k"] + 1) * int(L) for L in case["keys"])
    res = {"config": f"C3 verify B=8 q_len 7 (store + attention), {sets} page sets, "
                     f"{calls} calls per graph", "us": round(ms * 1e3, 2),
           "GBps": round(nbytes / ms / 1e6, 1), "frac": round(nbytes / ms / 1e6 / PEAK_HBM_GBS, 4),
           "TFLOPs": round(flops / ms / 1e9, 2), "seed": case["seed_used"],
           "algorithmic_bytes": nbytes, "minmax_us": [round(t[1] * 1e3, 2), round(t[2] * 1e3, 2)],
           "timing": "median of 5 groups of >= 20 calls"}
    # the plain (non-storing) call and its twins over the same keys
    for twin, key in ((None, "attention_us"), ("main", "main_us"), ("floor", "floor_us")):
        body, calls = chain(False, twin)
        tt = time_groups(graph_of(body, torch), calls, torch)
        res[key] = round(tt[0] * 1e3, 2)
        res[key.replace("_us", "_minmax_us")] = [round(tt[1] * 1e3, 2), round(tt[2] * 1e3, 2)]
    return res


def bench_decode_batch(ops, workloads, torch, B, steps):
    """C2 decode step (fused store + attention) at batch B over disjoint page
    sets, one graph of consecutive steps; plus the attention main kernel and its
    read-only floor over the same sets."""
    probe = workloads.decode_case(B, seed=B, sets=1, device="cpu", num_blocks=2048,
                                  num_q_heads=1, num_kv_heads=1, head_dim=8)
    pages = sum(math.ceil(int(L) / 256) for L in probe["lens"])
    sets = max(1, min(16, 2048 // pages))
    case = workloads.decode_case(B, seed=B, sets=sets)
    lens_d = case["lens"].cuda()
    tables = [t.cuda() for t in case["tables"]]
    slots = [x.cuda() for x in case["slots"]]
    out = torch.empty_like(case["q"])
    ws_bytes = ops.paged_attention_workspace_bytes(B, 1, 32, 8, tables[0].shape[1] * 256,
                                                   device="cuda")
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")

    def chain(**kw):
        fns = [lambda i=i: ops.paged_attention(case["q"], case["k_cache"], case["v_cache"],
                                               tables[i], case["scale"], context_lens=lens_d,
                                               out=out, **({"key": case["k_new"],
                                                            "value": case["v_new"],
                                                            "slot_mapping": slots[i]}
                                                           if kw.get("store") else
                                                           {"twin": kw.get("twin"),
                                                            "workspace": ws}))
               for i in range(sets)]
        return cycle(fns)
    del steps
    res = {"config": f"C2 decode step B={B} (store + attention), {sets} page sets cycled "
                     f"through >= {MIN_GRAPH_CALLS} calls per graph, median of 5 groups of "
                     ">= 20 calls"}
    for name, kw in (("step_us", {"store": True}), ("attention_us", {}),
                     ("main_us", {"twin": "main"}), ("floor_us", {"twin": "floor"})):
        body, calls = chain(**kw)
        g = graph_of(body, torch)
        t = time_groups(g, calls, torch)
        res[name] = round(t[0] * 1e3, 2)
        res[name.replace("_us", "_minmax_us")] = [round(t[1] * 1e3, 2), round(t[2] * 1e3, 2)]
        del g
    nbytes = decode_bytes(case["lens"].tolist(), 32, 8, 128, 2, B)
    res["GBps"] = round(nbytes / res["step_us"] / 1e3, 1)
    res["frac"] = round(res["GBps"] / PEAK_HBM_GBS, 4)
    res["algorithmic_bytes"] = nbytes
    del case
    torch.cuda.empty_cache()
    return res


def bench_ctx_sweep(ops, workloads, torch):
    """B = 1 decode at Qwen3-4B attention geometry over context lengths 256 -
    4096, the reference's latency curve (nanovllm/kernels/README.md:266-275):
    the attention op (main + combine) and the decode step (fused store +
    attention), us per call as the median of 5 groups over chains of 32
    calls, each call on its own page set."""
    sets = 32
    case = workloads.decode_case(1, seed=7, sets=sets, ctx_range=(4096, 4096))
    tables = [t.cuda() for t in case["tables"]]
    out = torch.empty_like(case["q"])
    ws = torch.empty(ops.paged_attention_workspace_bytes(1, 1, 32, 8, 4096, device="cuda"),
                     dtype=torch.uint8, device="cuda")
    rows = []
    for L in (256, 512, 1024, 2048, 4096):
        lens = torch.full((1,), L, dtype=torch.int32, device="cuda")
        slots = [(t[0, (L - 1) // 256].long() * 256 + (L - 1) % 256).to(torch.int32).view(1)
                 for t in tables]

        def chain(store):
            if store:
                return cycle([lambda i=i: ops.paged_attention(
                    case["q"], case["k_cache"], case["v_cache"], tables[i], case["scale"],
                    context_lens=lens, out=out, key=case["k_new"], value=case["v_new"],
                    slot_mapping=slots[i]) for i in range(sets)])
            return cycle([lambda i=i: ops.paged_attention(
                case["q"], case["k_cache"], case["v_cache"], tables[i], case["scale"],
                context_lens=lens, out=out, workspace=ws) for i in range(sets)])
        row = {"ctx": L}
        for key, store in (("attention_us", False), ("step_us", True)):
            body, calls = chain(store)
            g = graph_of(body, torch)
            t = time_groups(g, calls, torch, groups=5, min_launches=32)
            del g
            row[key] = round(t[0] * 1e3, 2)
            row[key.replace("_us", "_minmax_us")] = [round(t[1] * 1e3, 2), round(t[2] * 1e3, 2)]
        nbytes = attn_bytes([L], 32, 8, 128, 2)
        row["attention_GBps"] = round(nbytes / row["attention_us"] / 1e3, 1)
        rows.append(row)
    del case
    torch.cuda.empty_cache()
    return {"config": "B=1, 32q/8kv/128 bf16, 256-token pages, 32 page sets (one per call), "
                      "median of 5 groups of >= 32 calls", "rows": rows}


def preload_w8a16(workloads, torch):
    """The C4 weights, allocated first in the process, as a serving process loads
    its weights before it allocates its KV cache: per shape, `copies` distinct
    int8 weight copies (> 2 x the 256 MB MALL in total, so every call streams its
    weight from HBM, as a model forward does) with their per-channel scale, and
    the bf16 copies of the dense comparison. The same weights allocated after a
    large allocate-and-free read measurably slower (one process, lm_head: 25.8
    against 24.5 us per call at M = 1, 30.0 against 28.7 at M = 16, after an
    8 GB allocate-and-free), which a bench that frees its attention buffers first
    would charge to the kernel."""
    pre = {}
    for name, N, K in workloads.W8A16_SHAPES:
        copies = max(2, math.ceil(2 * 256e6 / (N * K)))
        base = workloads.w8a16_case(1, N, K, seed=N)
        ws = [base["w"]] + [torch.roll(base["w"], i, 0) for i in range(1, copies)]
        bcopies = max(2, math.ceil(2 * 256e6 / (2 * N * K)))
        gen = torch.Generator(device="cuda").manual_seed(N + K)
        wb = [(torch.randn((N, K), generator=gen, device="cuda") * 0.02).to(torch.bfloat16)
              for _ in range(bcopies)]
        pre[name] = {"ws": ws, "s": base["s"], "wb": wb}
    torch.cuda.synchronize()
    return pre


def bench_w8a16(ops, workloads, torch, steps, pre):
    """Each shape x M: one HIP graph holding a chain of calls cycling over the
    preloaded weight copies (`preload_w8a16`); us per call = the median over 5
    groups of >= 20 calls (min / max beside it). Beside each row: the load-only
    twin (sd_w8a16_floor, same plan and loads, no math) and, at M in {1, 16}, the
    dense bf16 linear torch runs for the same shape (F.linear, hipBLASLt) over
    bf16 weight copies, as the reference compares its int8 path with the bf16
    GEMM (docs/W8A16量化-开发记录.md:264-275, scripts/bench_int8_gemm.py:138-146)."""
    import torch.nn.functional as F
    rows = []
    del steps
    for name, N, K in workloads.W8A16_SHAPES:
        for M in workloads.W8A16_MS:
            ws = pre[name]["ws"]
            g = torch.Generator(device="cuda").manual_seed(N + M)
            base = {"s": pre[name]["s"],
                    "x": torch.randn((M, K), generator=g, device="cuda").to(torch.float16)}
            y = torch.empty((M, N), dtype=torch.float16, device="cuda")
            nbytes = N * K + 2 * N + 2 * M * K + 2 * M * N
            row = {"shape": name, "M": M, "N": N, "K": K}
            for key, twin in (("us", None), ("floor", "floor")):
                body, calls = cycle([lambda w=w: ops.w8a16_linear(base["x"], w, base["s"],
                                                                  out=y, twin=twin) for w in ws])
                g = graph_of(body, torch)
                t = time_groups(g, calls, torch)
                del g
                if twin is None:
                    row.update(us3(t))
                    row["GBps"] = round(nbytes / t[0] / 1e6, 1)
                    row["frac"] = round(nbytes / t[0] / 1e6 / PEAK_HBM_GBS, 4)
                else:
                    row["floor_us"] = round(t[0] * 1e3, 2)
            if M in (1, 16):
                wb = pre[name]["wb"]
                xb = base["x"].to(torch.bfloat16)
                try:
                    body, calls = cycle([lambda w=w: F.linear(xb, w) for w in wb])
                    g = graph_of(body, torch)
                    t = time_groups(g, calls, torch)
                    del g
                    bbytes = 2 * N * K + 2 * M * K + 2 * M * N
                    row["bf16_linear_us"] = round(t[0] * 1e3, 2)
                    row["bf16_linear_GBps"] = round(bbytes / t[0] / 1e6, 1)
                    row["int8_speedup_vs_bf16"] = round(t[0] * 1e3 / row["us"], 2)
                except RuntimeError as e:  # capture refused: say so, no number
                    row["bf16_linear_us"] = None
                    row["bf16_linear_note"] = str(e)[:120]
            rows.append(row)
            del base
    return rows


def bench_verify_batch(ops, torch, steps):
    """Rejection-sampling verification (spec_decode/verify.py) at the C3 verify
    shape: B = 8 sequences, k = 6 draft tokens, vocab 151936, fp32 draft and
    target logits. Bytes: every logit once (row statistics) + the two rows the
    residual race rereads per sequence."""
    B, k, V = 8, 6, 151936
    g = torch.Generator(device="cuda")
    g.manual_seed(0)
    tl = torch.randn((B, k + 1, V), generator=g, device="cuda") * 3
    dl = tl[:, :k] + torch.randn((B, k, V), generator=g, device="cuda")
    toks = torch.randint(0, V, (B, k), generator=g, device="cuda")
    temps = torch.ones(B, device="cuda")
    st = torch.tensor([1, 0], dtype=torch.int64, device="cuda")
    g_ = graph_of(lambda: ops.verify_batch(dl, tl, toks, temps, rng_state=st), torch)
    ms = time_replays([g_], steps, 5, torch)
    nbytes = B * (2 * k + 1) * V * 4 + B * 2 * V * 4
    return {"config": "verify_batch B=8 k=6 vocab 151936 fp32 logits", "us": round(ms * 1e3, 2),
            "GBps": round(nbytes / ms / 1e6, 1), "bytes": nbytes}


def bench_prefill(ops, torch, steps):
    """Prefill attention (flash_attn_varlen_func's causal varlen form): B = 4
    sequences of 2048 tokens, Qwen3-4B attention 32q/8kv/128, bf16, contiguous
    K/V. FLOPs: 4 D Hq per visible (query, key) pair, sum over t of (t + 1) keys."""
    B, L, hq, hkv = 4, 2048, 32, 8
    g = torch.Generator(device="cuda")
    g.manual_seed(0)
    q = torch.randn((B * L, hq, 128), generator=g, device="cuda").to(torch.bfloat16)
    k = torch.randn((B * L, hkv, 128), generator=g, device="cuda").to(torch.bfloat16)
    v = torch.randn((B * L, hkv, 128), generator=g, device="cuda").to(torch.bfloat16)
    cu = torch.arange(0, (B + 1) * L, L, dtype=torch.int32, device="cuda")
    out = torch.empty_like(q)
    g_ = graph_of(lambda: ops.prefill_attention(q, k, v, cu, cu, L, 128 ** -0.5, out=out), torch)
    ms = time_replays([g_], steps, 3, torch)
    flops = 4 * 128 * hq * B * (L * (L + 1) // 2)
    return {"config": "prefill B=4 x 2048 tokens, 32q/8kv/128 bf16, causal", "us": round(ms * 1e3, 2),
            "TFLOPs": round(flops / ms / 1e9, 1),
            "frac_of_bf16_peak": round(flops / ms / 1e9 / 2500.0, 4)}


def preload_draft_chains(torch):
    """The C5 draft models (weights, then their paged KV caches) for B in {1, 16},
    built first in the process with the C4 weights (see `preload_w8a16`)."""
    from specdec_nanovllm_amd.draft_chain import DraftChain
    chains = {B: DraftChain(B, ctx_len=2048, k=6, seed=B) for B in (1, 16)}
    torch.cuda.synchronize()
    return chains


def bench_draft_chain(workloads_mod, torch, chains, reps=5):
    """C5: hipGraph-captured k = 6 greedy draft steps of a random-init
    Qwen3-0.6B (28 layers, all linears W8A16, paged bf16 KV with a 2048-token
    context) at B in {1, 16}, with the neighbour ops as eager torch (the C5
    protocol) and as this library's fused kernels: us per draft step and
    algorithmic GB/s. The fused rows' attention / GEMV split comes from a kernel
    trace of the chain (`c5_kernel_split`); the graph-timed figures (attention =
    store + paged attention, GEMV = the W8A16 linears, each captured as its own
    graph over the same shapes) stay beside it as `*_graph_us`."""
    rows = []
    for B in (1, 16):
        ch = chains.pop(B)
        parts = {}
        for name, fn in (("attention", ch.attention_chain), ("gemv", ch.gemv_chain)):
            g = graph_of(fn, torch)
            parts[name] = time_groups(g, ch.k, torch, groups=5, min_launches=ch.k)[0] * 1e3
            del g
        for fused in (False, True):
            ch.fused = fused
            g = graph_of(ch.chain, torch)
            tt = time_groups(g, ch.k, torch, groups=5, min_launches=ch.k)
            step = tt[0] * 1e3
            del g
            out = {"config": f"C5 draft chain B={B} ctx 2048 k=6, neighbours "
                             + ("fused HIP kernels" if fused else "eager torch"),
                   "step_us": round(step, 2),
                   "step_minmax_us": [round(tt[1] * 1e3, 2), round(tt[2] * 1e3, 2)],
                   "attention_graph_us": round(parts["attention"], 2),
                   "gemv_graph_us": round(parts["gemv"], 2),
                   "GBps": round(ch.step_bytes() / step / 1e3, 1),
                   "attention_graph_share": round(parts["attention"] / step, 3),
                   "gemv_graph_share": round(parts["gemv"] / step, 3),
                   "bytes_per_step": ch.step_bytes()}
            rows.append(out)
        del ch
        torch.cuda.empty_cache()
    for out in rows:
        if out["config"].endswith("fused HIP kernels"):
            B = int(out["config"].split("B=")[1].split()[0])
            print(f"bench: C5 B={B} kernel trace (rocprofv3 child process)", file=sys.stderr,
                  flush=True)
            kt = c5_kernel_split(B)
            out["kernel_trace"] = kt
            if "error" not in kt:
                out["attention_share"] = kt["attention_share"]
                out["gemv_share"] = kt["gemv_share"]
    return rows


TRACED_REPLAYS = 4  # chain replays between the markers of --draft-chain-only
MARKER_KERNEL = "stream_read_kernel"


def c5_kernel_split(B, timeout_s=240):
    """The fused C5 chain's kernel time by class, from a kernel trace: this script
    re-run as a child process under `rocprofv3 --kernel-trace` with
    `--draft-chain-only B`, which replays the captured chain TRACED_REPLAYS times
    between two launches of the streaming-read kernel (a kernel the chain never
    launches); only the dispatches between the two markers count (no context
    prefill, no setup). Attention = the q/k norm + RoPE + store launch and both
    paged-attention launches; GEMV = every W8A16 launch (the decoder linears and
    lm_head); other = the rest (norms, sampler, embedding lookup). Returns us per
    draft step per class and the shares of the summed kernel time, or
    {"error": ...}."""
    import csv
    import glob
    import shutil
    import subprocess
    import tempfile
    prof = shutil.which("rocprofv3") or "/opt/rocm/bin/rocprofv3"
    tmp = tempfile.mkdtemp(prefix="c5trace_", dir="/tmp")
    cmd = [prof, "--kernel-trace", "--output-format", "csv", "-d", tmp, "-o", "c5", "--",
           sys.executable, os.path.abspath(__file__), "--draft-chain-only", str(B)]
    try:
        env = dict(os.environ, TMPDIR=tmp)
        r = subprocess.run(cmd, cwd=tmp, env=env, stdout=subprocess.PIPE,
                           stderr=subprocess.STDOUT, timeout=timeout_s, text=True)
        info = None
        for line in r.stdout.splitlines():
            if line.startswith("{") and "draft_chain_only" in line:
                info = json.loads(line)
        trace = glob.glob(os.path.join(tmp, "**", "c5_kernel_trace.csv"), recursive=True)
        if info is None or not trace:  # (rocprofv3 may end with 139 after whole results)
            return {"error": f"rocprofv3 rc={r.returncode}: " + r.stdout[-300:]}
        rows = sorted(((int(d["Start_Timestamp"]), int(d["End_Timestamp"]), d["Kernel_Name"])
                       for d in csv.DictReader(open(trace[0]))), key=lambda t: t[0])
        marks = [i for i, t in enumerate(rows) if MARKER_KERNEL in t[2]]
        if len(marks) < 2:
            return {"error": f"{len(marks)} marker dispatches in the trace"}
        chain = rows[marks[-2] + 1:marks[-1]]
        steps = info["traced_replays"] * info["steps_per_chain"]
        mains = sum("paged_attn_main" in t[2] for t in chain)
        if mains != steps * info["layers"]:
            return {"error": f"{mains} attention launches between the markers, expected "
                             f"{steps * info['layers']}"}
        ns = {"attention": 0, "gemv": 0, "other": 0}
        for t0, t1, name in chain:
            cls = ("attention" if "paged_attn" in name or "qk_norm_rope" in name
                   else "gemv" if "w8a16" in name else "other")
            ns[cls] += t1 - t0
        tot = sum(ns.values())
        out = {"source": f"rocprofv3 --kernel-trace, {info['traced_replays']} replays of the "
                         f"captured chain ({steps} draft steps, {len(chain)} dispatches)",
               "kernel_us_per_step": round(tot / steps / 1e3, 2),
               "launches_per_step": round(len(chain) / steps, 1),
               "span_us_per_step": round((chain[-1][1] - chain[0][0]) / steps / 1e3, 2)}
        for k, v in ns.items():
            out[f"{k}_us"] = round(v / steps / 1e3, 2)
            out[f"{k}_share"] = round(v / tot, 3) if tot else None
        return out
    except Exception as e:  # the split is a report; the bench line stands without it
        return {"error": f"{type(e).__name__}: {e}"}
    finally:
        shutil.rmtree(tmp, ignore_errors=True)


# ---------------------------------------------------------------------------- profile
def twin_pass(ops, workloads, torch):
    """The attention main kernel (`twin="main"`) and its read-only floor twin, three
    launches each: C2 decode B=32, then C3 verify (plain attention), so counter runs
    can set the main kernel's instructions and waits against its access pattern's."""
    dev = "cuda"
    c = workloads.decode_case(32, seed=0, sets=1)
    bt, lens = c["tables"][0].to(dev), c["lens"].to(dev)
    out = torch.empty_like(c["q"])
    ws = torch.empty(ops.paged_attention_workspace_bytes(32, 1, 32, 8, bt.shape[1] * 256,
                                                         device=dev),
                     dtype=torch.uint8, device=dev)
    for twin in ("main", "floor"):
        for _ in range(3):
            ops.paged_attention(c["q"], c["k_cache"], c["v_cache"], bt, c["scale"],
                                context_lens=lens, out=out, twin=twin, workspace=ws)
    v = workloads.verify_case(seed=0, sets=1)
    vt, cuq, cuk = v["tables"][0].to(dev), v["cu_q"].to(dev), v["cu_k"].to(dev)
    vo = torch.empty_like(v["q"])
    vws = torch.empty(ops.paged_attention_workspace_bytes(8, v["k"] + 1, 32, 8,
                                                          vt.shape[1] * 256, device=dev),
                      dtype=torch.uint8, device=dev)
    for twin in ("main", "floor"):
        for _ in range(3):
            ops.paged_attention(v["q"], v["k_cache"], v["v_cache"], vt, v["scale"],
                                cu_seqlens_k=cuk, cu_seqlens_q=cuq, max_seqlen_q=v["k"] + 1,
                                out=vo, twin=twin, workspace=vws)
    torch.cuda.synchronize()
    print(json.dumps({"twin_pass": True}))


def profile_pass(ops, workloads, torch):
    """A few launches of each kernel plus a 512 MiB device copy (known bytes) so
    rocprofv3 counter runs can be scaled; prints what ran."""
    case = workloads.decode_case(32, seed=0, sets=1)
    bt = case["tables"][0].cuda()
    lens = case["lens"].cuda()
    out = torch.empty_like(case["q"])
    for _ in range(3):
        ops.paged_attention(case["q"], case["k_cache"], case["v_cache"], bt, case["scale"],
                            context_lens=lens, out=out)
    src = torch.empty(512 * 2 ** 20, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    c = workloads.w8a16_case(1, 151936, 1024, seed=1)
    for _ in range(3):
        ops.w8a16_linear(c["x"], c["w"], c["s"])
    del src, dst
    # the kernels where MFMA does the contraction (for the MFMA-utilization pass):
    # C3 verify (fused store), lm_head at M = 56, prefill; in this order, 3 each
    v = workloads.verify_case(seed=0)
    vt, vcu_k, vcu_q, vsl = v["table"].cuda(), v["cu_k"].cuda(), v["cu_q"].cuda(), v["slots"].cuda()
    vo = torch.empty_like(v["q"])
    for _ in range(3):
        ops.paged_attention(v["q"], v["k_cache"], v["v_cache"], vt, v["scale"],
                            cu_seqlens_k=vcu_k, cu_seqlens_q=vcu_q, max_seqlen_q=v["k"] + 1,
                            out=vo, key=v["k_new"], value=v["v_new"], slot_mapping=vsl)
    c56 = workloads.w8a16_case(56, 151936, 1024, seed=2)
    for _ in range(3):
        ops.w8a16_linear(c56["x"], c56["w"], c56["s"])
    B, L, hq, hkv = 4, 2048, 32, 8
    g = torch.Generator(device="cuda").manual_seed(5)
    pq = torch.randn((B * L, hq, 128), generator=g, device="cuda").to(torch.bfloat16)
    pk = torch.randn((B * L, hkv, 128), generator=g, device="cuda").to(torch.bfloat16)
    pv = torch.randn((B * L, hkv, 128), generator=g, device="cuda").to(torch.bfloat16)
    cu = torch.arange(0, (B + 1) * L, L, dtype=torch.int32, device="cuda")
    po = torch.empty_like(pq)
    for _ in range(3):
        ops.prefill_attention(pq, pk, pv, cu, cu, L, 128 ** -0.5, out=po)
    torch.cuda.synchronize()
    print(json.dumps({"profile_pass": True, "attn_bytes": attn_bytes(case["lens"].tolist(),
                                                                     32, 8, 128, 2),
                      "copy_bytes": 2 * 512 * 2 ** 20,
                      "lm_head_bytes": 151936 * 1024 + 2 * 151936 + 2048 + 2 * 151936,
                      "verify_flops": 4 * 128 * hq * sum(
                          sum(int(K) - v["k"] + i for i in range(v["k"] + 1)) for K in v["keys"]),
                      "lm_head_m56_flops": 2 * 56 * 151936 * 1024,
                      "prefill_flops": 4 * 128 * hq * B * L * (L + 1) // 2}))


# ------------------------------------------------------------------------------- main
def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures the one-GPU hot path only: every box in this build has a "
              "single GPU; run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch
    import __graft_entry__
    __graft_entry__.load_package()
    from specdec_nanovllm_amd import ops, workloads

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(1)
    if args.profile_pass:
        profile_pass(ops, workloads, torch)
        return
    if args.twin_pass:
        twin_pass(ops, workloads, torch)
        return
    if args.draft_chain_only:
        from specdec_nanovllm_amd.draft_chain import DraftChain
        ch = DraftChain(args.draft_chain_only, ctx_len=2048, k=6, seed=args.draft_chain_only,
                        fused=True)
        g = graph_of(ch.chain, torch)
        step = time_replays([g], 5, 1, torch) * 1e3 / ch.k
        # the chain ran once eagerly before capture, then in the settle phase, once
        # more and 5 timed times; then TRACED_REPLAYS more between two launches of
        # the streaming-read kernel over 4 KiB, which the chain never launches: a
        # kernel trace's dispatches between the two markers are these replays
        marker = torch.zeros(4096, dtype=torch.uint8, device="cuda")
        sink = torch.zeros(4, dtype=torch.int32, device="cuda")
        ops.stream_read(marker, sink, 1)
        torch.cuda.synchronize()
        for _ in range(TRACED_REPLAYS):
            g.replay()
        torch.cuda.synchronize()
        ops.stream_read(marker, sink, 1)
        torch.cuda.synchronize()
        print(json.dumps({"draft_chain_only": args.draft_chain_only, "fused": True,
                          "step_us": round(step, 2), "steps_per_chain": ch.k,
                          "layers": ch.L, "traced_replays": TRACED_REPLAYS}), flush=True)
        return

    B = args.batch
    hq, hkv, d = 32, 8, 128
    probe = workloads.decode_case(B, seed=0, sets=1, device="cpu", num_blocks=2048,
                                  num_q_heads=1, num_kv_heads=1, head_dim=8)
    pages = sum(math.ceil(int(L) / 256) for L in probe["lens"])
    sets = max(1, min(6, 2048 // pages))
    del probe
    case = workloads.decode_case(B, seed=0, sets=sets)
    lens = case["lens"]
    lens_d = lens.cuda()
    tables = [t.cuda() for t in case["tables"]]
    slots = [s.cuda() for s in case["slots"]]
    kc, vc, q = case["k_cache"], case["v_cache"], case["q"]
    out = torch.empty_like(q)
    # the extras' weights (C4 copies, C5 draft models) right after the headline's
    # KV cache and before anything is freed: both allocations are fresh, as in a
    # serving process, which loads its weights and allocates its KV cache once
    w8_pre = preload_w8a16(workloads, torch) if not args.no_extra else None
    c5_pre = (preload_draft_chains(torch)
              if not args.no_extra and not args.no_draft_chain else None)

    def step_fn(i):
        # store_kvcache of the new rows + attention: one fused launch (+ combine)
        return lambda: ops.paged_attention(q, kc, vc, tables[i], case["scale"],
                                           context_lens=lens_d, out=out, key=case["k_new"],
                                           value=case["v_new"], slot_mapping=slots[i])

    def main_fn(i):
        return lambda: ops.paged_attention(q, kc, vc, tables[i], case["scale"],
                                           context_lens=lens_d, out=out, main_only=True)

    def attn_fn(i):
        return lambda: ops.paged_attention(q, kc, vc, tables[i], case["scale"],
                                           context_lens=lens_d, out=out)

    # measurement twins: the main kernel's loads alone (read-only floor), and the
    # merge alone over the workspace a main-only call left for each page set
    ws_bytes = ops.paged_attention_workspace_bytes(B, 1, hq, hkv,
                                                   tables[0].shape[1] * 256, device="cuda")
    twin_ws = [torch.empty(ws_bytes, dtype=torch.uint8, device="cuda") for _ in range(sets)]

    def floor_fn(i):
        return lambda: ops.paged_attention(q, kc, vc, tables[i], case["scale"],
                                           context_lens=lens_d, out=out, twin="floor",
                                           workspace=twin_ws[i])

    def combine_fn(i):
        return lambda: ops.paged_attention(q, kc, vc, tables[i], case["scale"],
                                           context_lens=lens_d, out=out, twin="combine",
                                           workspace=twin_ws[i])

    step_graphs = [graph_of(step_fn(i), torch) for i in range(sets)]

    def chain(make):
        # one graph launching the kernel once per page set, the cycle repeated to
        # >= MIN_GRAPH_CALLS launches: back-to-back launches with no host gap
        # between them, each on cold pages (the other sets stream more than the
        # MALL holds before a set comes back)
        return cycle([make(i) for i in range(sets)])[0]
    roof_calls = cycle([None] * sets)[1]
    main_graphs = [graph_of(chain(main_fn), torch)]
    attn_graphs = [graph_of(chain(attn_fn), torch)]
    floor_graphs = [graph_of(chain(floor_fn), torch)]
    for i in range(sets):  # fill each set's workspace once for the combine twin
        ops.paged_attention(q, kc, vc, tables[i], case["scale"], context_lens=lens_d, out=out,
                            twin="main", workspace=twin_ws[i])
    combine_graphs = [graph_of(chain(combine_fn), torch)]
    # the timed chain: chain_len(steps) consecutive steps cycling over the page
    # sets (each set's pages are cold again when it comes back: the other sets
    # stream more than the MALL holds in between)
    n_chain = chain_len(args.steps, sets)
    step_fns = [step_fn(i % sets) for i in range(n_chain)]
    step_chain = graph_of(lambda: [f() for f in step_fns], torch)
    step_chain.steps = n_chain

    # ---- timed region: exactly `steps` decode steps (each a full fused store +
    #      attention over its own page set), `sets` of them per graph
    torch.cuda.synchronize()
    ms_step = time_steps(step_chain, step_graphs, args.steps, args.warmup, torch)
    ms_step_graph = time_replays(step_graphs, args.steps, args.warmup, torch)
    step_bytes = decode_bytes(lens.tolist(), hq, hkv, d, 2, B)
    value = step_bytes / (ms_step * 1e-3) / 1e9

    # ---- dominant kernel: attention main kernel alone, HIP events on the launching
    #      (current) stream around graph chains of back-to-back launches: the median
    #      of 5 groups of >= 20 launches, whatever --steps is (min / max beside it)
    t_main = time_groups(main_graphs[0], roof_calls, torch)
    t_attn = time_groups(attn_graphs[0], roof_calls, torch)
    t_floor = time_groups(floor_graphs[0], roof_calls, torch)
    t_comb = time_groups(combine_graphs[0], roof_calls, torch)
    ms_main, ms_attn, ms_floor, ms_comb = t_main[0], t_attn[0], t_floor[0], t_comb[0]
    a_bytes = attn_bytes(lens.tolist(), hq, hkv, d, 2)
    achieved = a_bytes / (ms_main * 1e-3) / 1e9
    ceiling = read_ceiling(ops, torch)
    ceiling["frac"] = round(achieved / ceiling["read_GBps"], 4)

    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) q/K/V, seeded page permutations)",
        "config": {"workload": f"C2 decode step B={B}: store_kvcache + paged decode attention, "
                               "Qwen3-4B attention 32q/8kv/128, ctx U[512,4096], 256-token "
                               f"pages, 2048-page pool, {sets} disjoint page sets, one "
                               f"step per set in turn, {n_chain} consecutive steps per HIP graph",
                   "batch": B, "context_lens_sum": int(lens.sum()),
                   "steps_per_graph": n_chain,
                   "algorithmic_bytes_per_step": step_bytes,
                   "frac_of_peak": round(value / PEAK_HBM_GBS, 4)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4),
                     "traffic": load_traffic("paged_attn_main_c2_b32"),
                     "kernel": "paged_attn_main", "algorithmic_bytes": a_bytes,
                     "avg_us": round(ms_main * 1e3, 2),
                     "avg_minmax_us": [round(t_main[1] * 1e3, 2), round(t_main[2] * 1e3, 2)],
                     "timing": "median of 5 groups of >= 20 launches (graph chains of "
                               f"{roof_calls} launches cycling over {sets} page sets), HIP "
                               "events on the launching stream",
                     "floor_us": round(ms_floor * 1e3, 2),
                     "floor_minmax_us": [round(t_floor[1] * 1e3, 2),
                                         round(t_floor[2] * 1e3, 2)],
                     "ceiling": ceiling,
                     "floor_note": "sd_paged_attention_floor: the same grid, loads and "
                                   "prefetch with no math (the access pattern's time)",
                     "traffic_note": "bytes per launch from the committed rocprofv3 "
                                     "FETCH_SIZE/WRITE_SIZE passes (profiles/traffic.json), "
                                     "not measured in this run"},
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline_decode(case, torch)
    if not args.no_extra:
        del step_graphs, main_graphs, attn_graphs, step_chain, floor_graphs, combine_graphs
        del twin_ws
        extra = {"attention_op_us": round(ms_attn * 1e3, 2),
                 "attention_op_minmax_us": [round(t_attn[1] * 1e3, 2), round(t_attn[2] * 1e3, 2)],
                 "attention_main_us": round(ms_main * 1e3, 2),
                 "attention_combine_us": round(ms_comb * 1e3, 2),
                 "attention_combine_minmax_us": [round(t_comb[1] * 1e3, 2),
                                                 round(t_comb[2] * 1e3, 2)],
                 "attention_floor_us": round(ms_floor * 1e3, 2),
                 "step_us": round(ms_step * 1e3, 2),
                 "step_us_one_graph_per_step": round(ms_step_graph * 1e3, 2)}
        del case, kc, vc
        torch.cuda.empty_cache()
        extra["decode_batches"] = [bench_decode_batch(ops, workloads, torch, b, args.steps)
                                   for b in (1, 8)]
        torch.cuda.empty_cache()
        extra["decode_ctx_sweep_b1"] = bench_ctx_sweep(ops, workloads, torch)
        torch.cuda.empty_cache()
        extra["verify"] = bench_verify(ops, workloads, torch, args.steps)
        torch.cuda.empty_cache()
        extra["w8a16"] = bench_w8a16(ops, workloads, torch, min(args.steps, 100), w8_pre)
        del w8_pre
        if not args.no_cpu_baseline:
            extra["cpu_baselines"] = cpu_baselines_extra(torch, workloads,
                                                         workloads.verify_case(seed=0))
            torch.cuda.empty_cache()
        torch.cuda.empty_cache()
        extra["verify_batch"] = bench_verify_batch(ops, torch, min(args.steps, 100))
        torch.cuda.empty_cache()
        extra["prefill"] = bench_prefill(ops, torch, min(args.steps, 50))
        torch.cuda.empty_cache()
        if not args.no_draft_chain:
            extra["draft_chain"] = bench_draft_chain(workloads, torch, c5_pre)
        line["extra"] = extra
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
