#!/usr/bin/env python3
"""Benchmark of the trellis kernel layer on one MI355X ("us/layer & compressed-weight HBM GB/s (% of
peak) at batch 1/8/32; decode tok/s").

Headline (`value`): BASELINE config 2, the dense attention-block layer (qkv 2048->5120 int6, o 4096->2048 int6,
shared-expert gate/up 2048->2x512 int5 and down 512->2048 int5, all 4-bit trellis; four launches a layer, one per vLLM
layer) at batch 1, as compressed-weight GB/s: algorithmic bytes (trellis + suh + svh of the four launches) over the
time per layer. Weights are cold: a HIP graph replays the layer over enough distinct weight copies (>= 1 GiB) that
the 256 MB MALL cannot serve them. A step is one replay of that graph; inputs are resident in HBM.

Also reported: us/layer at batch 8 and 32; BASELINE config 1 (one 2048x2048 int6 matrix); config 3 (route_group);
config 4 (a 256-expert MoE layer, fused routing + six launches, T = 1, 4, 32); config 5 (the synthetic 40-layer decoder
of vllm_espalier/step.py: greedy decode us/step and tok/s, one HIP graph a step, and 512-token prefill in 32-row
windows); `roofline` of the dominant kernel (the qkv dense launch: average launch time from a graph of cold
launches, with HIP events on the launch stream); and
`cpu_baseline`: the reference's CPU path on this host (this repo's C restatement of the dequantisation, multithreaded,
then fp32 Hadamards and torch.matmul), on a bounded sample of the same layer.

usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-moe] [--no-decoder]

Comparing two builds (how changes are judged): `python bench.py --compare` times the workloads a change is decided
on (the dense block at 1 and 32 rows, the MoE layer at 1 / 4 / 32 tokens, the decode step, the config-2 prompt block
at 512 rows and the tile prefill) and prints one JSON line; `--package DIR` runs it (or any mode) on the package in
DIR (a directory holding `vllm_espalier`, e.g. another checkout's `vllm-espalier_amd`, built there) instead of this
repository's. Alternate the two builds in one session on one GPU: runs of one build agree to ~0.2 %, boxes ~1.5 %.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
PACKAGE_ROOT = REPO / "vllm-espalier_amd"
if "--package" in sys.argv[:-1]:              # before any import of vllm_espalier (see --package)
    PACKAGE_ROOT = Path(sys.argv[sys.argv.index("--package") + 1]).resolve()
sys.path.insert(0, str(PACKAGE_ROOT))

PEAK_GBS = 8000.0            # MI355X HBM3E, public spec
COLD_BYTES = 1 << 30         # distinct weight bytes a cold graph streams
CSRC = REPO / "vllm-espalier_amd" / "vllm_espalier" / "csrc"
# HBM bytes a qkv launch moves at batch 1, written by `bench.py --traffic-record` from the two rocprofv3 --pmc passes
# (FETCH_SIZE, then WRITE_SIZE) over `bench.py --traffic-probe`, each scaled by what the counter reads for a plain
# copy of known size. The record names the hash of the kernel sources it was measured on; the bench reports its
# traffic only while the sources still hash the same, and null otherwise.
TRAFFIC_RECORD = REPO / "profiles" / "dense_qkv_batch1_traffic.json"
ROOFLINE_KERNEL = "dense_kernel<23, 8, 1>"


def kernel_sources_sha() -> str:
    """sha256 of the sources the dense kernel is compiled from."""
    import hashlib
    h = hashlib.sha256()
    for name in ("dense.hip", "dense.hpp", "common.hpp", "trellis.hpp", "gemm.hpp", "norm.hpp"):
        h.update(name.encode())
        h.update((CSRC / name).read_bytes())
    return h.hexdigest()[:16]


def recorded_traffic():
    """(bytes per qkv launch, note): the record's traffic if it was measured on these kernel sources, else None."""
    if not TRAFFIC_RECORD.exists():
        return None, "no traffic record"
    rec = json.loads(TRAFFIC_RECORD.read_text())
    if rec.get("sources_sha") != kernel_sources_sha():
        return None, f"record measured on other kernel sources ({rec.get('sources_sha')}); unmeasured for this build"
    return rec["bytes"], f"rocprofv3 FETCH_SIZE x {rec['fetch_factor']:.3f} + WRITE_SIZE x {rec['write_factor']:.3f}"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def graph_of(fn):
    import torch
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


def time_graph(g, reps: int, warmup: int = 2) -> float:
    """ms per replay, from HIP events on the current stream."""
    import torch
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    st.record()
    for _ in range(reps):
        g.replay()
    en.record()
    torch.cuda.synchronize()
    return st.elapsed_time(en) / reps


# ---------------------------------------------------------------------------------------------------------------
# workloads
# ---------------------------------------------------------------------------------------------------------------
def dense_block(gen, dev):
    """BASELINE config 2's four launches: [qkv], [o], [shared gate, up], [shared down]."""
    from vllm_espalier import dense as D, workloads as WL
    q = [WL.matrix(2048, 4096, 4, "int6", gen, dev), WL.matrix(2048, 512, 4, "int6", gen, dev),
         WL.matrix(2048, 512, 4, "int6", gen, dev)]
    o = [WL.matrix(4096, 2048, 4, "int6", gen, dev)]
    gu = [WL.matrix(2048, 512, 4, "int5", gen, dev), WL.matrix(2048, 512, 4, "int5", gen, dev)]
    dn = [WL.matrix(512, 2048, 4, "int5", gen, dev)]
    return [D.Dense(q), D.Dense(o), D.Dense(gu), D.Dense(dn)]


def block_bytes(block) -> int:
    from vllm_espalier import workloads as WL
    return sum(WL.nbytes(d.mats) for d in block)


def dense_stack(copies: int, seed: int, dev):
    import torch
    gen = torch.Generator(device=dev).manual_seed(seed)
    return [dense_block(gen, dev) for _ in range(copies)]


def run_dense(stack, M: int, dev, which=None):
    """A graph over every copy of the block at M rows (which: the launch indices to include)."""
    import torch
    gen = torch.Generator(device=dev).manual_seed(1000 + M)
    xs = {K: torch.randn((M, K), generator=gen, device=dev).to(torch.bfloat16) for K in (512, 2048, 4096)}
    outs = [[torch.empty((M, d.n_out), dtype=torch.bfloat16, device=dev) for d in block] for block in stack]
    idx = range(4) if which is None else which

    def fn():
        for block, ob in zip(stack, outs):
            for i in idx:
                block[i].forward(xs[block[i].K], out=ob[i])
    return graph_of(fn)


CHAIN_W = 8                 # waves a workgroup of the chained block (step.ATTN_W, the decoder's qkv -> o launch)


def run_dense_multi(stack, M: int, dev, chain: bool, W: int = 16):
    """A graph over every copy of the block as ONE esp_dense_multi launch a copy (W waves a workgroup for every
    group): the four groups side by side on their own inputs ("in one launch per layer"), or
    chained, each group reading the previous group's output (o reads q, gate/up reads o's output, down reads the gate
    half), every consumer waiting for its producer inside the launch."""
    import torch
    from vllm_espalier import dense as D
    gen = torch.Generator(device=dev).manual_seed(2000 + M)
    xs = {K: torch.randn((M, K), generator=gen, device=dev).to(torch.bfloat16) for K in (512, 2048, 4096)}
    multis, ios = [], []
    for block in stack:
        m = D.DenseMulti(block, after=[False, chain, chain, chain], W=W)
        outs = [torch.empty((M, d.n_out), dtype=torch.bfloat16, device=dev) for d in block]
        if chain:
            ins = [xs[2048], outs[0][:, :4096], outs[1], outs[2][:, :512]]
        else:
            ins = [xs[d.K] for d in block]
        multis.append(m)
        ios.append((ins, outs))

    def fn():
        for m, (ins, outs) in zip(multis, ios):
            m.forward(ins, outs)
    return graph_of(fn)


def run_dense_prompt(stack, T: int, dev):
    """A graph over every copy of the block as prompt launches (Dense.forward_tile) over T rows."""
    import torch
    gen = torch.Generator(device=dev).manual_seed(3000 + T)
    xs = {K: torch.randn((T, K), generator=gen, device=dev).to(torch.bfloat16) for K in (512, 2048, 4096)}
    outs = [[torch.empty((T, d.n_out), dtype=torch.bfloat16, device=dev) for d in block] for block in stack]

    def fn():
        for block, ob in zip(stack, outs):
            for d, o in zip(block, ob):
                d.forward_tile(xs[d.K], out=o)
    return graph_of(fn)


# ---------------------------------------------------------------------------------------------------------------
# MoE (config 4)
# ---------------------------------------------------------------------------------------------------------------
def moe_layer(gen, dev, E=256, D=2048, I=512):
    import torch
    from vllm_espalier import experts as G, workloads as WL
    widths = torch.randint(1, 4, (E,), generator=gen, device=dev).tolist()
    grid = {1: "e2m1", 2: "e2m1", 3: "int5"}
    experts = [tuple(WL.matrix(k, n, b, grid[b], gen, dev) for k, n in ((D, I), (D, I), (I, D))) for b in widths]
    shared = tuple(WL.matrix(k, n, 4, "int5", gen, dev) for k, n in ((D, I), (D, I), (I, D)))
    gate_w = (torch.randn((D,), generator=gen, device=dev) * 0.05).to(torch.bfloat16)
    router = (torch.randn((E, D), generator=gen, device=dev) * 0.02).to(torch.bfloat16)
    L = G.prepare(experts, shared, gate_w)
    return L, experts, shared, router


def bench_moe(dev, steps: int, layers: int = 8, passes: int = 16, rows=(1, 4, 32)):
    """Config 4 (route_group + the six-launch MoE layer) and config 3 (route_group alone). A replay runs `passes`
    passes over `layers` distinct 256-expert layers (1.6 GB of expert weights), each (pass, layer) with its own input
    rows, so the experts picked change from one call to the next and a replay reads well over 1 GiB of picked-expert
    bytes at one token (the 256 MB MALL cannot serve them from one replay to the next). Algorithmic bytes: trellis +
    suh + svh of every distinct expert a call picks, plus the shared expert, summed over the calls."""
    import torch
    from vllm_espalier import experts as G, workloads as WL
    gen = torch.Generator(device=dev).manual_seed(4)
    stack = [moe_layer(gen, dev) for _ in range(layers)]
    calls = [(p, l) for p in range(passes) for l in range(layers)]
    res = {}
    for T in rows:
        xg = torch.Generator(device=dev).manual_seed(40 + T)
        xs = {c: torch.randn((T, 2048), generator=xg, device=dev).to(torch.bfloat16) for c in calls}
        s = G.scratch(stack[0][0], 32, 9, dev)
        outs = (torch.empty((T, 2048), dtype=torch.bfloat16, device=dev),
                torch.empty((T, 2048), dtype=torch.bfloat16, device=dev))
        nbytes = 0
        for c in calls:                       # the experts each call picks, for its algorithmic bytes
            L, experts, shared, router = stack[c[1]]
            G.route(xs[c], router, 8, L, s)
            torch.cuda.synchronize()
            ids = s.ids[:int(s.count.item())].tolist()
            nbytes += sum(WL.nbytes(experts[e]) if e < 256 else WL.nbytes(shared) for e in ids)

        def fn():
            for c in calls:
                L, experts, shared, router = stack[c[1]]
                G.route(xs[c], router, 8, L, s)
                G.routed2(xs[c], None, None, L, s, out=outs[0], out_shared=outs[1], k=8)
        g = graph_of(fn)
        ms = time_graph(g, steps)
        del g
        us = ms * 1000 / len(calls)
        gbs = nbytes / len(calls) / (us * 1e-6) / 1e9
        res[str(T)] = {"us_per_layer": round(us, 2), "bytes_per_layer": nbytes // len(calls), "GBps": round(gbs, 1),
                       "pct_peak": round(100 * gbs / PEAK_GBS, 1), "picked_bytes_per_replay": nbytes}
        log(f"moe T={T}: {us:.2f} us/layer, {gbs:.0f} GB/s ({100 * gbs / PEAK_GBS:.1f}% of peak), "
            f"{nbytes / 2**30:.2f} GiB of picked experts a replay")
    # the router alone (config 3): its 1 MiB bf16 weight a layer stays in the MALL (8 layers), so this is warm; then
    # cold, over 1024 distinct routers
    rt = {}
    for T in (1, 32):
        xg = torch.Generator(device=dev).manual_seed(70 + T)
        xs = [torch.randn((T, 2048), generator=xg, device=dev).to(torch.bfloat16) for _ in stack]
        s = G.scratch(stack[0][0], 32, 9, dev)

        def fr():
            for (L, experts, shared, router), x in zip(stack, xs):
                G.route(x, router, 8, L, s)
        ms = time_graph(graph_of(fr), steps)
        rt[str(T)] = {"us_per_call": round(ms * 1000 / len(stack), 2), "weights": "MALL-warm",
                      "entry": "esp_route_group_own (logits an all-ones hand-off buffer)"}
        log(f"route_group T={T}: {ms * 1000 / len(stack):.2f} us")
        # the reference's contract (esp_route_group: logits plain scratch, arrivals counted)
        plain = torch.zeros((T * 257,), dtype=torch.float32, device=dev)
        ids, members = s.window(T)

        def fp():
            for (L, experts, shared, router), x in zip(stack, xs):
                G.ext().route_group(x, router, L.gate_w, 8, L.shared_id, plain, s.route_counter, s.pick[:T * 9],
                                    s.wts[:T * 9], ids, s.count, members)
        ms = time_graph(graph_of(fp), steps)
        rt[str(T)]["plain_logits_us_per_call"] = round(ms * 1000 / len(stack), 2)
        log(f"route_group T={T}, plain logits (esp_route_group): {ms * 1000 / len(stack):.2f} us")
    # and cold: one call on each of 1024 distinct 1 MiB router weights (1 GiB a replay, past the 256 MB MALL)
    L0 = stack[0][0]
    routers = [(torch.randn((256, 2048), generator=gen, device=dev) * 0.02).to(torch.bfloat16) for _ in range(1024)]
    for T in (1, 32):
        xg = torch.Generator(device=dev).manual_seed(90 + T)
        x = torch.randn((T, 2048), generator=xg, device=dev).to(torch.bfloat16)
        s = G.scratch(L0, 32, 9, dev)

        def fc():
            for r in routers:
                G.route(x, r, 8, L0, s)
        ms = time_graph(graph_of(fc), max(3, steps // 2))
        rt[str(T)]["cold_us_per_call"] = round(ms * 1000 / len(routers), 2)
        log(f"route_group T={T}, cold router weights: {ms * 1000 / len(routers):.2f} us")
    # the decoder's routing launch at one token, route_group_rmsnorm: the residual add and RMSNorm inside, the logits
    # an all-ones hand-off polled by the last workgroup (no arrival count), over the same 1024 cold routers
    xg = torch.Generator(device=dev).manual_seed(95)
    h, d1 = (torch.randn((1, 2048), generator=xg, device=dev).to(torch.bfloat16) for _ in range(2))
    nw = (1 + 0.1 * torch.randn((2048,), generator=xg, device=dev)).to(torch.bfloat16)
    h_out, a_out = torch.empty_like(h), torch.empty_like(h)
    s = G.scratch(L0, 32, 9, dev)

    def fn_norm():
        for r in routers:
            G.route_rmsnorm(h, d1, nw, 1e-6, h_out, a_out, r, 8, L0, s)
    ms = time_graph(graph_of(fn_norm), max(3, steps // 2))
    rt["1"]["rmsnorm_cold_us_per_call"] = round(ms * 1000 / len(routers), 2)
    log(f"route_group_rmsnorm T=1, cold router weights: {ms * 1000 / len(routers):.2f} us")
    del stack, routers
    torch.cuda.empty_cache()
    return res, rt


# ---------------------------------------------------------------------------------------------------------------
# config 5: the synthetic 40-layer decoder (dense block + route + MoE a layer, mcg LM head), greedy decode and
# windowed prefill
# ---------------------------------------------------------------------------------------------------------------
def bench_decoder(dev, steps: int, warmup: int, layers: int = 40, prefill_tokens: int = 512):
    import torch
    from vllm_espalier import step as S
    t0 = time.perf_counter()
    dec = S.SyntheticDecoder(n_layers=layers, seed=5, device=dev)
    torch.cuda.synchronize()
    log(f"decoder: {layers} layers built in {time.perf_counter() - t0:.1f} s")
    b = dec.buffers(1)
    b.ids_in.fill_(1)
    picks = []
    dec.forward(1, picks=picks)                  # eager: the experts each layer reads, for the bytes of a step
    step_bytes = dec.algorithmic_bytes(picks, 1)

    def decode_step():
        dec.forward(1)
        b.ids_in.copy_(b.ids_out)                # greedy: the argmax is the next input, on the device
    g = graph_of(decode_step)
    ms = time_graph(g, steps, warmup)
    del g
    us = ms * 1000
    gbs = step_bytes / (us * 1e-6) / 1e9
    res = {"layers": layers, "us_per_step": round(us, 1), "tok_per_s": round(1e6 / us, 1),
           "bytes_per_step": step_bytes, "GBps": round(gbs, 1), "pct_peak": round(100 * gbs / PEAK_GBS, 1)}
    log(f"decode step: {us:.1f} us, {1e6 / us:.1f} tok/s, {step_bytes / 1e9:.3f} GB a step, {gbs:.0f} GB/s")

    # prefill: prefill_tokens ids in windows of 32 rows, the head on the last window only
    W = S.Dn.MAX_ROWS
    bw = dec.buffers(W)
    gen = torch.Generator(device=dev).manual_seed(55)
    ids_all = torch.randint(0, dec.vocab, (prefill_tokens,), generator=gen, device=dev, dtype=torch.int32)
    nwin = prefill_tokens // W

    def prefill():
        for w in range(nwin):
            bw.ids_in.copy_(ids_all[w * W:(w + 1) * W])
            dec.forward(W, head=(w == nwin - 1))
    g = graph_of(prefill)
    ms = time_graph(g, max(3, steps // 4), 1)
    del g
    res["prefill"] = {"tokens": nwin * W, "window": W, "ms": round(ms, 3), "tok_per_s": round(nwin * W / (ms * 1e-3), 1)}
    log(f"prefill: {nwin * W} tokens in {ms:.2f} ms, {nwin * W / (ms * 1e-3):.0f} tok/s")
    # the tile prefill: prompt launches for the dense layers and the head, the MoE over the whole prompt
    T = nwin * W
    bp = dec.prefill_buffers(T)
    bp.ids_in.copy_(ids_all[:T])

    def prefill_tile():
        dec.prefill(T)
    g = graph_of(prefill_tile)
    ms = time_graph(g, max(3, steps // 4), 1)
    del g
    res["prefill_tile"] = {"tokens": T, "ms": round(ms, 3), "tok_per_s": round(T / (ms * 1e-3), 1),
                           "mode": "dense layers and head as prompt launches (128 rows a workgroup), routing in one "
                                   "launch, each layer's MoE grouped over the whole prompt"}
    log(f"prefill (tile): {T} tokens in {ms:.2f} ms, {T / (ms * 1e-3):.0f} tok/s")
    del dec
    torch.cuda.empty_cache()
    return res


# ---------------------------------------------------------------------------------------------------------------
# CPU baseline: the reference's CPU path (dequantisation + torch matmul) on this host
# ---------------------------------------------------------------------------------------------------------------
def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(block, reps: int):
    import numpy as np
    import torch
    sys.path.insert(0, str(REPO / "oracle"))
    import oracle as O            # the C restatement of the reference dequantisation (cpu_baseline leg only)
    from vllm_espalier import experts as G
    affinity = len(os.sched_getaffinity(0))
    # the job's CPU share: OMP_NUM_THREADS where the host sets it (16 for one GPU on the MI355X boxes), else every
    # core of the affinity mask
    cores = min(affinity, int(os.environ.get("OMP_NUM_THREADS", affinity)))
    torch.set_num_threads(cores)
    H = torch.from_numpy(O.sylvester() / np.sqrt(128.0)).float()
    mats = [[(m.trellis.cpu().numpy(), 2 * m.K, G.KERNEL_CB[m.cb], m.suh.float().cpu(), m.svh.float().cpu())
             for m in d.mats] for d in block]
    x = {K: torch.randn((1, K)) for K in (512, 2048, 4096)}

    def had(v):
        return (v.view(*v.shape[:-1], -1, 128) @ H).view(v.shape)

    def layer():
        for launch in mats:
            for t, k2, cb, suh, svh in launch:
                W = torch.from_numpy(O.dequant_f32(t, k2, cb, cores))
                xv = x[W.shape[0]]
                _ = had(had(xv * suh) @ W) * svh
    layer()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        layer()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    return med, cores, affinity


# ---------------------------------------------------------------------------------------------------------------
# HBM traffic of the roofline kernel: the workload rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs read
# ---------------------------------------------------------------------------------------------------------------
CALIB_BYTES = 256 << 20


def traffic_probe(dev) -> None:
    """Two replays of the roofline graph (98 cold qkv launches at batch 1, as in the bench), one of the same launches
    at 32 rows, and two copies of CALIB_BYTES, the plain copy kernel whose counters scale the qkv launch's (a copy
    reads and writes its size)."""
    import torch
    probe = dense_stack(1, 1, dev)
    copies = max(2, -(-COLD_BYTES // block_bytes(probe[0])))
    del probe
    stack = dense_stack(copies, 2, dev)
    g = run_dense(stack, 1, dev, which=[0])
    for _ in range(2):
        g.replay()
    del g
    g = run_dense(stack, 32, dev, which=[0])          # the 32-row tiles (dense_kernel<23, 8, 2>), for MFMA use
    g.replay()
    del g
    src = torch.ones(CALIB_BYTES // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(2):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"traffic probe: {copies} qkv launches x 2 at 1 row, x 1 at 32 rows, copy of {CALIB_BYTES} B x 2")


def _counter_avgs(d: str, counter: str) -> dict:
    """Average per-dispatch value of `counter` by (kernel name with template arguments, grid size) in a rocprofv3
    csv directory."""
    import csv
    from collections import defaultdict
    f = next(Path(d).rglob("*counter_collection.csv"))
    acc = defaultdict(list)
    for r in csv.DictReader(open(f)):
        if r["Counter_Name"] == counter:
            grid = r.get("Grid_Size") or r.get("Grid_Size_X", "?")
            acc[(r["Kernel_Name"].replace("void ", "").split("(")[0], grid)].append(float(r["Counter_Value"]))
    return {k: sum(v) / len(v) for k, v in acc.items()}


def traffic_record(fetch_dir: str, write_dir: str) -> dict:
    """The traffic record from the FETCH_SIZE and WRITE_SIZE passes over --traffic-probe: the qkv launch's KiB a
    dispatch, each scaled by what the counter reads for the probe's copy of CALIB_BYTES (it reads and writes them;
    the copy is the copy kernel dispatch of the largest grid)."""
    fetch, write = _counter_avgs(fetch_dir, "FETCH_SIZE"), _counter_avgs(write_dir, "WRITE_SIZE")
    kern = next(k for k in fetch if k[0].endswith(ROOFLINE_KERNEL))
    copy = max((k for k in fetch if "copyBuffer" in k[0]), key=lambda k: int(k[1]) if k[1].isdigit() else 0)
    kib = CALIB_BYTES / 1024
    ff, wf = kib / fetch[copy], kib / write[copy]
    rec = {"kernel": kern[0], "grid": kern[1], "copy_grid": copy[1], "fetch_kib": round(fetch[kern], 1), "write_kib": round(write[kern], 1),
           "copy_fetch_kib": round(fetch[copy], 1), "copy_write_kib": round(write[copy], 1),
           "fetch_factor": round(ff, 4), "write_factor": round(wf, 4),
           "bytes": int(round((fetch[kern] * ff + write[kern] * wf) * 1024)), "sources_sha": kernel_sources_sha()}
    return rec


def counter_probe(dev) -> None:
    """The workload of the shader-counter passes over the expert kernels and the LM head: 8 cold 256-expert layers
    at 1 token (route_group, then the chained layer, esp_moe_chain) and at 32 tokens (route_group, rot_in, the
    grouped gate/up launch, its epilogue, the grouped down launch, down_combine2), one replay each, then 8 cold
    chained config-2 blocks at one row (esp_dense_multi), then two cold LM-head launches (2048 x 151936, 6-bit mcg) at one row, then two cold config-2 blocks
    as prompt launches over 512 rows (esp_dense_tile), then two cold 256-expert layers over a 512-token prompt
    (experts.prefill)."""
    import torch
    from vllm_espalier import dense as D, experts as G, workloads as WL
    gen = torch.Generator(device=dev).manual_seed(4)
    stack = [moe_layer(gen, dev) for _ in range(8)]
    for T in (1, 32):
        xs = [torch.randn((T, 2048), device=dev).to(torch.bfloat16) for _ in stack]
        s = G.scratch(stack[0][0], 32, 9, dev)
        o = (torch.empty((T, 2048), dtype=torch.bfloat16, device=dev), torch.empty((T, 2048), dtype=torch.bfloat16,
                                                                                   device=dev))

        def fn():
            for (L, experts, shared, router), x in zip(stack, xs):
                G.route(x, router, 8, L, s)
                G.routed2(x, None, None, L, s, out=o[0], out_shared=o[1], k=8)
        graph_of(fn).replay()
    del stack
    # the chained config-2 block at one row as the decoder runs it (esp_dense_multi, CHAIN_W waves: qkv -> o ->
    # shared gate/up -> down in one launch, consumers decoding ahead), 8 cold copies
    run_dense_multi(dense_stack(8, 13, dev), 1, dev, True, CHAIN_W).replay()
    heads = [D.Dense([WL.matrix(2048, 151936, 6, "mcg", gen, dev)]) for _ in range(2)]
    x = torch.randn((1, 2048), device=dev).to(torch.bfloat16)
    y = torch.empty((1, 151936), dtype=torch.bfloat16, device=dev)
    graph_of(lambda: [h.forward(x, out=y) for h in heads]).replay()
    del heads
    g = run_dense_prompt(dense_stack(2, 12, dev), 512, dev)
    g.replay()
    del g
    # two cold 256-expert layers over a whole 512-token prompt (experts.prefill: route_rows, one grouping, the tile
    # list, the grouped launches over it, the epilogues)
    stack = [moe_layer(gen, dev) for _ in range(2)]
    ps = G.prefill_scratch(stack[0][0], 512, 9, dev)
    xs = [torch.randn((512, 2048), device=dev).to(torch.bfloat16) for _ in stack]
    o = (torch.empty((512, 2048), dtype=torch.bfloat16, device=dev),
         torch.empty((512, 2048), dtype=torch.bfloat16, device=dev))

    def fp():
        for (L, experts, shared, router), x in zip(stack, xs):
            G.prefill(x, None, None, L, ps, 8, gate=router, out=o[0], out_shared=o[1])
    graph_of(fp).replay()
    torch.cuda.synchronize()
    log("counter probe: 8 MoE layers at 1 and 32 tokens, 8 chained dense blocks at one row, 2 LM-head launches at "
        "one row, 2 dense blocks over 512 rows, 2 MoE layers over a 512-token prompt")


# ---------------------------------------------------------------------------------------------------------------
# ceilings (--probes): launch floor, streaming read rate, VALU issue rates, from libespalier_probe.so
# ---------------------------------------------------------------------------------------------------------------
VALU_OPS = ["v_add_u32", "v_mul_lo_u32", "v_bfe_u32", "v_perm_b32", "v_fma_mix_f32", "v_pk_add_f16",
            "v_add_f16 (SDWA)"]


def probes(dev) -> dict:
    """The device ceilings the kernels are held to, measured here: (1) the launch floor, an empty kernel of
    256 workgroups, as us a launch in a graph of 1000; (2) the streaming read rate of a 2 GiB buffer (16-byte
    nontemporal loads, 8 workgroups of 256 threads a CU); (3) each decode instruction's issue rate, 8 independent
    chains a lane, one and four waves a SIMD, as lane operations a CU a clock (at the reported peak clock)."""
    import ctypes
    import torch
    L = ctypes.CDLL(str(REPO / "vllm-espalier_amd" / "vllm_espalier" / "libespalier_probe.so"))
    P, I64 = ctypes.c_void_p, ctypes.c_int64
    L.esp_probe_empty.argtypes = [I64, P]
    L.esp_probe_read.argtypes = [P, I64, P, I64, P]
    L.esp_probe_valu.argtypes = [ctypes.c_int, ctypes.c_int, I64, ctypes.c_int, P, P]
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    khz = L.esp_probe_clock_khz()
    out = {"cus": cus, "clock_mhz": khz / 1000}

    def stream():
        return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    n = 1000
    g = graph_of(lambda: [L.esp_probe_empty(256, stream()) for _ in range(n)])
    out["launch_floor_us"] = round(time_graph(g, 5) * 1000 / n, 3)
    del g
    nbytes = 2 << 30
    buf = torch.ones(nbytes // 4, dtype=torch.int32, device=dev)
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    g = graph_of(lambda: L.esp_probe_read(buf.data_ptr(), nbytes, sink.data_ptr(), 8 * cus, stream()))
    ms = time_graph(g, 10)
    out["read_GBps"] = round(nbytes / (ms * 1e-3) / 1e9, 1)
    del g, buf
    rates = {}
    iters = 20000
    for op, name in enumerate(VALU_OPS):
        for waves_per_simd in (1, 4):
            g = graph_of(lambda: L.esp_probe_valu(op, iters, cus, 4 * waves_per_simd, sink.data_ptr(), stream()))
            ms = time_graph(g, 5)
            lane_ops = cus * 4 * waves_per_simd * 64 * 8 * iters
            rates[f"{name} @{waves_per_simd}w"] = round(lane_ops / (ms * 1e-3) / (cus * khz * 1e3), 1)
            del g
    out["valu_lane_ops_per_cu_clk"] = rates
    # random lookups into a shared-memory table (the codebook-table decode's inner operation), lookups a CU a clock
    L.esp_probe_lds.argtypes = [ctypes.c_int, ctypes.c_int, I64, ctypes.c_int, P, P]
    lds = {}
    for wide, name in ((0, "u8 of 64 KiB"), (1, "u16 of 128 KiB")):
        for waves in (4, 16):
            iters = 4000
            if L.esp_probe_lds(wide, iters, cus, waves, sink.data_ptr(), stream()) != 0:
                raise RuntimeError("esp_probe_lds failed")
            g = graph_of(lambda: L.esp_probe_lds(wide, iters, cus, waves, sink.data_ptr(), stream()))
            ms = time_graph(g, 5)
            lookups = cus * waves * 64 * 8 * iters
            lds[f"{name} @{waves} waves"] = round(lookups / (ms * 1e-3) / (cus * khz * 1e3), 1)
            del g
    out["lds_lookups_per_cu_clk"] = lds
    for k, v in out.items():
        log(f"probe {k}: {v}")
    return out


# ---------------------------------------------------------------------------------------------------------------
# rocprofv3 summaries (the text kept under profiles/)
# ---------------------------------------------------------------------------------------------------------------
def rocprof_summary(d: str, top: int = 80) -> str:
    """Markdown from a `rocprofv3 --kernel-trace --stats --output-format csv -o run` directory: the --stats table
    of this library's kernels, then per-dispatch durations grouped by kernel and launch shape (grid and workgroup, in
    threads), from the kernel trace. Durations in microseconds."""
    import csv
    from collections import defaultdict
    root = Path(d)
    stats = next(root.rglob("*kernel_stats.csv"), None)
    trace = next(root.rglob("*kernel_trace.csv"), None)
    out = []
    if stats is not None:
        rows = [r for r in csv.DictReader(open(stats)) if "esp::" in r["Name"]]
        rows.sort(key=lambda r: -float(r["TotalDurationNs"]))
        out += ["`rocprofv3 --stats` (kernel_stats.csv), kernels of this library:", "",
                "| kernel | calls | avg us | min us | max us | total ms |", "|---|---:|---:|---:|---:|---:|"]
        for r in rows[:top]:
            n = r["Name"].replace("void ", "").split("(")[0]
            out.append(f"| `{n}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | {float(r['MinNs']) / 1e3:.2f} | "
                       f"{float(r['MaxNs']) / 1e3:.2f} | {float(r['TotalDurationNs']) / 1e6:.2f} |")
        out.append("")
    if trace is not None:
        groups = defaultdict(list)
        for r in csv.DictReader(open(trace)):
            if "esp::" not in r["Kernel_Name"]:
                continue
            n = r["Kernel_Name"].replace("void ", "").split("(")[0]
            shape = (f"{r.get('Grid_Size_X', '?')}x{r.get('Grid_Size_Y', '?')}x{r.get('Grid_Size_Z', '?')} / "
                     f"{r.get('Workgroup_Size_X', '?')}")
            groups[(n, shape)].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
        items = sorted(groups.items(), key=lambda kv: -sum(kv[1]))
        out += ["Kernel trace (kernel_trace.csv), dispatches grouped by kernel and launch shape (grid x*y*z threads / "
                "workgroup threads):", "", "| kernel | launch shape | calls | avg us | median us | min us | max us |",
                "|---|---|---:|---:|---:|---:|---:|"]
        for (n, shape), v in items[:top]:
            v = sorted(v)
            out.append(f"| `{n}` | {shape} | {len(v)} | {sum(v) / len(v):.2f} | {v[len(v) // 2]:.2f} | {v[0]:.2f} | "
                       f"{v[-1]:.2f} |")
        out.append("")
    pmc = next(root.rglob("*counter_collection.csv"), None)
    if pmc is not None:
        groups = defaultdict(list)
        for r in csv.DictReader(open(pmc)):
            if "esp::" not in r["Kernel_Name"] and "copyBuffer" not in r["Kernel_Name"]:
                continue
            n = r["Kernel_Name"].replace("void ", "").split("(")[0]
            shape = r.get("Grid_Size") or f"{r.get('Grid_Size_X', '?')}x{r.get('Grid_Size_Y', '?')}x{r.get('Grid_Size_Z', '?')}"
            groups[(n[:80], shape, r["Counter_Name"])].append(float(r["Counter_Value"]))
        items = sorted(groups.items(), key=lambda kv: (kv[0][0], kv[0][1], kv[0][2]))
        out += ["Counters (counter_collection.csv), per dispatch, grouped by kernel, grid size (threads) and counter:", "",
                "| kernel | grid | counter | dispatches | average | min | max |", "|---|---|---|---:|---:|---:|---:|"]
        for (n, shape, c), v in items[:8 * top]:
            out.append(f"| `{n}` | {shape} | {c} | {len(v)} | {sum(v) / len(v):.1f} | {min(v):.1f} | {max(v):.1f} |")
        out.append("")
    return "\n".join(out)


# ---------------------------------------------------------------------------------------------------------------
PHASE_ROOT = CSRC / "_phase"         # csrc/build.py --phase-trace puts the timing copy of the package here
PHASE_NAMES = ("start", "copies issued", "rows ready", "K loop (wave 0)", "partials stored", "arrived last",
               "finished")


def phase_trace(dev) -> dict:
    """Where a batch-1 dense launch spends its time, from the timing build (csrc/build.py --phase-trace: thread 0 of
    every workgroup records the 100 MHz real-time counter at each phase of the launch, dense.hpp). Each of config 2's
    four launches runs in a graph of 24 back-to-back launches over one weight copy (timed with HIP events), then one
    more replay whose last launch's records are read back. Times are ns from the launch's first workgroup start;
    each phase is the median (and 90th percentile) over workgroups of the time since the previous phase, the
    finisher's phases over the finishers (the last split of each column block to arrive)."""
    import ctypes
    import numpy as np
    import torch
    import vllm_espalier
    pkg = Path(vllm_espalier.__file__).resolve().parent
    if pkg.parent != PHASE_ROOT.resolve():
        raise RuntimeError(f"--phase-trace needs the timing build (csrc/build.py --phase-trace); imported {pkg}")
    lib = ctypes.CDLL(str(pkg / "libespalier_hip.so"))
    lib.esp_phase_read.argtypes = [ctypes.c_void_p, ctypes.c_int64]
    words = 8192 * 8
    buf = np.zeros(words, dtype=np.uint64)
    gen = torch.Generator(device=dev).manual_seed(3)
    block = dense_block(gen, dev)
    res = {}
    for M in (1, 32):
        for d, nm in zip(block, ("qkv", "o", "shared gate/up", "shared down")):
            x = torch.randn((M, d.K), generator=gen, device=dev).to(torch.bfloat16)
            y = torch.empty((M, d.n_out), dtype=torch.bfloat16, device=dev)
            reps = 24

            def fn():
                for _ in range(reps):
                    d.forward(x, out=y)
            g = graph_of(fn)
            us = time_graph(g, 20) * 1000 / reps
            if lib.esp_phase_clear() != 0:
                raise RuntimeError("esp_phase_clear failed")
            g.replay()
            torch.cuda.synchronize()
            if lib.esp_phase_read(buf.ctypes.data, words) != 0:
                raise RuntimeError("esp_phase_read failed")
            del g
            t = buf.reshape(-1, 8).astype(np.int64)
            wg = np.nonzero(t[:, 0] > 0)[0]
            T = t[wg]
            rel = (T[:, :7] - T[:, 0].min()) * 10
            fin = (T[:, 7] >> 8) & 1 == 1
            xcd = T[:, 7] & 0xF

            def stat(v):
                return {"p50": float(np.median(v)), "p90": float(np.percentile(v, 90))}
            ph = {PHASE_NAMES[0]: stat(rel[:, 0])}
            for i in range(1, 5):
                ph[PHASE_NAMES[i]] = stat(rel[:, i] - rel[:, i - 1])
            for i in (5, 6):
                ph[PHASE_NAMES[i]] = stat(rel[fin, i] - rel[fin, i - 1])
            res[f"{nm}, M={M}"] = {
                "us_per_launch": round(us, 2), "workgroups": int(len(wg)), "finishers": int(fin.sum()),
                "span_us": round(float(rel[fin, 6].max()) / 1000, 2),
                "stored_p50_us": round(float(np.median(rel[:, 4])) / 1000, 2),
                "xcd_is_workgroup_mod_8": bool(np.all(xcd == wg % 8)), "phases_ns": ph}
            log(f"phase trace {nm} M={M}: {us:.2f} us a launch, span {res[f'{nm}, M={M}']['span_us']} us")
    return res


# ---------------------------------------------------------------------------------------------------------------
# --sweep: the measurements behind the shape rules dense.plan, dense.tile_plan and experts.tile_config (the
# reference's --sweep / --cold, tests/gpu_dense.py:127-202, and tests/gpu_grouped_sweep.py, with its --force-cb)
# ---------------------------------------------------------------------------------------------------------------
def sweep(dev, force_cb: int = -1) -> dict:
    """Cold sweeps on the BASELINE shapes, each candidate timed as a graph over >= 1 GiB of distinct weights (so
    nothing is served from the 256 MB MALL):
      * dense decode plan (dense.plan): config 2's four launches at 1 and 32 rows, every K split SK (uneven splits
        allowed) and 4 / 8 / 16 waves a workgroup; the LM head (2048 x 151936, 6-bit mcg) at one row, 1-4 splits;
      * prompt K splits (dense.tile_plan): the same launches as prompt launches over 128, 512 and 2048 rows;
      * grouped tile config (experts.tile_config): the config-4 MoE layer (8 cold 256-expert layers, fused routing)
        at 1, 4 and 32 tokens, gate/up and down each at 4 / 8 waves and every power-of-two K split. force_cb >= 0
        decodes every expert with that kernel codebook (the same bytes, wrong values), to see what share of the time
        is decode arithmetic.
    Each line gives the best candidates and the rule's choice; the rules themselves depend on the shape alone, so a
    row's bits never depend on the batch."""
    import torch
    from vllm_espalier import dense as D, experts as G
    sms = torch.cuda.get_device_properties(dev).multi_processor_count
    out = {"dense_plan": {}, "tile_plan": {}, "tile_config": {}}
    probe = dense_stack(1, 1, dev)
    copies = max(2, -(-COLD_BYTES // block_bytes(probe[0])))
    del probe
    stack = dense_stack(copies, 5, dev)
    names = ("qkv", "o", "shared gate/up", "shared down")
    for M in (1, 32):
        for i, nm in enumerate(names):
            ds = [blk[i] for blk in stack]
            K, N = ds[0].K, ds[0].N
            x = torch.randn((M, K), device=dev).to(torch.bfloat16)
            ys = [torch.empty((M, d.n_out), dtype=torch.bfloat16, device=dev) for d in ds]
            keep = [d.plans for d in ds]
            res = []
            for sk in sorted({1, 2, 3, 4, 6, 8, 12, 16, 24, 32} & set(range(1, K // 128 + 1))):
                for w in (4, 8, 16):
                    for d in ds:
                        d.plans = [(sk, w, 2)] * len(d.launches)
                    D.scratch(dev, sk * D.MAX_ROWS * N, 0)
                    g = graph_of(lambda: [d.forward(x, out=y) for d, y in zip(ds, ys)])
                    res.append((round(time_graph(g, 10, 2) * 1000 / len(ds), 3), sk, w))
                    del g
            for d, p in zip(ds, keep):
                d.plans = p
            res.sort()
            rule = D.plan(K, N, sms)[:2]
            t_rule = next(t for t, sk, w in res if (sk, w) == rule)
            out["dense_plan"][f"{nm}, M={M}"] = {"rule": list(rule), "rule_us": t_rule,
                                                "best": [list(r) for r in res[:6]]}
            log(f"sweep dense plan {nm} M={M}: rule {rule} {t_rule} us; best " +
                ", ".join(f"{t}({sk},{w})" for t, sk, w in res[:6]))
    # the LM head (2048 x 151936, 6-bit mcg) at one row: 4 cold copies (934 MB)
    from vllm_espalier import workloads as WL
    hgen = torch.Generator(device=dev).manual_seed(3)
    heads = [D.Dense([WL.matrix(2048, 151936, 6, "mcg", hgen, dev)]) for _ in range(4)]
    hx = torch.randn((1, 2048), device=dev).to(torch.bfloat16)
    hy = torch.empty((1, 151936), dtype=torch.bfloat16, device=dev)
    keep = heads[0].plans
    res = []
    for sk in (1, 2, 3, 4):
        for w in (4, 8, 16):
            for h in heads:
                h.plans = [(sk, w, 2)]
            D.scratch(dev, sk * D.MAX_ROWS * 151936, 0)
            g = graph_of(lambda: [h.forward(hx, out=hy) for h in heads])
            res.append((round(time_graph(g, 5, 1) * 1000 / len(heads), 2), sk, w))
            del g
    res.sort()
    rule = tuple(keep[0][:2])
    t_rule = next(t for t, sk, w in res if (sk, w) == rule)
    out["dense_plan"]["LM head, M=1"] = {"rule": list(rule), "rule_us": t_rule, "best": [list(r) for r in res[:6]]}
    log(f"sweep dense plan LM head M=1: rule {rule} {t_rule} us; best " +
        ", ".join(f"{t}({sk},{w})" for t, sk, w in res[:6]))
    del heads
    for T in (128, 512, 2048):
        for i, nm in enumerate(names):
            ds = [blk[i] for blk in stack[:8]]
            K, N = ds[0].K, ds[0].N
            x = torch.randn((T, K), device=dev).to(torch.bfloat16)
            ys = [torch.empty((T, d.n_out), dtype=torch.bfloat16, device=dev) for d in ds]
            res = []
            for sk in sorted({1, 2, 3, 4, 6, 8, 12, 16} & set(range(1, K // 128 + 1))):
                os.environ["ESPALIER_DENSE_PROMPT_SK"] = str(sk)
                for d in ds:
                    d.reserve_prompt(T)
                g = graph_of(lambda: [d.forward_tile(x, out=y) for d, y in zip(ds, ys)])
                res.append((round(time_graph(g, 5, 1) * 1000 / len(ds), 2), sk))
                del g
            os.environ.pop("ESPALIER_DENSE_PROMPT_SK", None)
            res.sort()
            rule = D.tile_plan(K, N)
            t_rule = next(t for t, sk in res if sk == rule)
            out["tile_plan"][f"{nm}, T={T}"] = {"rule": rule, "rule_us": t_rule, "best": [list(r) for r in res[:5]]}
            log(f"sweep prompt SK {nm} T={T}: rule {rule} {t_rule} us; best " +
                ", ".join(f"{t}({sk})" for t, sk in res[:5]))
    del stack
    torch.cuda.empty_cache()
    gen = torch.Generator(device=dev).manual_seed(4)
    layers = [moe_layer(gen, dev) for _ in range(8)]
    if force_cb >= 0:
        for L, *_ in layers:
            for c in L.cb:
                c.fill_(force_cb)
    for T in (1, 4, 32):
        xg = torch.Generator(device=dev).manual_seed(40 + T)
        xs = [torch.randn((T, 2048), generator=xg, device=dev).to(torch.bfloat16) for _ in range(16 * len(layers))]
        o = (torch.empty((T, 2048), dtype=torch.bfloat16, device=dev),
             torch.empty((T, 2048), dtype=torch.bfloat16, device=dev))
        res = []
        for wgu, skgu in ((4, 2), (4, 4), (4, 8), (4, 16), (8, 4), (8, 8)):
            for wd, skd in ((4, 1), (4, 2), (4, 4), (8, 2), (8, 4)):
                os.environ["ESPALIER_GROUPED_TILE_PLAN"] = f"{wgu},{skgu};{wd},{skd}"
                s = G.Scratch(256 + 1, 2048, 512, 32, 9, dev)
                calls = [(xs[i], layers[i % len(layers)]) for i in range(len(xs))]

                def fn():
                    for x, (L, _, _, router) in calls:
                        G.route(x, router, 8, L, s)
                        G.routed2(x, None, None, L, s, out=o[0], out_shared=o[1], k=8)
                g = graph_of(fn)
                res.append((round(time_graph(g, 5, 1) * 1000 / len(calls), 2), wgu, skgu, wd, skd))
                del g, s
        os.environ.pop("ESPALIER_GROUPED_TILE_PLAN", None)
        res.sort()
        rule = (G.tile_config(2048, 512, True)[1:3], G.tile_config(512, 2048, False)[1:3])
        key = (rule[0][0], rule[0][1], rule[1][0], rule[1][1])
        t_rule = next(r[0] for r in res if tuple(r[1:]) == key)
        out["tile_config"][f"T={T}"] = {"rule": list(key), "rule_us": t_rule, "best": [list(r) for r in res[:6]],
                                        "force_cb": force_cb}
        log(f"sweep grouped tile config T={T}: rule (w,sk gate/up; w,sk down) {key} {t_rule} us; best " +
            ", ".join(f"{r[0]}{tuple(r[1:])}" for r in res[:6]))
    return out


TILE_PHASE_NAMES = ("first stage landed", "K loop (wave 0)", "of which stage waits", "sums in shared memory",
                    "stored and arrived", "finisher")


def tile_phase_trace(dev) -> dict:
    """Where a prompt launch (esp_dense_tile) spends its time, from the same timing build (dense_tile.hip: thread 0 of
    every workgroup records the real-time counter at each phase, and sums its waits for the later stages). Config 2's
    four matrices at 512 rows and the LM head at one row, each in a graph of 8 back-to-back prompt launches (the
    rotation launch included in the time a launch), then one more replay whose last launch's records are read back.
    Each phase is the median (and 90th percentile) over workgroups of the ns since the previous phase; the
    finisher's over the finishers (the last split of each column block and row tile to arrive)."""
    import ctypes
    import numpy as np
    import torch
    import vllm_espalier
    from vllm_espalier import dense as D, workloads as WL
    pkg = Path(vllm_espalier.__file__).resolve().parent
    if pkg.parent != PHASE_ROOT.resolve():
        raise RuntimeError(f"--phase-trace needs the timing build (csrc/build.py --phase-trace); imported {pkg}")
    lib = ctypes.CDLL(str(pkg / "libespalier_hip.so"))
    lib.esp_tile_phase_read.argtypes = [ctypes.c_void_p, ctypes.c_int64]
    words = 8192 * 8
    buf = np.zeros(words, dtype=np.uint64)
    gen = torch.Generator(device=dev).manual_seed(3)
    block = dense_block(gen, dev)
    head = D.Dense([WL.matrix(2048, 151936, 6, "mcg", gen, dev)])
    cases = [(d, nm, 512) for d, nm in zip(block, ("qkv", "o", "shared gate/up", "shared down"))] + [(head, "head", 1)]
    res = {}
    for d, nm, T in cases:
        x = torch.randn((T, d.K), generator=gen, device=dev).to(torch.bfloat16)
        y = torch.empty((T, d.n_out), dtype=torch.bfloat16, device=dev)
        d.reserve_prompt(T)
        reps = 8
        g = graph_of(lambda: [d.forward_tile(x, out=y) for _ in range(reps)])
        us = time_graph(g, 10) * 1000 / reps
        if lib.esp_tile_phase_clear() != 0:
            raise RuntimeError("esp_tile_phase_clear failed")
        g.replay()
        torch.cuda.synchronize()
        if lib.esp_tile_phase_read(buf.ctypes.data, words) != 0:
            raise RuntimeError("esp_tile_phase_read failed")
        del g
        t = buf.reshape(-1, 8).astype(np.int64)
        wg = np.nonzero(t[:, 0] > 0)[0]
        R = t[wg]
        rel = (R[:, [0, 1, 3, 4, 5, 6]] - R[:, 0].min()) * 10
        waits = R[:, 2] * 10
        fin = (R[:, 7] >> 8) & 1 == 1

        def stat(v):
            return {"p50": float(np.median(v)), "p90": float(np.percentile(v, 90))}
        ph = {"first stage landed": stat(rel[:, 1] - rel[:, 0]), "K loop (wave 0)": stat(rel[:, 2] - rel[:, 1]),
              "of which stage waits": stat(waits), "sums in shared memory": stat(rel[:, 3] - rel[:, 2]),
              "stored and arrived": stat(rel[:, 4] - rel[:, 3])}
        if fin.any():
            ph["finisher"] = stat(rel[fin, 5] - rel[fin, 4])
            span = float(rel[fin, 5].max())
        else:
            span = float(rel[:, 4].max())
        res[f"{nm}, T={T}"] = {"us_per_launch": round(us, 2), "workgroups": int(len(wg)),
                               "stages": int(np.median((R[:, 7] >> 16) & 0xFFFF)), "span_us": round(span / 1000, 2),
                               "phases_ns": ph}
        log(f"tile phase trace {nm} T={T}: {us:.2f} us a launch, span {span / 1000:.2f} us")
    return res


def tile_phase_table(res: dict) -> str:
    """The markdown table of tile_phase_trace's result (medians, ns)."""
    head = ["prompt launch", "us a launch (graph, with its rotation)", "workgroups", "stages", *TILE_PHASE_NAMES,
            "last done (us)"]
    lines = ["| " + " | ".join(head) + " |", "|" + "---|" * len(head)]
    for k, r in res.items():
        ph = r["phases_ns"]
        cells = [k, f"{r['us_per_launch']:.2f}", f"{r['workgroups']}", f"{r['stages']}",
                 *(f"{ph[n]['p50']:.0f} ({ph[n]['p90']:.0f})" if n in ph else "-" for n in TILE_PHASE_NAMES),
                 f"{r['span_us']:.2f}"]
        lines.append("| " + " | ".join(cells) + " |")
    return "\n".join(lines)


def phase_table(res: dict) -> str:
    """The markdown table of phase_trace's result (medians, ns)."""
    head = ["launch", "us a launch (graph)", "workgroups", *PHASE_NAMES[1:], "last finisher done (us)"]
    lines = ["| " + " | ".join(head) + " |", "|" + "---|" * len(head)]
    for k, r in res.items():
        ph = r["phases_ns"]
        cells = [k, f"{r['us_per_launch']:.2f}", f"{r['workgroups']}",
                 *(f"{ph[n]['p50']:.0f} ({ph[n]['p90']:.0f})" for n in PHASE_NAMES[1:]), f"{r['span_us']:.2f}"]
        lines.append("| " + " | ".join(cells) + " |")
    return "\n".join(lines)


def compare(dev) -> dict:
    """The workloads a change is decided on, timed as graphs of cold weights (the bench's own helpers): us a layer for
    the dense block at 1 and 32 rows, the MoE layer at 1 / 4 / 32 tokens and the config-2 prompt block at 512 rows; us a
    decode step; ms and tok/s of the 512-token tile prefill."""
    import torch
    from vllm_espalier import step as S
    res = {}
    stack = dense_stack(98, 11, dev)
    for M in (1, 32):
        g = run_dense(stack, M, dev)
        res[f"dense_block_{M}_us"] = round(min(time_graph(g, 10, 2) for _ in range(2)) * 1000 / len(stack), 2)
        del g
    del stack
    moe = bench_moe(dev, 10, rows=(1, 4, 32))[0]
    for T, v in moe.items():
        res[f"moe_layer_{T}_us"] = v["us_per_layer"]
    stack = dense_stack(8, 11, dev)
    g = run_dense_prompt(stack, 512, dev)
    res["prompt_block_512_us"] = round(min(time_graph(g, 5, 1) for _ in range(2)) * 1000 / len(stack), 2)
    del g, stack
    dec = S.SyntheticDecoder(n_layers=40, seed=5, device=dev)
    b = dec.buffers(1)
    b.ids_in.fill_(1)
    dec.forward(1)

    def decode_step():
        dec.forward(1)
        b.ids_in.copy_(b.ids_out)
    g = graph_of(decode_step)
    res["decode_step_us"] = round(min(time_graph(g, 10, 3) for _ in range(3)) * 1000, 1)
    del g
    bp = dec.prefill_buffers(512)
    bp.ids_in.copy_(torch.arange(512, dtype=torch.int32, device=dev))
    dec.prefill(512)
    torch.cuda.synchronize()
    g = graph_of(lambda: dec.prefill(512))
    ms = min(time_graph(g, 3, 1) for _ in range(2))
    res["tile_prefill_512_ms"] = round(ms, 3)
    res["tile_prefill_512_tok_per_s"] = round(512 / ms * 1000, 1)
    for k, v in res.items():
        log(f"compare {k}: {v}")
    return res


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-moe", action="store_true")
    ap.add_argument("--no-decoder", action="store_true")
    ap.add_argument("--cpu-reps", type=int, default=20)
    ap.add_argument("--rocprof-summary", metavar="DIR", help="print the markdown summary of a rocprofv3 csv output "
                    "directory and exit (no GPU work)")
    ap.add_argument("--traffic-probe", action="store_true", help="run only the workload of the FETCH_SIZE / "
                    "WRITE_SIZE counter passes (the roofline graph and a calibration copy) and exit")
    ap.add_argument("--traffic-record", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"), help="write the traffic record "
                    f"({TRAFFIC_RECORD.relative_to(REPO)}) from the two rocprofv3 csv directories and exit")
    ap.add_argument("--counter-probe", action="store_true", help="run only the workload of the shader-counter "
                    "passes over the expert kernels and the LM head, and exit")
    ap.add_argument("--probes", action="store_true", help="measure the ceilings the kernels are held to (graph "
                    "launch floor, streaming read bandwidth, VALU issue rates) and exit")
    ap.add_argument("--phase-trace", action="store_true", help="time the phases of config 2's batch-1 launches and "
                    "of its prompt launches at 512 rows with the timing build (csrc/build.py --phase-trace) and exit")
    ap.add_argument("--sweep", action="store_true", help="cold sweeps behind dense.plan, dense.tile_plan and "
                    "experts.tile_config (one JSON line), and exit")
    ap.add_argument("--force-cb", type=int, default=-1, help="with --sweep: decode every expert with this kernel "
                    "codebook (same bytes, wrong values) to see the decode arithmetic's share")
    ap.add_argument("--compare", action="store_true", help="time the workloads two builds are compared on (one "
                    "JSON line), and exit")
    ap.add_argument("--package", metavar="DIR", help="import vllm_espalier from DIR instead of this repository")
    a = ap.parse_args()
    if a.rocprof_summary:
        print(rocprof_summary(a.rocprof_summary))
        return 0
    if a.traffic_record:
        rec = traffic_record(*a.traffic_record)
        TRAFFIC_RECORD.write_text(json.dumps(rec, indent=1) + "\n")
        print(json.dumps(rec))
        return 0
    if a.gpus != 1:
        print(f"bench.py: this build runs on one GPU (the reference path is single-GPU, TP=1); --gpus {a.gpus} is "
              "not supported", file=sys.stderr)
        return 2
    import torch
    if not torch.cuda.is_available():
        print("bench.py: no GPU", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    if a.phase_trace:                         # the timing copy of the package, in place of the product one
        sys.path[:] = [p for p in sys.path if Path(p).resolve() != (REPO / "vllm-espalier_amd").resolve()]
        sys.path.insert(0, str(PHASE_ROOT))
    from vllm_espalier import experts as G
    G.ext()                                   # the HIP extension must be there: no fallback
    name = torch.cuda.get_device_name(dev)
    log(f"device {name}")
    if a.compare:
        import vllm_espalier
        res = compare(dev)
        print(json.dumps({"compare": res, "package": str(Path(vllm_espalier.__file__).parent), "device": name}),
              flush=True)
        return 0
    if a.traffic_probe:
        traffic_probe(dev)
        return 0
    if a.counter_probe:
        counter_probe(dev)
        return 0
    if a.probes:
        print(json.dumps({"probes": probes(dev), "device": name}), flush=True)
        return 0
    if a.sweep:
        print(json.dumps({"sweep": sweep(dev, a.force_cb), "device": name}), flush=True)
        return 0
    if a.phase_trace:
        res = phase_trace(dev)
        tres = tile_phase_trace(dev)
        print(phase_table(res), flush=True)
        print(tile_phase_table(tres), flush=True)
        print(json.dumps({"phase_trace": res, "tile_phase_trace": tres, "device": name}), flush=True)
        return 0

    # ---- config 2 dense block, cold stack
    probe = dense_stack(1, 1, dev)
    bpl = block_bytes(probe[0])
    copies = max(2, -(-COLD_BYTES // bpl))
    del probe
    stack = dense_stack(copies, 2, dev)
    log(f"dense block: {bpl} algorithmic bytes a layer, {copies} cold copies ({copies * bpl / 2**30:.2f} GiB)")
    per_m = {}
    g1 = None
    for M in (1, 8, 32):
        g = run_dense(stack, M, dev)
        ms = time_graph(g, a.steps if M == 1 else max(5, a.steps // 2), a.warmup)
        us = ms * 1000 / copies
        gbs = bpl / (us * 1e-6) / 1e9
        per_m[str(M)] = {"us_per_layer": round(us, 3), "GBps": round(gbs, 1), "pct_peak": round(100 * gbs / PEAK_GBS, 1)}
        log(f"dense block M={M}: {us:.3f} us/layer, {gbs:.0f} GB/s ({100 * gbs / PEAK_GBS:.1f}% of peak)")
        if M == 1:
            g1 = g
        else:
            del g
    # the same block as one esp_dense_multi launch a layer: side by side (16 waves a workgroup), and chained (8, the
    # decoder's: two workgroups a CU, so a consumer that decoded ahead and waits leaves the other slot to a producer)
    multi = {"waves": {"independent": 16, "chain": CHAIN_W}}
    for chain in (False, True):
        key = "chain" if chain else "independent"
        multi[key] = {}
        for M in (1, 8, 32):
            g = run_dense_multi(stack, M, dev, chain, CHAIN_W if chain else 16)
            us = time_graph(g, a.steps if M == 1 else max(5, a.steps // 2), a.warmup) * 1000 / copies
            del g
            multi[key][str(M)] = {"us_per_layer": round(us, 3), "GBps": round(bpl / (us * 1e-6) / 1e9, 1)}
            log(f"dense block, one multi launch ({key}) M={M}: {us:.3f} us/layer, {bpl / (us * 1e-6) / 1e9:.0f} GB/s")
    # the same block over a prompt: the prompt launches (each weight decoded once for every 128 rows)
    prompt = {}
    flops_row = 2 * sum(d.K * d.N for d in stack[0])
    for T in (128, 512):
        g = run_dense_prompt(stack, T, dev)
        us = time_graph(g, max(3, a.steps // 4), 1) * 1000 / copies
        del g
        tf = flops_row * T / (us * 1e-6) / 1e12
        prompt[str(T)] = {"us_per_layer": round(us, 2), "tok_per_s": round(T / (us * 1e-6), 1),
                          "TFLOPs": round(tf, 1), "GBps": round(bpl / (us * 1e-6) / 1e9, 1)}
        log(f"dense block, prompt launches T={T}: {us:.2f} us/layer, {T / (us * 1e-6):.0f} rows/s, {tf:.1f} TFLOP/s")
    # the timed steps of the headline: a step = one replay over the cold stack at batch 1
    for _ in range(a.warmup):
        g1.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    st.record()
    for _ in range(a.steps):
        g1.replay()
    en.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = st.elapsed_time(en) / a.steps
    value = copies * bpl / (ms_step * 1e-3) / 1e9
    log(f"headline: {ms_step:.3f} ms a step ({copies} layers), {value:.0f} GB/s; wall {wall:.3f} s")
    del g1

    # ---- roofline of the dominant kernel: the qkv launch (5.27 MB), a graph of cold launches at batch 1
    gq = run_dense(stack, 1, dev, which=[0])
    ms = time_graph(gq, a.steps, a.warmup)
    from vllm_espalier import dense as D, workloads as WL
    qkv_bytes = WL.nbytes(stack[0][0].mats)
    q_us = ms * 1000 / copies
    achieved = qkv_bytes / (q_us * 1e-6) / 1e9
    log(f"qkv launch: {q_us:.3f} us, {achieved:.0f} GB/s")
    del gq
    per_launch = {}
    for i, nm in enumerate(("qkv", "o", "shared_gate_up", "shared_down")):
        if i == 0:
            per_launch[nm] = round(q_us, 3)
            continue
        gi = run_dense(stack, 1, dev, which=[i])
        per_launch[nm] = round(time_graph(gi, a.steps, a.warmup) * 1000 / copies, 3)
        del gi

    # ---- config 1: one 2048x2048 4-bit int6 matrix, cold
    gen = torch.Generator(device=dev).manual_seed(11)
    m1 = [D.Dense([WL.matrix(2048, 2048, 4, "int6", gen, dev)]) for _ in range(max(2, COLD_BYTES // 2105344))]
    x1 = torch.randn((1, 2048), device=dev).to(torch.bfloat16)
    o1 = torch.empty((1, 2048), dtype=torch.bfloat16, device=dev)
    g = graph_of(lambda: [d.forward(x1, out=o1) for d in m1])
    c1_us = time_graph(g, a.steps, a.warmup) * 1000 / len(m1)
    c1_gbs = WL.nbytes(m1[0].mats) / (c1_us * 1e-6) / 1e9
    log(f"config 1: {c1_us:.3f} us, {c1_gbs:.0f} GB/s")
    del g, m1

    cpu_block = stack[0]
    del stack
    torch.cuda.empty_cache()

    moe = route = None
    if not a.no_moe:
        moe, route = bench_moe(dev, max(5, a.steps // 2))
    decoder = None
    if not a.no_decoder:
        decoder = bench_decoder(dev, max(5, a.steps // 2), a.warmup)

    cpu = None
    if not a.no_cpu:
        med, cores, affinity = cpu_baseline(cpu_block, a.cpu_reps)
        cpu = {"value": round(bpl / med / 1e9, 4), "unit": "GB/s", "cores": cores, "kind": "port",
               "us_per_layer": round(med * 1e6, 1), "affinity_cores": affinity, "cpu_model": cpu_model(),
               "sample": f"median of {a.cpu_reps} forwards of one config-2 block at batch 1: C dequantisation "
                         f"(oracle/, {cores} threads) + fp32 Hadamards + torch.matmul"}
        log(f"cpu baseline: {med * 1e3:.1f} ms/layer on {cores} cores")

    traffic, traffic_note = recorded_traffic()
    out = {
        "metric": "compressed-weight HBM GB/s, config-2 dense block at batch 1 (us/layer at batch 1/8/32 and the MoE "
                  "layer alongside)",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded random trellis codes, N(0,1) bf16 activations)",
        "config": {"workload": f"BASELINE config 2 dense block (qkv/o int6, shared gate/up/down int5, 4-bit), batch 1, "
                               f"{copies} cold copies a step",
                   "bytes_per_layer": bpl, "layers_per_step": copies, "device": name},
        "dense_block": per_m,
        "dense_block_one_launch": multi,
        "dense_block_prompt": prompt,
        "dense_launch_us_batch1": per_launch,
        "config1_us": round(c1_us, 3),
        "config1_GBps": round(c1_gbs, 1),
        "moe_layer": moe,
        "route_group": route,
        "decoder": decoder,
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_GBS, 4), "traffic": traffic, "traffic_source": traffic_note,
                     "kernel": f"{ROOFLINE_KERNEL} (qkv launch, {qkv_bytes:,} B a launch)"},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
