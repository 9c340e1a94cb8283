#!/usr/bin/env python
"""Per-layer Bigger Bird v3 sparse prefill on one MI355X: the BASELINE metric (ms/layer @128K, effective TFLOP/s).

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--T 131072] [--no-cpu-baseline]

Workload: one attention layer, B=1, T=131072, 32 query / 8 KV heads, d=128, bf16 Q/K/V ~ N(0,1)
with Llama RoPE (theta 500000) on Q and K, 64 planted keys per KV head (4x the group-mean of the last 64 post-RoPE
queries, at seeded positions in [sink, T - window)), cfg {sink 64, window 16384, vertical 512, exact_tail 256}.
A step is RDAttention.sparse_prefill(q, k, v) -- routes, V^T, the sink+window+routed kernel, the exact tail -- with
the inputs resident in HBM (the reference's timed region, modal_rd/attn_bench.py:48). Q/K/V come from the device
generator (seed 0), so no host->device copy is timed.

Printed JSON (one line): value = ms per layer (lower is better); effective TFLOP/s over attended (q, k) pairs with
4*d FLOP per pair counted from the actual routes; `roofline` for the dominant kernel (the main sparse kernel) from
HIP events around its launches on the stream it runs on; `cpu_baseline` = the CPU restatement of the reference's
PyTorch path (oracle.routes_reference_order + oracle.flash_ref) timed on a bounded sample and scaled to a layer.
Also reported, next to the headline: `tail_roofline` (the exact 256-row tail, TFLOP/s and HBM GB/s), `decode`
(INT8-KV decode: microseconds per step and HBM GB/s against 8 TB/s and against
`hbm_read_ceiling`, the rate of a non-temporal 16-byte streaming read over 4 GiB measured in the same run) and `short_arm`
(B=4 at T=32768: sparse prefill, with its stage split, against dense causal SDPA on the same
inputs).
"""
import argparse
import json
import sys
import time
from pathlib import Path
from types import SimpleNamespace

ROOT = Path(__file__).resolve().parent
for _p in (str(ROOT), str(ROOT / "utmist-bigger-bird_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "ms/layer sparse prefill @128K; effective TFLOP/s and % of bf16 MFMA peak"
PEAK_BF16_TFLOPS = 2500.0      # MI355X dense bf16 MFMA
PEAK_HBM_GBPS = 8000.0         # MI355X HBM3E
H100_REFERENCE_MS = 124.6      # the reference's published sparse ms/layer at 131072 tokens (H100)


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--T", type=int, default=131072)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-decode", action="store_true", help="skip the decode legs (INT8 exact decode of BASELINE configs[4], sparse decode)")
    ap.add_argument("--full-model", action="store_true",
                    help="only run the full-model prefill (BASELINE configs[2]): random-init Llama-3-8B, sparse and exact arms")
    ap.add_argument("--no-full-model", action="store_true",
                    help="skip the full-model leg (BASELINE configs[2]) that the default run adds after the headline")
    ap.add_argument("--no-length-sweep", action="store_true",
                    help="skip the per-layer sparse time at 32K..1M tokens (the reference's attn_bench sweep)")
    ap.add_argument("--no-short-arm", action="store_true",
                    help="skip the B=4, T=32768 sparse-vs-dense leg (BASELINE configs[3])")
    ap.add_argument("--copy-probe", action="store_true",
                    help="only run kernels of known traffic, 5 launches each: a 1 GiB device copy, a 1 GiB read "
                         "(sum) and a 1 GiB write (fill); calibrates rocprofv3 FETCH_SIZE / WRITE_SIZE")
    ap.add_argument("--cpu-sample-blocks", type=int, default=96,
                    help="64-row blocks (of 4 heads each) timed for the CPU baseline")
    return ap.parse_args()


def stub_base(H, Hkv, d):
    cfg = SimpleNamespace(num_attention_heads=H, num_key_value_heads=Hkv)
    return SimpleNamespace(config=cfg, layer_idx=0, head_dim=d, scaling=d ** -0.5, q_proj=None, k_proj=None,
                           v_proj=None, o_proj=None)


def staged_prefill(attn, q, k, v, ev):
    """RDAttention.sparse_prefill split into its launches with an event pair around each stage (same calls, same
    order; the output is checked bit-identical to sparse_prefill once before timing)."""
    import torch
    from bigger_bird_amd import bigger_bird_flash, transpose_v
    from bigger_bird_amd.attention import _flat_heads

    n = k.shape[-2]
    bsz = q.shape[0]
    bh = bsz * attn.num_heads
    kw = dict(num_heads=attn.num_heads, kv_groups=attn.groups, scale=attn.scaling)
    ev["routes"][0].record()
    idx = attn.routes(q, k)
    ev["routes"][1].record()
    Q, K, V = _flat_heads(q), _flat_heads(k), _flat_heads(v)  # B > 1: one batch of B * H heads, as sparse_prefill
    ev["transpose_v"][0].record()
    vt = transpose_v(V)
    ev["transpose_v"][1].record()
    r = min(attn.exact_tail, n)
    ev["main"][0].record()
    out = bigger_bird_flash(Q, K, V, idx.view(bh, 1, -1), front=attn.sink, window=attn.window, row_end=n - r, vt=vt,
                            **kw)
    ev["main"][1].record()
    if r:
        none = torch.full((bh, 1, 1), -1, dtype=torch.int32, device=q.device)
        ev["tail"][0].record()
        bigger_bird_flash(Q[:, n - r:], K, V, none, front=0, window=n, vt=vt, out=out[:, n - r:], **kw)
        ev["tail"][1].record()
    return out.unflatten(0, (bsz, attn.num_heads)), idx if bsz == 1 else idx.view(bsz, attn.num_heads, -1)


def hbm_read_ceiling(dev, gib=4, workgroups=4096, reps=10):
    """HBM read rate of a non-temporal 16-byte streaming read (bb_stream_read: one contiguous range per workgroup)
    over `gib` GiB, far past the 256 MB Infinity Cache: the ceiling the decode kernels are reported against next to
    the published 8 TB/s. Best of `reps`."""
    import torch
    from bigger_bird_amd import _lib

    nbytes = gib << 30
    buf = torch.ones(nbytes // 4, dtype=torch.float32, device=dev)
    sink = torch.empty(workgroups, dtype=torch.int32, device=dev)
    L = _lib.lib()
    run = lambda: _lib.check(L.bb_stream_read(_lib.ptr(buf), nbytes, _lib.ptr(sink), workgroups,  # noqa: E731
                                              _lib.stream_of(buf)))
    run()
    torch.cuda.synchronize()
    best = float("inf")
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        run()
        b.record()
        torch.cuda.synchronize()
        best = min(best, a.elapsed_time(b))
    del buf
    return {"gbps": round(nbytes / (best * 1e-3) / 1e9, 1), "bytes": nbytes, "workgroups": workgroups,
            "kernel": "stream_read_kernel (bb_stream_read): non-temporal 16-byte loads, 8 in flight per thread, "
                      "one contiguous range per workgroup"}


def main_traffic():
    """HBM bytes per launch of the main kernel from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary
    (profiles/prefill_128k_hbm_traffic.json, scaled by calibrating kernels of known traffic); None when absent."""
    path = ROOT / "profiles" / "prefill_128k_hbm_traffic.json"
    try:
        data = json.loads(path.read_text())
        keys = [k for k in data["kernels"] if k.startswith("flash_ping_kernel") and k.endswith("[main]")]
        return int(data["kernels"][keys[0]]["bytes"])
    except (OSError, KeyError, ValueError):
        return None


def main_activity():
    """Clock and matrix-core busy fraction of the main kernel from the committed rocprofv3 counter summary
    (profiles/prefill_128k_mfma_busy.json: GRBM_GUI_ACTIVE, SQ_VALU_MFMA_BUSY_CYCLES); empty when absent."""
    path = ROOT / "profiles" / "prefill_128k_mfma_busy.json"
    try:
        m = json.loads(path.read_text())["flash_ping_kernel [main]"]
        return {"mfma_busy": m["mfma_busy"], "clock_ghz": m["clock_ghz"],
                "activity_source": "profiles/prefill_128k_mfma_busy.md"}
    except (OSError, KeyError, ValueError):
        return {}


def cpu_model():
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(q, k, v, routes, cfg, args):
    """The reference's CPU path (routes() op sequence + bigger_bird_flash_ref masked-dense semantics), restated in
    torch CPU ops by the oracle, timed on a bounded sample and scaled to one layer:
      routes: one KV head group (4 query heads) of the 8, x8;
      attention: `cpu_sample_blocks` blocks of 64 query rows x 4 heads; every row of the reference's masked-dense
      CPU path costs O(N) whatever its position, so the blocks are scaled by (H / 4) * (T / 64) / blocks."""
    import torch
    import oracle

    H, T, d = q.shape[1], q.shape[2], q.shape[3]
    Hkv = k.shape[1]
    G = H // Hkv
    qc, kc, vc = q[:, :G].cpu(), k[:, :1].cpu(), v[:, :1].cpu()
    rc = routes[:G].cpu()
    budget = rc.shape[1]
    threads = torch.get_num_threads()
    t0 = time.perf_counter()
    oracle.routes_reference_order(qc, kc, num_heads=G, num_kv_heads=1, sink=cfg["sink"], window=cfg["window"],
                                  budget=budget, scaling=d ** -0.5)
    t_routes = (time.perf_counter() - t0) * Hkv
    blocks = max(1, args.cpu_sample_blocks)
    t0 = time.perf_counter()
    for b in range(blocks):
        # last 64 rows of the prompt (full-length rows, like every row of the masked-dense path)
        oracle.flash_ref(qc[0][:, T - 64:], kc[0], vc[0], rc.view(G, 1, -1), front=cfg["sink"], window=cfg["window"],
                         num_heads=G, kv_groups=G, scale=d ** -0.5)
    t_blocks = time.perf_counter() - t0
    t_attn = t_blocks / blocks * (H / G) * (T / 64)
    ms = (t_routes + t_attn) * 1e3
    return {"value": round(ms, 1), "unit": "ms/layer", "cores": threads, "kind": "port",
            "cpu_model": cpu_model(),
            "sample": (f"torch CPU restatement of the reference path: routes for 1 of {Hkv} KV groups (x{Hkv}) + "
                       f"masked-dense attention for {blocks} blocks of 64 rows x {G} heads over all {T} keys, "
                       f"scaled x{(H // G) * (T // 64) / blocks:.0f}; extrapolated, measured "
                       f"{(t_routes / Hkv + t_blocks):.1f} s")}


def config1_side_by_side(dev, seed):
    """BASELINE configs[0] (T=8192, {64, 2048, 128, 256}, 32 q / 8 KV heads, d=128) timed in full on both sides: the
    CPU restatement of the reference's path (oracle.routes_reference_order for every head, then the masked-dense
    oracle.flash_ref over every row, outputs and int32 routes) on the host cores, and RDAttention.sparse_prefill on
    the GPU, on the same inputs. The routes are compared (set-exact), and the GPU output against the CPU one."""
    import torch
    import oracle
    from bigger_bird_amd import RDAttention
    from bigger_bird_amd.synth import attended_pairs, make_inputs

    T, H, Hkv, d = 8192, 32, 8, 128
    cfg = dict(sink=64, window=2048, vertical=128, exact_tail=256)
    inp = make_inputs(T, H, Hkv, d, seed=seed + 11, sink=cfg["sink"], window=cfg["window"], device=dev, rng="device")
    q, k, v = inp["q"], inp["k"], inp["v"]
    attn = RDAttention(stub_base(H, Hkv, d), **cfg)
    with torch.inference_mode():
        out = attn.sparse_prefill(q, k, v)
        torch.cuda.synchronize()
        best = float("inf")
        for _ in range(5):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            attn.sparse_prefill(q, k, v)
            b.record()
            torch.cuda.synchronize()
            best = min(best, a.elapsed_time(b))
    routes_gpu = attn.last_routes.cpu()
    qc, kc, vc = q[0].cpu(), k[0].cpu(), v[0].cpu()
    t0 = time.perf_counter()
    routes_cpu = oracle.routes_reference_order(q.cpu(), k.cpu(), num_heads=H, num_kv_heads=Hkv, sink=cfg["sink"],
                                               window=cfg["window"], budget=cfg["vertical"], scaling=d ** -0.5)
    t_routes = time.perf_counter() - t0
    r = cfg["exact_tail"]
    t0 = time.perf_counter()
    main = oracle.flash_ref(qc, kc, vc, routes_cpu.view(H, 1, -1), front=cfg["sink"], window=cfg["window"],
                            num_heads=H, kv_groups=H // Hkv, scale=d ** -0.5)
    none = torch.full((H, 1, 1), -1, dtype=torch.int32)
    tail = oracle.flash_ref(qc[:, T - r:], kc, vc, none, front=0, window=T, num_heads=H, kv_groups=H // Hkv,
                            scale=d ** -0.5)
    main[:, T - r:] = tail
    t_attn = time.perf_counter() - t0
    err = (out[0].float().cpu() - main.float()).abs()
    cpu_ms = (t_routes + t_attn) * 1e3
    flop = 4 * d * attended_pairs(T, H, cfg["sink"], cfg["window"], routes_gpu, r)
    return {"workload": "BASELINE configs[0]: T=8192, 32q/8kv heads, d=128, cfg {64, 2048, 128, 256}; routes + "
                        "sparse attention + exact tail, whole layer on both sides",
            "cpu_ms": round(cpu_ms, 1), "cpu_routes_ms": round(t_routes * 1e3, 1),
            "cpu_threads": torch.get_num_threads(), "cpu_model": cpu_model(),
            "gpu_ms": round(best, 3), "speedup": round(cpu_ms / best, 1),
            "gpu_effective_tflops": round(flop / (best * 1e-3) / 1e12, 1),
            "routes_equal": bool(torch.equal(routes_gpu, routes_cpu)),
            "max_abs_gpu_vs_cpu": round(err.max().item(), 5), "mean_abs_gpu_vs_cpu": round(err.mean().item(), 6)}


def decode_leg(dev, seed, ceiling):
    """exact decode over an INT8 cache of 131072 tokens (32 q / 8 KV heads, d=128, per-token
    per-head fp32 scales = absmax/127), 256 steps; each step quantises one new token into the cache and attends to
    all n + 1 rows with a fresh bf16 query. Reported per step with the cache bytes a step must read."""
    import torch
    from bigger_bird_amd import decode_int8_append, quantize

    n0, steps, H, Hkv, d = 131072, 256, 32, 8, 128
    g = torch.Generator(device=dev).manual_seed(seed + 5)
    k = torch.randn(n0 + steps, Hkv, d, device=dev, generator=g).to(torch.bfloat16)
    v = torch.randn(n0 + steps, Hkv, d, device=dev, generator=g).to(torch.bfloat16)
    qs = torch.randn(steps, H, d, device=dev, generator=g).to(torch.bfloat16)
    k8 = torch.empty(n0 + steps, Hkv, d, dtype=torch.int8, device=dev)
    v8 = torch.empty_like(k8)
    ks = torch.empty(n0 + steps, Hkv, 1, dtype=torch.float32, device=dev)
    vs = torch.empty_like(ks)
    quantize(k[:n0], out=(k8[:n0], ks[:n0]), scale_dtype=torch.float32)
    quantize(v[:n0], out=(v8[:n0], vs[:n0]), scale_dtype=torch.float32)
    scale = d ** -0.5

    def step(i):
        # the new token's K / V rows are quantised into row n0 + i by the decode kernel itself (bb_decode_append)
        return decode_int8_append(qs[i], k8, ks, v8, vs, k[n0 + i], v[n0 + i], n0 + i + 1, scale)

    with torch.inference_mode():
        for i in range(8):  # warm-up (rewrites the same rows)
            step(i)
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for i in range(steps):
            step(i)
        b.record()
        torch.cuda.synchronize()
    us = a.elapsed_time(b) * 1e3 / steps
    n_mean = n0 + (steps + 1) / 2
    bytes_step = 2 * Hkv * n_mean * (d + 4) + 2 * H * d * 2  # int8 K and V rows + fp32 scales, q in + out
    gbps = bytes_step / (us * 1e-6) / 1e9
    return {"workload": "BASELINE configs[4]: INT8-KV exact decode, 131072 cached tokens (+1 per step), 32q/8kv heads, "
                        "d=128, fp32 per-token per-head scales, 256 steps",
            "us_per_step": round(us, 2), "bytes_per_step": int(bytes_step), "achieved_gbps": round(gbps, 1),
            "peak_gbps": PEAK_HBM_GBPS, "frac": round(gbps / PEAK_HBM_GBPS, 4),
            "read_ceiling_gbps": ceiling["gbps"], "frac_of_read_ceiling": round(gbps / ceiling["gbps"], 4),
            "kernels": "per step decode_mfma_kernel (new-row quantisation + split-K decode) + decode_merge_kernel"}


def sparse_decode_leg(dev, seed, ceiling):
    """Sparse decode after a 128K prefill (the reference's kernels/bigger_bird_decode.py + bigger_bird_route.py):
    bf16 cache of 131072 tokens (+1 per step), 32 q / 8 KV heads, d=128; a step appends the new K/V row at the
    device-side length, routes (pooled decode routing over every cached key, top 512 per KV head outside the sink
    and the 16384-key window) and attends sink 64 + window 16384 + the 512 routed keys. The step's inputs are fixed
    buffers (in a model they come from the projections inside the same graph). Timed eagerly, as a captured HIP
    graph of one step replayed per step, and as a graph of 8 consecutive steps (the length advances on the device,
    so 8 steps need no host work between them; a replay has a fixed cost of about 5 us that 8 steps share); bytes =
    the K rows the routing reads + its fp32 score round trip + what the sparse decode reads: the V rows of its key
    list and their scores (the fused step's decode takes the routing pass's scores instead of re-reading K rows)."""
    import torch
    from bigger_bird_amd.decode import decode_step

    n0, steps, H, Hkv, d = 131072, 64, 32, 8, 128
    front, window, routed = 64, 16384, 512
    cap = n0 + 2 * steps + 8
    g = torch.Generator(device=dev).manual_seed(seed + 9)
    k = torch.randn(Hkv, cap, d, device=dev, generator=g).to(torch.bfloat16)
    v = torch.randn(Hkv, cap, d, device=dev, generator=g).to(torch.bfloat16)
    qb = torch.randn(H, d, device=dev, generator=g).to(torch.bfloat16)
    kb = torch.randn(Hkv, d, device=dev, generator=g).to(torch.bfloat16)
    vb = torch.randn(Hkv, d, device=dev, generator=g).to(torch.bfloat16)
    scale = d ** -0.5

    def step(length):
        # length counts the new row: it becomes row length - 1 inside the routing scores pass, and the sparse decode's
        # merge advances the length for the next step (bb_decode_step: 6 launches)
        return decode_step(qb, k, v, kb, vb, length, routed=routed, front=front, window=window, scale=scale,
                           advance=1)

    def timed(fn, reps=steps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record()
        for _ in range(reps):
            fn()
        b.record()
        torch.cuda.synchronize()
        return round(a.elapsed_time(b) * 1e3 / reps, 2)

    res = {"workload": "sparse decode after a 131072-token prefill: bf16 cache, 32q/8kv heads, d=128; per step append + "
                       "pooled decode routing (top 512 per KV head) + split-K decode over sink 64 + window 16384 + 512 "
                       "routed keys"}
    with torch.inference_mode():
        length = torch.tensor([n0 + 1], device=dev)
        for _ in range(4):
            step(length)
        length.fill_(n0 + 1)
        res["eager_us_per_step"] = timed(lambda: step(length))
        length.fill_(n0 + 1)
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            step(length)
        torch.cuda.current_stream().wait_stream(s)
        for per, key in ((1, "graph_us_per_step"), (8, "graph8_us_per_step")):
            length.fill_(n0 + 1)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                for _ in range(per):
                    step(length)
            length.fill_(n0 + 1)
            res[key] = round(timed(graph.replay, steps // per) / per, 2)
            del graph
    n_mean = n0 + (steps + 1) / 2
    route_bytes = Hkv * n_mean * d * 2 + 2 * H * n_mean * 4          # K read once + fp32 scores written and read
    n_list = front + window + routed
    decode_bytes = Hkv * n_list * d * 2 + H * n_list * 4               # V rows of the key list + their fp32 scores
    res["bytes_per_step"] = int(route_bytes + decode_bytes)
    us = min(res["eager_us_per_step"], res["graph_us_per_step"], res["graph8_us_per_step"])
    res["achieved_gbps"] = round(res["bytes_per_step"] / (us * 1e-6) / 1e9, 1)
    res["peak_gbps"] = PEAK_HBM_GBPS
    res["frac"] = round(res["achieved_gbps"] / PEAK_HBM_GBPS, 4)
    res["read_ceiling_gbps"] = ceiling["gbps"]
    res["frac_of_read_ceiling"] = round(res["achieved_gbps"] / ceiling["gbps"], 4)
    return res


def short_arm_leg(dev, seed):
    """B=4, T=32768, cfg {64, 4096, 512, 256}: sparse_prefill (routes + main + tail, each batch
    element a layer call) against dense causal attention on the same inputs (torch SDPA, flash backend forced so that
    no [T, T] matrix is ever formed; K/V repeated to the query heads)."""
    import torch
    import torch.nn.functional as F
    from bigger_bird_amd import RDAttention
    from bigger_bird_amd.synth import make_inputs

    B, H, Hkv, T, d = 4, 32, 8, 32768, 128
    cfg = dict(sink=64, window=4096, vertical=512, exact_tail=256)
    inp = make_inputs(T, H, Hkv, d, batch=B, seed=seed + 3, sink=cfg["sink"], window=cfg["window"], device=dev,
                      rng="device")
    q, k, v = inp["q"], inp["k"], inp["v"]
    attn = RDAttention(stub_base(H, Hkv, d), **cfg)

    def timed(fn, reps=3):
        fn()
        torch.cuda.synchronize()
        best = float("inf")
        for _ in range(reps):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            fn()
            b.record()
            torch.cuda.synchronize()
            best = min(best, a.elapsed_time(b))
        return best

    from bigger_bird_amd.synth import attended_pairs

    res = {"workload": "BASELINE configs[3]: B=4, T=32768, 32q/8kv heads, d=128, cfg {64, 4096, 512, 256}"}
    with torch.inference_mode():
        sparse_ms = timed(lambda: attn.sparse_prefill(q, k, v))
        res["sparse_ms"] = round(sparse_ms, 3)
        # the same launches one stage at a time (checked bit-identical to sparse_prefill): best of 3 per stage
        ref = attn.sparse_prefill(q, k, v)
        mk = lambda: (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))  # noqa: E731
        stages = ("routes", "transpose_v", "main", "tail")
        best = {st: float("inf") for st in stages}
        for i in range(4):
            ev = {st: mk() for st in stages}
            out, _ = staged_prefill(attn, q, k, v, ev)
            torch.cuda.synchronize()
            if i == 0 and not torch.equal(out, ref):
                raise SystemExit("staged prefill (B=4) differs from sparse_prefill")
            if i > 0:
                for st in stages:
                    best[st] = min(best[st], ev[st][0].elapsed_time(ev[st][1]))
        del ref, out
        res["stage_ms"] = {st: round(x, 3) for st, x in best.items()}
        # 4 d FLOP per attended (q, k) pair, pairs counted from each batch element's actual routes
        flop = sum(4 * d * attended_pairs(T, H, cfg["sink"], cfg["window"], attn.last_routes[b].cpu(),
                                          cfg["exact_tail"]) for b in range(B))
        res["flop"] = flop
        res["effective_tflops"] = round(flop / (sparse_ms * 1e-3) / 1e12, 1)
        res["frac"] = round(res["effective_tflops"] / PEAK_BF16_TFLOPS, 4)
        try:
            from torch.nn.attention import SDPBackend, sdpa_kernel
            kr = k.repeat_interleave(H // Hkv, dim=1)
            vr = v.repeat_interleave(H // Hkv, dim=1)
            with sdpa_kernel(SDPBackend.FLASH_ATTENTION):
                res["dense_ms"] = round(timed(lambda: F.scaled_dot_product_attention(q, kr, vr, is_causal=True,
                                                                                      scale=d ** -0.5)), 3)
            res["speedup"] = round(res["dense_ms"] / res["sparse_ms"], 2)
            dense_flop = B * 4 * d * H * T * (T + 1) // 2
            res["dense_effective_tflops"] = round(dense_flop / (res["dense_ms"] * 1e-3) / 1e12, 1)
            res["dense"] = "torch SDPA flash backend (ROCm), causal, K/V repeated to 32 heads"
        except RuntimeError as e:  # no flash backend for this shape: report the sparse time only
            res["dense_ms"] = None
            res["dense"] = f"unavailable: {str(e)[:120]}"
    return res


# The reference's attention-only per-layer sparse cost on H100 (modal_rd/RESULTS.md:56-62), in ms.
H100_SWEEP_MS = {32768: 30, 65536: 61, 131072: 125, 262144: 251, 524288: 508, 1048576: 1038}


def length_sweep_leg(dev, seed, cfg, dense_max=131072):
    """The reference's attn_bench sweep (modal_rd/attn_bench.py:31-54): one RDAttention layer with cfg
    {64, 16384, 512, 256} on N(0, 1) bf16 Q/K/V (32q/8kv heads, d=128, no RoPE) at 32K..1M tokens, best of 3 after
    a warm-up call, routes + V^T + main + tail. Dense causal attention (torch SDPA, flash backend, K/V repeated) is
    timed up to `dense_max` tokens only: past that it costs seconds per call."""
    import torch
    import torch.nn.functional as F
    from bigger_bird_amd import RDAttention

    H, Hkv, d = 32, 8, 128
    attn = RDAttention(stub_base(H, Hkv, d), **cfg)

    def timed(fn, reps=3):
        fn()
        torch.cuda.synchronize()
        best = float("inf")
        for _ in range(reps):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            fn()
            b.record()
            torch.cuda.synchronize()
            best = min(best, a.elapsed_time(b))
        return best

    rows = []
    for n in sorted(H100_SWEEP_MS):
        print(f"bench: length sweep T={n}", file=sys.stderr, flush=True)
        g = torch.Generator(device=dev).manual_seed(seed + n)
        q = torch.randn(1, H, n, d, device=dev, dtype=torch.bfloat16, generator=g)
        k = torch.randn(1, Hkv, n, d, device=dev, dtype=torch.bfloat16, generator=g)
        v = torch.randn(1, Hkv, n, d, device=dev, dtype=torch.bfloat16, generator=g)
        row = {"tokens": n}
        with torch.inference_mode():
            row["sparse_ms"] = round(timed(lambda: attn.sparse_prefill(q, k, v)), 3)
            if n <= dense_max:
                from torch.nn.attention import SDPBackend, sdpa_kernel
                kr, vr = k.repeat_interleave(H // Hkv, dim=1), v.repeat_interleave(H // Hkv, dim=1)
                with sdpa_kernel(SDPBackend.FLASH_ATTENTION):
                    row["dense_ms"] = round(timed(lambda: F.scaled_dot_product_attention(
                        q, kr, vr, is_causal=True, scale=d ** -0.5)), 3)
                row["speedup"] = round(row["dense_ms"] / row["sparse_ms"], 2)
                del kr, vr
        row["h100_sparse_ms"] = H100_SWEEP_MS[n]
        row["vs_h100"] = round(row["sparse_ms"] / H100_SWEEP_MS[n], 4)
        rows.append(row)
        del q, k, v
        torch.cuda.empty_cache()
    return {"workload": "modal_rd/attn_bench.py sweep: 1 layer, B=1, 32q/8kv, d=128, cfg {64, 16384, 512, 256}, "
                        "N(0,1) bf16 Q/K/V, best of 3", "rows": rows}


def graph_decode_leg(model, ids, steps=32):
    """Greedy decode after the sparse prefill (modal_rd/graph_decode.py): prefill into the decoder's buffers, then
    one HIP graph per token (32 layers of split-K flash decoding over the whole cache + projections, MLP, lm_head,
    argmax), timed per token; the same step run eagerly (one launch per op) beside it."""
    import torch
    from bigger_bird_amd.graph_decode import graph_prefill

    dec, out, prefill_s = graph_prefill(model, ids, 2 * steps + 16, headroom=0)
    del out
    dec.capture()
    dec.run(2)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    dec.run(steps)
    torch.cuda.synchronize()
    graph_ms = (time.perf_counter() - t0) / steps * 1e3
    t0 = time.perf_counter()
    dec.run(steps // 4, graph=False)
    torch.cuda.synchronize()
    eager_ms = (time.perf_counter() - t0) / (steps // 4) * 1e3
    res = {"context_tokens": int(ids.shape[1]), "prefill_s": round(prefill_s, 3),
           "graph_ms_per_token": round(graph_ms, 3), "eager_step_ms_per_token": round(eager_ms, 3),
           "h100_reference_ms_per_token": {"eager": 25.5, "graph": 15.1, "context": "~128K, v3"}}
    print(f"graph decode: {graph_ms:.3f} ms/token (eager step {eager_ms:.3f})", file=sys.stderr, flush=True)
    del dec
    from bigger_bird_amd import graph_decode as gd
    gd.release()
    return res


def full_model_leg(dev, seed, T=131072):
    """prefill of a random-init Llama-3-8B-architecture model in bf16 (32 layers,
    hidden 4096, 32 q / 8 KV heads, FFN 14336, vocab 128256, RoPE theta 500000) at T uniform-random token ids, with
    RDAttention on every layer: the sparse arm (final cfg {64, 16384, 512, 256}) and the exact arm (`dense_rd`: the
    same module with exact causal attention on the HIP kernel). KV cache on, last-token logits only, as the
    reference's long-context prefill runs (modal_rd/RESULTS.md:37-43). Projections, MLP and norms are PyTorch."""
    import torch
    from transformers import LlamaConfig, LlamaForCausalLM
    from bigger_bird_amd import install

    cfg = LlamaConfig(vocab_size=128256, hidden_size=4096, intermediate_size=14336, num_hidden_layers=32,
                      num_attention_heads=32, num_key_value_heads=8, max_position_embeddings=T, rope_theta=500000.0,
                      rms_norm_eps=1e-5, attn_implementation="sdpa")
    old = torch.get_default_dtype()
    torch.manual_seed(seed)
    try:
        torch.set_default_dtype(torch.bfloat16)
        with torch.device(dev):
            model = LlamaForCausalLM(cfg)
    finally:
        torch.set_default_dtype(old)
    model.eval()
    g = torch.Generator(device=dev).manual_seed(seed + 7)
    ids = torch.randint(0, cfg.vocab_size, (1, T), generator=g, device=dev)
    print("full model built", file=sys.stderr, flush=True)

    def run():
        with torch.inference_mode():
            return model(input_ids=ids, use_cache=True, logits_to_keep=1).logits[0, -1].float()

    def timed(reps, arm):
        best, logits = float("inf"), None
        for _ in range(reps):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            logits = run()
            torch.cuda.synchronize()
            best = min(best, time.perf_counter() - t0)
            print(f"full model {arm}: {time.perf_counter() - t0:.3f} s", file=sys.stderr, flush=True)
        return best, logits

    res = {"workload": f"BASELINE configs[2]: random-init Llama-3-8B architecture, bf16, T={T}, KV cache on, "
                       "last-token logits; arms: HF sdpa (unmodified model), RDAttention sparse final cfg on all 32 "
                       "layers, RDAttention exact (dense_rd)"}
    # Arm 1: the unmodified HF model (sdpa attention; flash or memory-efficient backend, never the math one).
    from torch.nn.attention import SDPBackend, sdpa_kernel
    lh = None
    try:
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            run()
            res["hf_sdpa_s"], lh = timed(1, "hf sdpa")
            res["hf_sdpa_s"] = round(res["hf_sdpa_s"], 3)
    except RuntimeError as e:  # no fused SDPA kernel for this shape: report, keep going with the RD arms
        res["hf_sdpa_s"] = f"unavailable: {str(e)[:160]}"
    attn_cfg = dict(sink=64, window=16384, vertical=512, exact_tail=256)
    install(model, "rd", **attn_cfg)
    run()  # warm-up: kernels loaded, allocator sized
    sparse_s, ls = timed(2, "rd sparse")
    res["graph_decode"] = graph_decode_leg(model, ids)
    install(model, "dense_rd", **attn_cfg)
    dense_s, ld = timed(1, "dense_rd")
    cos = torch.nn.functional.cosine_similarity
    res.update({"sparse_s": round(sparse_s, 3), "exact_rd_s": round(dense_s, 3),
                "h100_reference_s": {"sparse_final_cfg": 8.50, "dense": 16.22, "tokens": 127545},
                "logits_cosine_sparse_vs_exact_rd": round(cos(ls, ld, dim=0).item(), 5),
                "top1_sparse_eq_exact_rd": bool(ls.argmax().item() == ld.argmax().item())})
    if lh is not None:
        res["logits_cosine_exact_rd_vs_hf_sdpa"] = round(cos(ld, lh, dim=0).item(), 5)
        res["logits_max_abs_exact_rd_vs_hf_sdpa"] = round((ld - lh).abs().max().item(), 5)
    return res


def main():
    args = parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "bench.py measures one GPU: this build has no multi-GPU path (every box has one "
                                   "GPU); run with --gpus 1"}), flush=True)
        sys.exit(2)
    import torch

    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs a ROCm GPU")
    if args.full_model:
        print(json.dumps({"full_model": full_model_leg(torch.device("cuda:0"), args.seed, args.T)}), flush=True)
        return
    if args.copy_probe:
        src = torch.ones(1 << 28, dtype=torch.float32, device="cuda")  # 1 GiB
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)  # reads and writes 1 GiB
        for _ in range(5):
            src.sum()  # reads 1 GiB
        for _ in range(5):
            dst.fill_(2.0)  # writes 1 GiB
        torch.cuda.synchronize()
        print(json.dumps({"probe_bytes": src.numel() * 4, "launches_each": 5, "kernels": ["copy", "sum", "fill"]}),
              flush=True)
        return
    from bigger_bird_amd import RDAttention, _lib
    from bigger_bird_amd.synth import attended_pairs, make_inputs

    _lib.lib()  # the HIP library must be present: no fallback path exists
    dev = torch.device("cuda:0")
    T, H, Hkv, d = args.T, 32, 8, 128
    cfg = dict(sink=64, window=16384, vertical=512, exact_tail=256)
    if T <= cfg["window"] + cfg["sink"] + 64:
        raise SystemExit("T must exceed sink + window + 64 planted keys")
    print(f"bench: T={T} H={H}/{Hkv} d={d} cfg={cfg} steps={args.steps} warmup={args.warmup}", file=sys.stderr,
          flush=True)
    inp = make_inputs(T, H, Hkv, d, seed=args.seed, planted=64, sink=cfg["sink"], window=cfg["window"],
                      device=dev, rng="device")
    q, k, v = inp["q"], inp["k"], inp["v"]
    attn = RDAttention(stub_base(H, Hkv, d), **cfg)
    torch.cuda.synchronize()

    with torch.inference_mode():
        ref_out = attn.sparse_prefill(q, k, v)
        mk = lambda: (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))  # noqa: E731
        ev = {s: mk() for s in ("routes", "transpose_v", "main", "tail")}
        out, routes = staged_prefill(attn, q, k, v, ev)
        torch.cuda.synchronize()
        if not torch.equal(out, ref_out) or not torch.equal(routes, attn.last_routes):
            raise SystemExit("staged prefill differs from sparse_prefill")
        planted = inp["planted_pos"][0]
        missed = sum(len(set(planted[h // (H // Hkv)].tolist()) - set(routes[h].tolist())) for h in range(H))
        print(f"bench: planted keys missed by routing: {missed}", file=sys.stderr, flush=True)
        del ref_out, out

        for _ in range(args.warmup):
            staged_prefill(attn, q, k, v, ev)
        torch.cuda.synchronize()
        # timed region: K steps, each stage bracketed by its own event pair on the current stream (where every
        # library launch goes); the outer pair gives ms/step
        evs = [{s: mk() for s in ev} for _ in range(args.steps)]
        t_start, t_end = mk()
        wall0 = time.perf_counter()
        t_start.record()
        for i in range(args.steps):
            staged_prefill(attn, q, k, v, evs[i])
        t_end.record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - wall0
        ms_per_step = t_start.elapsed_time(t_end) / args.steps
        stage_avg = {s: sum(e[s][0].elapsed_time(e[s][1]) for e in evs) / args.steps for s in ev}

    ceiling = None if args.no_decode else hbm_read_ceiling(dev)
    r = cfg["exact_tail"]
    pairs_total = attended_pairs(T, H, cfg["sink"], cfg["window"], routes, r)
    pairs_tail = H * sum(i + 1 for i in range(T - r, T))
    pairs_main = pairs_total - pairs_tail
    flops_total, flops_main, flops_tail = 4 * d * pairs_total, 4 * d * pairs_main, 4 * d * pairs_tail
    tflops = flops_total / (ms_per_step * 1e-3) / 1e12
    main_tflops = flops_main / (stage_avg["main"] * 1e-3) / 1e12
    tail_tflops = flops_tail / (stage_avg["tail"] * 1e-3) / 1e12
    # the tail reads every K and V row of the layer once per KV head (plus its 256 query rows in and out)
    tail_bytes = 2 * Hkv * T * d * 2 + 2 * H * r * d * 2
    result = {
        "metric": METRIC,
        "value": round(ms_per_step, 3),
        "unit": "ms/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": round(ms_per_step / H100_REFERENCE_MS, 4),
        "dtype": "bf16",
        "data": "synthetic (device RNG seed 0, RoPE theta 5e5, 64 planted keys per KV head)",
        "config": {"workload": f"BASELINE configs[1]: single-layer Bigger Bird v3 sparse prefill, B=1, T={T}, "
                               f"32q/8kv heads, d=128, sink 64, window 16384, vertical 512, exact_tail 256",
                   "T": T, "heads": H, "kv_heads": Hkv, "head_dim": d, **cfg},
        "effective_tflops": round(tflops, 1),
        "pct_bf16_peak": round(100 * tflops / PEAK_BF16_TFLOPS, 2),
        "attended_pairs": pairs_total,
        "flop": flops_total,
        "stage_ms": {s: round(x, 3) for s, x in stage_avg.items()},
        "stage_tflops": {"main": round(main_tflops, 1), "tail": round(tail_tflops, 1)},
        "wall_s_timed": round(wall, 3),
        "h100_reference_ms": H100_REFERENCE_MS,
        "roofline": {"bound": "mfma", "kernel": "flash_ping_kernel (main sink+window+routed pass)",
                     "achieved": round(main_tflops, 1), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(main_tflops / PEAK_BF16_TFLOPS, 4), "traffic": main_traffic(),
                     "traffic_unit": "bytes per launch (rocprofv3 FETCH_SIZE/WRITE_SIZE, copy-calibrated)",
                     "flop_per_launch": flops_main, "avg_launch_ms": round(stage_avg["main"], 4),
                     **main_activity()},
        "tail_roofline": {"bound": "mfma", "achieved": round(tail_tflops, 1), "peak": PEAK_BF16_TFLOPS,
                          "unit": "TFLOP/s", "frac": round(tail_tflops / PEAK_BF16_TFLOPS, 4),
                          "hbm_gbps": round(tail_bytes / (stage_avg["tail"] * 1e-3) / 1e9, 1),
                          "hbm_frac": round(tail_bytes / (stage_avg["tail"] * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4),
                          "bytes": tail_bytes},
        "decode": None if args.no_decode else decode_leg(dev, args.seed, ceiling),
        "sparse_decode": None if args.no_decode else sparse_decode_leg(dev, args.seed, ceiling),
        "hbm_read_ceiling": ceiling,
        "short_arm": None if args.no_short_arm else short_arm_leg(dev, args.seed),
        "cpu_baseline": None,
    }
    if not args.no_length_sweep:
        result["length_sweep"] = length_sweep_leg(dev, args.seed, cfg)
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(q, k, v, routes, cfg, args)
        result["cpu_baseline"]["config1_full_layer"] = config1_side_by_side(dev, args.seed)
    if not args.no_full_model:
        del q, k, v, inp, attn
        torch.cuda.empty_cache()
        result["full_model"] = full_model_leg(dev, args.seed, T)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
