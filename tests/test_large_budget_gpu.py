"""Routed budgets above 512 slots per head on the production kernel (flash_ping_kernel: head_dim 128, 32 query / 8 KV
heads, no token mask), against the float64 oracle.

The kernel stages a head's route slots in LDS 512 at a time, so budgets above 512 take several passes over the slot
list, each starting at batch sb / 64 of the pre-gathered routed tiles. The module's own default is vertical=2048
(modal_rd/attention.py:79), and the reference checks its kernel at budgets 1024..8192 (modal_rd/kernelcheck.py:7-32)
and at the full budget (modal_rd/selfcheck.py:36-41). Tolerance: max-abs 2e-2, mean-abs 2e-3.

Rows checked per case: the kernelcheck rows (64 evenly spaced rows and the last 8) for every head, and for one head
per KV group the 64-row tile boundaries around the window edge, random rows, and for every slot s at the start or end
of a 512-slot pass (s = 512 m - 1, 512 m) the first row that attends routed key idx[h, s] (idx + window) and the row
before it.
"""
from types import SimpleNamespace

import pytest
import torch

import oracle
from bigger_bird_amd import RDAttention, bigger_bird_flash

pytestmark = pytest.mark.gpu

MAX_ABS, MEAN_ABS = 2e-2, 2e-3
H, HKV, D = 32, 8, 128


def _check(got, ref, what):
    err = (got.double().cpu() - ref).abs()
    print(f"{what}: rows={ref.shape[0]} max_abs={err.max().item():.3e} mean_abs={err.mean().item():.3e}", flush=True)
    assert err.max().item() < MAX_ABS and err.mean().item() < MEAN_ABS, what


def _sample_pairs(n, window, idx, gen, heads_dense=range(H)):
    """(head, row) pairs: kernelcheck rows for every head; pass-boundary, window and random rows for one head per KV
    group (head 4 kv + kv % 4, a different slot of each group)."""
    kc = torch.cat([torch.linspace(0, n - 1, 64).long(), torch.arange(n - 8, n)])
    pairs = [torch.stack([torch.full_like(kc, h), kc], -1) for h in heads_dense]
    budget = idx.shape[-1]
    slots = sorted({s for m in range(1, budget // 512 + 1) for s in (512 * m - 1, 512 * m) if s < budget} | {0})
    for kv in range(HKV):
        h = 4 * kv + kv % 4
        first = idx[h, slots].long() + window  # first row that attends the routed key
        edges = torch.tensor([window - 65, window - 64, window - 1, window, window + 63, window + 64])
        rows = torch.cat([first, first - 1, edges, torch.randint(0, n, (16,), generator=gen)])
        rows = rows[(rows >= 0) & (rows < n)].unique()
        pairs.append(torch.stack([torch.full_like(rows, h), rows], -1))
    return torch.cat(pairs)


def _random_routes(n, sink, window, budget, gen):
    return torch.stack([torch.randperm(n - window - sink, generator=gen)[:budget].sort().values + sink
                        for _ in range(H)]).to(torch.int32)


# modal_rd/kernelcheck.py:30-32 shapes (n, window, budget), at GQA 32 / 8 so that the pipelined kernel runs
KERNELCHECK = [(4096, 512, 256), (131072, 4096, 2048), (131072, 4096, 4096), (131072, 8192, 8192),
               (65536, 4096, 4096), (131072, 2048, 1024)]


@pytest.mark.parametrize("n,window,budget", KERNELCHECK, ids=[f"n{n}_w{w}_b{b}" for n, w, b in KERNELCHECK])
def test_kernelcheck_budgets(n, window, budget, dev):
    """modal_rd/kernelcheck.py:7-27: Q ~ N(0,1) * d^-0.5 * 3 with scale 1.0 (peaked rows), random sorted routes per
    head, sink 64; sampled rows against the float64 union oracle."""
    sink = 64
    print(f"case kernelcheck n={n} window={window} budget={budget}", flush=True)
    gd = torch.Generator(device=dev).manual_seed(n + window + budget)
    q = (torch.randn(H, n, D, device=dev, generator=gd) * D ** -0.5 * 3).to(torch.bfloat16)
    k = torch.randn(HKV, n, D, device=dev, generator=gd).to(torch.bfloat16)
    v = torch.randn(HKV, n, D, device=dev, generator=gd).to(torch.bfloat16)
    gen = torch.Generator().manual_seed(budget)
    idx = _random_routes(n, sink, window, budget, gen)
    out = bigger_bird_flash(q, k, v, idx.view(H, 1, budget).to(dev), front=sink, window=window, num_heads=H,
                            kv_groups=H // HKV, scale=1.0)
    torch.cuda.synchronize()
    pairs = _sample_pairs(n, window, idx, gen)
    ref = oracle.attn_rows(q.cpu(), k.cpu(), v.cpu(), idx.view(H, 1, budget), pairs, front=sink, window=window,
                           num_heads=H, kv_groups=H // HKV, scale=1.0)
    _check(out[pairs[:, 0].to(dev), pairs[:, 1].to(dev)], ref, f"kernelcheck n={n} w={window} b={budget}")


def test_full_budget_gqa_equals_dense_causal(dev):
    """modal_rd/selfcheck.py:36-41 at 32 query / 8 KV heads: every column outside sink / window routed (3520 slots,
    seven 512-slot passes) gives exact causal attention; checked in full against float64 SDPA."""
    n, sink, window = 4096, 64, 512
    print(f"case full_budget_gqa n={n} routes={n - sink - window}", flush=True)
    g = torch.Generator().manual_seed(36)
    q = (torch.randn(H, n, D, generator=g) * D ** -0.5).to(torch.bfloat16)
    k = torch.randn(HKV, n, D, generator=g).to(torch.bfloat16)
    v = torch.randn(HKV, n, D, generator=g).to(torch.bfloat16)
    full = torch.arange(sink, n - window, dtype=torch.int32).expand(H, -1).contiguous()
    out = bigger_bird_flash(q.to(dev), k.to(dev), v.to(dev), full.view(H, 1, -1).to(dev), front=sink, window=window,
                            num_heads=H, kv_groups=H // HKV, scale=1.0)
    ref = oracle.sdpa_ref(q, k, v, causal=True, scale=1.0, groups=H // HKV)
    _check(out.reshape(-1, D), ref.reshape(-1, D), "full_budget_gqa")


def test_rdattention_default_vertical(dev):
    """One RDAttention layer with the module defaults (sink 64, window 4096, vertical 2048; modal_rd/attention.py:79)
    at T = 16384, 32 / 8 heads: routes set-exact with the oracle's (pooled values bit-equal), and sampled output rows
    (including each pass boundary's first routed row and the exact tail) against the float64 oracle."""
    from bigger_bird_amd.attention import routes as bb_routes
    from bigger_bird_amd.synth import make_inputs

    T, r = 16384, 256
    print(f"case rdattention_default T={T}", flush=True)
    base = SimpleNamespace(config=SimpleNamespace(num_attention_heads=H, num_key_value_heads=HKV), layer_idx=0,
                           head_dim=D, scaling=D ** -0.5, q_proj=None, k_proj=None, v_proj=None, o_proj=None)
    attn = RDAttention(base, exact_tail=r)
    assert (attn.sink, attn.window, attn.vertical) == (64, 4096, 2048)
    inp = make_inputs(T, H, HKV, D, seed=79, planted=64, sink=64, window=4096, device=dev)
    q, k, v = inp["q"], inp["k"], inp["v"]
    with torch.inference_mode():
        out = attn.sparse_prefill(q, k, v)
    torch.cuda.synchronize()
    routes = attn.last_routes.cpu()
    assert routes.shape == (H, 2048)
    want, want_pooled = oracle.routes(q[0], k[0], sink=64, window=4096, budget=2048, scaling=D ** -0.5,
                                      return_pooled=True)
    assert torch.equal(routes, want), "routes differ from the oracle"
    _, pooled = bb_routes(q, k, num_heads=H, num_kv_heads=HKV, sink=64, window=4096, budget=2048, scaling=D ** -0.5,
                          return_pooled=True)
    prob = (want_pooled.double() * 2.0 ** -40 / 64).float()  # mean over the 64 route queries, as routes() returns
    assert torch.equal(pooled.cpu()[:, 64:T - 4096], prob[:, 64:T - 4096]), "pooled values differ from the oracle"
    planted = inp["planted_pos"][0]
    for kv in range(HKV):
        for h in range(4 * kv, 4 * kv + 4):
            assert set(planted[kv].tolist()) <= set(routes[h].tolist()), h
    gen = torch.Generator().manual_seed(80)
    pairs = _sample_pairs(T, 4096, routes, gen)
    main, tail = pairs[pairs[:, 1] < T - r], pairs[pairs[:, 1] >= T - r]
    tail = torch.cat([tail, torch.stack([torch.arange(H), torch.full((H,), T - r)], -1)])
    qc, kc, vc = q[0].cpu(), k[0].cpu(), v[0].cpu()
    ref_main = oracle.attn_rows(qc, kc, vc, routes[:, None], main, front=64, window=4096, num_heads=H,
                                kv_groups=H // HKV, scale=D ** -0.5)
    none = torch.full((H, 1, 1), -1, dtype=torch.int32)
    ref_tail = oracle.attn_rows(qc, kc, vc, none, tail, front=0, window=T, num_heads=H, kv_groups=H // HKV,
                                scale=D ** -0.5)
    o = out[0]
    _check(o[main[:, 0].to(dev), main[:, 1].to(dev)], ref_main, "rdattention_default main")
    _check(o[tail[:, 0].to(dev), tail[:, 1].to(dev)], ref_tail, "rdattention_default tail")


def test_vertical_scope_default_budget(dev):
    """vertical_scope with the default budget (2048 slots, four passes) and 4 route groups of 4096 rows: the kernel
    gathers the routed rows of the active groups itself (no pre-gathered tiles), against the float64 oracle with the
    same per-group lists."""
    T, chunk, scope = 16384, 4096, 6000
    print(f"case vertical_scope_default T={T}", flush=True)
    base = SimpleNamespace(config=SimpleNamespace(num_attention_heads=H, num_key_value_heads=HKV), layer_idx=0,
                           head_dim=D, scaling=D ** -0.5, q_proj=None, k_proj=None, v_proj=None, o_proj=None)
    attn = RDAttention(base, vertical_scope=scope, scope_chunk=chunk)
    from bigger_bird_amd.synth import make_inputs
    inp = make_inputs(T, H, HKV, D, seed=81, sink=64, window=4096, device=dev)
    q, k, v = inp["q"], inp["k"], inp["v"]
    with torch.inference_mode():
        out = attn.sparse_prefill(q, k, v)
    torch.cuda.synchronize()
    routes = attn.last_routes.cpu()
    active = [(c + 1) * chunk > T - scope for c in range(T // chunk)]
    assert active == [False, False, True, True]
    idx = torch.stack([routes if a else torch.full_like(routes, -1) for a in active], 1)
    gen = torch.Generator().manual_seed(82)
    pairs = _sample_pairs(T, 4096, routes, gen, heads_dense=range(0, H, 3))
    extra = torch.tensor([2 * chunk - 1, 2 * chunk, 3 * chunk - 1, 3 * chunk, T - 1])
    pairs = torch.cat([pairs, torch.stack([torch.arange(H).repeat_interleave(5), extra.repeat(H)], -1)])
    ref = oracle.attn_rows(q[0].cpu(), k[0].cpu(), v[0].cpu(), idx, pairs, front=64, window=4096, num_heads=H,
                           kv_groups=H // HKV, scale=D ** -0.5, route_chunk=chunk)
    _check(out[0][pairs[:, 0].to(dev), pairs[:, 1].to(dev)], ref, "vertical_scope_default")
