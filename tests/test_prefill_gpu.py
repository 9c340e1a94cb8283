"""End-to-end RDAttention.sparse_prefill on the GPU (routes + sparse kernel + exact tail, modal_rd/attention.py:176-206)
at BASELINE config 1 (T=8192, {64, 2048, 128, 256}; also with fp16 inputs) and config 2 (T=131072,
{64, 16384, 512, 256}, 64 planted keys per KV head) on the inputs the reference's routes() saw (tests/golden): routes
set-exact against the reference, and
output rows within max-abs 2e-2 / mean-abs 2e-3 of the float64 oracle over the union mask -- every (head, row) at
config 1; at config 2, 8 heads (one per KV group) at every 64-row tile boundary, the window edges, routed keys' first
rows, 4096 random rows and every exact-tail row. Config 4 (B=4) checks sampled rows of all 32 heads, and each
element's routes set-exact (pooled values bit-equal) against the oracle on that element's inputs.
"""
from types import SimpleNamespace

import pytest
import torch

import golden_routes
import oracle
from bigger_bird_amd import RDAttention

pytestmark = pytest.mark.gpu


def _base(H, Hkv, d):
    return SimpleNamespace(config=SimpleNamespace(num_attention_heads=H, num_key_value_heads=Hkv), layer_idx=0,
                           head_dim=d, scaling=d ** -0.5, q_proj=None, k_proj=None, v_proj=None, o_proj=None)


CFG = {"config1": dict(sink=64, window=2048, vertical=128, exact_tail=256),
       "config2": dict(sink=64, window=16384, vertical=512, exact_tail=256),
       "config1_f16": dict(sink=64, window=2048, vertical=128, exact_tail=256)}


def _rows_for(name, T, H, cfg, routes, gen):
    """(head, row) pairs checked at each config.
    config1: every row of every head (262144 pairs).
    config2: 8 heads (one per KV group): every 64-row tile boundary (rows 64j - 1 and 64j), the window edges, the
    first row each of every 8th routed key reaches, 4096 random rows, and all 256 exact-tail rows."""
    W, r = cfg["window"], cfg["exact_tail"]
    if name.startswith("config1"):
        return torch.stack(torch.meshgrid(torch.arange(H), torch.arange(T), indexing="ij"), -1).reshape(-1, 2)
    heads = torch.arange(0, H, 4) + torch.arange(H // 4) % 4  # 0, 5, 10, 15, 16, 21, 26, 31
    edges = torch.tensor([0, 1, 2, W - 2, W - 1, W, W + 1, W + 63, W + 64, T - r - 1])
    tiles = torch.arange(64, T - r + 64, 64)
    boundaries = torch.cat([tiles - 1, tiles])
    pairs = []
    for h in heads.tolist():
        seen = routes[h, ::8].long() + W
        rows = torch.cat([edges, boundaries, seen, torch.randint(0, T - r, (4096 // len(heads),), generator=gen),
                          torch.arange(T - r, T)])
        rows = rows[(rows >= 0) & (rows < T)].unique()
        pairs.append(torch.stack([torch.full_like(rows, h), rows], -1))
    return torch.cat(pairs)


@pytest.mark.parametrize("name", ["config1", "config2", "config1_f16"])
def test_sparse_prefill_matches_oracle(name, dev):
    print(f"case prefill {name}", flush=True)
    g = golden_routes.case(name)
    H, Hkv, T, d = g["H"], g["Hkv"], g["T"], g["d"]
    cfg = CFG[name]
    attn = RDAttention(_base(H, Hkv, d), **cfg)
    gen = torch.Generator().manual_seed(7)
    q, k = g["q"], g["k"]
    v = torch.randn(1, Hkv, T, d, generator=gen).to(q.dtype)
    with torch.inference_mode():
        out = attn.sparse_prefill(q.to(dev), k.to(dev), v.to(dev))
    torch.cuda.synchronize()
    assert out.shape == (1, H, T, d)
    routes = attn.last_routes.cpu()
    assert torch.equal(routes, g["routes"]), "routes differ from the reference's"
    W, r = cfg["window"], cfg["exact_tail"]
    pairs = _rows_for(name, T, H, cfg, routes, gen)
    main = pairs[pairs[:, 1] < T - r]
    tail = pairs[pairs[:, 1] >= T - r]
    G = H // Hkv
    ref_main = oracle.attn_rows(q[0], k[0], v[0], routes[:, None], main, front=cfg["sink"], window=W, num_heads=H,
                                kv_groups=G, scale=d ** -0.5)
    none = torch.full((H, 1, 1), -1, dtype=torch.int32)
    ref_tail = oracle.attn_rows(q[0], k[0], v[0], none, tail, front=0, window=T, num_heads=H, kv_groups=G,
                                scale=d ** -0.5)
    o = out[0].cpu()
    for what, pr, ref in (("main", main, ref_main), ("tail", tail, ref_tail)):
        err = (o[pr[:, 0], pr[:, 1]].double() - ref).abs()
        worst = err.amax(-1).argmax().item()
        print(f"{name} {what}: rows={pr.shape[0]} max_abs={err.max().item():.3e} mean_abs={err.mean().item():.3e} "
              f"worst at (head, row) {tuple(pr[worst].tolist())}", flush=True)
        assert err.max().item() < 2e-2 and err.mean().item() < 2e-3


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_config4_batch_sampled_rows(dtype, dev):
    """BASELINE configs[3] shape: B=4, T=32768, {64, 4096, 512, 256}, bf16 and fp16 inputs; each batch element against
    the float64 oracle on sampled rows (main pass, window edges, tail) of all 32 heads, with that element's own
    routes, and the routes themselves against the oracle's."""
    print(f"case prefill config4 B=4 T=32768 {dtype}", flush=True)
    from bigger_bird_amd.synth import make_inputs
    B, H, Hkv, T, d = 4, 32, 8, 32768, 128
    cfg = dict(sink=64, window=4096, vertical=512, exact_tail=256)
    inp = make_inputs(T, H, Hkv, d, batch=B, seed=4, sink=cfg["sink"], window=cfg["window"], device=dev,
                      rng="device", dtype=dtype)
    attn = RDAttention(_base(H, Hkv, d), **cfg)
    with torch.inference_mode():
        out = attn.sparse_prefill(inp["q"], inp["k"], inp["v"])
    torch.cuda.synchronize()
    assert out.shape == (B, H, T, d) and attn.last_routes.shape == (B, H, 512)
    W, r, G = cfg["window"], cfg["exact_tail"], H // Hkv
    # the batched launch equals one layer call per element: routes and main-pass rows bitwise; the exact tail's
    # key-chunk split depends on the launch's work count, so its rows agree to fp32 merge-order rounding
    routes_all = attn.last_routes.clone()
    with torch.inference_mode():
        for b in (0, B - 1):
            one = attn.sparse_prefill(inp["q"][b:b + 1], inp["k"][b:b + 1], inp["v"][b:b + 1])
            assert torch.equal(attn.last_routes, routes_all[b]), b
            assert torch.equal(one[0, :, :T - r], out[b, :, :T - r]), b
            assert (one[0, :, T - r:].float() - out[b, :, T - r:].float()).abs().max().item() < 4e-3, b
    attn.last_routes = routes_all
    # every element's routes at this shape against the oracle on that element's own inputs: set-exact, and the
    # pooled values of the batched launch bit-equal to the oracle's (eligible columns [sink, T - window))
    from bigger_bird_amd.attention import routes as hip_routes
    with torch.inference_mode():
        idx_b, pooled_b = hip_routes(inp["q"], inp["k"], num_heads=H, num_kv_heads=Hkv, sink=cfg["sink"], window=W,
                                     budget=512, scaling=d ** -0.5, return_pooled=True)
    assert torch.equal(idx_b.view(B, H, -1), routes_all)
    for b in range(B):
        want, want_pooled = oracle.routes(inp["q"][b], inp["k"][b], sink=cfg["sink"], window=W, budget=512,
                                          scaling=d ** -0.5, return_pooled=True)
        assert torch.equal(routes_all[b].cpu(), want), f"config4 b={b}: routes differ from the oracle"
        prob = (want_pooled.double() * 2.0 ** -40 / 64).float()
        got = pooled_b.view(B, H, -1)[b].cpu()
        assert torch.equal(got[:, cfg["sink"]:T - W], prob[:, cfg["sink"]:T - W]), f"config4 b={b}: pooled differ"
    gen = torch.Generator().manual_seed(9)
    rows = torch.tensor([0, 63, 64, W - 1, W, W + 64, T // 2, T - r - 1, T - r, T - 1])
    rows = torch.cat([rows, torch.randint(0, T, (4,), generator=gen)])
    for b in range(B):
        q, k, v = inp["q"][b].cpu(), inp["k"][b].cpu(), inp["v"][b].cpu()
        routes = attn.last_routes[b].cpu()
        heads = torch.arange(H)
        pairs = torch.stack([heads.repeat_interleave(rows.numel()), rows.repeat(heads.numel())], -1)
        main, tail = pairs[pairs[:, 1] < T - r], pairs[pairs[:, 1] >= T - r]
        ref_main = oracle.attn_rows(q, k, v, routes[:, None], main, front=cfg["sink"], window=W, num_heads=H,
                                    kv_groups=G, scale=d ** -0.5)
        none = torch.full((H, 1, 1), -1, dtype=torch.int32)
        ref_tail = oracle.attn_rows(q, k, v, none, tail, front=0, window=T, num_heads=H, kv_groups=G,
                                    scale=d ** -0.5)
        o = out[b].cpu()
        for what, pr, ref in (("main", main, ref_main), ("tail", tail, ref_tail)):
            err = (o[pr[:, 0], pr[:, 1]].double() - ref).abs()
            print(f"config4 b={b} {what}: max_abs={err.max().item():.3e} mean_abs={err.mean().item():.3e}", flush=True)
            assert err.max().item() < 2e-2 and err.mean().item() < 2e-3


@pytest.mark.parametrize("name", ["config1", "config1_f16"])
def test_vertical_scope_matches_oracle(name, dev):
    """vertical_scope (modal_rd/attention.py:187-196): routed keys only for the query chunks of `scope_chunk` rows that
    end inside the last `vertical_scope` rows; earlier chunks attend sink + window only. The oracle gets the same
    per-chunk route lists ([H, groups, K], -1 for inactive chunks) and route_chunk = scope_chunk. bf16 and fp16
    inputs (the routes equal the reference's golden routes for each)."""
    print(f"case prefill vertical_scope {name}", flush=True)
    g = golden_routes.case(name)
    H, Hkv, T, d = g["H"], g["Hkv"], g["T"], g["d"]
    cfg = dict(sink=64, window=2048, vertical=128, exact_tail=256, vertical_scope=3000, scope_chunk=1024)
    attn = RDAttention(_base(H, Hkv, d), **cfg)
    gen = torch.Generator().manual_seed(9)
    q, k = g["q"], g["k"]
    v = torch.randn(1, Hkv, T, d, generator=gen).to(q.dtype)
    with torch.inference_mode():
        out = attn.sparse_prefill(q.to(dev), k.to(dev), v.to(dev))
    torch.cuda.synchronize()
    routes = attn.last_routes.cpu()
    assert torch.equal(routes, g["routes"])
    chunk, groups = 1024, T // 1024
    active = [(c + 1) * chunk > T - cfg["vertical_scope"] for c in range(groups)]
    assert active == [False] * 5 + [True] * 3
    idx = torch.stack([routes if a else torch.full_like(routes, -1) for a in active], 1)  # [H, groups, K]
    r = cfg["exact_tail"]
    rows = torch.tensor([100, 2047, 2048, 4095, 4200, 5119, 5120, 5121, 6000, 7000, T - r - 1, T - r, T - 1])
    pairs = torch.stack([torch.arange(H).repeat_interleave(rows.numel()), rows.repeat(H)], -1)
    main, tail = pairs[pairs[:, 1] < T - r], pairs[pairs[:, 1] >= T - r]
    G = H // Hkv
    ref_main = oracle.attn_rows(q[0], k[0], v[0], idx, main, front=64, window=2048, num_heads=H, kv_groups=G,
                                scale=d ** -0.5, route_chunk=chunk)
    none = torch.full((H, 1, 1), -1, dtype=torch.int32)
    ref_tail = oracle.attn_rows(q[0], k[0], v[0], none, tail, front=0, window=T, num_heads=H, kv_groups=G,
                                scale=d ** -0.5)
    o = out[0].cpu()
    for what, pr, ref in (("main", main, ref_main), ("tail", tail, ref_tail)):
        err = (o[pr[:, 0], pr[:, 1]].double() - ref).abs()
        print(f"vertical_scope {what}: max_abs={err.max().item():.3e} mean_abs={err.mean().item():.3e}", flush=True)
        assert err.max().item() < 2e-2 and err.mean().item() < 2e-3
