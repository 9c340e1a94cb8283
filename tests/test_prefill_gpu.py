"""End-to-end RDAttention.sparse_prefill on the GPU (routes + sparse kernel + exact tail, modal_rd/attention.py:176-206)
at BASELINE config 1 (T=8192, {64, 2048, 128, 256}) and config 2 (T=131072, {64, 16384, 512, 256}, 64 planted keys
per KV head) on the inputs the reference's routes() saw (tests/golden): routes set-exact against the reference, and
sampled output rows (main-pass rows, window edges, the exact tail) within max-abs 2e-2 / mean-abs 2e-3 of the float64
oracle over the union mask.
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
       "config2": dict(sink=64, window=16384, vertical=512, exact_tail=256)}


@pytest.mark.parametrize("name", ["config1", "config2"])
def test_sparse_prefill_matches_oracle(name, dev):
    print(f"case prefill {name}", flush=True)
    g = golden_routes.case(name)
    H, Hkv, T, d = g["H"], g["Hkv"], g["T"], g["d"]
    cfg = CFG[name]
    attn = RDAttention(_base(H, Hkv, d), **cfg)
    gen = torch.Generator().manual_seed(7)
    v = torch.randn(1, Hkv, T, d, generator=gen).to(torch.bfloat16)
    q, k = g["q"], g["k"]
    with torch.inference_mode():
        out = attn.sparse_prefill(q.to(dev), k.to(dev), v.to(dev))
    torch.cuda.synchronize()
    assert out.shape == (1, H, T, d)
    routes = attn.last_routes.cpu()
    assert torch.equal(routes, g["routes"]), "routes differ from the reference's"
    W, r = cfg["window"], cfg["exact_tail"]
    rows = torch.tensor([0, 1, 63, 64, 65, W - 1, W, W + 1, W + 64, T // 2, T - r - 1, T - r, T - r + 1, T - 2, T - 1])
    rows = torch.cat([rows, torch.randint(0, T, (9,), generator=gen)])
    pairs = torch.stack([torch.arange(H).repeat_interleave(rows.numel()), rows.repeat(H)], -1)
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
        print(f"{name} {what}: rows={pr.shape[0]} max_abs={err.max().item():.3e} mean_abs={err.mean().item():.3e}",
              flush=True)
        assert err.max().item() < 2e-2 and err.mean().item() < 2e-3


def test_config4_batch_sampled_rows(dev):
    """BASELINE configs[3] shape: B=4, T=32768, {64, 4096, 512, 256}; each batch element against the float64 oracle
    on sampled rows (main pass, window edges, tail), with that element's own routes."""
    print("case prefill config4 B=4 T=32768", flush=True)
    from bigger_bird_amd.synth import make_inputs
    B, H, Hkv, T, d = 4, 32, 8, 32768, 128
    cfg = dict(sink=64, window=4096, vertical=512, exact_tail=256)
    inp = make_inputs(T, H, Hkv, d, batch=B, seed=4, sink=cfg["sink"], window=cfg["window"], device=dev,
                      rng="device")
    attn = RDAttention(_base(H, Hkv, d), **cfg)
    with torch.inference_mode():
        out = attn.sparse_prefill(inp["q"], inp["k"], inp["v"])
    torch.cuda.synchronize()
    assert out.shape == (B, H, T, d) and attn.last_routes.shape == (B, H, 512)
    W, r, G = cfg["window"], cfg["exact_tail"], H // Hkv
    gen = torch.Generator().manual_seed(9)
    rows = torch.tensor([0, 63, 64, W - 1, W, W + 64, T // 2, T - r - 1, T - r, T - 1])
    rows = torch.cat([rows, torch.randint(0, T, (4,), generator=gen)])
    for b in range(B):
        q, k, v = inp["q"][b].cpu(), inp["k"][b].cpu(), inp["v"][b].cpu()
        routes = attn.last_routes[b].cpu()
        heads = torch.tensor([0, 5, 17, 31])
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


def test_vertical_scope_matches_oracle(dev):
    """vertical_scope (modal_rd/attention.py:187-196): routed keys only for the query chunks of `scope_chunk` rows that
    end inside the last `vertical_scope` rows; earlier chunks attend sink + window only. The oracle gets the same
    per-chunk route lists ([H, groups, K], -1 for inactive chunks) and route_chunk = scope_chunk."""
    print("case prefill vertical_scope", flush=True)
    g = golden_routes.case("config1")
    H, Hkv, T, d = g["H"], g["Hkv"], g["T"], g["d"]
    cfg = dict(sink=64, window=2048, vertical=128, exact_tail=256, vertical_scope=3000, scope_chunk=1024)
    attn = RDAttention(_base(H, Hkv, d), **cfg)
    gen = torch.Generator().manual_seed(9)
    v = torch.randn(1, Hkv, T, d, generator=gen).to(torch.bfloat16)
    q, k = g["q"], g["k"]
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
