"""bb_routes (HIP) against the CPU oracle: the deterministic contract makes them bit-identical, so route indices
are compared set-exactly (sorted int32 equality) and the pooled fixed-point scores value-exactly; for bf16 and for
fp16 inputs (fp16 scores follow torch's CPU fp16 matmul order, checked against the reference's fp16 golden routes)."""
import pytest
import torch

import oracle
from bigger_bird_amd.attention import routes as hip_routes
from bigger_bird_amd.synth import make_inputs

pytestmark = pytest.mark.gpu

CASES = [
    # name, T, H, Hkv, d, sink, window, budget, n_route, pool, queries, planted
    ("small_d64", 1024, 8, 2, 64, 16, 256, 64, 64, "mean", "last", 0),
    ("odd_len_d128", 3001, 8, 2, 128, 64, 512, 100, 64, "mean", "last", 8),
    ("max_pool", 2048, 16, 4, 128, 64, 512, 128, 64, "max", "last", 0),
    ("spread", 2048, 16, 4, 128, 64, 512, 128, 64, "mean", "spread", 0),
    ("mha_d32", 777, 4, 4, 32, 8, 96, 24, 16, "mean", "last", 0),
    ("config1", 8192, 32, 8, 128, 64, 2048, 128, 64, "mean", "last", 64),
    # head_dim 128 with 48, 128 and 96 route rows per KV head (MFMA scorer workgroups of 2, 4 and 4 waves)
    ("mha_d128_48rows", 2500, 4, 4, 128, 32, 256, 64, 48, "mean", "last", 8),
    ("gqa2_d128", 3001, 8, 4, 128, 64, 512, 100, 64, "mean", "spread", 0),
    ("gqa3_d128_96rows", 2049, 12, 4, 128, 64, 512, 100, 32, "max", "last", 0),
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_routes_bit_exact(case, dtype, dev):
    name, T, H, Hkv, d, sink, window, budget, nr, pool, qmode, planted = case
    print(f"case {name} {dtype}", flush=True)
    inp = make_inputs(T, H, Hkv, d, seed=3, window=window, sink=sink, planted=planted, dtype=dtype)
    q, k = inp["q"], inp["k"]
    idx, pooled = hip_routes(q.to(dev), k.to(dev), num_heads=H, num_kv_heads=Hkv, sink=sink, window=window,
                             budget=budget, n_route=nr, route_pool=pool, route_queries=qmode, scaling=d ** -0.5,
                             return_pooled=True)
    torch.cuda.synchronize()
    r = min(nr, T)
    qpos = (torch.linspace(sink + window, T - 1, r).long() if qmode == "spread" else torch.arange(T - r, T))
    want, want_pooled = oracle.routes(q[0], k[0], sink=sink, window=window, budget=budget, scaling=d ** -0.5,
                                      n_route=nr, route_pool=pool, qpos=qpos, return_pooled=True)
    got = idx.cpu()
    assert torch.equal(got, want), f"{name}: route indices differ"
    scale = 2.0 ** -40 / (r if pool == "mean" else 1)
    prob = (want_pooled.double() * scale).float()
    lo, hi = sink, T - window  # pooled scores are defined on the eligible columns
    assert torch.equal(pooled.cpu()[:, lo:hi], prob[:, lo:hi]), f"{name}: pooled scores differ"
    if planted:
        for h in range(H):
            assert set(inp["planted_pos"][0, h // (H // Hkv)].tolist()) <= set(got[h].tolist()), "planted key missed"


def test_ties_go_to_lower_index(dev):
    """Identical keys give identical pooled probabilities; the lower index must win (the contract's tie-break)."""
    print("case ties", flush=True)
    T, H, Hkv, d, sink, window, budget = 512, 4, 1, 64, 8, 64, 10
    g = torch.Generator().manual_seed(5)
    q = torch.randn(1, H, T, d, generator=g).to(torch.bfloat16)
    k = torch.randn(1, Hkv, T, d, generator=g).to(torch.bfloat16)
    k[0, 0, sink:T - window] = k[0, 0, 100]  # every eligible key identical -> all pooled values tie
    idx = hip_routes(q.to(dev), k.to(dev), num_heads=H, num_kv_heads=Hkv, sink=sink, window=window, budget=budget,
                     scaling=d ** -0.5).cpu()
    want = torch.arange(sink, sink + budget, dtype=torch.int32).expand(H, -1)
    assert torch.equal(idx, want)


def test_budget_covers_all_eligible(dev):
    """budget == n - sink - window -> every eligible column (modal_rd/selfcheck.py:38)."""
    print("case full_budget_routes", flush=True)
    T, H, Hkv, d, sink, window = 700, 8, 2, 128, 16, 128
    inp = make_inputs(T, H, Hkv, d, seed=9, window=window)
    idx = hip_routes(inp["q"].to(dev), inp["k"].to(dev), num_heads=H, num_kv_heads=Hkv, sink=sink, window=window,
                     budget=T - sink - window, scaling=d ** -0.5).cpu()
    assert torch.equal(idx, torch.arange(sink, T - window, dtype=torch.int32).expand(H, -1))


GOLDEN = ["config1", "small_mean", "odd_planted", "max_pool", "spread", "mha_d32", "vertical_sqrt", "config2",
          "config1_f16", "config2_f16", "small_mean_f16", "max_pool_f16"]


@pytest.mark.parametrize("name", GOLDEN)
def test_routes_match_reference_golden(name, dev):
    """HIP routes against the reference's own routes() on the same seeded inputs (tests/golden): set-exact, with
    the documented lower-index rule only where the reference's pooled values tie exactly at the boundary."""
    import golden_routes

    print(f"case golden {name}", flush=True)
    g = golden_routes.case(name)
    idx, pooled = hip_routes(g["q"].to(dev), g["k"].to(dev), num_heads=g["H"], num_kv_heads=g["Hkv"], sink=g["sink"],
                             window=g["window"], budget=g["budget"], n_route=g["n_route"], route_pool=g["route_pool"],
                             route_queries=g["route_queries"], scaling=g["scaling"], return_pooled=True)
    torch.cuda.synchronize()
    tied = golden_routes.check_against_golden(idx.cpu(), g, pooled=pooled.cpu(), what=name)
    if not name.startswith("max_pool"):
        assert tied == 0 and torch.equal(idx.cpu(), g["routes"])
    if g["planted"] is not None:
        G = g["H"] // g["Hkv"]
        for h in range(g["H"]):
            assert set(g["planted"][0, h // G].tolist()) <= set(idx[h].cpu().tolist())


@pytest.mark.parametrize("name,T,scale_q,scale_k", [
    ("config2_shape", 131072, 1.0, 1.0),
    ("large_values", 16384, 40.0, 25.0),
    ("tiny_values", 16384, 1e-3, 2e-3),
    ("mixed_rows", 16384, 1.0, 1.0),
    ("mixed_rows_gqa2", 16384, 1.0, 1.0),
    ("mixed_rows_mha", 16384, 1.0, 1.0),
])
def test_mfma_scores_match_reference_order(name, T, scale_q, scale_k, dev, monkeypatch):
    """The MFMA score path with exact fix-up must give the same bf16 scores as computing every score in the
    reference order; compared through the pooled fixed-point values (every unmasked score of a row enters them)
    and the selected indices, at production size and at magnitudes that put many scores near rounding boundaries."""
    print(f"case mfma_scores {name} T={T}", flush=True)
    H, d, sink, window, budget = 32, 128, 64, min(16384, T // 4), 512
    Hkv = 32 if name.endswith("_mha") else (16 if name.endswith("_gqa2") else 8)
    inp = make_inputs(T, H, Hkv, d, seed=11, planted=64 if name == "config2_shape" else 0, sink=sink, window=window,
                      device=dev, rng="device")
    q, k = inp["q"] * scale_q, inp["k"] * scale_k
    if name.startswith("mixed_rows"):  # rows and keys spanning many binades, some exact zeros and repeated keys
        g = torch.Generator(device=dev).manual_seed(3)
        q = q * torch.exp2(torch.randint(-12, 8, (1, H, T, 1), device=dev, generator=g).to(q.dtype))
        k = k * torch.exp2(torch.randint(-12, 8, (1, Hkv, T, 1), device=dev, generator=g).to(k.dtype))
        k[:, :, 1000:1100] = 0
        k[:, :, 2000:2100] = k[:, :, 3000:3001]
    kw = dict(num_heads=H, num_kv_heads=Hkv, sink=sink, window=window, budget=budget, scaling=d ** -0.5,
              return_pooled=True)
    idx, pooled = hip_routes(q, k, **kw)
    monkeypatch.setenv("BB_ROUTES_REFERENCE_ORDER", "1")
    idx_ref, pooled_ref = hip_routes(q, k, **kw)
    monkeypatch.delenv("BB_ROUTES_REFERENCE_ORDER")
    torch.cuda.synchronize()
    assert torch.equal(pooled.cpu(), pooled_ref.cpu()), f"{name}: pooled values differ"
    assert torch.equal(idx.cpu(), idx_ref.cpu()), f"{name}: route indices differ"
