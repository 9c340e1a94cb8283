"""Pins the routing oracle (oracle/bb_oracle.c orc_routes) before it is trusted as the GPU router's checker.

  * against the reference's own routes() indices (tests/golden, written by golden/make_golden.py) -- set-exact, for
    bf16 and for fp16 inputs;
  * the score arithmetic against torch's CPU bf16 and fp16 matmuls (the library routine the reference calls);
  * the pooled probabilities against float64 brute force and against the reference's pooled values;
  * closed-form special cases (full budget, ties, planted keys) and planted mistakes that those checks must catch.
"""
import subprocess

import numpy as np
import pytest
import torch

import golden_routes
import oracle
from bigger_bird_amd.synth import make_inputs


def _amx_host():
    try:
        return "amx_bf16" in subprocess.run(["lscpu"], capture_output=True, text=True).stdout
    except OSError:
        return False


def _route_case_kwargs(g):
    return dict(sink=g["sink"], window=g["window"], budget=g["budget"], scaling=g["scaling"], n_route=g["n_route"],
                route_pool=g["route_pool"], qpos=g["qpos"])


SMALL_GOLDEN = ["config1", "small_mean", "odd_planted", "max_pool", "spread", "mha_d32", "vertical_sqrt", "config1_f16",
                "small_mean_f16", "max_pool_f16"]


@pytest.mark.parametrize("name", SMALL_GOLDEN)
def test_oracle_matches_reference_routes(name):
    g = golden_routes.case(name)
    got, pooled = oracle.routes(g["q"][0], g["k"][0], return_pooled=True, **_route_case_kwargs(g))
    golden_routes.check_against_golden(got, g, pooled=pooled, what=name)
    if not name.startswith("max_pool"):
        assert torch.equal(got, g["routes"]), name


@pytest.mark.parametrize("name", ["config2", "config2_f16"])
def test_oracle_matches_reference_routes_128k(name):
    """BASELINE config 2 (T=131072, 32/8 heads, 64 planted keys per KV head): set-exact at the production shape, for
    bf16 and fp16 inputs."""
    g = golden_routes.case(name)
    got = oracle.routes(g["q"][0], g["k"][0], **_route_case_kwargs(g))
    assert torch.equal(got, g["routes"])
    for h in range(g["H"]):
        assert set(g["planted"][0, h // (g["H"] // g["Hkv"])].tolist()) <= set(got[h].tolist())


@pytest.mark.skipif(not _amx_host(), reason="the reference's CPU matmul order is pinned on AMX-BF16 hosts")
@pytest.mark.parametrize("d", [32, 64, 128])
def test_score_order_matches_torch_cpu_matmul(d):
    """orc_amx_dot reproduces torch.matmul on bf16 CPU tensors bit for bit (the reference's score arithmetic)."""
    gen = torch.Generator().manual_seed(d)
    q = torch.randn(2, 256, d, generator=gen).to(torch.bfloat16)
    k = (3 * torch.randn(2, 1024, d, generator=gen)).to(torch.bfloat16)
    s = torch.matmul(q, k.transpose(-1, -2))
    L = oracle.lib()
    qn, kn = q.contiguous(), k.contiguous()
    mism = 0
    for b in range(2):
        for i in range(0, 256, 7):
            for j in range(0, 1024, 5):
                v = L.orc_amx_dot(qn[b, i].data_ptr(), kn[b, j].data_ptr(), d)
                mism += torch.tensor(v).to(torch.bfloat16).item() != s[b, i, j].item()
    assert mism == 0


@pytest.mark.parametrize("d,n", [(32, 1024), (64, 1024), (128, 4096)])
def test_f16_score_order_matches_torch_cpu_matmul(d, n):
    """fp16 inputs: orc_f16_dot (one sequential fp32 chain over d) rounded to fp16 reproduces torch.matmul on fp16 CPU
    tensors bit for bit, with K passed as a transposed view as the reference does (modal_rd/attention.py:164)."""
    gen = torch.Generator().manual_seed(d + n)
    q = torch.randn(2, 256, d, generator=gen).to(torch.float16)
    k = (2 * torch.randn(2, n, d, generator=gen)).to(torch.float16)
    s = torch.matmul(q, k.transpose(-1, -2))
    L = oracle.lib()
    mism = 0
    for b in range(2):
        for i in range(0, 256, 5):
            for j in range(0, n, 7):
                v = L.orc_f16_round(L.orc_f16_dot(q[b, i].data_ptr(), k[b, j].data_ptr(), d))
                mism += v != s[b, i, j].item()
    assert mism == 0


def test_f16_score_order_is_not_the_bf16_order():
    """Planted check for the fp16 score model: the bf16 path's block order (even / odd chains per 32 elements) on the
    same fp16 values differs from torch's fp16 matmul on some scores, so mixing the two orders is caught."""
    gen = torch.Generator().manual_seed(3)
    q = torch.randn(64, 128, generator=gen).to(torch.float16)
    k = (3 * torch.randn(2048, 128, generator=gen)).to(torch.float16)
    s = torch.matmul(q[None], k.T[None])[0].float().numpy()
    qf, kf = q.float().numpy(), k.float().numpy()
    L = oracle.lib()
    flips = 0
    for i in range(0, 64, 3):
        for j in range(0, 2048, 3):
            acc = np.float32(0)
            for b0 in range(0, 128, 32):
                e, o = np.float32(0), np.float32(0)
                for t in range(b0, b0 + 32, 2):
                    e = np.float32(e + np.float32(qf[i, t] * kf[j, t]))
                    o = np.float32(o + np.float32(qf[i, t + 1] * kf[j, t + 1]))
                acc = np.float32(acc + np.float32(e + o))
            flips += L.orc_f16_round(float(acc)) != s[i, j]
    assert flips > 0


def test_score_order_is_not_exact_rounding():
    """The planted check for the score model: exact rounding (score mode 1) differs from torch on some scores, so a
    model mistake of that kind would fail test_score_order_matches_torch_cpu_matmul."""
    gen = torch.Generator().manual_seed(1)
    q = torch.randn(64, 128, generator=gen).to(torch.bfloat16)
    k = torch.randn(4096, 128, generator=gen).to(torch.bfloat16)
    exact = (q.double() @ k.double().T)
    amx = torch.matmul(q[None], k.T[None])[0]
    # round exact to bf16 through the oracle's one-step rounding
    L = oracle.lib()
    flips = 0
    for i in range(0, 64, 3):
        for j in range(0, 4096, 3):
            bits = L.orc_bf16_from_double(exact[i, j].item())
            flips += bits != amx[i, j].view(torch.int16).item() & 0xFFFF
    assert flips > 0


def _fp64_pooled(q, k, qpos, scaling, pool):
    """float64 softmax of the bf16-rounded (torch CPU) scores, pooled over the route queries."""
    H, n, d = q.shape
    G = H // k.shape[0]
    out = np.zeros((H, n))
    for h in range(H):
        s = torch.matmul(q[h, qpos][None], k[h // G].T[None])[0].double() * np.float32(scaling)
        s = s.numpy()
        s[np.arange(n)[None, :] > qpos.numpy()[:, None]] = -np.inf
        p = np.exp(s - s.max(1, keepdims=True))
        p /= p.sum(1, keepdims=True)
        out[h] = p.max(0) if pool == "max" else p.mean(0)
    return out


@pytest.mark.parametrize("pool", ["mean", "max"])
def test_pooled_scores_match_fp64_brute_force(pool):
    T, H, Hkv, d = 600, 4, 2, 64
    inp = make_inputs(T, H, Hkv, d, seed=21, window=100, sink=8)
    q, k = inp["q"][0], inp["k"][0]
    qpos = torch.arange(T - 32, T)
    _, pooled = oracle.routes(q, k, sink=8, window=100, budget=50, scaling=d ** -0.5, n_route=32, route_pool=pool,
                              qpos=qpos, return_pooled=True)
    got = pooled.double().numpy() * 2.0 ** -40 / (32 if pool == "mean" else 1)
    want = _fp64_pooled(q, k, qpos, d ** -0.5, pool)
    sel = want > 1e-7
    rel = np.abs(got[sel] - want[sel]) / want[sel]
    assert rel.max() < 2e-5, rel.max()


def test_pooled_scores_match_reference_col():
    for name in ("small_mean", "mha_d32"):
        g = golden_routes.case(name)
        _, pooled = oracle.routes(g["q"][0], g["k"][0], return_pooled=True, **_route_case_kwargs(g))
        got = pooled.double() * 2.0 ** -40 / g["n_route"]
        col = g["col"].double()
        lo, hi = g["sink"], g["T"] - g["window"]
        sel = col[:, lo:hi] > 1e-6
        rel = ((got[:, lo:hi] - col[:, lo:hi]).abs() / col[:, lo:hi].clamp_min(1e-30))[sel]
        assert rel.max().item() < 1e-5, (name, rel.max().item())


def test_full_budget_is_every_eligible_column():
    T, H, Hkv, d, sink, window = 700, 8, 2, 128, 16, 128
    inp = make_inputs(T, H, Hkv, d, seed=9, window=window, sink=sink)
    idx = oracle.routes(inp["q"][0], inp["k"][0], sink=sink, window=window, budget=T - sink - window,
                        scaling=d ** -0.5)
    assert torch.equal(idx, torch.arange(sink, T - window, dtype=torch.int32).expand(H, -1))


def _tie_inputs():
    T, H, Hkv, d, sink, window = 512, 4, 1, 64, 8, 64
    gen = torch.Generator().manual_seed(5)
    q = torch.randn(H, T, d, generator=gen).to(torch.bfloat16)
    k = torch.randn(Hkv, T, d, generator=gen).to(torch.bfloat16)
    k[0, sink:T - window] = k[0, 100]
    return q, k, sink, window


def test_ties_go_to_lower_index():
    q, k, sink, window = _tie_inputs()
    idx = oracle.routes(q, k, sink=sink, window=window, budget=10, scaling=0.125)
    assert torch.equal(idx, torch.arange(sink, sink + 10, dtype=torch.int32).expand(4, -1))


def test_planted_mistakes_are_caught():
    q, k, sink, window = _tie_inputs()
    with oracle.mutation(4):  # ties to the higher index
        idx = oracle.routes(q, k, sink=sink, window=window, budget=10, scaling=0.125)
    assert not torch.equal(idx, torch.arange(sink, sink + 10, dtype=torch.int32).expand(4, -1))
    T, H, Hkv, d = 700, 8, 2, 128
    inp = make_inputs(T, H, Hkv, d, seed=9, window=128, sink=16)
    with oracle.mutation(5):  # sink columns eligible
        idx = oracle.routes(inp["q"][0], inp["k"][0], sink=16, window=128, budget=T - 16 - 128, scaling=d ** -0.5)
    assert not torch.equal(idx, torch.arange(16, T - 128, dtype=torch.int32).expand(H, -1))


def test_reference_order_restatement_matches_reference():
    """oracle.routes_reference_order (torch CPU ops in the reference's order) reproduces the reference's indices."""
    if not _amx_host():
        pytest.skip("the golden routes were written on an AMX-BF16 host")
    for name in ("config1", "small_mean", "spread", "mha_d32", "vertical_sqrt", "odd_planted"):
        g = golden_routes.case(name)
        idx = oracle.routes_reference_order(g["q"], g["k"], num_heads=g["H"], num_kv_heads=g["Hkv"], sink=g["sink"],
                                            window=g["window"], budget=g["budget"], scaling=g["scaling"],
                                            n_route=g["n_route"], route_pool=g["route_pool"],
                                            route_queries=g["route_queries"])
        assert torch.equal(idx, g["routes"]), name
