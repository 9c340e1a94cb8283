"""Split-K sparse decode and fused decode routing on the GPU (through the C ABI) against the float64 oracles.

Mirrors the reference's kernels/tests/test_bigger_bird_decode.py and test_bigger_bird_route.py: the same shapes,
strided cache views, pooled and per-head route rows, the device-side length with garbage past it, dense mode, the
short-cache error, and the same bars (decode: atol = rtol = 1e-2; pooled probabilities: atol 1e-6, rtol 2e-3;
routes: at least 99% overlap with the oracle's top-k, near-ties may swap). Beyond the reference: the routed keys
must be exactly the top-k of the kernel's own probabilities with ties to the lower index, and a captured HIP graph
of a whole decode step (append to the cache, route, decode) replays with a growing device-side length and matches
the same step run eagerly.
"""
import pytest
import torch

import oracle
from bigger_bird_amd import bigger_bird_decode, bigger_bird_route, pooled_probs
from bigger_bird_amd.decode import kv_append

pytestmark = pytest.mark.gpu


def _cache(n, hk, d, dtype, seed, scale_k=2.0):
    g = torch.Generator().manual_seed(seed)
    cache = torch.randn(2, 1, hk, n, d, generator=g).to(dtype)
    return cache[0, 0] * scale_k, cache[1, 0]


def _routes(rows, n, front, window, r, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.stack([front + torch.randperm(n - window - front, generator=g)[:r] for _ in range(rows)])


@pytest.mark.parametrize("n,front,window,routed,pooled,splits,dtype,d,hk", [
    (4096, 64, 1024, 256, True, None, torch.bfloat16, 128, 8),
    (4096, 64, 1024, 256, False, None, torch.bfloat16, 128, 8),
    (20000, 64, 4096, 512, True, 7, torch.float16, 128, 8),
    (20000, 16, 333, 1000, False, 1, torch.bfloat16, 128, 8),
    (70000, 64, 16384, 512, True, None, torch.bfloat16, 128, 8),
    (9000, 32, 2048, 300, True, None, torch.bfloat16, 64, 4),     # head_dim 64, 8 query heads per KV head
    (9000, 32, 2048, 300, False, 3, torch.float16, 64, 16),       # head_dim 64, 2 query heads per KV head
])
def test_sparse_decode_matches_oracle(n, front, window, routed, pooled, splits, dtype, d, hk, dev):
    print(f"case sparse_decode n={n} pooled={pooled} splits={splits} {dtype} d={d} hk={hk}", flush=True)
    h = 32
    k, v = _cache(n, hk, d, dtype, 0)
    g = torch.Generator().manual_seed(1)
    q = torch.randn(h, d, generator=g).to(dtype)
    idx = _routes(hk if pooled else h, n, front, window, routed, 2)
    kd, vd = k.to(dev), v.to(dev)  # strided views of one [2, 1, Hkv, n, d] buffer on the host; copies keep strides
    out = bigger_bird_decode(q.to(dev), kd, vd, idx.to(dev), front=front, window=window, scale=d ** -0.5,
                             splits=splits)
    ref = oracle.sparse_decode(q, k, v, idx, front=front, window=window, scale=d ** -0.5)
    assert out.dtype == dtype and out.shape == (h, d)
    torch.testing.assert_close(out.float().cpu().double(), ref, atol=1e-2, rtol=1e-2)


def test_strided_cache_view(dev):
    """K/V as views of one [2, 1, Hkv, cap, d] device buffer (the reference's cache layout), with a per-head list."""
    print("case strided_view", flush=True)
    h, hk, d, n = 32, 8, 128, 6000
    g = torch.Generator().manual_seed(3)
    cache = torch.randn(2, 1, hk, n, d, generator=g).to(torch.bfloat16).to(dev)
    k, v = cache[0, 0], cache[1, 0]
    q = torch.randn(h, d, generator=g).to(torch.bfloat16).to(dev)
    idx = _routes(h, n, 32, 512, 200, 4).to(dev)
    out = bigger_bird_decode(q, k, v, idx, front=32, window=512, scale=0.09)
    ref = oracle.sparse_decode(q.cpu(), k.cpu(), v.cpu(), idx.cpu(), front=32, window=512, scale=0.09)
    torch.testing.assert_close(out.float().cpu().double(), ref, atol=1e-2, rtol=1e-2)


def test_device_length_and_dense_mode(dev):
    """n as a GPU tensor inside a larger buffer (garbage past it); front=0 / window=cap / no routes = dense."""
    print("case device_length_dense", flush=True)
    h, hk, d, cap, n = 32, 8, 128, 9000, 7777
    g = torch.Generator().manual_seed(5)
    k = torch.randn(hk, cap, d, generator=g).to(torch.bfloat16)
    v = torch.randn(hk, cap, d, generator=g).to(torch.bfloat16)
    k[:, n:] = 100
    q = torch.randn(h, d, generator=g).to(torch.bfloat16)
    length = torch.tensor([n], device=dev)
    idx = _routes(hk, n, 64, 1024, 300, 6)
    sparse = bigger_bird_decode(q.to(dev), k.to(dev), v.to(dev), idx.to(dev), front=64, window=1024, scale=d ** -0.5,
                                n=length)
    ref = oracle.sparse_decode(q, k[:, :n], v[:, :n], idx, front=64, window=1024, scale=d ** -0.5)
    torch.testing.assert_close(sparse.float().cpu().double(), ref, atol=1e-2, rtol=1e-2)
    none = torch.empty(hk, 0, dtype=torch.long, device=dev)
    dense = bigger_bird_decode(q.to(dev), k.to(dev), v.to(dev), none, front=0, window=cap, scale=d ** -0.5, n=length)
    exact = oracle.sparse_decode(q, k[:, :n], v[:, :n], torch.empty(hk, 0, dtype=torch.long), front=0, window=n,
                                 scale=d ** -0.5)
    torch.testing.assert_close(dense.float().cpu().double(), exact, atol=1e-2, rtol=1e-2)


def test_rejects_short_cache(dev):
    k = torch.zeros(8, 100, 128, device=dev, dtype=torch.bfloat16)
    q = torch.zeros(32, 128, device=dev, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="cache shorter than front"):
        bigger_bird_decode(q, k, k, torch.zeros(8, 4, dtype=torch.long, device=dev), front=64, window=64)
    with pytest.raises(ValueError, match="indices must be"):
        bigger_bird_decode(q, k, k, torch.zeros(3, 4, dtype=torch.long, device=dev), front=8, window=8)
    with pytest.raises(ValueError, match="FP16/BF16"):
        bigger_bird_decode(q.float(), k, k, torch.zeros(8, 4, dtype=torch.long, device=dev), front=8, window=8)


@pytest.mark.parametrize("cap,n,front,window,routed,dtype,device_n,d,hk", [
    (5000, 5000, 64, 1024, 256, torch.bfloat16, False, 128, 8),
    (40000, 40000, 64, 4096, 1024, torch.bfloat16, False, 128, 8),
    (40000, 33333, 16, 1000, 512, torch.float16, True, 128, 8),
    (131072, 131072, 64, 1024, 1024, torch.bfloat16, False, 128, 8),
    (12000, 11000, 32, 2048, 400, torch.bfloat16, True, 64, 4),   # head_dim 64, 8 query heads per KV head
    (12000, 12000, 32, 2048, 400, torch.float16, False, 64, 32),  # one query head per KV head
])
def test_route_matches_oracle(cap, n, front, window, routed, dtype, device_n, d, hk, dev):
    print(f"case route cap={cap} n={n} device_n={device_n} {dtype} d={d} hk={hk}", flush=True)
    h = 32
    g = torch.Generator().manual_seed(0)
    k = (torch.randn(hk, cap, d, generator=g) * 2).to(dtype)
    k[:, n:] = 50
    q = torch.randn(h, d, generator=g).to(dtype)
    scale = d ** -0.5
    kw = dict(front=front, window=window, scale=scale, n=torch.tensor([n], device=dev) if device_n else None)
    k_in = (k if device_n else k[:, :n]).to(dev)
    p = pooled_probs(q.to(dev), k_in, **kw).cpu()
    ref = oracle.pooled_probs(q, k[:, :n], front=front, window=window, scale=scale)
    torch.testing.assert_close(p[:, :n].double(), ref, atol=1e-6, rtol=2e-3)
    if device_n:
        assert (p[:, n:] == -1).all()
    idx = bigger_bird_route(q.to(dev), k_in, routed, **kw).cpu()
    want = ref.topk(routed, dim=-1).indices
    for kv, (a, b) in enumerate(zip(idx.tolist(), want.tolist())):
        assert len(set(a) & set(b)) >= 0.99 * routed, kv  # near-ties may swap at the boundary
        # exactly the top-k of the kernel's own probabilities (value desc, index asc), ascending
        vals = p[kv, front:n - window]
        order = torch.argsort(-vals, stable=True)[:routed] + front
        assert a == sorted(order.tolist()), kv


def test_route_fewer_eligible_than_budget(dev):
    """Fewer eligible keys than k_route: all of them, ascending, then -1."""
    h, hk, d, n = 8, 2, 64, 300
    g = torch.Generator().manual_seed(9)
    k = torch.randn(hk, n, d, generator=g).to(torch.bfloat16).to(dev)
    q = torch.randn(h, d, generator=g).to(torch.bfloat16).to(dev)
    idx = bigger_bird_route(q, k, 64, front=10, window=250, scale=0.1).cpu()
    want = torch.cat([torch.arange(10, 50), torch.full((24,), -1)]).to(torch.int32)
    assert torch.equal(idx, want.expand(hk, -1))


def test_graph_captured_decode_step(dev):
    """A whole decode step -- append the new K/V row at the device-side length, route on the grown cache, sparse
    decode -- captured once in a HIP graph and replayed with a growing length; every replay equals the same step run
    eagerly (no memset nodes: the kernels clear their own histograms and counters)."""
    print("case graph_decode", flush=True)
    h, hk, d, cap, n0 = 32, 8, 128, 12000, 9000
    front, window, routed = 64, 2048, 256
    g = torch.Generator().manual_seed(11)
    k0 = torch.randn(hk, cap, d, generator=g).to(torch.bfloat16).to(dev)
    v0 = torch.randn(hk, cap, d, generator=g).to(torch.bfloat16).to(dev)
    steps = [(torch.randn(h, d, generator=g).to(torch.bfloat16).to(dev),
              torch.randn(hk, d, generator=g).to(torch.bfloat16).to(dev),
              torch.randn(hk, d, generator=g).to(torch.bfloat16).to(dev)) for _ in range(4)]
    scale = d ** -0.5

    def step(k, v, length, q, kn, vn):
        kv_append(k, v, kn, vn, length)
        idx = bigger_bird_route(q, k, routed, front=front, window=window, scale=scale, n=length)
        return bigger_bird_decode(q, k, v, idx, front=front, window=window, scale=scale, n=length), idx

    # eager reference of the four steps
    ke, ve, le = k0.clone(), v0.clone(), torch.tensor([n0], device=dev)
    eager = [step(ke, ve, le, *s) for s in steps]
    # graph: static inputs, captured once (after a warm-up on a side stream), replayed per step
    kg, vg, lg = k0.clone(), v0.clone(), torch.tensor([n0], device=dev)
    qs, ks_, vs_ = (torch.empty_like(t) for t in steps[0])
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        kw_, vw_, lw_ = kg.clone(), vg.clone(), lg.clone()
        step(kw_, vw_, lw_, *steps[0])
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_g, idx_g = step(kg, vg, lg, qs, ks_, vs_)
    for i, (q, kn, vn) in enumerate(steps):
        qs.copy_(q)
        ks_.copy_(kn)
        vs_.copy_(vn)
        graph.replay()
        torch.cuda.synchronize()
        assert int(lg.item()) == n0 + i + 1
        assert torch.equal(idx_g, eager[i][1]), i
        assert torch.equal(out_g, eager[i][0]), i
        _ = torch.zeros(1, device=dev).sum().item()  # unrelated eager work between replays


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_kv_append_matches_index_copy(dtype, dev):
    """bb_kv_append writes the new rows at the device-side length and advances it: bitwise what two index_copy_ calls
    and the add do, on strided cache views and strided new rows; a length at the capacity writes nothing."""
    print(f"case kv_append {dtype}", flush=True)
    hk, cap, d = 8, 300, 128
    g = torch.Generator().manual_seed(3)
    arena = torch.randn(2, hk, cap, 2 * d, generator=g).to(dtype).to(dev)
    k, v = arena[0, :, :, :d], arena[1, :, :, d:]  # [hk, cap, d] views with row stride 2 d
    ref = arena.clone()
    kr, vr = ref[0, :, :, :d], ref[1, :, :, d:]
    length, lref = torch.tensor([123], device=dev), torch.tensor([123], device=dev)
    for step in range(3):
        rows = torch.randn(hk, 3 * d, generator=g).to(dtype).to(dev)
        kn, vn = rows[:, :d], rows[:, 2 * d:]
        kv_append(k, v, kn, vn, length)
        kr.index_copy_(1, lref, kn[:, None])
        vr.index_copy_(1, lref, vn[:, None])
        lref.add_(1)
        torch.cuda.synchronize()
        assert torch.equal(arena, ref) and int(length.item()) == 124 + step
    full = torch.tensor([cap], device=dev)
    before = arena.clone()
    kv_append(k, v, kn, vn, full)
    torch.cuda.synchronize()
    assert torch.equal(arena, before) and int(full.item()) == cap


@pytest.mark.parametrize("routed,dtype,d,hk", [
    (256, torch.bfloat16, 128, 8),
    (300, torch.float16, 128, 8),
    (128, torch.bfloat16, 64, 4),    # head_dim 64, 8 query heads per KV head
    (0, torch.bfloat16, 128, 8),     # dense: every cached row
    (0, torch.float16, 64, 16),      # dense, 2 query heads per KV head
])
def test_decode_step_matches_separate_launches(routed, dtype, d, hk, dev):
    """bb_decode_step (the new row appended by the first kernel that reads the cache, the length advanced by the
    last) against the same step as separate launches: kv_append at length - 1, then routing + sparse decode (or dense
    decode over the cache), then the length add. Bitwise on the routed indices, the whole cache buffer (strided
    views) and the length, over consecutive steps up to and past the capacity (a length past it appends nothing and
    stays). The output is bitwise for the dense step; the routed step's decode takes its scores from the routing
    pass (the same q.k in another fp32 summation order) instead of recomputing them, so there it may differ from the
    separate launches by one unit in the last place of the output type."""
    print(f"case decode_step routed={routed} {dtype} d={d} hk={hk}", flush=True)
    from bigger_bird_amd.decode import decode_step
    h, cap = 32, 5000
    front, window = 64, 1024
    g = torch.Generator().manual_seed(21)
    arena = torch.randn(2, hk, cap, 2 * d, generator=g).to(dtype).to(dev)
    ref = arena.clone()
    k, v = arena[0, :, :, :d], arena[1, :, :, d:]  # [hk, cap, d] views, row stride 2 d
    kr, vr = ref[0, :, :, :d], ref[1, :, :, d:]
    scale = d ** -0.5
    length, lref = torch.tensor([cap - 3], device=dev), torch.tensor([cap - 3], device=dev)
    for i in range(5):  # lengths cap - 3 .. cap, then cap + 1 (no append)
        q = torch.randn(h, d, generator=g).to(dtype).to(dev)
        rows = torch.randn(2, hk, d, generator=g).to(dtype).to(dev)
        kn, vn = rows[0], rows[1]
        res = decode_step(q, k, v, kn, vn, length, routed=routed, front=front, window=window, scale=scale, advance=1)
        kv_append(kr, vr, kn, vn, lref - 1, advance=0)
        if routed:
            idx_r = bigger_bird_route(q, kr, routed, front=front, window=window, scale=scale, n=lref)
            out_r = bigger_bird_decode(q, kr, vr, idx_r, front=front, window=window, scale=scale, n=lref)
            out, idx = res
            assert torch.equal(idx, idx_r), i
        else:
            out_r = bigger_bird_decode(q, kr, vr, torch.empty(hk, 0, dtype=torch.int32, device=dev), front=0,
                                       window=cap, scale=scale, n=lref)
            out = res
        appended = 1 <= int(lref.item()) <= cap
        if appended:
            lref.add_(1)
        torch.cuda.synchronize()
        if routed:
            ulp = 2.0 ** (-7 if dtype == torch.bfloat16 else -10)
            err = (out.float() - out_r.float()).abs()
            assert bool((err <= out_r.float().abs() * ulp + 1e-6).all()), (i, err.max().item())
        else:
            assert torch.equal(out, out_r), i
        assert torch.equal(arena, ref), i
        assert int(length.item()) == int(lref.item()), i
    assert int(length.item()) == cap + 1


def test_decode_step_in_graph(dev):
    """The fused step captured once and replayed with the length advancing on the device: every replay equals the
    same fused step run eagerly (the kernels write the new row and the length themselves; no memset or copy nodes)."""
    print("case decode_step_graph", flush=True)
    from bigger_bird_amd.decode import decode_step
    h, hk, d, cap, n0 = 32, 8, 128, 12000, 9001
    front, window, routed = 64, 2048, 256
    g = torch.Generator().manual_seed(12)
    k0 = torch.randn(hk, cap, d, generator=g).to(torch.bfloat16).to(dev)
    v0 = torch.randn(hk, cap, d, generator=g).to(torch.bfloat16).to(dev)
    steps = [tuple(torch.randn(*shape, generator=g).to(torch.bfloat16).to(dev) for shape in ((h, d), (hk, d), (hk, d)))
             for _ in range(4)]
    scale = d ** -0.5

    def step(k, v, length, q, kn, vn):
        return decode_step(q, k, v, kn, vn, length, routed=routed, front=front, window=window, scale=scale, advance=1)

    ke, ve, le = k0.clone(), v0.clone(), torch.tensor([n0], device=dev)
    eager = [tuple(t.clone() for t in step(ke, ve, le, *s)) for s in steps]
    kg, vg, lg = k0.clone(), v0.clone(), torch.tensor([n0], device=dev)
    qs, ks_, vs_ = (torch.empty_like(t) for t in steps[0])
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step(kg.clone(), vg.clone(), lg.clone(), *steps[0])
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_g, idx_g = step(kg, vg, lg, qs, ks_, vs_)
    for i, (q, kn, vn) in enumerate(steps):
        qs.copy_(q)
        ks_.copy_(kn)
        vs_.copy_(vn)
        graph.replay()
        torch.cuda.synchronize()
        assert int(lg.item()) == n0 + i + 1
        assert torch.equal(idx_g, eager[i][1]), i
        assert torch.equal(out_g, eager[i][0]), i
        _ = torch.zeros(1, device=dev).sum().item()  # unrelated eager work between replays
    assert torch.equal(kg, ke) and torch.equal(vg, ve)
