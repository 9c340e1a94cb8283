"""bb_sparse_flash (through the C ABI via bigger_bird_flash) against the float64 CPU oracle.

Tolerance: max-abs 2e-2 and mean-abs 2e-3 against the float64 masked-dense oracle for bf16;
fp16 inputs (the reference kernel accepts both, kernels/bigger_bird_flash.py:110) are held to the same bound.
Cases mirror the reference's own checks: tests/test_rd_attention_gqa.py (grouped == repeated, tail == masked SDPA),
modal_rd/selfcheck.py (full budget == dense causal), modal_rd/check_long_indexing.py (identity attention is exact),
tests/test_bigger_bird_flash.py (route chunks, token masks, odd lengths).
"""
import pytest
import torch

import oracle
from bigger_bird_amd import bigger_bird_flash

pytestmark = pytest.mark.gpu

MAX_ABS, MEAN_ABS = 2e-2, 2e-3


def _rand(shape, seed, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).to(dtype)


def _routes(h, n, front, window, k, seed, groups=1, chunk=None):
    g = torch.Generator().manual_seed(seed)
    span = max(n - window - front, 1)
    rows = []
    for _ in range(h * groups):
        perm = torch.randperm(span, generator=g)[:k] + front
        if perm.numel() < k:
            perm = torch.cat([perm, torch.full((k - perm.numel(),), -1)])
        rows.append(perm.sort().values)
    return torch.stack(rows).view(h, groups, k).to(torch.int32)


def _check(got, ref, what):
    err = (got.double().cpu() - ref).abs()
    print(f"{what}: max_abs={err.max().item():.3e} mean_abs={err.mean().item():.3e}", flush=True)
    assert err.max().item() < MAX_ABS and err.mean().item() < MEAN_ABS, what


CASES = [
    # name, H, Hkv, T, N, d, front, window, route_k, scale
    ("gqa4_d32", 8, 2, 384, 384, 32, 16, 64, 24, 0.2),
    ("gqa2_d64_odd", 8, 4, 1000, 1000, 64, 7, 97, 40, 0.125),
    ("gqa4_d128", 32, 8, 2048, 2048, 128, 64, 512, 128, 128 ** -0.5),
    ("mha_d128", 4, 4, 513, 513, 128, 3, 100, 33, 0.1),
    ("gqa8_d128", 16, 2, 700, 700, 128, 64, 128, 64, 128 ** -0.5),
    ("offset_d128", 8, 2, 300, 1100, 128, 32, 200, 50, 128 ** -0.5),
    # the pipelined kernel with 2 and 1 query heads per workgroup (128- and 256-row tiles), and past 512 route slots
    ("gqa2_d128", 16, 8, 1500, 1500, 128, 64, 256, 130, 128 ** -0.5),
    ("mha_d128_600routes", 8, 8, 3000, 3000, 128, 64, 512, 600, 128 ** -0.5),
    ("gqa3_d128", 12, 4, 700, 900, 128, 16, 160, 70, 128 ** -0.5),
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_matches_oracle(case, dtype, dev):
    name, H, Hkv, T, N, d, front, window, rk, scale = case
    print(f"case {name} {dtype}", flush=True)
    q, k, v = _rand((H, T, d), 1, dtype), _rand((Hkv, N, d), 2, dtype), _rand((Hkv, N, d), 3, dtype)
    idx = _routes(H, N, front, window, rk, 4)
    out = bigger_bird_flash(q.to(dev), k.to(dev), v.to(dev), idx.to(dev), front=front, window=window, num_heads=H,
                            kv_groups=H // Hkv, scale=scale)
    torch.cuda.synchronize()
    assert out.shape == (H, T, d) and out.stride() == (d, H * d, 1) and out.dtype == dtype
    ref = oracle.attn_all(q, k, v, idx, front=front, window=window, num_heads=H, kv_groups=H // Hkv, scale=scale)
    _check(out, ref, name)


def test_grouped_equals_repeated(dev):
    print("case grouped_equals_repeated", flush=True)
    h, g, n, d = 8, 4, 384, 32
    q, k, v = _rand((h, n, d), 11), _rand((h // g, n, d), 12), _rand((h // g, n, d), 13)
    idx = _routes(h, n, 16, 64, 24, 14)
    kw = dict(front=16, window=64, num_heads=h, scale=0.2)
    grouped = bigger_bird_flash(q.to(dev), k.to(dev), v.to(dev), idx.to(dev), kv_groups=g, **kw)
    repeated = bigger_bird_flash(q.to(dev), k.repeat_interleave(g, 0).to(dev), v.repeat_interleave(g, 0).to(dev),
                                 idx.to(dev), **kw)
    torch.testing.assert_close(grouped, repeated, atol=2e-2, rtol=1e-3)


@pytest.mark.parametrize("heads", [(32, 8), (32, 16), (32, 32)], ids=["gqa4", "gqa2", "mha"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_tail_window_n_is_dense_causal_rows(dtype, heads, dev):
    """Exact tail: front=0, window=N, no routes == dense causal rows (split-key schedule + merge)."""
    print(f"case tail_split {dtype} {heads}", flush=True)
    (H, Hkv), N, r, d = heads, 4096, 256, 128
    q, k, v = _rand((H, N, d), 21, dtype), _rand((Hkv, N, d), 22, dtype), _rand((Hkv, N, d), 23, dtype)
    none = torch.full((H, 1, 1), -1, dtype=torch.int32)
    Q = q.to(dev)
    out = bigger_bird_flash(Q[:, N - r:], k.to(dev), v.to(dev), none.to(dev), front=0, window=N, num_heads=H,
                            kv_groups=H // Hkv, scale=d ** -0.5)
    torch.cuda.synchronize()
    qp = torch.arange(N - r, N)[:, None]
    mask = torch.arange(N)[None] <= qp
    ref = torch.nn.functional.scaled_dot_product_attention(
        q[:, N - r:].double()[None], k.double().repeat_interleave(H // Hkv, 0)[None],
        v.double().repeat_interleave(H // Hkv, 0)[None], attn_mask=mask, scale=d ** -0.5)[0]
    assert out.dtype == dtype
    _check(out, ref, "tail_split")


def test_full_budget_equals_dense_causal(dev):
    """modal_rd/selfcheck.py:36-41: routing every column outside sink/window gives exact causal attention."""
    print("case full_budget", flush=True)
    h, n, d, sink, window = 8, 1024, 128, 64, 256
    q, k, v = _rand((h, n, d), 31), _rand((h, n, d), 32), _rand((h, n, d), 33)
    full = torch.arange(sink, n - window, dtype=torch.int32).expand(h, -1).contiguous()
    out = bigger_bird_flash(q.to(dev), k.to(dev), v.to(dev), full.view(h, 1, -1).to(dev), front=sink, window=window,
                            num_heads=h, scale=d ** -0.5)
    ref = oracle.sdpa_ref(q, k, v, causal=True, scale=d ** -0.5)
    _check(out, ref, "full_budget")


def test_identity_attention_is_exact(dev):
    """modal_rd/check_long_indexing.py:50-54: front=0, window=1 -> every query sees only its own key: out == V."""
    print("case identity", flush=True)
    h, hk, n, d = 32, 8, 5000, 128
    q = torch.zeros(n, h, d, dtype=torch.bfloat16).permute(1, 0, 2)
    k = torch.zeros(n, hk, d, dtype=torch.bfloat16).permute(1, 0, 2)
    v = torch.stack([((torch.arange(n) % 97).float() + head * 0.25)[:, None].expand(n, d) for head in range(hk)])
    v = v.to(torch.bfloat16)
    idx = torch.empty(h, 1, 0, dtype=torch.int32)
    out = bigger_bird_flash(q.to(dev), k.to(dev), v.to(dev), idx.to(dev), front=0, window=1, num_heads=h, kv_groups=4)
    out = out.cpu()
    for head in range(h):
        assert torch.equal(out[head], v[head // 4]), head


@pytest.mark.parametrize("n,masked", [(524288, False), (995993, False), (1048576, False), (1048576, True),
                                      (2097152, False)])
def test_identity_long_strided(n, masked, dev):
    """modal_rd/check_long_indexing.py:32-56: identity attention (front 0, window 1) on model-strided views
    (q [n, 32, 128], k / v [n, 8, 128] permuted to head-major) past the 2^31-byte mark of a KV head's K rows: every
    output row must equal its V row exactly. The pipelined kernel takes up to 2^32 bytes of one head's K rows
    (2097088 tokens at this stride); an all-true token mask (at 1048576) and the 2097152-token case route the call to
    the generic kernel (flash_kernel), so both kernels' addressing is exercised past 2^31 bytes."""
    print(f"case identity_long n={n} masked={masked}", flush=True)
    h, hk, d = 32, 8, 128
    q = torch.zeros((n, h, d), device=dev, dtype=torch.bfloat16).permute(1, 0, 2)
    k = torch.zeros((n, hk, d), device=dev, dtype=torch.bfloat16).permute(1, 0, 2)
    pattern = (torch.arange(n, device=dev) % 97).float()[:, None] + 0.25 * torch.arange(hk, device=dev)[None, :]
    v = pattern[:, :, None].expand(n, hk, d).to(torch.bfloat16).permute(1, 0, 2)
    del pattern
    idx = torch.empty(h, 1, 0, dtype=torch.int32, device=dev)
    mask = torch.ones(1, n, dtype=torch.bool, device=dev) if masked else None
    out = bigger_bird_flash(q, k, v, idx, front=0, window=1, num_heads=h, kv_groups=4, token_mask=mask)
    torch.cuda.synchronize()
    assert out.stride() == (d, h * d, 1)
    for head in range(h):
        assert torch.equal(out[head], v[head // 4]), (n, head)


def test_million_token_rows_match_oracle(dev):
    """A full sparse layer at 1048576 tokens on model-strided views ({64, 16384}, 512 routes per head): sampled rows
    of one KV group (heads 28..31), including the last rows, against the float64 oracle."""
    n, h, hk, d, front, window, rk = 1048576, 32, 8, 128, 64, 16384, 512
    print(f"case million_rows n={n}", flush=True)
    g = torch.Generator(device=dev).manual_seed(61)
    q = torch.randn((n, h, d), device=dev, generator=g).to(torch.bfloat16).permute(1, 0, 2)
    k = torch.randn((n, hk, d), device=dev, generator=g).to(torch.bfloat16).permute(1, 0, 2)
    v = torch.randn((n, hk, d), device=dev, generator=g).to(torch.bfloat16).permute(1, 0, 2)
    gc = torch.Generator().manual_seed(62)
    idx = torch.stack([torch.randperm(n - window - front, generator=gc)[:rk].sort().values + front
                       for _ in range(h)]).to(torch.int32)
    out = bigger_bird_flash(q, k, v, idx.view(h, 1, rk).to(dev), front=front, window=window, num_heads=h, kv_groups=4,
                            scale=d ** -0.5)
    torch.cuda.synchronize()
    heads = slice(28, 32)
    rows = torch.cat([torch.tensor([0, 63, 64, window - 1, window, window + 1, n // 2, n - 65, n - 64, n - 2, n - 1]),
                      idx[28:32, ::64].reshape(-1).long() + window, torch.randint(0, n, (24,), generator=gc)])
    pairs = torch.stack([torch.arange(4).repeat_interleave(rows.numel()), rows.repeat(4)], -1)
    ref = oracle.attn_rows(q[heads].cpu(), k[7:8].cpu(), v[7:8].cpu(), idx[heads].view(4, 1, rk), pairs, front=front,
                           window=window, num_heads=4, kv_groups=4, scale=d ** -0.5)
    got = out[heads].cpu()[pairs[:, 0], pairs[:, 1]]
    _check(got, ref, "million_rows")


@pytest.mark.parametrize("t,n,H,Hkv,d,dtype", [(2, 20000, 32, 8, 128, torch.bfloat16),
                                               (65, 131072, 32, 8, 128, torch.bfloat16),
                                               (300, 5000, 32, 8, 128, torch.bfloat16),
                                               (7, 3000, 8, 2, 64, torch.bfloat16),
                                               (300, 5000, 32, 8, 128, torch.float16),
                                               (7, 3000, 8, 2, 64, torch.float16),
                                               (300, 5000, 16, 8, 128, torch.bfloat16),
                                               (65, 5000, 16, 16, 128, torch.bfloat16)])
def test_exact_attention_noncausal(t, n, H, Hkv, d, dtype, dev):
    """bb_exact_attention: t query rows, each attending all n cached keys (the reference's SDPA with is_causal=False
    for 1 < t < n, modal_rd/attention.py:140-141), in one call, against float64 SDPA; also through
    RDAttention.exact_attention on [1, H, t, d] / [1, Hkv, n, d] views."""
    print(f"case exact_noncausal t={t} n={n} H={H}/{Hkv} d={d} {dtype}", flush=True)
    from types import SimpleNamespace

    from bigger_bird_amd import RDAttention, exact_attention

    q, k, v = _rand((H, t, d), 71 + t, dtype), _rand((Hkv, n, d), 72, dtype), _rand((Hkv, n, d), 73, dtype)
    ref = oracle.sdpa_ref(q, k, v, causal=False, scale=d ** -0.5, groups=H // Hkv)
    out = exact_attention(q.to(dev), k.to(dev), v.to(dev), num_heads=H, kv_groups=H // Hkv, scale=d ** -0.5)
    _check(out, ref, f"exact_noncausal t={t} n={n}")
    base = SimpleNamespace(config=SimpleNamespace(num_attention_heads=H, num_key_value_heads=Hkv), layer_idx=0,
                           head_dim=d, scaling=d ** -0.5, q_proj=None, k_proj=None, v_proj=None, o_proj=None)
    attn = RDAttention(base, sink=64, window=1024, vertical=64)
    out2 = attn.exact_attention(q.to(dev)[None], k.to(dev)[None], v.to(dev)[None], t, n)
    assert torch.equal(out2[0], out)


def test_route_groups_and_token_mask(dev):
    """Per-query route groups (vertical_scope layout) and a padding mask (tests/test_bigger_bird_flash.py)."""
    print("case groups_mask", flush=True)
    H, Hkv, n, d, front, window, chunk = 8, 2, 1024, 64, 8, 128, 256
    q, k, v = _rand((H, n, d), 41), _rand((Hkv, n, d), 42), _rand((Hkv, n, d), 43)
    G = n // chunk
    idx = _routes(H, n, front, window, 48, 44, groups=G)
    idx[:, 0] = -1  # first group routes nothing
    mask = torch.ones(H // H, n, dtype=torch.bool)
    mask[0, 100:140] = False
    out = bigger_bird_flash(q.to(dev), k.to(dev), v.to(dev), idx.to(dev), front=front, window=window, num_heads=H,
                            kv_groups=H // Hkv, scale=0.125, route_chunk=chunk, token_mask=mask.to(dev))
    ref = oracle.attn_all(q, k, v, idx, front=front, window=window, num_heads=H, kv_groups=H // Hkv, scale=0.125,
                          route_chunk=chunk, token_mask=mask)
    _check(out, ref, "groups_mask")


def test_config1_sampled_rows(dev):
    """BASELINE config 1 shape (T=8192, 32/8 heads, d=128, {64, 2048, 128}) on random routes, 64 rows per head."""
    print("case config1_rows", flush=True)
    H, Hkv, n, d, front, window, rk = 32, 8, 8192, 128, 64, 2048, 128
    q, k, v = _rand((H, n, d), 51), _rand((Hkv, n, d), 52), _rand((Hkv, n, d), 53)
    idx = _routes(H, n, front, window, rk, 54)
    out = bigger_bird_flash(q.to(dev), k.to(dev), v.to(dev), idx.to(dev), front=front, window=window, num_heads=H,
                            kv_groups=4, scale=d ** -0.5).cpu()
    g = torch.Generator().manual_seed(55)
    rows = torch.cat([torch.randint(0, n, (56,), generator=g), torch.tensor([0, 1, 63, 64, 2047, 2048, n - 2, n - 1])])
    pairs = torch.stack([torch.arange(H).repeat_interleave(rows.numel()), rows.repeat(H)], -1)
    ref = oracle.attn_rows(q, k, v, idx, pairs, front=front, window=window, num_heads=H, kv_groups=4, scale=d ** -0.5)
    _check(out[pairs[:, 0], pairs[:, 1]], ref, "config1_rows")


def test_argument_errors(dev):
    q = torch.zeros(8, 64, 32, dtype=torch.bfloat16, device=dev)
    k = torch.zeros(2, 64, 32, dtype=torch.bfloat16, device=dev)
    idx = torch.zeros(8, 1, 4, dtype=torch.int32, device=dev)
    with pytest.raises(ValueError, match="front >= 0"):
        bigger_bird_flash(q, k, k, idx, front=-1, window=8, num_heads=8, kv_groups=4)
    with pytest.raises(ValueError, match="matching heads"):
        bigger_bird_flash(q, k, k, idx, front=0, window=8, num_heads=8, kv_groups=2)
    with pytest.raises(ValueError, match="at least as long"):
        bigger_bird_flash(q, k[:, :32], k[:, :32], idx, front=0, window=8, num_heads=8, kv_groups=4)
    with pytest.raises(ValueError, match="Routing groups"):
        bigger_bird_flash(q, k, k, idx, front=0, window=8, num_heads=8, kv_groups=4, route_chunk=48)
    with pytest.raises(ValueError):
        bigger_bird_flash(q.cpu(), k.cpu(), k.cpu(), idx.cpu(), front=0, window=8, num_heads=8, kv_groups=4)
