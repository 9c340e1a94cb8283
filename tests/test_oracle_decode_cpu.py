"""Pins the decode oracles (oracle.sparse_decode, oracle.pooled_probs) before they check the HIP kernels.

Independent checks, each chosen so that a plausible mistake fails one of them:
  * dense mode (front=0, window=n, no routes) equals torch SDPA in float64 over the first n keys, grouped query heads
    over repeated K/V (kernels/tests/test_bigger_bird_decode.py:63-68 of the reference);
  * with disjoint front / window / routed sets, the decode of the last token equals the prefill union-mask oracle
    (oracle.attn_rows, pinned in test_oracle_attention_cpu.py) for the query row at position n - 1: two
    independent formulations of the same key set;
  * pooled (route rows = KV heads) and per-head rows agree when every head of a group gets the same list;
  * pooled probabilities: q = 0 gives 1/n on every kept key (uniform softmax), one query head per KV head gives the
    plain softmax, the masked ranges read -1, and each KV head's kept mass plus its masked mass sums to 1;
  * planted mistakes (a window off by one, routed keys dropped, the group mean replaced by the first head) each fail
    one of the above.
"""
import pytest
import torch

import oracle


def _rand(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16)


def _routes(rows, n, front, window, r, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.stack([front + torch.randperm(n - window - front, generator=g)[:r] for _ in range(rows)])


def test_dense_mode_equals_sdpa():
    H, Hkv, n, d = 8, 2, 333, 64
    q, k, v = _rand((H, d), 1), _rand((Hkv, n, d), 2), _rand((Hkv, n, d), 3)
    none = torch.empty(Hkv, 0, dtype=torch.long)
    got = oracle.sparse_decode(q, k, v, none, front=0, window=n, scale=0.125)
    want = torch.nn.functional.scaled_dot_product_attention(
        q.double()[None, :, None], k.double().repeat_interleave(4, 0)[None], v.double().repeat_interleave(4, 0)[None],
        scale=0.125)[0, :, 0]
    assert (got - want).abs().max().item() < 1e-12


def _prefill_last_row(q, k, v, idx_heads, front, window, scale):
    """The decode query as row n-1 of a prefill call with per-head routes (union semantics)."""
    H, d = q.shape
    Hkv, n, _ = k.shape
    qf = torch.zeros(H, n, d, dtype=torch.bfloat16)
    qf[:, n - 1] = q
    rows = torch.stack([torch.arange(H), torch.full((H,), n - 1)], -1)
    return oracle.attn_rows(qf, k, v, idx_heads[:, None, :].to(torch.int32), rows, front=front, window=window,
                            num_heads=H, kv_groups=H // Hkv, scale=scale)


@pytest.mark.parametrize("pooled", [True, False])
def test_matches_prefill_union_oracle(pooled):
    H, Hkv, n, d, front, window, r = 8, 2, 600, 32, 16, 128, 40
    q, k, v = _rand((H, d), 4), _rand((Hkv, n, d), 5), _rand((Hkv, n, d), 6)
    idx = _routes(Hkv if pooled else H, n, front, window, r, 7)
    got = oracle.sparse_decode(q, k, v, idx, front=front, window=window, scale=0.2)
    per_head = idx.repeat_interleave(H // Hkv, 0) if pooled else idx
    want = _prefill_last_row(q, k, v, per_head, front, window, 0.2)
    assert (got - want).abs().max().item() < 1e-9


def test_pooled_equals_per_head_with_shared_lists():
    H, Hkv, n, d = 8, 2, 400, 32
    q, k, v = _rand((H, d), 8), _rand((Hkv, n, d), 9), _rand((Hkv, n, d), 10)
    idx = _routes(Hkv, n, 8, 64, 30, 11)
    a = oracle.sparse_decode(q, k, v, idx, front=8, window=64, scale=0.3)
    b = oracle.sparse_decode(q, k, v, idx.repeat_interleave(4, 0), front=8, window=64, scale=0.3)
    assert torch.equal(a, b)


def test_planted_decode_mistakes_fail(monkeypatch):
    H, Hkv, n, d, front, window, r = 8, 2, 600, 32, 16, 128, 40
    q, k, v = _rand((H, d), 4), _rand((Hkv, n, d), 5), _rand((Hkv, n, d), 6)
    idx = _routes(Hkv, n, front, window, r, 7)
    want = _prefill_last_row(q, k, v, idx.repeat_interleave(4, 0), front, window, 0.2)
    good = oracle.decode_positions
    for bad in (lambda f, w, n_, rt: good(f, w + 1, n_, rt),      # window one key too long
                lambda f, w, n_, rt: good(f, w, n_, [])):         # routed keys dropped
        monkeypatch.setattr(oracle, "decode_positions", bad)
        got = oracle.sparse_decode(q, k, v, idx, front=front, window=window, scale=0.2)
        assert (got - want).abs().max().item() > 1e-4
    monkeypatch.setattr(oracle, "decode_positions", good)


def test_pooled_probs_closed_forms():
    H, Hkv, cap, d, front, window = 8, 2, 300, 32, 10, 50
    k = _rand((Hkv, cap, d), 12)
    n = 250
    zero = torch.zeros(H, d, dtype=torch.bfloat16)
    p = oracle.pooled_probs(zero, k, front=front, window=window, scale=0.1, n=n)
    assert torch.all(p[:, front:n - window] == 1.0 / n)
    assert torch.all(p[:, :front] == -1) and torch.all(p[:, n - window:] == -1)
    # one query head per KV head: the plain softmax over the first n keys
    q1 = _rand((Hkv, d), 13)
    p1 = oracle.pooled_probs(q1, k, front=0, window=0, scale=0.1, n=n)
    for kv in range(Hkv):
        sm = torch.softmax(k[kv, :n].double() @ q1[kv].double() * 0.1, 0)
        assert (p1[kv, :n] - sm).abs().max().item() < 1e-15
    # full mass: kept probabilities plus the masked keys' (recomputed) probabilities sum to one per KV head
    q = _rand((H, d), 14)
    pk = oracle.pooled_probs(q, k, front=front, window=window, scale=0.1, n=n)
    full = oracle.pooled_probs(q, k, front=0, window=0, scale=0.1, n=n)
    assert torch.allclose(full[:, :n].sum(1), torch.ones(Hkv, dtype=torch.float64), atol=1e-12)
    assert torch.equal(pk[:, front:n - window], full[:, front:n - window])


def test_pooled_probs_planted_first_head_fails():
    H, Hkv, cap, d = 8, 2, 200, 32
    q, k = _rand((H, d), 15), _rand((Hkv, cap, d), 16)
    p = oracle.pooled_probs(q, k, front=0, window=0, scale=0.2)
    first = oracle.pooled_probs(q[::4].contiguous(), k, front=0, window=0, scale=0.2)  # group mean -> first head
    assert (p - first).abs().max().item() > 1e-4
