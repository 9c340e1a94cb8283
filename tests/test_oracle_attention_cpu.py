"""Pins the attention oracle (oracle/bb_oracle.c orc_attn_rows, float64 per row) before it checks the HIP kernel.

Independent checks, each chosen so that a plausible mistake fails one of them:
  * torch's own SDPA in float64 (full routing budget == dense causal, modal_rd/selfcheck.py:36-41; exact tail
    front=0/window=N == causal rows, tests/test_rd_attention_gqa.py:90-102 of the reference);
  * the selfcheck masked-union formula (modal_rd/selfcheck.py:18-26) and the masked-dense restatement of
    kernels/bigger_bird_flash_ref.py (oracle.flash_ref);
  * identity attention front=0/window=1 returns V exactly (modal_rd/check_long_indexing.py:50-54);
  * GQA grouped == repeated K/V (tests/test_rd_attention_gqa.py:63-73);
  * planted mistakes (window edge, GQA map, routed causality) each fail at least one of the above.
"""
import pytest
import torch

import oracle


def _rand(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).to(torch.bfloat16)


def _routes(h, n, front, window, k, seed, groups=1):
    g = torch.Generator().manual_seed(seed)
    span = max(n - window - front, 1)
    rows = [(torch.randperm(span, generator=g)[:k] + front).sort().values for _ in range(h * groups)]
    return torch.stack(rows).view(h, groups, -1).to(torch.int32)


def test_full_budget_equals_dense_causal_sdpa():
    h, n, d, sink, window = 4, 300, 64, 16, 64
    q, k, v = _rand((h, n, d), 1), _rand((h, n, d), 2), _rand((h, n, d), 3)
    full = torch.arange(sink, n - window, dtype=torch.int32).expand(h, -1).contiguous()
    got = oracle.attn_all(q, k, v, full, front=sink, window=window, num_heads=h, scale=d ** -0.5)
    want = oracle.sdpa_ref(q, k, v, causal=True, scale=d ** -0.5)
    assert (got - want).abs().max().item() < 1e-12


def test_fp16_decode_matches_torch_on_every_bit_pattern():
    bits = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.float16)
    want = bits.float()
    got = torch.tensor([oracle.lib().orc_f16_to_f32(i) for i in range(65536)], dtype=torch.float32)
    nan = want.isnan()
    assert torch.equal(got.isnan(), nan)
    assert torch.equal(got[~nan].view(torch.int32), want[~nan].view(torch.int32))


@pytest.mark.parametrize("groups", [1, 4])
def test_fp16_full_budget_equals_dense_causal_sdpa(groups):
    H, n, d, sink, window = 8, 260, 64, 16, 64
    g = torch.Generator().manual_seed(21)
    q = torch.randn(H, n, d, generator=g).half()
    k = torch.randn(H // groups, n, d, generator=g).half()
    v = torch.randn(H // groups, n, d, generator=g).half()
    full = torch.arange(sink, n - window, dtype=torch.int32).expand(H, -1).contiguous()
    got = oracle.attn_all(q, k, v, full, front=sink, window=window, num_heads=H, kv_groups=groups, scale=d ** -0.5)
    want = oracle.sdpa_ref(q, k, v, causal=True, scale=d ** -0.5, groups=groups)
    assert (got - want).abs().max().item() < 1e-12
    # The same bits read as bf16 are different numbers: the element type is not ignored.
    wrong = oracle.attn_all(q.view(torch.bfloat16), k.view(torch.bfloat16), v.view(torch.bfloat16), full, front=sink,
                            window=window, num_heads=H, kv_groups=groups, scale=d ** -0.5)
    assert not torch.allclose(wrong, want, atol=1e-3)
    with pytest.raises(ValueError):
        oracle.attn_all(q, k.view(torch.bfloat16), v, full, front=sink, window=window, num_heads=H, kv_groups=groups)


def test_tail_window_n_equals_causal_rows():
    H, Hkv, N, r, d = 8, 2, 400, 37, 64
    q, k, v = _rand((H, N, d), 4), _rand((Hkv, N, d), 5), _rand((Hkv, N, d), 6)
    none = torch.full((H, 1, 1), -1, dtype=torch.int32)
    got = oracle.attn_all(q[:, N - r:], k, v, none, front=0, window=N, num_heads=H, kv_groups=4, scale=0.1)
    want = oracle.sdpa_ref(q, k, v, causal=True, scale=0.1, groups=4)[:, N - r:]
    assert (got - want).abs().max().item() < 1e-12


@pytest.mark.parametrize("front,window", [(16, 64), (0, 1), (5, 300), (64, 7)])
def test_matches_selfcheck_masked_union(front, window):
    h, n, d = 4, 256, 32
    q, k, v = _rand((h, n, d), 7), _rand((h, n, d), 8), _rand((h, n, d), 9)
    idx = _routes(h, n, front, window, 20, 10)
    got = oracle.attn_all(q, k, v, idx, front=front, window=window, num_heads=h, scale=0.2)
    want = oracle.masked_union_reference(q, k, v, front, window, idx[:, 0], scale=0.2)
    assert (got - want.double()).abs().max().item() < 2e-5


def test_matches_masked_dense_restatement_gqa_groups_mask_offset():
    H, Hkv, T, N, d, front, window, chunk = 8, 2, 150, 256, 32, 8, 40, 64
    q, k, v = _rand((H, T, d), 11), _rand((Hkv, N, d), 12), _rand((Hkv, N, d), 13)
    idx = _routes(H, N, front, window, 12, 14, groups=N // chunk)
    idx[:, 1, :3] = -1
    mask = torch.ones(1, N, dtype=torch.bool)
    mask[0, 120:140] = False
    kw = dict(front=front, window=window, num_heads=H, kv_groups=4, scale=0.15, route_chunk=chunk)
    got = oracle.attn_all(q, k, v, idx, token_mask=mask, **kw)
    want = oracle.flash_ref(q, k, v, idx, token_mask=mask, **kw)
    assert (got - want.double()).abs().max().item() < 8e-3  # bf16 output rounding of the restatement
    want32 = oracle.flash_ref(q.float(), k.float(), v.float(), idx, token_mask=mask, **kw)
    assert (got - want32.double()).abs().max().item() < 2e-5


def test_identity_attention_is_exact():
    h, n, d = 8, 500, 32
    q, k = torch.zeros(h, n, d, dtype=torch.bfloat16), torch.zeros(2, n, d, dtype=torch.bfloat16)
    v = _rand((2, n, d), 15)
    idx = torch.empty(h, 1, 0, dtype=torch.int32)
    got = oracle.attn_all(q, k, v, idx, front=0, window=1, num_heads=h, kv_groups=4)
    assert torch.equal(got, v.double().repeat_interleave(4, 0))


def test_grouped_equals_repeated():
    h, g, n, d = 8, 4, 200, 32
    q, k, v = _rand((h, n, d), 16), _rand((h // g, n, d), 17), _rand((h // g, n, d), 18)
    idx = _routes(h, n, 16, 64, 24, 19)
    kw = dict(front=16, window=64, num_heads=h, scale=0.2)
    a = oracle.attn_all(q, k, v, idx, kv_groups=g, **kw)
    b = oracle.attn_all(q, k.repeat_interleave(g, 0), v.repeat_interleave(g, 0), idx, **kw)
    assert torch.equal(a, b)


def test_planted_mistakes_are_caught():
    h, n, d, front, window = 4, 256, 32, 16, 64
    q, k, v = _rand((h, n, d), 7), _rand((h, n, d), 8), _rand((h, n, d), 9)
    idx = _routes(h, n, front, window, 20, 10)
    want = oracle.masked_union_reference(q, k, v, front, window, idx[:, 0], scale=0.2).double()
    for code in (1, 3):  # window edge off by one; routed keys ignore causality
        with oracle.mutation(code):
            got = oracle.attn_all(q, k, v, idx, front=front, window=window, num_heads=h, scale=0.2)
        assert (got - want).abs().max().item() > 1e-3, code
    hq, g = 8, 4
    q2, k2, v2 = _rand((hq, n, d), 16), _rand((hq // g, n, d), 17), _rand((hq // g, n, d), 18)
    idx2 = _routes(hq, n, 16, 64, 24, 19)
    kw = dict(front=16, window=64, num_heads=hq, scale=0.2)
    rep = oracle.attn_all(q2, k2.repeat_interleave(g, 0), v2.repeat_interleave(g, 0), idx2, **kw)
    with oracle.mutation(2):  # transposed GQA head map
        got = oracle.attn_all(q2, k2, v2, idx2, kv_groups=g, **kw)
    assert (got - rep).abs().max().item() > 1e-3
