"""kv_evict on the GPU (mirrors the reference's tests/test_kv_evict.py:26-100 with a tiny random-init Llama):
prefill logits are unchanged by eviction, every layer's cache shrinks to sink + window + groups * vertical rows, the
kept positions are sorted and unique with the sink, the window and every routed column of the layer's query heads,
and the compacted cache equals the full cache gathered at the kept positions (torch's own gather). The two HIP
helpers evict runs on (topk_columns, gather_rows) are also checked against torch.topk / torch.gather directly."""
import pytest
import torch

from bigger_bird_amd import install
from bigger_bird_amd.decode import gather_rows, topk_columns

pytestmark = pytest.mark.gpu

KW = dict(sink=8, window=96, vertical=24, n_route=16, exact_tail=24, block_m=16, block_n=16)
N = 400


def _tiny(dev, dtype=torch.bfloat16):
    from transformers import LlamaConfig, LlamaForCausalLM

    cfg = LlamaConfig(vocab_size=512, hidden_size=512, intermediate_size=1024, num_hidden_layers=2,
                      num_attention_heads=16, num_key_value_heads=4, max_position_embeddings=8192,
                      attn_implementation="sdpa")
    torch.manual_seed(0)
    return LlamaForCausalLM(cfg).to(dev, dtype).eval()


def _prefill(model, ids):
    from transformers import DynamicCache

    cache = DynamicCache()
    with torch.inference_mode():
        logits = model(ids, past_key_values=cache, use_cache=True).logits
    return logits, cache


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_prefill_unchanged_cache_shrinks_and_retained_set(dtype, dev):
    print(f"case kv_evict_model {dtype}", flush=True)
    torch.manual_seed(4)
    ids = torch.randint(0, 512, (1, N), device=dev)
    model = _tiny(dev, dtype)
    install(model, "rd", **KW)
    want, full = _prefill(model, ids)
    install(model, "rd", kv_evict=True, **KW)
    got, cache = _prefill(model, ids)
    assert torch.equal(got, want), "eviction must not change prefill output"
    cfg = model.config
    g = cfg.num_attention_heads // cfg.num_key_value_heads
    d = cfg.hidden_size // cfg.num_attention_heads
    m = KW["sink"] + KW["window"] + g * KW["vertical"]
    for i, layer in enumerate(model.model.layers):
        assert cache.layers[i].keys.shape == (1, cfg.num_key_value_heads, m, d)
        assert full.layers[i].keys.shape[-2] == N
        a = layer.self_attn
        kept = a.kept
        assert (kept[:, :-1] < kept[:, 1:]).all(), "positions sorted and unique"
        assert (kept[:, :KW["sink"]] == torch.arange(KW["sink"], device=dev)).all()
        assert (kept[:, -KW["window"]:] == torch.arange(N - KW["window"], N, device=dev)).all()
        for h in range(cfg.num_attention_heads):  # every routed column survives
            assert torch.isin(a.last_routes[h].long(), kept[h // g]).all()
        gi = kept[None, :, :, None].expand(1, -1, -1, d)
        assert torch.equal(cache.layers[i].keys, full.layers[i].keys.gather(2, gi))
        assert torch.equal(cache.layers[i].values, full.layers[i].values.gather(2, gi))


def test_helpers_match_torch(dev):
    g = torch.Generator().manual_seed(3)
    vals = torch.rand(6, 5000, generator=g).to(dev)  # distinct values: no ties
    vals[2, 100:200] = 0.0                           # zeros rank last but are still selectable
    front, tail, budget = 37, 900, 700
    got = topk_columns(vals, budget, front=front, tail=tail)
    for r in range(6):
        seg = vals[r, front:5000 - tail]
        want = (seg.topk(budget).indices + front).sort().values.to(torch.int32)
        assert torch.equal(got[r], want), r
    x = torch.randn(4, 3000, 128, generator=g).to(torch.bfloat16).to(dev)
    idx = torch.randint(0, 3000, (4, 517), generator=g).to(dev)
    out = gather_rows(x, idx)
    assert torch.equal(out, x.gather(1, idx[:, :, None].expand(-1, -1, 128)))


def _topk_ref(vals, budget, front, tail):
    """(value desc, index asc) over [front, n - tail), ascending indices; values <= 0 / NaN rank last."""
    out = []
    for row in vals.double().cpu():
        seg = row[front:row.shape[0] - tail].clone()
        seg[~(seg > 0)] = 0.0
        order = torch.argsort(-seg, stable=True)[:budget] + front
        out.append(order.sort().values)
    return torch.stack(out).to(torch.int32)


@pytest.mark.parametrize("case", ["wide_range", "ties", "above_clamp", "below_clamp", "mixed_signs", "one_bin"])
def test_topk_columns_float_bins(case, dev):
    """The float-key histogram bins 32 per octave over [2^-40, 2^25) and clamps outside; clamped bins, heavy ties
    (candidate overflow -> radix select) and non-positive values must still give the exact top-k. `one_bin` puts
    every key in one bin with distinct values inside sub-bins and exact duplicates (the final kernel's sub-bin
    refinement and its pairwise ranking of the threshold sub-bin)."""
    print(f"case topk_float_bins {case}", flush=True)
    g = torch.Generator().manual_seed(11)
    rows, n, front, tail, budget = 4, 20000, 5, 300, 700
    if case == "wide_range":
        vals = torch.exp2(torch.rand(rows, n, generator=g) * 110 - 65)          # 2^-65 .. 2^45
    elif case == "ties":
        vals = torch.randint(0, 6, (rows, n), generator=g).float() * 0.25     # six values, 3000+ ties each
    elif case == "above_clamp":
        vals = 2.0 ** 30 * (1 + torch.rand(rows, n, generator=g))             # one clamped bin, distinct values
    elif case == "below_clamp":
        vals = 2.0 ** -50 * (1 + torch.rand(rows, n, generator=g))
    elif case == "one_bin":
        vals = 1.0 + torch.randint(0, 4096, (rows, n), generator=g).float() * 2.0 ** -19
    else:
        vals = torch.randn(rows, n, generator=g)                                # half non-positive
        vals[:, ::7] = float("nan")
    got = topk_columns(vals.to(dev), budget, front=front, tail=tail).cpu()
    assert torch.equal(got, _topk_ref(vals, budget, front, tail))


def test_evict_options_match_torch_topk(dev, monkeypatch):
    """kv_evict with its tuning options (evict_keep, evict_pool / evict_pool_back span pooling, evict_obs exact
    scoring with mean and max pooling, evict_window, evict_full_layers; modal_rd/attention.py:226-259): the kept
    positions and the compacted caches equal those of the same policy with torch's topk + sort in place of the HIP
    top-k and torch's gather in place of the HIP row gather."""
    print("case kv_evict_options", flush=True)
    from bigger_bird_amd import attention as rd

    def torch_topk(vals, budget, *, front=0, tail=0):
        seg = vals[:, front:vals.shape[1] - tail]
        return (seg.topk(budget, dim=-1).indices + front).sort(-1).values.to(torch.int32)

    def torch_gather(x, idx):
        return x.gather(1, idx[:, :, None].expand(-1, -1, x.shape[-1]))

    torch.manual_seed(5)
    ids = torch.randint(0, 512, (1, N), device=dev)
    model = _tiny(dev)
    for opts in (dict(evict_keep=150, evict_pool=3, evict_pool_back=1, evict_window=128, evict_full_layers=1),
                 dict(evict_obs=16, evict_obs_max=True, evict_pool=2),
                 dict(evict_obs=8)):
        install(model, "rd", kv_evict=True, **KW, **opts)
        _, got = _prefill(model, ids)
        kept = [layer.self_attn.kept.clone() for layer in model.model.layers]
        with monkeypatch.context() as m:
            m.setattr(rd, "topk_columns", torch_topk)
            m.setattr(rd, "gather_rows", torch_gather)
            _, want = _prefill(model, ids)
        for i, layer in enumerate(model.model.layers):
            assert torch.equal(kept[i], layer.self_attn.kept), (opts, i)
            assert torch.equal(got.layers[i].keys, want.layers[i].keys), (opts, i)
            assert torch.equal(got.layers[i].values, want.layers[i].values), (opts, i)
        if opts.get("evict_full_layers"):
            assert kept[0].shape[-1] == N and got.layers[0].keys.shape[-2] == N


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_decode_matches_masked_full_cache(dtype, dev):
    """tests/test_kv_evict.py:67-100 of the reference: 6 greedy tokens through HF generate on the evicted cache (the
    HIP decode over the compacted rows; this also checks that RoPE positions continue from the prompt length) equal
    those of a full-cache model whose decode attention is masked to the same kept positions plus every generated
    token. The masked reference runs float32 SDPA; scores within 2e-2, sequences equal; bf16 and fp16 models."""
    import types

    import torch.nn.functional as F

    print(f"case kv_evict_decode {dtype}", flush=True)
    torch.manual_seed(4)
    ids = torch.randint(0, 512, (1, N), device=dev)
    gen = dict(max_new_tokens=6, min_new_tokens=6, do_sample=False, use_cache=True, pad_token_id=0,
               output_scores=True, return_dict_in_generate=True)
    ev = _tiny(dev, dtype)
    install(ev, "rd", kv_evict=True, **KW)
    with torch.inference_mode():
        out = ev.generate(ids, **gen)
    kept = [layer.self_attn.kept for layer in ev.model.layers]
    g = ev.config.num_attention_heads // ev.config.num_key_value_heads
    m = KW["sink"] + KW["window"] + g * KW["vertical"]
    assert all(kp.shape[-1] == m for kp in kept)

    ref = _tiny(dev, dtype)
    install(ref, "rd", **KW)
    for layer, kp in zip(ref.model.layers, kept):
        attn = layer.self_attn
        orig = attn.exact_attention

        def masked(self, q, k, v, t, n, _orig=orig, _kp=kp):
            if t == n:
                return _orig(q, k, v, t, n)
            keep = torch.zeros(self.num_kv_heads, n, dtype=torch.bool, device=q.device)
            keep.scatter_(1, _kp, True)
            keep[:, N:] = True  # every generated token
            mask = keep.repeat_interleave(self.groups, 0)[None, :, None, :]
            kf = k.float().repeat_interleave(self.groups, 1)
            vf = v.float().repeat_interleave(self.groups, 1)
            o = F.scaled_dot_product_attention(q.float(), kf, vf, attn_mask=mask, scale=self.scaling)
            return o.to(q.dtype)

        attn.exact_attention = types.MethodType(masked, attn)
    with torch.inference_mode():
        want = ref.generate(ids, **gen)
    assert len(out.scores) == 6, "all decode steps must run"
    assert torch.equal(out.sequences, want.sequences)
    for a, b in zip(out.scores, want.scores):
        torch.testing.assert_close(a.float(), b.float(), atol=2e-2, rtol=2e-2)
