"""Int8KVLayer (bigger_bird_amd.kv_int8, drop-in for modal_rd/kv_int8.py) inside a model and on its own, on the GPU,
mirroring the reference's tests/test_kv_int8.py:44-94:

* prefill logits are identical to a bf16 DynamicCache (the layer returns the full-precision inputs at prefill), and
  greedy-decode logits stay within 0.05 of it, with RDAttention taking the fused int8 decode (Int8Handle.attend ->
  bb_decode) and with a stock HF attention module taking the dequantised tensors;
* kv_evict composes: the layer holds the evicted length, and decode stays within 0.05;
* token-by-token appends across several GROW reallocations equal a one-shot quantisation, bitwise (and equal the CPU
  oracle's quantise / dequantise); crop drops rows and appends continue after them;
* BASELINE configs[4] through the layer: 131072 cached tokens, fp32 scales, 256 one-token updates + exact_attention,
  sampled steps against the float64 oracle over the same int8 rows (max-abs 2e-2, mean-abs 2e-3).
"""
from types import SimpleNamespace

import pytest
import torch

import oracle
from bigger_bird_amd import RDAttention, install
from bigger_bird_amd import kv_int8
from bigger_bird_amd.kv_int8 import GROW, Int8KVLayer, dequantize, make_int8_cache, quantize

pytestmark = pytest.mark.gpu

KW = dict(sink=8, window=96, vertical=24, n_route=16, exact_tail=24, block_m=16, block_n=16)
N = 400


def _tiny(dev, dtype=torch.bfloat16):
    from transformers import LlamaConfig, LlamaForCausalLM

    # 8 query / 2 KV heads, head_dim 64 (the decode kernels take 64 or 128)
    cfg = LlamaConfig(vocab_size=512, hidden_size=512, intermediate_size=1024, num_hidden_layers=2,
                      num_attention_heads=8, num_key_value_heads=2, max_position_embeddings=8192,
                      attn_implementation="sdpa")
    torch.manual_seed(0)
    return LlamaForCausalLM(cfg).to(dev, dtype).eval()


def _prompt(dev):
    g = torch.Generator().manual_seed(4)
    return torch.randint(0, 512, (1, N), generator=g).to(dev)


def _gen(model, ids, cache):
    with torch.inference_mode():
        return model.generate(ids, max_new_tokens=6, min_new_tokens=6, do_sample=False, pad_token_id=0,
                              past_key_values=cache, output_scores=True, return_dict_in_generate=True)


def _max_diff(a, b):
    ok = torch.isfinite(a) & torch.isfinite(b)  # min_new_tokens puts -inf on EOS in both
    assert torch.equal(torch.isfinite(a), torch.isfinite(b))
    return (a.float() - b.float())[ok].abs().max().item()


class _CountAttend:
    """Counts Int8Handle.attend calls (the fused int8 decode) while active."""

    def __init__(self, monkeypatch):
        self.calls = 0
        real = kv_int8.Int8Handle.attend

        def attend(handle, q, scale):
            self.calls += 1
            return real(handle, q, scale)

        monkeypatch.setattr(kv_int8.Int8Handle, "attend", attend)


@pytest.mark.parametrize("installed", [True, False])
def test_prefill_unchanged_and_decode_close(installed, dev, monkeypatch):
    print(f"case int8_layer_generate installed={installed}", flush=True)
    from transformers import DynamicCache

    model = _tiny(dev)
    if installed:
        install(model, "rd", **KW)
    ids = _prompt(dev)
    want = _gen(model, ids, DynamicCache(config=model.config))
    counter = _CountAttend(monkeypatch)
    cache = make_int8_cache(model.config)
    got = _gen(model, ids, cache)
    assert torch.equal(got.scores[0], want.scores[0]), "prefill logits must be identical"
    diffs = [_max_diff(a, b) for a, b in zip(got.scores, want.scores)]
    print("max |logit diff| per step, int8 vs bf16 cache:", [round(d, 5) for d in diffs], flush=True)
    assert max(diffs) < 0.05
    assert all(isinstance(x, Int8KVLayer) and x.get_seq_length() == N + 5 for x in cache.layers)
    # RDAttention opts in to the fused decode (5 decode steps x 2 layers); a stock HF module never gets handles
    assert counter.calls == (10 if installed else 0)


@pytest.mark.parametrize("installed", [True, False])
def test_fp16_model(installed, dev, monkeypatch):
    """An fp16 model with the int8 cache (the reference's layer quantises any float dtype and dequantises to it): the
    fp16 rows quantise and dequantise on the HIP kernels, prefill logits are identical to an fp16 DynamicCache and
    greedy decode stays within 0.05 of it. The fused int8 decode takes bf16 queries, so an fp16 model's decode
    attends the dequantised fp16 cache (RDAttention's exact path, or the stock HF module)."""
    print(f"case int8_layer_fp16 installed={installed}", flush=True)
    from transformers import DynamicCache

    model = _tiny(dev, torch.float16)
    if installed:
        install(model, "rd", **KW)
    ids = _prompt(dev)
    want = _gen(model, ids, DynamicCache(config=model.config))
    counter = _CountAttend(monkeypatch)
    cache = make_int8_cache(model.config)
    got = _gen(model, ids, cache)
    assert torch.equal(got.scores[0], want.scores[0]), "prefill logits must be identical"
    diffs = [_max_diff(a, b) for a, b in zip(got.scores, want.scores)]
    print("max |logit diff| per step, int8 vs fp16 cache:", [round(d, 5) for d in diffs], flush=True)
    assert max(diffs) < 0.05
    assert counter.calls == 0
    layer = cache.layers[0]
    assert layer.keys.dtype == torch.float16 and layer.get_seq_length() == N + 5


def test_fused_off_gives_tensors_to_rd_attention(dev, monkeypatch):
    print("case int8_layer_fused_off", flush=True)
    model = _tiny(dev)
    install(model, "rd", **KW)
    ids = _prompt(dev)
    counter = _CountAttend(monkeypatch)
    fused = _gen(model, ids, make_int8_cache(model.config))
    calls = counter.calls
    plain = _gen(model, ids, make_int8_cache(model.config, fused=False))
    assert calls == 10 and counter.calls == calls
    assert torch.equal(plain.scores[0], fused.scores[0])
    assert max(_max_diff(a, b) for a, b in zip(plain.scores, fused.scores)) < 0.05


def test_composes_with_kv_evict(dev):
    print("case int8_layer_kv_evict", flush=True)
    from transformers import DynamicCache

    model = _tiny(dev)
    install(model, "rd", kv_evict=True, **KW)
    ids = _prompt(dev)
    want = _gen(model, ids, DynamicCache(config=model.config))
    cache = make_int8_cache(model.config)
    got = _gen(model, ids, cache)
    cfg = model.config
    g = cfg.num_attention_heads // cfg.num_key_value_heads
    m = KW["sink"] + KW["window"] + g * KW["vertical"]
    assert all(x.get_seq_length() == m + 5 for x in cache.layers), "int8 layer must hold the evicted length"
    diffs = [_max_diff(a, b) for a, b in zip(got.scores, want.scores)]
    print("evict+int8 vs evict-only, max |logit diff| per step:", [round(d, 5) for d in diffs], flush=True)
    assert torch.equal(got.scores[0], want.scores[0]) and max(diffs) < 0.05
    head_dim = cfg.hidden_size // cfg.num_attention_heads
    assert cache.layers[0].nbytes() == 2 * (m + 5) * cfg.num_key_value_heads * (head_dim + 2)


def test_appends_across_growth_and_crop(dev):
    print("case int8_layer_appends_crop", flush=True)
    g = torch.Generator().manual_seed(1)
    k = torch.randn(1, 2, 700, 64, generator=g).to(dev)
    v = torch.randn(1, 2, 700, 64, generator=g).to(dev)
    layer = Int8KVLayer()
    pk, pv = layer.update(k[..., :100, :], v[..., :100, :])
    assert torch.equal(pk, k[..., :100, :]) and torch.equal(pv, v[..., :100, :]), "prefill returns full precision"
    buffers = {layer.store_k.q.data_ptr()}
    for i in range(100, 700):
        got_k, got_v = layer.update(k[..., i:i + 1, :], v[..., i:i + 1, :])
        buffers.add(layer.store_k.q.data_ptr())
    assert len(buffers) >= 1 + (700 - 100 - GROW) // GROW, "appends must have crossed several reallocations"
    want_k, want_v = (dequantize(*quantize(x), torch.float32) for x in (k, v))
    assert layer.get_seq_length() == 700 and got_k.shape == (1, 2, 700, 64)
    assert torch.equal(got_k, want_k) and torch.equal(got_v, want_v)
    # and the one-shot quantisation itself equals the CPU oracle
    q8, s16, _ = oracle.quantize(k[0].transpose(0, 1).contiguous().cpu())
    assert torch.equal(want_k[0].transpose(0, 1).cpu(), oracle.dequantize(q8, s16).float())
    assert layer.nbytes() == 2 * (700 * 2 * 64 + 700 * 2 * 2)
    layer.crop(-50)
    assert layer.get_seq_length() == 650 and torch.equal(layer.keys, want_k[..., :650, :])
    layer.update(k[..., :1, :], v[..., :1, :])
    assert torch.equal(layer.keys[..., 650:, :], want_k[..., :1, :])
    assert torch.equal(layer.values[..., :650, :], want_v[..., :650, :])
    with pytest.raises(NotImplementedError):
        layer.crop(3)


def test_deferred_row_is_quantised_on_every_path(dev):
    """A one-token bf16 step handed out as Int8Handle keeps its row unquantised until the handle is attended (the
    decode kernel quantises it, bb_decode_append). Reading the cache, a further update, crop or nbytes before that
    quantises it first, so every path sees the same int8 rows as a one-shot quantisation."""
    print("case int8_layer_deferred_rows", flush=True)
    g = torch.Generator().manual_seed(8)
    H, Hkv, d = 32, 8, 128
    k = torch.randn(1, Hkv, 303, d, generator=g).to(torch.bfloat16).to(dev)
    v = torch.randn(1, Hkv, 303, d, generator=g).to(torch.bfloat16).to(dev)
    q = torch.randn(1, H, 1, d, generator=g).to(torch.bfloat16).to(dev)
    want_k, want_v = (dequantize(*quantize(x[0].transpose(0, 1)), torch.bfloat16).transpose(0, 1)[None]
                      for x in (k, v))
    layer = Int8KVLayer()
    layer.update(k[..., :300, :], v[..., :300, :])
    hk, _ = layer.update(k[..., 300:301, :], v[..., 300:301, :], {"bb_attend": True})
    assert isinstance(hk, kv_int8.Int8Handle) and layer._pending is not None
    assert torch.equal(layer.keys, want_k[..., :301, :]) and layer._pending is None  # read -> quantised first
    layer.update(k[..., 301:302, :], v[..., 301:302, :], {"bb_attend": True})
    layer.update(k[..., 302:303, :], v[..., 302:303, :], {"bb_attend": True})  # update -> previous row first
    out = hk.attend(q, d ** -0.5)  # a stale handle attends the whole current cache
    assert layer._pending is None
    assert torch.equal(layer.values, want_v) and torch.equal(layer.keys, want_k)
    st_k, st_v = layer.store_k, layer.store_v
    ref = oracle.decode(q[0, :, 0], st_k.q, st_k.s, st_v.q, st_v.s, 303, d ** -0.5)
    assert (out[0, :, 0].double().cpu() - ref).abs().max().item() < 2e-2


def test_config5_decode_through_the_layer(dev):
    """131072 cached tokens, 32 q / 8 KV heads, d 128, fp32 per-token scales, 256 decode steps:
    each step's K/V row goes in through Int8KVLayer.update and attention runs through RDAttention.exact_attention ->
    Int8Handle.attend; steps 0, 127 and 255 are checked against the float64 oracle over the layer's own int8 rows."""
    n0, H, Hkv, d, steps = 131072, 32, 8, 128, 256
    print(f"case int8_layer_config5 n={n0} steps={steps}", flush=True)
    base = SimpleNamespace(config=SimpleNamespace(num_attention_heads=H, num_key_value_heads=Hkv), layer_idx=0,
                           head_dim=d, scaling=d ** -0.5, q_proj=None, k_proj=None, v_proj=None, o_proj=None)
    attn = RDAttention(base, sink=64, window=16384, vertical=512, exact_tail=256)
    g = torch.Generator(device=dev).manual_seed(5)
    layer = Int8KVLayer()
    layer.scale_dtype = torch.float32
    k = torch.randn(1, Hkv, n0, d, device=dev, generator=g).to(torch.bfloat16)
    v = torch.randn(1, Hkv, n0, d, device=dev, generator=g).to(torch.bfloat16)
    layer.update(k, v)
    del k, v
    checked = 0
    for s in range(steps):
        kn = torch.randn(1, Hkv, 1, d, device=dev, generator=g).to(torch.bfloat16)
        vn = torch.randn(1, Hkv, 1, d, device=dev, generator=g).to(torch.bfloat16)
        q = torch.randn(1, H, 1, d, device=dev, generator=g).to(torch.bfloat16)
        hk, hv = layer.update(kn, vn, {"bb_attend": True})
        n = layer.get_seq_length()
        assert n == n0 + s + 1 and hk.shape == (1, Hkv, n, d)
        out = attn.exact_attention(q, hk, hv, 1, n)
        if s in (0, 127, steps - 1):
            torch.cuda.synchronize()
            st_k, st_v = layer.store_k, layer.store_v
            assert st_k.s.dtype == torch.float32
            ref = oracle.decode(q[0, :, 0], st_k.q, st_k.s, st_v.q, st_v.s, n, d ** -0.5)
            err = (out[0, :, 0].double().cpu() - ref).abs()
            print(f"step {s}: n={n} max_abs={err.max().item():.3e} mean_abs={err.mean().item():.3e}", flush=True)
            assert err.max().item() < 2e-2 and err.mean().item() < 2e-3
            # the new row is the quantised input row (bitwise, as the oracle quantises it)
            q8, _, s32 = oracle.quantize(kn[0].transpose(0, 1).contiguous().cpu())
            assert torch.equal(st_k.q[n - 1:n].cpu(), q8) and torch.equal(st_k.s[n - 1:n].cpu(), s32)
            checked += 1
    assert checked == 3
