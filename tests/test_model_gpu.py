"""RDAttention installed in a (small, random-init) Hugging Face Llama model on the GPU, as the reference's experiments
use it (modal_rd/attention.py:262-270 install, the decoder layer calling self_attn with position embeddings and the
KV cache): every layer's attention output, captured at o_proj's input, against float32 attention recomputed from the
same layer input with the same projections, the HF rotary embedding and the mask the arm defines:
  * "dense_rd": causal attention over all keys;
  * "rd": sink | window | the layer's chosen routes (before the window) for rows below n - exact_tail, causal for the
    exact tail (modal_rd/attention.py:176-206);
  * one decode step after the prefill: attention of the new token over every cached key.
The model runs in bf16 and in fp16 (routes, RoPE, the flash kernels and decode on fp16 inputs). Bar: max-abs 2e-2
and mean-abs 2e-3 per layer. Logits are not compared across precisions: with the enlarged q/k
projections below the bf16 and float32 models diverge by themselves (last-token cosine 0.17 for HF's own bf16 model),
so the per-layer comparison from a common bf16 input is the meaningful one.
"""
import pytest
import torch

from bigger_bird_amd import install

pytestmark = pytest.mark.gpu

T = 2048
SPARSE = dict(sink=64, window=512, vertical=128, exact_tail=64)


def _model(dev, dtype=torch.bfloat16):
    from transformers import LlamaConfig, LlamaForCausalLM

    cfg = LlamaConfig(vocab_size=512, hidden_size=1024, intermediate_size=1024, num_hidden_layers=2,
                      num_attention_heads=8, num_key_value_heads=2, max_position_embeddings=4096,
                      rope_theta=500000.0, rms_norm_eps=1e-5, attn_implementation="sdpa")
    torch.manual_seed(0)
    m32 = LlamaForCausalLM(cfg).eval()
    # larger q/k projections than the 0.02 init so that the softmax is far from uniform and routes matter
    with torch.no_grad():
        for layer in m32.model.layers:
            layer.self_attn.q_proj.weight.mul_(4.0)
            layer.self_attn.k_proj.weight.mul_(4.0)
    return m32.to(dev, dtype)


class _Capture:
    """Per layer: the attention input (hidden states, rotary cos/sin) and the attention output at o_proj's input."""

    def __init__(self, model):
        self.calls, self.handles = [], []
        for i, layer in enumerate(model.model.layers):
            attn = layer.self_attn
            self.handles.append(attn.register_forward_pre_hook(self._pre(i, attn), with_kwargs=True))
            self.handles.append(attn.o_proj.register_forward_pre_hook(self._out(i)))

    def _pre(self, i, attn):
        def hook(_mod, args, kwargs):
            hs = kwargs.get("hidden_states", args[0] if args else None)
            self.calls.append({"layer": i, "attn": attn, "h": hs.detach().clone(),
                               "pe": tuple(x.detach().clone() for x in kwargs["position_embeddings"]),
                               "cache": kwargs.get("past_key_values")})
        return hook

    def _out(self, i):
        def hook(_mod, args):
            assert self.calls[-1]["layer"] == i
            self.calls[-1]["out"] = args[0].detach().float().clone()
        return hook

    def close(self):
        for h in self.handles:
            h.remove()


def _heads(attn):
    cfg = attn.config if hasattr(attn, "config") else None
    H = getattr(attn, "num_heads", None) or cfg.num_attention_heads
    Hkv = getattr(attn, "num_kv_heads", None) or cfg.num_key_value_heads
    return H, Hkv


def _reference(call, mask_fn):
    """float32 attention of one captured layer call; mask_fn(attn, t, n) -> bool [H, t, n] or None (all keys)."""
    from transformers.models.llama.modeling_llama import apply_rotary_pos_emb

    attn, h = call["attn"], call["h"]
    b, t, _ = h.shape
    (H, Hkv), d = _heads(attn), attn.head_dim
    q = attn.q_proj(h).view(b, t, H, d).transpose(1, 2)
    k = attn.k_proj(h).view(b, t, Hkv, d).transpose(1, 2)
    v = attn.v_proj(h).view(b, t, Hkv, d).transpose(1, 2)
    q, k = apply_rotary_pos_emb(q, k, *call["pe"])
    if t == 1:  # decode: the cache (after this call's update) holds every key, the new one last
        layer = call["cache"].layers[call["layer"]]
        k, v = layer.keys, layer.values
    n = k.shape[-2]
    g = H // Hkv
    kf = k[0].float().repeat_interleave(g, 0)
    vf = v[0].float().repeat_interleave(g, 0)
    s = torch.matmul(q[0].float(), kf.transpose(-1, -2).contiguous()) * attn.scaling  # [H, t, n]
    mask = mask_fn(attn, t, n)
    if mask is not None:
        s = s.masked_fill(~mask, -float("inf"))
    o = torch.matmul(s.softmax(-1), vf)  # [H, t, d]
    return o.transpose(0, 1).reshape(1, t, H * d)


def _causal(attn, t, n):
    if t == 1:
        return None
    i = torch.arange(t, device=attn.o_proj.weight.device)[:, None] + (n - t)
    j = torch.arange(n, device=i.device)[None, :]
    return (j <= i)[None].expand(_heads(attn)[0], t, n)


def _sparse(attn, t, n):
    if t == 1:
        return None
    dev = attn.o_proj.weight.device
    i = torch.arange(t, device=dev)[:, None]
    j = torch.arange(n, device=dev)[None, :]
    causal = j <= i
    local = causal & ((j < attn.sink) | (i - j < attn.window))
    routes = attn.last_routes.long()  # [H, budget], -1 = unused slot
    member = torch.zeros(attn.num_heads, n + 1, dtype=torch.bool, device=dev)
    member.scatter_(1, torch.where(routes >= 0, routes, n), True)
    mask = local[None] | (causal & (i - j >= attn.window))[None] & member[:, None, :n]
    tail = i[:, 0] >= n - attn.exact_tail
    mask[:, tail] = causal[tail][None]
    return mask


def _check(calls, mask_fn, what):
    assert calls, what
    for c in calls:
        ref = _reference(c, mask_fn)
        err = (c["out"] - ref).abs()
        print(f"{what} layer {c['layer']} t={c['h'].shape[1]}: max {err.max().item():.3e} mean {err.mean().item():.3e}",
              flush=True)
        assert err.max().item() <= 2e-2 and err.mean().item() <= 2e-3, (what, c["layer"])


@pytest.mark.parametrize("arm,dtype", [("dense_rd", torch.bfloat16), ("rd", torch.bfloat16), ("dense_rd", torch.float16),
                                       ("rd", torch.float16)])
def test_installed_model_layers_match_reference(arm, dtype, dev):
    print(f"case model {arm} {dtype} T={T}", flush=True)
    mbf = _model(dev, dtype)
    g = torch.Generator(device=dev).manual_seed(1)
    ids = torch.randint(0, 512, (1, T + 1), generator=g, device=dev)
    install(mbf, arm, **SPARSE)
    cap = _Capture(mbf)
    try:
        with torch.inference_mode():
            out = mbf(input_ids=ids[:, :T], use_cache=True, logits_to_keep=1)
            prefill = list(cap.calls)
            cap.calls.clear()
            mbf(input_ids=ids[:, T:], past_key_values=out.past_key_values, use_cache=True, logits_to_keep=1)
            decode = list(cap.calls)
            _check(prefill, _causal if arm == "dense_rd" else _sparse, f"{arm} prefill")
            _check(decode, _causal, f"{arm} decode")
            for layer in out.past_key_values.layers:  # every layer's cache grew by the decode token
                assert layer.keys.shape[-2] == T + 1 and layer.values.shape[-2] == T + 1
            if arm == "rd":
                for c in prefill:
                    r = c["attn"].last_routes
                    assert r.shape[0] == 8 and r.shape[1] > 0 and bool((r[:, 1:] > r[:, :-1]).all())
    finally:
        cap.close()


def test_autograd_mode_as_the_reference(dev):
    """forward with autograd on (modal_rd/attention.py:118-119, 140-141): exact layers run RoPE out of place and
    torch's differentiable SDPA, so an installed dense_rd model backpropagates like the unmodified HF model (same
    loss, same weight gradients within float32 rounding); sparse layers run the HIP prefill forward-only, so their
    logits equal the inference-mode logits bit for bit and no gradient reaches q / k / v through them."""
    import copy

    print("case model autograd", flush=True)
    from transformers import LlamaConfig, LlamaForCausalLM

    cfg = LlamaConfig(vocab_size=256, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=4096,
                      rope_theta=500000.0, attn_implementation="sdpa")
    torch.manual_seed(3)
    ref = LlamaForCausalLM(cfg).to(dev).train(False)
    mine = copy.deepcopy(ref)
    install(mine, "dense_rd", **SPARSE)
    ids = torch.randint(0, 256, (1, 300), device=dev)
    losses, grads = [], []
    for m in (ref, mine):
        m.zero_grad()
        loss = m(input_ids=ids, use_cache=False).logits.float().square().mean()
        loss.backward()
        losses.append(loss.item())
        grads.append({n: p.grad.clone() for n, p in m.named_parameters() if p.grad is not None})
    assert abs(losses[0] - losses[1]) <= 1e-5 * abs(losses[0])
    assert set(grads[0]) == set(grads[1])
    for name, g0 in grads[0].items():
        torch.testing.assert_close(grads[1][name], g0, rtol=1e-3, atol=1e-6, msg=name)

    # sparse layers (bf16, T > sink + window): forward-only through the HIP path
    mbf = _model(dev)
    install(mbf, "rd", **SPARSE)
    g = torch.Generator(device=dev).manual_seed(2)
    ids = torch.randint(0, 512, (1, T), generator=g, device=dev)
    with torch.inference_mode():
        want = mbf(input_ids=ids, use_cache=False).logits
    mbf.zero_grad()
    out = mbf(input_ids=ids, use_cache=False).logits
    assert torch.equal(out.detach(), want)
    out.float().square().mean().backward()
    for layer in mbf.model.layers:
        a = layer.self_attn
        assert a.o_proj.weight.grad is not None and a.o_proj.weight.grad.abs().sum() > 0
        assert a.q_proj.weight.grad is None or not a.q_proj.weight.grad.any()
