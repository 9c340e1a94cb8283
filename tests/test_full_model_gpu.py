"""BASELINE configs[2] at its real size: a random-init Llama-3-8B-architecture model in bf16 (32 layers, hidden 4096,
32 q / 8 KV heads, d 128, FFN 14336, vocab 128256, RoPE theta 5e5) with RDAttention installed on every layer
(modal_rd/attention.py:262-270) and the final cfg {sink 64, window 16384, vertical 512, exact_tail 256}, prefilled
at T = 131072 uniform-random token ids with the KV cache on and last-token logits, as the reference's long-context
prefill runs it (modal_rd/eval_niah.py:65-120, modal_rd/RESULTS.md:43).

For layers 0 and 31 the post-RoPE q/k/v the layer's sparse_prefill received, its routes and its output are captured:
* routes: [32, 512] int32, strictly ascending per head, inside [sink, n - window);
* output rows of 4 heads (one per KV group 0, 2, 5, 7) against the float64 union-mask oracle on the same inputs:
  row-tile and window edges, the first row each of a few routed keys becomes visible to, random main rows, and all
  256 exact-tail rows; max-abs 2e-2, mean-abs 2e-3.
The logits must be finite. (Random-init weights give nearly uniform attention, so the model-level output is a
smoke check; the masks themselves are pinned at the kernel level by the other prefill tests.)
"""
import pytest
import torch

import oracle
from bigger_bird_amd import install

pytestmark = pytest.mark.gpu

T = 131072
CFG = dict(sink=64, window=16384, vertical=512, exact_tail=256)
HEADS = torch.tensor([0, 9, 22, 31])
LAYERS = (0, 31)


def _model(dev):
    from transformers import LlamaConfig, LlamaForCausalLM

    cfg = LlamaConfig(vocab_size=128256, hidden_size=4096, intermediate_size=14336, num_hidden_layers=32,
                      num_attention_heads=32, num_key_value_heads=8, max_position_embeddings=T, rope_theta=500000.0,
                      rms_norm_eps=1e-5, attn_implementation="sdpa")
    torch.manual_seed(0)
    old = torch.get_default_dtype()
    try:
        torch.set_default_dtype(torch.bfloat16)
        with torch.device(dev):
            model = LlamaForCausalLM(cfg)
    finally:
        torch.set_default_dtype(old)
    return model.eval()


def test_llama3_8b_prefill_128k(dev):
    print(f"case full_model llama3-8b random-init T={T} cfg={CFG}", flush=True)
    model = _model(dev)
    install(model, "rd", **CFG)
    captured = {}
    for li in LAYERS:
        attn = model.model.layers[li].self_attn
        real = attn.sparse_prefill

        def spy(q, k, v, _real=real, _li=li, _attn=attn):
            out = _real(q, k, v)
            captured[_li] = dict(q=q[0].cpu(), k=k[0].cpu(), v=v[0].cpu(), routes=_attn.last_routes.cpu(),
                                 out=out[0, HEADS.to(out.device)].cpu())
            return out

        attn.sparse_prefill = spy
    g = torch.Generator(device=dev).manual_seed(7)
    ids = torch.randint(0, model.config.vocab_size, (1, T), generator=g, device=dev)
    with torch.inference_mode():
        logits = model(input_ids=ids, use_cache=True, logits_to_keep=1).logits[0, -1].float()
    torch.cuda.synchronize()
    print("prefill done", flush=True)
    assert torch.isfinite(logits).all()
    assert set(captured) == set(LAYERS)
    W, S, r = CFG["window"], CFG["sink"], CFG["exact_tail"]
    gen = torch.Generator().manual_seed(3)
    for li in LAYERS:
        c = captured[li]
        routes = c["routes"]
        assert routes.shape == (32, 512) and routes.dtype == torch.int32
        assert (routes[:, 1:] > routes[:, :-1]).all(), "routes must be strictly ascending"
        assert routes.min().item() >= S and routes.max().item() < T - W
        fixed = [0, 1, 63, 64, 65, S, W - 1, W, W + 1, W + 63, W + 64, T // 2, T - r - 65, T - r - 64, T - r - 1]
        rows_main = []
        for hi, h in enumerate(HEADS.tolist()):
            first_seen = (routes[h, ::97].long() + W).tolist()  # the first row each sampled routed key reaches
            rand = torch.randint(0, T - r, (24,), generator=gen).tolist()
            rows_main += [(hi, h, x) for x in fixed + first_seen + rand if x < T - r]
        rows_tail = [(hi, h, x) for hi, h in enumerate(HEADS.tolist()) for x in range(T - r, T)]
        G = 4
        main_pairs = torch.tensor([[h, x] for _, h, x in rows_main])
        ref_main = oracle.attn_rows(c["q"], c["k"], c["v"], routes[:, None], main_pairs, front=S, window=W,
                                    num_heads=32, kv_groups=G, scale=128 ** -0.5)
        none = torch.full((32, 1, 1), -1, dtype=torch.int32)
        tail_pairs = torch.tensor([[h, x] for _, h, x in rows_tail])
        ref_tail = oracle.attn_rows(c["q"], c["k"], c["v"], none, tail_pairs, front=0, window=T, num_heads=32,
                                    kv_groups=G, scale=128 ** -0.5)
        for what, rows, ref in (("main", rows_main, ref_main), ("tail", rows_tail, ref_tail)):
            got = torch.stack([c["out"][hi, x] for hi, _, x in rows]).double()
            err = (got - ref).abs()
            print(f"layer {li} {what}: rows={len(rows)} max_abs={err.max().item():.3e} "
                  f"mean_abs={err.mean().item():.3e}", flush=True)
            assert err.max().item() < 2e-2 and err.mean().item() < 2e-3
