"""Argument checks of the decode-side Python surface that run before any GPU work (no GPU needed): the HIP-only
operators refuse CPU tensors loudly (no CPU fallback), and the graph decoder validates its configuration."""
import pytest
import torch

from bigger_bird_amd.decode import argmax_index, bigger_bird_decode, bigger_bird_route, decode_step, gather_rows, \
    rms_norm, topk_columns
from bigger_bird_amd.kv_int8 import quantize_pair


def test_decode_ops_refuse_cpu_tensors():
    q = torch.zeros(32, 128, dtype=torch.bfloat16)
    k = torch.zeros(8, 300, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="requires CUDA"):
        bigger_bird_decode(q, k, k, torch.zeros(8, 4, dtype=torch.long), front=8, window=8)
    with pytest.raises(ValueError, match="requires CUDA"):
        bigger_bird_route(q, k, 16, front=8, window=8)
    with pytest.raises(ValueError, match="requires CUDA"):
        decode_step(q, k, k, k[:, 0], k[:, 0], torch.tensor([10]), routed=16, front=8, window=8)
    with pytest.raises(ValueError, match="GPU"):
        gather_rows(k, torch.zeros(8, 4, dtype=torch.long))
    with pytest.raises(ValueError, match="GPU"):
        topk_columns(torch.rand(2, 100), 10)
    with pytest.raises(ValueError, match="1-D"):
        argmax_index(torch.rand(10))
    with pytest.raises(ValueError, match="GPU"):
        rms_norm(torch.zeros(4, 64, dtype=torch.bfloat16), torch.ones(64, dtype=torch.bfloat16), 1e-5)
    with pytest.raises((ValueError, RuntimeError)):
        quantize_pair(k, k, None, None)


def test_route_rejects_nonpositive_budget():
    q = torch.zeros(32, 128, dtype=torch.bfloat16)
    k = torch.zeros(8, 300, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        bigger_bird_route(q, k, 0, front=8, window=8)


def test_static_decoder_validates_sparse_config():
    from transformers import LlamaConfig, LlamaForCausalLM

    from bigger_bird_amd.graph_decode import StaticDecoder

    cfg = LlamaConfig(vocab_size=64, hidden_size=64, intermediate_size=128, num_hidden_layers=1,
                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=256)
    model = LlamaForCausalLM(cfg).to(torch.bfloat16).eval()
    dec = StaticDecoder(model, 32)  # buffers on the model's device; nothing runs yet
    assert dec.k[0].shape == (2, 32, 16) and dec.sparse == [False]
    with pytest.raises(ValueError, match="front, window and routed"):
        StaticDecoder(model, 32, sparse_decode={"front": 8, "window": 16})


def test_forward_pool_keeps_span_continuation():
    """tests/test_kv_evict.py:134-142 of the reference: with p = 4 the 3 keys after a high-scoring key inherit its
    score; other keys keep theirs."""
    from bigger_bird_amd import forward_pool

    score = torch.zeros(2, 20)
    score[0, 5] = 1.0
    score[1, 18] = 0.5
    pooled = forward_pool(score, 4)
    assert pooled.shape == score.shape
    assert pooled[0, 5:9].eq(1).all() and pooled[0, :5].eq(0).all() and pooled[0, 9:].eq(0).all()
    assert pooled[1, 18:].eq(0.5).all() and pooled[1, :18].eq(0).all()


def test_forward_pool_back_keeps_span_lead_in():
    """tests/test_kv_evict.py:145-151 of the reference: `back` = b also gives the b keys before a high-scoring key its
    score, and p = 0 counts as 1 (the key itself)."""
    from bigger_bird_amd import forward_pool

    score = torch.zeros(1, 20)
    score[0, 10] = 1.0
    pooled = forward_pool(score, 3, back=4)
    assert pooled[0, 6:13].eq(1).all() and pooled[0, :6].eq(0).all() and pooled[0, 13:].eq(0).all()
    assert forward_pool(score, 0, back=2)[0, 8:11].eq(1).all()
    assert forward_pool(score, 0, back=2)[0, :8].eq(0).all() and forward_pool(score, 0, back=2)[0, 11:].eq(0).all()


def test_forward_pool_matches_brute_force():
    """Closed form on random rows: out[h, j] = max(score[h, max(0, j - p + 1) : j + back + 1])."""
    from bigger_bird_amd import forward_pool

    g = torch.Generator().manual_seed(1)
    score = torch.rand(3, 57, generator=g)
    for p, back in ((1, 0), (2, 0), (5, 3), (9, 1), (1, 6)):
        got = forward_pool(score, p, back)
        for j in range(57):
            want = score[:, max(0, j - p + 1):j + back + 1].amax(-1)
            assert torch.equal(got[:, j], want), (p, back, j)


def test_fused_qkv_weights_share_storage():
    """The graph decoder's fused QKV matrix holds the q / k / v weights as row blocks of one buffer: the parameters
    become views of it (same values, no second copy), and a second fusion reuses that buffer."""
    from bigger_bird_amd.graph_decode import _fuse_rows

    lin = [torch.nn.Linear(16, n, bias=False) for n in (8, 4, 4)]
    before = [m.weight.detach().clone() for m in lin]
    fused = _fuse_rows([m.weight for m in lin])
    assert fused.shape == (16, 16)
    for m, w in zip(lin, before):
        assert isinstance(m.weight, torch.nn.Parameter) and torch.equal(m.weight, w)
        assert m.weight.untyped_storage().data_ptr() == fused.untyped_storage().data_ptr()
    again = _fuse_rows([m.weight for m in lin])
    assert again.data_ptr() == fused.data_ptr() and torch.equal(again, fused)
    x = torch.randn(3, 16)
    assert torch.equal(torch.cat([m(x) for m in lin], -1), x @ fused.T)
