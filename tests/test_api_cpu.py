"""Argument checks of the decode-side Python surface that run before any GPU work (no GPU needed): the HIP-only
operators refuse CPU tensors loudly (no CPU fallback), and the graph decoder validates its configuration."""
import pytest
import torch

from bigger_bird_amd.decode import argmax_index, bigger_bird_decode, bigger_bird_route, gather_rows, rms_norm, \
    topk_columns
from bigger_bird_amd.kv_int8 import quantize_pair


def test_decode_ops_refuse_cpu_tensors():
    q = torch.zeros(32, 128, dtype=torch.bfloat16)
    k = torch.zeros(8, 300, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="requires CUDA"):
        bigger_bird_decode(q, k, k, torch.zeros(8, 4, dtype=torch.long), front=8, window=8)
    with pytest.raises(ValueError, match="requires CUDA"):
        bigger_bird_route(q, k, 16, front=8, window=8)
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
