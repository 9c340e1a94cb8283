"""Pins the INT8 / decode / RoPE parts of the oracle and of the host-side input generator.

  * int8 quantise: bitwise against torch ops restating modal_rd/kv_int8.py:19-22, plus the error bounds of
    tests/test_kv_int8.py:24-33 (err <= 0.6 * scale, rel-RMS < 1%) and the storage ratio (35-41);
  * decode: float64 exact attention over the dequantised cache against torch's float64 SDPA;
  * RoPE: synth.rope_cos_sin / rope_host bit-identical to transformers' LlamaRotaryEmbedding and
    apply_rotary_pos_emb (the functions the reference's rope_inplace wraps, modal_rd/attention.py:51-60).
"""
import pytest
import torch

import oracle
from bigger_bird_amd.synth import rope_cos_sin, rope_host


def _torch_quantize(x):
    scale = (x.float().abs().amax(-1, keepdim=True) / 127).clamp_min(1e-4)
    q = (x.float() / scale).round().clamp(-127, 127).to(torch.int8)
    return q, scale.to(torch.float16), scale


def test_quantize_bitwise_matches_torch_formula():
    g = torch.Generator().manual_seed(0)
    x = (torch.randn(300, 8, 128, generator=g) * torch.rand(300, 8, 1, generator=g) * 3).to(torch.bfloat16)
    x[5, 3] = 0  # all-zero row -> min scale
    x[7, 1, :4] = torch.tensor([1e-6, -1e-6, 0.0, 2e-6])
    q, s16, s32 = oracle.quantize(x)
    tq, t16, t32 = _torch_quantize(x)
    assert torch.equal(q, tq)
    assert torch.equal(s16.view(torch.int16), t16.view(torch.int16))
    assert torch.equal(s32, t32)
    xf = torch.randn(64, 128, generator=g) * 50
    q, s16, _ = oracle.quantize(xf)
    tq, t16, _ = _torch_quantize(xf)
    assert torch.equal(q, tq) and torch.equal(s16.view(torch.int16), t16.view(torch.int16))
    # fp16 input (an fp16 model's cache): values down to fp16 subnormals and up to its largest finite magnitudes
    xh = (torch.randn(200, 8, 128, generator=g) * torch.rand(200, 8, 1, generator=g) * 3).to(torch.float16)
    xh[0, 0, :3] = torch.tensor([6e-8, -3e-5, 65504.0], dtype=torch.float16)
    xh[1, 2] = 0
    q, s16, s32 = oracle.quantize(xh)
    tq, t16, t32 = _torch_quantize(xh)
    assert torch.equal(q, tq) and torch.equal(s16.view(torch.int16), t16.view(torch.int16)) and torch.equal(s32, t32)


def test_quantize_error_bounds_and_storage():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(1000, 8, 128, generator=g).to(torch.bfloat16)
    q, s16, _ = oracle.quantize(x)
    deq = oracle.dequantize(q, s16)
    err = (deq - x.float()).abs()
    assert (err <= 0.6 * s16.float()).all()
    rel_rms = ((deq - x.float()).pow(2).mean().sqrt() / x.float().pow(2).mean().sqrt()).item()
    assert rel_rms < 0.01
    stored = q.numel() * q.element_size() + s16.numel() * s16.element_size()
    assert abs(stored / (x.numel() * 2) - (1 + 2 / 128) / 2) < 1e-12


def test_dequantize_is_int_times_scale():
    q = torch.tensor([[-127, -1, 0, 1, 127, 64, -64, 3]], dtype=torch.int8)
    s = torch.tensor([[0.5]], dtype=torch.float16)
    assert torch.equal(oracle.dequantize(q, s), q.float() * 0.5)


def test_decode_matches_sdpa_over_dequantised_cache():
    g = torch.Generator().manual_seed(2)
    n, H, Hkv, d = 777, 8, 2, 64
    k = torch.randn(n, Hkv, d, generator=g).to(torch.bfloat16)
    v = torch.randn(n, Hkv, d, generator=g).to(torch.bfloat16)
    q = torch.randn(H, d, generator=g).to(torch.bfloat16)
    for scale_is_f16 in (True, False):
        k8, ks16, ks32 = oracle.quantize(k)
        v8, vs16, vs32 = oracle.quantize(v)
        ks, vs = (ks16, vs16) if scale_is_f16 else (ks32, vs32)
        got = oracle.decode(q, k8, ks, v8, vs, n, d ** -0.5)
        kd = oracle.dequantize(k8, ks).double().permute(1, 0, 2).repeat_interleave(H // Hkv, 0)
        vd = oracle.dequantize(v8, vs).double().permute(1, 0, 2).repeat_interleave(H // Hkv, 0)
        want = torch.nn.functional.scaled_dot_product_attention(q.double()[:, None], kd, vd, scale=d ** -0.5)[:, 0]
        assert (got - want).abs().max().item() < 1e-12


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_rope_matches_transformers_bitwise(dtype):
    from transformers import LlamaConfig
    from transformers.models.llama.modeling_llama import LlamaRotaryEmbedding, apply_rotary_pos_emb

    T, d = 3000, 128
    cfg = LlamaConfig(hidden_size=32 * d, num_attention_heads=32, num_key_value_heads=8, head_dim=d,
                      rope_theta=500000.0, max_position_embeddings=131072)
    rot = LlamaRotaryEmbedding(cfg)
    cos, sin = rot(torch.zeros(1, T, 8, dtype=dtype), torch.arange(T)[None])
    c2, s2 = rope_cos_sin(T, d, dtype=dtype)
    assert torch.equal(cos[0], c2) and torch.equal(sin[0], s2)
    g = torch.Generator().manual_seed(3)
    q = (torch.randn(1, 4, T, d, generator=g) * 3).to(dtype)
    k = (torch.randn(1, 2, T, d, generator=g) * 3).to(dtype)
    hq, hk = apply_rotary_pos_emb(q, k, cos, sin)
    assert torch.equal(rope_host(q, c2, s2), hq) and torch.equal(rope_host(k, c2, s2), hk)
