"""HIP int8 quantise/dequantise, exact decode (int8 and bf16 caches) and in-place RoPE against the CPU oracle.

Bars: quantise/dequantise/RoPE are integer-exact or single-rounding ops -> bitwise; decode is floating point ->
max-abs 2e-2 / mean-abs 2e-3 against the float64 oracle (the north-star bf16 tolerance).
"""
import pytest
import torch

import oracle
from bigger_bird_amd import decode_bf16, decode_int8, dequantize, quantize, rope_inplace
from bigger_bird_amd.synth import rope_cos_sin, rope_host

pytestmark = pytest.mark.gpu


def _rand(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16)


@pytest.mark.parametrize("scale_dtype", [torch.float16, torch.float32])
def test_quantize_bitwise(scale_dtype, dev):
    print(f"case quantize {scale_dtype}", flush=True)
    x = _rand((1, 8, 777, 128), 1, 2.0)
    x[0, 3, 5] = 0
    q8, s = quantize(x.to(dev)[0].transpose(0, 1), scale_dtype=scale_dtype)  # strided rows -> token-major
    want_q, want16, want32 = oracle.quantize(x[0].transpose(0, 1).contiguous())
    assert torch.equal(q8.cpu(), want_q)
    want_s = want16 if scale_dtype == torch.float16 else want32
    assert torch.equal(s.cpu().view(torch.int16 if scale_dtype == torch.float16 else torch.int32),
                       want_s.view(torch.int16 if scale_dtype == torch.float16 else torch.int32))
    deq = dequantize(q8, s, torch.float32).cpu()
    assert torch.equal(deq, oracle.dequantize(want_q, want_s))


def test_quantize_fp16_input_and_output(dev):
    """An fp16 model's cache: fp16 rows quantised bitwise as the oracle (the reference's formula on x.float()), and
    dequantised to fp16 as torch rounds the fp32 product (modal_rd/kv_int8.py:25-26, `.to(dtype)`)."""
    print("case quantize_fp16", flush=True)
    g = torch.Generator().manual_seed(5)
    x = (torch.randn(1, 8, 513, 128, generator=g) * torch.rand(1, 8, 513, 1, generator=g) * 4).to(torch.float16)
    x[0, 2, 7] = 0
    x[0, 1, 9, :3] = torch.tensor([6e-8, -3e-5, 65504.0], dtype=torch.float16)
    q8, s = quantize(x.to(dev)[0].transpose(0, 1))  # strided rows -> token-major
    want_q, want16, _ = oracle.quantize(x[0].transpose(0, 1).contiguous())
    assert torch.equal(q8.cpu(), want_q) and torch.equal(s.cpu().view(torch.int16), want16.view(torch.int16))
    deq = dequantize(q8, s, torch.float16).cpu()
    assert torch.equal(deq.view(torch.int16), oracle.dequantize(want_q, want16).to(torch.float16).view(torch.int16))
    deq_bf = dequantize(q8, s, torch.bfloat16).cpu()
    assert torch.equal(deq_bf.view(torch.int16), oracle.dequantize(want_q, want16).to(torch.bfloat16).view(torch.int16))


def test_quantize_fp32_input(dev):
    print("case quantize_fp32", flush=True)
    g = torch.Generator().manual_seed(2)
    x = torch.randn(300, 8, 64, generator=g) * 7
    q8, s = quantize(x.to(dev))
    want_q, want16, _ = oracle.quantize(x)
    assert torch.equal(q8.cpu(), want_q) and torch.equal(s.cpu().view(torch.int16), want16.view(torch.int16))


def _check(got, ref, what):
    err = (got.double().cpu() - ref).abs()
    print(f"{what}: max_abs={err.max().item():.3e} mean_abs={err.mean().item():.3e}", flush=True)
    assert err.max().item() < 2e-2 and err.mean().item() < 2e-3, what


# 32769 and 131329 keys: 128 splits of 257 / 1027 keys (not a multiple of the 32-key chunk), the last one short
@pytest.mark.parametrize("n,H,Hkv,d,f16", [(1, 32, 8, 128, True), (300, 32, 8, 128, True), (4099, 32, 8, 128, False),
                                           (20000, 16, 2, 64, True), (32769, 32, 8, 128, True),
                                           (131072, 32, 8, 128, False), (131329, 32, 8, 128, False)])
def test_decode_int8_matches_oracle(n, H, Hkv, d, f16, dev):
    print(f"case decode_int8 n={n} H={H}/{Hkv} d={d} f16={f16}", flush=True)
    cap = n + 5  # spare capacity past n must be ignored
    g = torch.Generator(device=dev).manual_seed(n)
    k = torch.randn(cap, Hkv, d, device=dev, generator=g).to(torch.bfloat16)
    v = torch.randn(cap, Hkv, d, device=dev, generator=g).to(torch.bfloat16)
    q = torch.randn(H, d, device=dev, generator=g).to(torch.bfloat16)
    sd = torch.float16 if f16 else torch.float32
    k8, ks = quantize(k, scale_dtype=sd)
    v8, vs = quantize(v, scale_dtype=sd)
    k8[n:] = 127  # garbage past n
    out = decode_int8(q, k8, ks, v8, vs, n, d ** -0.5)
    torch.cuda.synchronize()
    ref = oracle.decode(q, k8, ks, v8, vs, n, d ** -0.5)
    _check(out, ref, f"decode_int8 n={n}")


@pytest.mark.parametrize("n,H,Hkv,d,f16", [(1, 32, 8, 128, True), (2049, 32, 8, 128, False),
                                           (131073, 32, 8, 128, True), (5000, 16, 2, 64, False),
                                           (700, 16, 8, 128, True)])
def test_decode_int8_append_matches_separate_steps(n, H, Hkv, d, f16, dev):
    """decode_int8_append (the new token's K / V rows quantised into row n - 1 by the decode kernel at d = 128 with 4
    query heads per KV head, and the whole cache attended) equals quantize_pair into that row followed by decode_int8: the
    cache rows and scales bitwise against the oracle's quantisation, the output bitwise against the separate
    steps and within tolerance of the float64 oracle. The new rows are strided [Hkv, d] views as a model's k_proj
    output gives them; shapes other than d = 128 / 4 groups take the quantise-then-decode path."""
    print(f"case decode_append n={n} H={H}/{Hkv} d={d} f16={f16}", flush=True)
    from bigger_bird_amd import decode_int8_append
    from bigger_bird_amd.kv_int8 import quantize_pair

    cap = n + 3
    g = torch.Generator(device=dev).manual_seed(n + 17)
    k = torch.randn(cap, Hkv, d, device=dev, generator=g).to(torch.bfloat16)
    v = torch.randn(cap, Hkv, d, device=dev, generator=g).to(torch.bfloat16)
    q = torch.randn(H, d, device=dev, generator=g).to(torch.bfloat16)
    new = torch.randn(2, 1, Hkv, 1, 3 * d, device=dev, generator=g).to(torch.bfloat16)
    knew, vnew = new[0, 0, :, 0, d:2 * d], new[1, 0, :, 0, d:2 * d]  # [Hkv, d], head stride 3 d
    assert knew.stride() == (3 * d, 1)
    sd = torch.float16 if f16 else torch.float32
    k8, ks = quantize(k, scale_dtype=sd)
    v8, vs = quantize(v, scale_dtype=sd)
    k8[n - 1:] = 77  # stale bytes where the new row goes and past it
    a8, as_, b8, bs = k8.clone(), ks.clone(), v8.clone(), vs.clone()
    out = decode_int8_append(q, k8, ks, v8, vs, knew, vnew, n, d ** -0.5)
    quantize_pair(knew[None], vnew[None], (a8[n - 1:n], as_[n - 1:n]), (b8[n - 1:n], bs[n - 1:n]), scale_dtype=sd)
    want = decode_int8(q, a8, as_, b8, bs, n, d ** -0.5)
    torch.cuda.synchronize()
    qk, sk16, sk32 = oracle.quantize(knew[None].cpu())
    qv, sv16, sv32 = oracle.quantize(vnew[None].cpu())
    assert torch.equal(k8[n - 1:n].cpu(), qk) and torch.equal(v8[n - 1:n].cpu(), qv)
    sk, sv = (sk16, sv16) if f16 else (sk32, sv32)
    bits = torch.int16 if f16 else torch.int32
    assert torch.equal(ks[n - 1:n].cpu().view(bits), sk.view(bits))
    assert torch.equal(vs[n - 1:n].cpu().view(bits), sv.view(bits))
    assert torch.equal(k8[:n - 1], a8[:n - 1]) and torch.equal(k8[n:], a8[n:])  # nothing else written
    assert torch.equal(out, want)
    _check(out, oracle.decode(q, k8, ks, v8, vs, n, d ** -0.5), f"decode_append n={n}")


def test_decode_bf16_matches_sdpa(dev):
    print("case decode_bf16", flush=True)
    n, H, Hkv, d = 5000, 32, 8, 128
    k, v, q = _rand((Hkv, n, d), 3), _rand((Hkv, n, d), 4), _rand((H, d), 5)
    out = decode_bf16(q.to(dev), k.to(dev), v.to(dev), d ** -0.5)
    ref = oracle.sdpa_ref(q[:, None], k, v, causal=False, scale=d ** -0.5, groups=H // Hkv)[:, 0]
    _check(out, ref, "decode_bf16")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_rope_inplace_bitwise(dtype, dev):
    print(f"case rope {dtype}", flush=True)
    T, d = 5000, 128
    cos, sin = rope_cos_sin(T, d, dtype=dtype)
    x = _rand((1, 8, T, d), 6, 3.0).to(dtype)
    y = x.to(dev).transpose(1, 2).contiguous().transpose(1, 2)  # strided [1, H, T, d] view like q_proj output
    rope_inplace(y, cos.to(dev), sin.to(dev))
    assert torch.equal(y.cpu(), rope_host(x, cos, sin))


@pytest.mark.parametrize("scale_dtype,f32", [(torch.float16, False), (torch.float32, False), (torch.float32, True),
                                             (torch.float16, "f16")])
def test_quantize_pair_matches_oracle(scale_dtype, f32, dev):
    """K and V rows quantised in one launch (bb_int8_quantize_pair) equal the oracle for each tensor, bitwise, into
    slices of cache buffers; inputs that differ in strides take the two-launch path with the same results."""
    print(f"case quantize_pair {scale_dtype} f32={f32}", flush=True)
    from bigger_bird_amd.kv_int8 import quantize_pair

    k, v = _rand((1, 8, 5, 128), 3, 3.0), _rand((1, 8, 5, 128), 4, 0.5)
    if f32 == "f16":  # fp16 inputs
        k, v = (_rand((1, 8, 5, 128), 3, 3.0).float() * 1.37).half(), (_rand((1, 8, 5, 128), 4, 0.5).float() * 0.71).half()
    elif f32:
        k, v = k.float(), v.float()
    kd, vd = k.to(dev)[0].transpose(0, 1), v.to(dev)[0].transpose(0, 1)  # [t, Hkv, d] strided views
    qk = torch.zeros(20, 8, 128, dtype=torch.int8, device=dev)
    qv = torch.zeros_like(qk)
    sk = torch.zeros(20, 8, 1, dtype=scale_dtype, device=dev)
    sv = torch.zeros_like(sk)
    rows = slice(7, 12)
    quantize_pair(kd, vd, (qk[rows], sk[rows]), (qv[rows], sv[rows]), scale_dtype=scale_dtype)
    for x, q8, s in ((k, qk, sk), (v, qv, sv)):
        want_q, want16, want32 = oracle.quantize(x[0].transpose(0, 1).contiguous())
        want_s = want16 if scale_dtype == torch.float16 else want32
        assert torch.equal(q8[rows].cpu(), want_q)
        assert torch.equal(s[rows].cpu().float(), want_s.float())
        assert (q8[:7] == 0).all() and (q8[12:] == 0).all()  # nothing outside the rows
    # different strides (V contiguous): two launches, same bytes
    qk2, qv2 = torch.zeros_like(qk), torch.zeros_like(qv)
    sk2, sv2 = torch.zeros_like(sk), torch.zeros_like(sv)
    quantize_pair(kd, vd.contiguous(), (qk2[rows], sk2[rows]), (qv2[rows], sv2[rows]), scale_dtype=scale_dtype)
    assert torch.equal(qk2, qk) and torch.equal(qv2, qv) and torch.equal(sk2, sk) and torch.equal(sv2, sv)
