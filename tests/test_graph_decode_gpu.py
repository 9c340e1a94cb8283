"""HIP-graph greedy decode (bigger_bird_amd.graph_decode, drop-in for modal_rd/graph_decode.py) on a tiny random-init
Llama, as the reference's GPU self-check modal_rd/graphcheck.py:22-37 runs it: for the dense_rd, rd and rd + kv_evict
arms the captured decode must produce what eager decoding produces.

* Graph replay vs the same step run eagerly (a second decoder, graph=False): token ids and logits bit-identical for
  every step, with unrelated eager work and host synchronisation between replays (captured graphs have given wrong
  results on replays after the first when they recorded memset nodes; the step records none).
* Graph decode vs the model's own eager forward (HF layer stack, RDAttention's exact decode over a DynamicCache),
  teacher-forced with the graph's tokens: logits close at every step (the attention kernels differ: split-K flash
  decoding vs the INT8-path kernel in bf16 mode), and the same greedy token wherever the eager top-2 margin is clear.
* generate(): stops after the block that produced an EOS, returns the tokens through it, rewinds the cache to right
  after the EOS's input and makes the EOS the next input; the HIP argmax equals torch.argmax (incl. ties, NaN).
"""
import pytest
import torch

from bigger_bird_amd import install
from bigger_bird_amd.decode import argmax_index
from bigger_bird_amd.graph_decode import StaticDecoder, graph_prefill

pytestmark = pytest.mark.gpu

KW = dict(sink=8, window=96, vertical=24, n_route=16, exact_tail=24, block_m=16, block_n=16)
EVICT = dict(kv_evict=True)
N, STEPS = 400, 12


def _tiny(dev, dtype=torch.bfloat16):
    from transformers import LlamaConfig, LlamaForCausalLM

    # head_dim 64: the decode kernels take 64 or 128
    cfg = LlamaConfig(vocab_size=512, hidden_size=512, intermediate_size=1024, num_hidden_layers=2,
                      num_attention_heads=8, num_key_value_heads=2, max_position_embeddings=8192,
                      attn_implementation="sdpa")
    torch.manual_seed(0)
    return LlamaForCausalLM(cfg).to(dev, dtype).eval()


def _ids(dev):
    g = torch.Generator().manual_seed(4)
    return torch.randint(0, 512, (1, N), generator=g).to(dev)


SPARSE = dict(front=8, window=64, routed=32)


@pytest.mark.parametrize("arm,extra,sparse,dtype", [("dense_rd", {}, None, torch.bfloat16), ("rd", {}, None, torch.bfloat16),
                                                    ("rd", EVICT, None, torch.bfloat16), ("rd", {}, SPARSE, torch.bfloat16),
                                                    ("rd", {}, SPARSE, torch.float16)])
def test_graph_matches_eager_step_bitwise(arm, extra, sparse, dtype, dev):
    print(f"case graph_vs_eager_step {arm} evict={bool(extra)} sparse={bool(sparse)} {dtype}", flush=True)
    model = _tiny(dev, dtype)
    install(model, arm, **KW, **extra)
    ids = _ids(dev)
    dec, out, _ = graph_prefill(model, ids, STEPS + 4, headroom=64, sparse_decode=sparse)
    assert int(dec.token) == out.logits[0, -1].argmax().item()
    assert dec.sparse == [bool(sparse)] * len(model.model.layers)
    # a second, eager decoder over the same prefill (deterministic kernels: identical cache)
    eager = StaticDecoder(model, dec.capacity, sparse_decode=sparse)
    with torch.inference_mode():
        from transformers import DynamicCache
        cache = eager.buffer_cache() if not extra else DynamicCache(config=model.config)
        o2 = model(input_ids=ids, position_ids=torch.arange(N, device=dev)[None], past_key_values=cache,
                   use_cache=True, logits_to_keep=1)
        assert torch.equal(o2.logits, out.logits)
        eager.load(cache, N, o2.logits[0, -1].argmax().item())
    m = int(dec.length)
    if extra:
        g = model.config.num_attention_heads // model.config.num_key_value_heads
        assert m == KW["sink"] + KW["window"] + g * KW["vertical"]
    else:
        assert m == N
    for i in range(STEPS):
        dec.run(1)
        eager.run(1, graph=False)
        torch.cuda.synchronize()
        assert int(dec.length) == m + i + 1 and int(dec.position) == N + i + 1
        assert torch.equal(dec.logits, eager.logits), i
        assert dec.generated() == eager.generated(), i
        _ = torch.randn(1000, device=dev).sum().item()  # unrelated eager work between replays


@pytest.mark.parametrize("arm,extra", [("dense_rd", {}), ("rd", {}), ("rd", EVICT)])
def test_graph_matches_model_forward(arm, extra, dev):
    print(f"case graph_vs_model {arm} evict={bool(extra)}", flush=True)
    from transformers import DynamicCache

    model = _tiny(dev)
    install(model, arm, **KW, **extra)
    ids = _ids(dev)
    dec, out, _ = graph_prefill(model, ids, STEPS + 4, headroom=64)
    cache = DynamicCache(config=model.config)
    with torch.inference_mode():
        ref = model(input_ids=ids, past_key_values=cache, use_cache=True, logits_to_keep=1).logits[0, -1]
        tok = ref.argmax().item()
        for i in range(STEPS):
            dec.run(1)
            got = dec.logits.float()
            step_ids = torch.tensor([[tok]], device=dev)
            pos = torch.tensor([[N + i]], device=dev)
            want = model(input_ids=step_ids, position_ids=pos, past_key_values=cache, use_cache=True).logits[0, -1]
            want = want.float()
            err = (got - want).abs().max().item()
            assert err <= 2e-2 * want.abs().max().item() + 1e-3, (i, err)
            top2 = want.topk(2).values
            nxt = dec.generated()[-1]
            if (top2[0] - top2[1]).item() > 4 * err + 1e-3:
                assert nxt == want.argmax().item(), i
            tok = nxt  # teacher forcing with the graph's token


def test_generate_eos_and_rewind(dev):
    print("case generate_eos", flush=True)
    model = _tiny(dev)
    install(model, "dense_rd", **KW)
    ids = _ids(dev)
    dec, _, _ = graph_prefill(model, ids, 40, headroom=64)
    first = int(dec.token)
    toks, steps = dec.generate(10, block=4)
    assert steps == 12 - 2 and len(toks) == 10  # max_steps caps the last block
    # replay from the same prefill with the 6th token as EOS
    dec2, _, _ = graph_prefill(model, ids, 40, headroom=64)
    assert dec2 is dec and int(dec.token) == first and int(dec.length) == N
    eos = toks[5]
    cut = toks.index(eos) + 1
    got, steps = dec.generate(10, eos=[eos], block=4)
    assert got == toks[:cut] and steps == 4 * ((cut + 3) // 4)  # whole blocks, stopping after the EOS's block
    assert int(dec.length) == N + cut and int(dec.position) == N + cut and int(dec.step_i) == cut
    assert int(dec.token) == eos
    # a further turn appends after the rewound point and continues as the uninterrupted run would
    more, _ = dec.generate(10 - cut, block=4)
    assert more == toks[cut:]
    with pytest.raises(ValueError, match="buffer full"):
        dec.run(dec.capacity)


def test_argmax_matches_torch(dev):
    g = torch.Generator().manual_seed(5)
    for dt in (torch.float32, torch.bfloat16, torch.float16):
        for n in (1, 7, 1000, 128256, 300001):
            x = torch.randn(n, generator=g).to(dt).to(dev)
            assert argmax_index(x).item() == x.argmax().item(), (dt, n)
        x = torch.zeros(5000, dtype=dt, device=dev)
        x[[17, 300, 4000]] = 3.0  # ties: first index
        assert argmax_index(x).item() == 17
        x[2500] = float("nan")
        x[4500] = float("nan")
        assert argmax_index(x).item() == 2500
        x = torch.full((999,), -float("inf"), dtype=dt, device=dev)
        assert argmax_index(x).item() == 0
    x = torch.randn(2, 4097, generator=g).to(torch.bfloat16).to(dev)[:, 1:].reshape(-1)  # offset, unaligned start
    assert argmax_index(x[3:]).item() == x[3:].argmax().item()


@pytest.mark.parametrize("dtype,d", [(torch.bfloat16, 4096), (torch.bfloat16, 512), (torch.float16, 4096)])
def test_rms_norm_matches_hf(dtype, d, dev):
    """bb_rms_norm against transformers' LlamaRMSNorm: the same arithmetic except the fp32 summation order of the
    mean of squares, so results agree to one unit in the last place of the model dtype (and mostly bitwise)."""
    from transformers.models.llama.modeling_llama import LlamaRMSNorm

    from bigger_bird_amd.decode import rms_norm

    g = torch.Generator().manual_seed(6)
    norm = LlamaRMSNorm(d, eps=1e-5).to(dev, dtype)
    with torch.no_grad():
        norm.weight.copy_((1 + 0.1 * torch.randn(d, generator=g)).to(dtype))
    x = (torch.randn(3, 5, d, generator=g) * 3).to(dtype).to(dev)
    want = norm(x)
    got = rms_norm(x, norm.weight, norm.variance_epsilon)
    diff = (got.float() - want.float()).abs()
    ulp = want.float().abs() * (2.0 ** -7 if dtype == torch.bfloat16 else 2.0 ** -10) + 1e-30
    assert (diff <= ulp).all()
    assert (diff == 0).float().mean() > 0.95


@pytest.mark.parametrize("dtype,d", [(torch.bfloat16, 4096), (torch.float16, 4096), (torch.bfloat16, 520)])
def test_add_rms_norm_matches_torch_and_hf(dtype, d, dev):
    """bb_add_rms_norm: the sum is the 16-bit tensor add bit for bit, and the norm of it is bb_rms_norm's bit for bit
    (so within one unit in the last place of transformers' LlamaRMSNorm, as bb_rms_norm)."""
    from transformers.models.llama.modeling_llama import LlamaRMSNorm

    from bigger_bird_amd.decode import add_rms_norm, rms_norm

    g = torch.Generator().manual_seed(8)
    norm = LlamaRMSNorm(d, eps=1e-5).to(dev, dtype)
    with torch.no_grad():
        norm.weight.copy_((1 + 0.1 * torch.randn(d, generator=g)).to(dtype))
    x = (torch.randn(1, 3, d, generator=g) * 3).to(dtype).to(dev)
    r = (torch.randn(1, 3, d, generator=g) * 2).to(dtype).to(dev)
    total, got = add_rms_norm(x, r, norm.weight, norm.variance_epsilon)
    assert torch.equal(total, x + r)
    assert torch.equal(got, rms_norm(x + r, norm.weight, norm.variance_epsilon))
    want = norm(x + r)
    diff = (got.float() - want.float()).abs()
    assert (diff <= want.float().abs() * (2.0 ** -7 if dtype == torch.bfloat16 else 2.0 ** -10) + 1e-30).all()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_silu_mul_matches_torch(dtype, dev):
    """bb_silu_mul against F.silu(g) * u on the same 16-bit inputs (wide range, signed zeros, +-inf, large
    negative gates): the same fp32 arithmetic, so the results are bitwise equal (NaNs compared as NaNs)."""
    from bigger_bird_amd.decode import silu_mul

    gen = torch.Generator().manual_seed(9)
    n = 14336 * 2
    g = (torch.randn(n, generator=gen) * torch.exp2(torch.randint(-8, 7, (n,), generator=gen).float()))
    u = torch.randn(n, generator=gen) * 4
    g[:8] = torch.tensor([0.0, -0.0, float("inf"), -float("inf"), -100.0, 100.0, 1e-30, -1e-30])
    g, u = g.to(dtype).to(dev), u.to(dtype).to(dev)
    y = torch.empty(2 * n, dtype=dtype, device=dev)  # g and u as the two halves of one projection's output
    y[:n], y[n:] = g, u
    got = silu_mul(y[:n], y[n:])
    want = torch.nn.functional.silu(g) * u
    assert torch.equal(got.isnan(), want.isnan())
    ok = ~want.isnan()
    assert torch.equal(got[ok], want[ok])


def test_fused_mlp_engaged_and_close_to_module(dev):
    """The decode step's MLP on a Llama layer takes the fused path (gate and up as one projection whose weights are
    views of one buffer, run as two HIP GEMVs) and agrees with the HF module to bf16 rounding of the projections."""
    model = _tiny(dev)
    dec = StaticDecoder(model, 64)
    plan = dec.plans[0]
    mlp = plan.layer.mlp
    assert plan.gate_up_w is not None and plan.inter == mlp.gate_proj.weight.shape[0]
    assert mlp.gate_proj.weight.data_ptr() == plan.gate_up_w.data_ptr()
    assert plan.mlp_vec and plan.qkv_vec and plan.o_vec
    x = torch.randn(1, 1, 512, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16).to(dev)
    with torch.no_grad():
        got, want = StaticDecoder._mlp(plan, x), mlp(x)
    assert (got.float() - want.float()).abs().max().item() <= 2e-2 * want.float().abs().max().item()



@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("n,k,stride", [(6144, 4096, 4096), (4096, 14336, 14336), (1001, 520, 520),
                                        (37, 1000, 1024), (3, 16384, 16384)])
def test_linear_vec_matches_fp32(n, k, stride, dtype, dev):
    """bb_gemv (one token through a linear layer) against the fp32 product of the same 16-bit operands: fp32
    accumulation of exact products and one rounding, so within half a unit in the last place of the result plus the
    accumulation's own error; ragged N and K, a row stride larger than K, and the largest K."""
    from bigger_bird_amd.decode import linear_vec

    g = torch.Generator().manual_seed(n + k)
    wfull = (torch.randn(n, stride, generator=g) * 0.05).to(dtype).to(dev)
    w = wfull[:, :k]
    x = torch.randn(1, 1, k, generator=g).to(dtype).to(dev)
    got = linear_vec(x, w).float()
    ref = x.float() @ w.float().t()
    mag = x.float().abs() @ w.float().abs().t()
    half_ulp = 2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -11  # relative, at most
    assert ((got - ref).abs() <= ref.abs() * half_ulp * 1.01 + mag * 2.0 ** -16 + 1e-30).all()
    assert ((got - ref).abs() <= ref.abs() * 2.0 ** -9).float().mean() > 0.5  # not a looser rounding


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("n,k", [(14336, 4096), (100, 520), (3, 64)])
def test_linear_vec_glu_matches_gate_up(n, k, dtype, dev):
    """bb_gemv with the SiLU gate on a fused [gate; up] weight: a row's sum does not depend on which rows share its
    wave, so the gated output is F.silu(gate) * up of the plain GEMV's gate and up outputs, bit for bit (the same
    arithmetic as bb_silu_mul, `test_silu_mul_matches_torch`); odd N included."""
    from bigger_bird_amd.decode import linear_vec

    g = torch.Generator().manual_seed(n)
    w = (torch.randn(2 * n, k, generator=g) * 0.05).to(dtype).to(dev)
    x = torch.randn(1, 1, k, generator=g).to(dtype).to(dev)
    got = linear_vec(x, w, glu=True)
    both = linear_vec(x, w)  # the same rows without the gate
    want = torch.nn.functional.silu(both[..., :n]) * both[..., n:]
    assert torch.equal(got, want)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("n,k,glu,with_res", [(6144, 4096, False, True), (1000, 4096, True, True),
                                              (37, 520, False, False), (64, 8192, True, False)])
def test_linear_vec_norm_is_norm_then_gemv(n, k, glu, with_res, dtype, dev):
    """bb_gemv_norm: every workgroup normalises the hidden row with bb_rms_norm's arithmetic, so (sum, y) equal
    bb_add_rms_norm (or bb_rms_norm) followed by bb_gemv bit for bit."""
    from bigger_bird_amd.decode import add_rms_norm, linear_vec, linear_vec_norm, rms_norm

    g = torch.Generator().manual_seed(k + n)
    w = (torch.randn(2 * n if glu else n, k, generator=g) * 0.05).to(dtype).to(dev)
    nw = (1 + 0.1 * torch.randn(k, generator=g)).to(dtype).to(dev)
    x = (torch.randn(1, 1, k, generator=g) * 3).to(dtype).to(dev)
    r = (torch.randn(1, 1, k, generator=g) * 2).to(dtype).to(dev) if with_res else None
    total, y = linear_vec_norm(x, r, nw, 1e-5, w, glu=glu)
    if with_res:
        want_total, xn = add_rms_norm(x, r, nw, 1e-5)
        assert torch.equal(total, want_total)
    else:
        xn = rms_norm(x, nw, 1e-5)
        assert total is x
    assert torch.equal(y, linear_vec(xn, w, glu=glu))
