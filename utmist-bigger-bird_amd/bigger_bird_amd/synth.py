"""Synthetic Llama-3-8B-geometry attention inputs (the benchmark workloads).

Q [B, H, T, d], K/V [B, Hkv, T, d] ~ N(0, 1) drawn on the host from a seeded torch.Generator (identical bytes on
every machine running this torch build), rounded to bf16 (or fp16), with HF Llama RoPE (theta 500000) applied to Q
and K.
Optionally `planted` keys per KV head: key m is 4 x the mean over the group's query heads of post-RoPE Q at position
T - planted + m, written post-RoPE at `planted` distinct seeded positions in [sink, T - window) -- they must be routed.
"""
import torch


def rope_cos_sin(T, d, theta=500000.0, dtype=torch.bfloat16):
    """HF LlamaRotaryEmbedding (default rope type) on the host: fp32 angles, cos/sin rounded to `dtype`. [T, d]."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, d, 2, dtype=torch.int64).to(torch.float32) / d))
    pos = torch.arange(T, dtype=torch.float32)
    freqs = pos[:, None] * inv_freq[None, :]
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def rope_host(x, cos, sin):
    """HF apply_rotary_pos_emb arithmetic on bf16 or fp16 host tensors: x*cos + rotate_half(x)*sin, rounding per
    op."""
    half = x.shape[-1] // 2
    rot = torch.cat((-x[..., half:], x[..., :half]), dim=-1)
    return x * cos + rot * sin


def make_inputs(T, H=32, Hkv=8, d=128, *, batch=1, seed=0, theta=500000.0, rope=True, planted=0, sink=64,
                window=16384, device="cpu", rope_on_device=True, rng="host", dtype=torch.bfloat16):
    """Returns dict(q, k, v, planted_pos) with q [B,H,T,d], k/v [B,Hkv,T,d] in `dtype` (bf16 or fp16) on `device`.

    rng="host" draws Q/K/V from a CPU generator (identical bytes on every machine); rng="device" draws them with the
    device's generator (fast at 128K tokens, reproducible on one torch build and GPU model). Planted positions always
    come from the host generator. RoPE runs on the device through the HIP kernel when `device` is a GPU and
    `rope_on_device` (bit-identical to the host formula), otherwise on the host."""
    g = torch.Generator().manual_seed(seed)
    if rng == "device":
        gd = torch.Generator(device=device).manual_seed(seed)
        q = torch.randn(batch, H, T, d, generator=gd, device=device).to(dtype)
        k = torch.randn(batch, Hkv, T, d, generator=gd, device=device).to(dtype)
        v = torch.randn(batch, Hkv, T, d, generator=gd, device=device).to(dtype)
    elif rng == "host":
        q = torch.randn(batch, H, T, d, generator=g).to(dtype)
        k = torch.randn(batch, Hkv, T, d, generator=g).to(dtype)
        v = torch.randn(batch, Hkv, T, d, generator=g).to(dtype)
    else:
        raise ValueError("rng must be 'host' or 'device'")
    pos = None
    if planted:
        span = T - window - sink
        if span < planted:
            raise ValueError("not enough room to plant keys")
        pos = torch.stack([torch.randperm(span, generator=g)[:planted].sort().values + sink
                           for _ in range(batch * Hkv)]).view(batch, Hkv, planted)
    on_gpu = torch.device(device).type == "cuda"
    if on_gpu:
        q, k, v = q.to(device), k.to(device), v.to(device)
    if rope:
        cos, sin = rope_cos_sin(T, d, theta, dtype)
        if on_gpu and rope_on_device:
            from .attention import rope_inplace
            cos, sin = cos.to(device), sin.to(device)
            rope_inplace(q, cos, sin)
            rope_inplace(k, cos, sin)
        else:
            cos, sin = cos.to(q.device), sin.to(q.device)
            q, k = rope_host(q, cos, sin), rope_host(k, cos, sin)
    if planted:
        G = H // Hkv
        tail = q[:, :, T - planted:, :].float().view(batch, Hkv, G, planted, d).mean(2)  # [B, Hkv, planted, d]
        keys = (4.0 * tail).to(dtype)
        p = pos.to(k.device)
        k.scatter_(2, p[..., None].expand(-1, -1, -1, d), keys)
    return dict(q=q, k=k, v=v, planted_pos=pos)


def attended_pairs(T, H, sink, window, routes, exact_tail, N=None):
    """Attended (query, key) pairs of one Bigger Bird v3 layer: front | window | routed union per row, plus the exact
    tail's causal rows. `routes` [H, K] int (ascending or not, -1 ignored). FLOPs = 4 * d * pairs."""
    N = T if N is None else N
    r = min(exact_tail, T)
    main_rows = T - r
    off = N - T
    total = 0
    i = torch.arange(main_rows, dtype=torch.int64) + off  # absolute positions of the main rows
    front = torch.clamp(torch.minimum(torch.full_like(i, sink), i + 1), min=0)
    win_lo = torch.maximum(torch.full_like(i, sink), i - window + 1)
    win = torch.clamp(i - win_lo + 1, min=0)
    total += int(front.sum() + win.sum()) * H
    rc = routes.detach().to("cpu", torch.int64)
    for h in range(rc.shape[0]):
        j = rc[h][(rc[h] >= sink)]
        # routed key j counts for main rows q >= j + window
        first = j + window - off
        total += int(torch.clamp(main_rows - first, min=0).sum())
    tail_rows = torch.arange(T - r, T, dtype=torch.int64) + off
    total += int((tail_rows + 1).sum()) * H
    return total
