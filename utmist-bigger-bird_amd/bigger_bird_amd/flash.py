"""`bigger_bird_flash`: the sparse attention operator, HIP-backed (drop-in for kernels/bigger_bird_flash.py:99-138).

Same arguments, shapes, output layout and ValueError conditions as the reference; fp16 and bf16 inputs, as the
reference's kernel takes (kernels/bigger_bird_flash.py:110). One joint softmax over front
anchors, a causal local window and routed key columns; Q [BH, T, D], K/V [BH / kv_groups, N, D] (any strides with a
contiguous head_dim), indices [BH, G, K] int32 with -1 for empty slots; the output is a [BH, T, D] view of a
[T, BH, D] buffer. Query row t sits at absolute position t + N - T.

`block_m`, `block_n`, `num_warps` and `num_stages` are accepted for signature compatibility; the gfx950 kernel's tile
shapes are fixed (64-key tiles, 256 query rows per workgroup), and `block_m` only enters the route_chunk alignment
check, exactly as in the reference.
"""
import torch

from . import _lib


def _next_pow2(n: int) -> int:
    return 1 << max(0, (int(n) - 1).bit_length())


def _same_dtype(q, *others):
    """q, k, v (and V^T / out when given) share one 16-bit dtype: the kernels read and write that type."""
    if any(x is not None and x.dtype != q.dtype for x in others):
        raise ValueError("q, k and v must share a dtype")


def _operand(x: torch.Tensor) -> torch.Tensor:
    """The kernel reads 16-byte rows: head_dim contiguous, row strides multiples of 8 elements, 16-byte base."""
    ok = (x.stride(-1) == 1 and all(s % 8 == 0 for s in x.stride()[:-1]) and x.data_ptr() % 16 == 0)
    return x if ok else x.contiguous()


def transpose_v(v: torch.Tensor) -> torch.Tensor:
    """V [BKV, N, D] -> V^T [BKV, D, N rounded up to 64] (zero columns past N), reusable across flash calls."""
    _lib.require_gpu(v, what="transpose_v")
    v = _operand(v)
    bkv, n, d = v.shape
    cols = _lib.lib().bb_transpose_v_cols(n)
    vt = torch.empty(bkv, d, cols, dtype=v.dtype, device=v.device)
    _lib.check(_lib.lib().bb_transpose_v(_lib.ptr(v), _lib.i64s(*v.stride()), bkv, n, d, _lib.ptr(vt),
                                         _lib.stream_of(v)))
    return vt


def bigger_bird_flash(q, k, v, indices, *, front=64, window=256, token_mask=None, num_heads=32, route_chunk=None,
                      kv_groups=1, scale=1.0, block_m=64, block_n=64, num_warps=4, num_stages=2, row_end=None,
                      vt=None, out=None):
    """Q [BH,T,D], K/V [BH/kv_groups,N,D]; unique route indices [BH,G,K], -1 marks invalid.

    Extensions over the reference signature (all optional): `row_end` leaves rows >= row_end unwritten (the exact
    tail overwrites them), `vt` passes a precomputed `transpose_v(v)`, `out` a preallocated [BH,T,D] destination.
    """
    if not q.is_cuda or q.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("HIP Bigger Bird requires ROCm FP16/BF16")
    if (k.shape != v.shape or q.ndim != 3 or q.shape[0] != k.shape[0] * kv_groups
            or q.shape[-1] != k.shape[-1] or num_heads % kv_groups):
        raise ValueError("Q [BH,T,D] and K/V [BH/kv_groups,N,D] must have matching heads and dimensions")
    _same_dtype(q, k, v, vt, out)
    if front < 0 or window < 1:
        raise ValueError("front >= 0 and window >= 1 required")
    bh, t, d = q.shape
    n = k.shape[1]
    if n - t < 0:
        raise ValueError("Key sequence must be at least as long as query sequence")
    if indices.ndim == 2:
        indices = indices[:, None, :]
    route_chunk = route_chunk or max(block_m, _next_pow2(n))
    if route_chunk % block_m or tuple(indices.shape[:2]) != (bh, -(-n // route_chunk)):
        raise ValueError("Routing groups must cover the sequence and align with query tiles")
    indices = indices.contiguous().to(torch.int32)
    if token_mask is not None:
        if tuple(token_mask.shape) != (bh // num_heads, n) or token_mask.dtype != torch.bool:
            raise ValueError("token_mask must be boolean [batch,N]")
    _lib.require_gpu(k, v, indices, token_mask, vt, what="bigger_bird_flash")
    if out is None:
        out = torch.empty((t, bh, d), dtype=q.dtype, device=q.device).permute(1, 0, 2)
    if t == 0:
        return out
    q, k, v = _operand(q), _operand(k), _operand(v)
    mask = token_mask.contiguous().view(torch.uint8) if token_mask is not None else None
    route_k = indices.shape[-1]
    re = t if row_end is None else int(row_end)
    L = _lib.lib()
    ws_bytes = L.bb_sparse_flash_workspace(bh, t, n, d, num_heads, kv_groups, min(front, n), window, route_k,
                                           indices.shape[1], re, int(vt is not None), int(mask is not None))
    ws = _lib.workspace(ws_bytes, q.device) if ws_bytes else None
    _lib.check(L.bb_sparse_flash(
        _lib.ptr(q), _lib.i64s(*q.stride()), _lib.ptr(k), _lib.i64s(*k.stride()), _lib.ptr(v), _lib.i64s(*v.stride()),
        _lib.ptr(vt), _lib.ptr(indices) if route_k else None, _lib.i64s(*indices.stride()), indices.shape[1], route_k,
        _lib.ptr(mask), mask.stride(0) if mask is not None else 0,
        _lib.ptr(out), _lib.i64s(*out.stride()), bh, t, n, d, int(q.dtype == torch.float16), num_heads, kv_groups,
        min(front, n), window, route_chunk, float(scale), re, _lib.ptr(ws), ws_bytes, _lib.stream_of(q)))
    return out


def exact_attention(q, k, v, *, num_heads, kv_groups=1, scale=1.0, vt=None, out=None):
    """Non-causal exact attention in one launch: every row of Q [BH, T, D] attends all N keys of K/V [BH/kv_groups, N,
    D] (T <= N). The operator behind RDAttention.exact_attention for 1 < t < n, where the reference calls
    F.scaled_dot_product_attention(q, k, v, is_causal=False, enable_gqa=True) (modal_rd/attention.py:140-141). Returns
    a [BH, T, D] view of a [T, BH, D] buffer (or writes `out`); `vt` may pass a precomputed transpose_v(v)."""
    if not q.is_cuda or q.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("HIP Bigger Bird requires ROCm FP16/BF16")
    if (k.shape != v.shape or q.ndim != 3 or q.shape[0] != k.shape[0] * kv_groups
            or q.shape[-1] != k.shape[-1] or num_heads % kv_groups):
        raise ValueError("Q [BH,T,D] and K/V [BH/kv_groups,N,D] must have matching heads and dimensions")
    _same_dtype(q, k, v, vt, out)
    bh, t, d = q.shape
    n = k.shape[1]
    if n - t < 0:
        raise ValueError("Key sequence must be at least as long as query sequence")
    _lib.require_gpu(k, v, vt, what="exact_attention")
    if out is None:
        out = torch.empty((t, bh, d), dtype=q.dtype, device=q.device).permute(1, 0, 2)
    if t == 0:
        return out
    q, k, v = _operand(q), _operand(k), _operand(v)
    L = _lib.lib()
    ws_bytes = L.bb_exact_attention_workspace(bh, t, n, d, num_heads, kv_groups, int(vt is not None))
    ws = _lib.workspace(ws_bytes, q.device) if ws_bytes else None
    _lib.check(L.bb_exact_attention(
        _lib.ptr(q), _lib.i64s(*q.stride()), _lib.ptr(k), _lib.i64s(*k.stride()), _lib.ptr(v), _lib.i64s(*v.stride()),
        _lib.ptr(vt), _lib.ptr(out), _lib.i64s(*out.stride()), bh, t, n, d, int(q.dtype == torch.float16), num_heads,
        kv_groups, float(scale), _lib.ptr(ws), ws_bytes, _lib.stream_of(q)))
    return out
