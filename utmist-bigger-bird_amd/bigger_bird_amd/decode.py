"""Decode-time operators for one new query token, HIP-backed: drop-ins for kernels/bigger_bird_decode.py (split-K
sparse decode) and kernels/bigger_bird_route.py (fused decode routing).

Same arguments, shapes and ValueError conditions as the reference. `n` may be a 1-element int64 tensor on the GPU
holding the current cache length (keys at >= n are ignored), so a HIP graph captured once stays valid as the cache
grows inside a fixed-capacity buffer; every other argument fixes the launch shapes. `block_n`, `num_warps` and
`num_stages` are accepted for signature compatibility (the gfx950 kernels use fixed 64-key chunks).
"""
import torch

from . import _lib


def _len_arg(n, device):
    """(host length or None, device pointer or None) for the C ABI."""
    if n is None:
        return None, None
    if isinstance(n, torch.Tensor):
        if not n.is_cuda or n.numel() != 1:
            raise ValueError("n must be a 1-element int tensor on the GPU")
        if n.dtype != torch.int64:
            raise ValueError("n must be an int64 tensor (it is read in place by the kernels)")
        return None, _lib.ptr(n)
    return int(n), None


def _rows16(x):
    """head_dim contiguous with 16-byte aligned rows (a cache view qualifies); otherwise a contiguous copy."""
    ok = x.stride(-1) == 1 and all(s % 8 == 0 for s in x.stride()[:-1]) and x.data_ptr() % 16 == 0
    return x if ok else x.contiguous()


def bigger_bird_decode(q, k, v, indices, *, front=64, window=4096, scale=1.0, n=None, splits=None, block_n=64,
                       num_warps=4, num_stages=2):
    """q [H, D] (one token), k / v [Hkv, N, D] (any strides, e.g. a cache view), indices int [Hkv or H, R].
    `n`: current length as a 1-element GPU int64 tensor (graph safe); default all N keys. Returns [H, D] in q's dtype.
    Attends each route group to front keys + the last `window` keys + its routed keys (positions outside [0, n) and
    -1 entries are skipped)."""
    if not q.is_cuda or q.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("bigger_bird_decode requires CUDA FP16/BF16")
    h, d = q.shape
    hk, cap, _ = k.shape
    if k.shape != v.shape or h % hk or k.shape[-1] != d:
        raise ValueError("q [H,D] and k/v [Hkv,N,D] must match")
    if n is None and cap < front + window:
        raise ValueError("cache shorter than front + window: use dense attention")
    if indices.ndim != 2 or indices.shape[0] not in (hk, h):
        raise ValueError("indices must be [Hkv, R] (pooled) or [H, R] (per head)")
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("q, k and v must share a dtype")
    _lib.require_gpu(k, v, indices, n if isinstance(n, torch.Tensor) else None, what="bigger_bird_decode")
    k, v = _rows16(k), _rows16(v)
    q = q if q.stride(-1) == 1 else q.contiguous()
    idx = indices.to(torch.int32)
    rows, route_k = idx.shape
    n_host, n_dev = _len_arg(n, q.device)
    if n_host is None:
        n_host = cap
    out = torch.empty(h, d, dtype=q.dtype, device=q.device)
    L = _lib.lib()
    sp = int(splits or 0)
    ws_bytes = L.bb_sparse_decode_workspace(h, hk, d, rows, front, window, route_k, sp)
    ws = _lib.workspace(ws_bytes, q.device)
    _lib.check(L.bb_sparse_decode(
        _lib.ptr(q), q.stride(0), _lib.ptr(k), _lib.i64s(*k.stride()[:2]), _lib.ptr(v), _lib.i64s(*v.stride()[:2]),
        _lib.ptr(idx) if route_k else None, _lib.i64s(*idx.stride()), rows, route_k, n_host, n_dev, cap, h, hk, d,
        int(front), int(window), float(scale), sp, int(q.dtype == torch.float16), _lib.ptr(out), out.stride(0),
        _lib.ptr(ws), ws_bytes, _lib.stream_of(q)))
    return out


def _route(q, k, k_route, front, window, scale, n, splits):
    if not q.is_cuda or q.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("bigger_bird_route requires CUDA FP16/BF16")
    h, d = q.shape
    hk, cap, _ = k.shape
    if h % hk or k.shape[-1] != d:
        raise ValueError("q [H,D] and k [Hkv,CAP,D] must match")
    if k.dtype != q.dtype:
        raise ValueError("q and k must share a dtype")
    _lib.require_gpu(k, n if isinstance(n, torch.Tensor) else None, what="bigger_bird_route")
    k = _rows16(k)
    q = q if q.stride(-1) == 1 else q.contiguous()
    n_host, n_dev = _len_arg(n, q.device)
    if n_host is None:
        n_host = cap
    probs = torch.empty(hk, cap, dtype=torch.float32, device=q.device)
    idx = torch.empty(hk, k_route, dtype=torch.int32, device=q.device) if k_route else None
    L = _lib.lib()
    sp = int(splits or 0)
    ws_bytes = L.bb_decode_route_workspace(cap, h, hk, sp, k_route)
    ws = _lib.workspace(ws_bytes, q.device)
    _lib.check(L.bb_decode_route(
        _lib.ptr(q), q.stride(0), _lib.ptr(k), _lib.i64s(*k.stride()[:2]), n_host, n_dev, cap, h, hk, d, int(front),
        int(window), float(scale), sp, int(q.dtype == torch.float16), _lib.ptr(probs), int(k_route), _lib.ptr(idx),
        _lib.ptr(ws), ws_bytes, _lib.stream_of(q)))
    return probs, idx


def pooled_probs(q, k, *, front=64, window=4096, scale=1.0, n=None, splits=None, block_n=64, num_warps=4):
    """q [H, D], k [Hkv, CAP, D] -> [Hkv, CAP] fp32 pooled probabilities; -1 outside [front, n - window)."""
    return _route(q, k, 0, front, window, scale, n, splits)[0]


def bigger_bird_route(q, k, k_route, *, front=64, window=4096, scale=1.0, n=None, splits=None, **kw):
    """Indices [Hkv, k_route] of the highest pooled-probability keys in [front, n - window): int32, ascending (the
    reference returns them unsorted), ties to the lower index, -1 past the eligible count."""
    if k_route <= 0:
        raise ValueError("k_route must be positive")
    return _route(q, k, int(k_route), front, window, scale, n, splits)[1]


def gather_rows(x, idx):
    """x [heads, n, D] (16-bit dtype, any 16-byte aligned row strides), idx int [heads, m] -> [heads, m, D] with
    out[h, i] = x[h, idx[h, i]] (a zero row for an index outside [0, n)): the cache compaction of kv_evict
    (modal_rd/attention.py:253-257)."""
    if not x.is_cuda or x.element_size() != 2:
        raise ValueError("gather_rows needs a 16-bit GPU tensor")
    heads, n, d = x.shape
    if idx.ndim != 2 or idx.shape[0] != heads:
        raise ValueError("idx must be [heads, m]")
    x = _rows16(x)
    ix = idx.to(torch.int64).contiguous()
    out = torch.empty(heads, ix.shape[1], d, dtype=x.dtype, device=x.device)
    _lib.check(_lib.lib().bb_gather_rows(_lib.ptr(x), _lib.i64s(*x.stride()[:2]), n, heads, _lib.ptr(ix), ix.stride(0),
                                         ix.shape[1], d, _lib.ptr(out), _lib.i64s(*out.stride()[:2]),
                                         _lib.stream_of(x)))
    return out


def kv_append(k, v, knew, vnew, length, advance=1):
    """One decode step's append: k[:, n] = knew and v[:, n] = vnew at n = length (an int64 GPU tensor of one element),
    then length += advance, in one launch (the two index_copy_ calls and the add of a decode step). k / v [Hkv, cap, D]
    (any cache view with 16-byte aligned rows), knew / vnew [Hkv, D]. A length outside [0, cap) writes nothing."""
    if not (k.is_cuda and v.is_cuda and knew.is_cuda and vnew.is_cuda and length.is_cuda):
        raise ValueError("kv_append needs GPU tensors")
    if k.element_size() != 2 or v.dtype != k.dtype or knew.dtype != k.dtype or vnew.dtype != k.dtype:
        raise ValueError("kv_append: one 16-bit dtype")
    hk, cap, d = k.shape
    if v.shape != k.shape or tuple(knew.shape) != (hk, d) or tuple(vnew.shape) != (hk, d):
        raise ValueError("kv_append: k / v [Hkv, cap, D] and new rows [Hkv, D]")
    if length.dtype != torch.int64 or length.numel() != 1:
        raise ValueError("kv_append: length must be one int64")
    if knew.stride(-1) != 1 or vnew.stride(-1) != 1 or k.stride(-1) != 1 or v.stride(-1) != 1:
        raise ValueError("kv_append: rows need a contiguous head_dim")
    _lib.check(_lib.lib().bb_kv_append(_lib.ptr(k), _lib.i64s(k.stride(0), k.stride(1)), _lib.ptr(v),
                                       _lib.i64s(v.stride(0), v.stride(1)), _lib.ptr(knew), knew.stride(0),
                                       _lib.ptr(vnew), vnew.stride(0), hk, d, cap, _lib.ptr(length), int(advance),
                                       _lib.stream_of(k)))


def decode_step(q, k, v, knew, vnew, length, *, routed=0, front=64, window=4096, scale=1.0, advance=0, out=None):
    """One decode step over a cache whose length (an int64 GPU tensor of one element) already counts the new row:
    knew / vnew [Hkv, D] become row length - 1 of k / v [Hkv, cap, D] (a length outside [1, cap] appends nothing),
    the token q [H, D] attends (routed > 0: top `routed` keys per KV head by pooled decode routing outside the front
    and the last `window` keys, then sparse decode over front | window | routed; routed = 0: all rows), and length +=
    advance afterwards (only when the row was appended). Bit-identical to kv_append(..., advance=0) at length - 1,
    bigger_bird_route and bigger_bird_decode (or bigger_bird_decode with front 0, window cap), in two launches fewer.
    Returns out [H, D], and the routed indices [Hkv, routed] (int32, ascending) when routed > 0."""
    if not q.is_cuda or q.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("decode_step requires CUDA FP16/BF16")
    h, d = q.shape
    hk, cap, _ = k.shape
    if k.shape != v.shape or h % hk or k.shape[-1] != d:
        raise ValueError("q [H,D] and k/v [Hkv,N,D] must match")
    if tuple(knew.shape) != (hk, d) or tuple(vnew.shape) != (hk, d):
        raise ValueError("decode_step: new rows must be [Hkv, D]")
    if any(x.dtype != q.dtype for x in (k, v, knew, vnew)):
        raise ValueError("q, k, v and the new rows must share a dtype")
    if not isinstance(length, torch.Tensor) or length.dtype != torch.int64 or length.numel() != 1:
        raise ValueError("decode_step: length must be one int64 GPU tensor")
    _lib.require_gpu(k, v, knew, vnew, length, what="decode_step")
    if any(x.stride(-1) != 1 or any(s % 8 for s in x.stride()[:-1]) or x.data_ptr() % 16 for x in (k, v, knew, vnew)):
        raise ValueError("decode_step: k / v and the new rows need 16-byte aligned rows (the cache is written in place)")
    q = q if q.stride(-1) == 1 else q.contiguous()
    routed = int(routed)
    idx = torch.empty(hk, routed, dtype=torch.int32, device=q.device) if routed > 0 else None
    if out is None:
        out = torch.empty(h, d, dtype=q.dtype, device=q.device)
    elif tuple(out.shape) != (h, d) or out.dtype != q.dtype or out.stride(-1) != 1 or out.device != q.device:
        raise ValueError("decode_step: out must be [H, D] in q's dtype with a contiguous head_dim")
    L = _lib.lib()
    ws_bytes = L.bb_decode_step_workspace(cap, h, hk, d, int(front), int(window), routed)
    ws = _lib.workspace(ws_bytes, q.device)
    _lib.check(L.bb_decode_step(
        _lib.ptr(q), q.stride(0), _lib.ptr(k), _lib.i64s(*k.stride()[:2]), _lib.ptr(v), _lib.i64s(*v.stride()[:2]),
        _lib.ptr(knew), knew.stride(0), _lib.ptr(vnew), vnew.stride(0), _lib.ptr(length), int(advance), cap, h, hk, d,
        int(front), int(window), routed, float(scale), int(q.dtype == torch.float16), _lib.ptr(idx), _lib.ptr(out),
        out.stride(0), _lib.ptr(ws), ws_bytes, _lib.stream_of(q)))
    return (out, idx) if routed > 0 else out


def topk_columns(vals, budget, *, front=0, tail=0):
    """Per row of vals [rows, n] (fp32): the `budget` columns of [front, n - tail) with the largest values (values
    <= 0 and NaN last, ties to the lower index), ascending int32 [rows, budget], -1 past the eligible count: the
    prio.topk(extra).indices.sort() of kv_evict (modal_rd/attention.py:251-252)."""
    if not vals.is_cuda:
        raise ValueError("topk_columns runs on the GPU")
    rows, n = vals.shape
    out = torch.empty(rows, budget, dtype=torch.int32, device=vals.device)
    if budget <= 0 or rows == 0:
        return out
    v = vals.to(torch.float32)
    v = v if v.stride(-1) == 1 else v.contiguous()
    L = _lib.lib()
    ws_bytes = L.bb_topk_f32_workspace(rows, n)
    ws = _lib.workspace(ws_bytes, vals.device)
    _lib.check(L.bb_topk_f32(_lib.ptr(v), v.stride(0), rows, n, int(front), int(tail), int(budget), _lib.ptr(out),
                             _lib.ptr(ws), ws_bytes, _lib.stream_of(v)))
    return out


_ARGMAX_KIND = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}


def argmax_index(x, out=None):
    """Index of the largest element of a 1-D GPU tensor (fp32 / bf16 / fp16) as an int64 [1] GPU tensor (written into
    `out` when given): torch.argmax semantics (NaN largest, first index on ties), one workgroup and no workspace, so
    a captured decode step needs no multi-workgroup reduction (modal_rd/graph_decode.py:201-202)."""
    if not x.is_cuda or x.ndim != 1 or x.dtype not in _ARGMAX_KIND:
        raise ValueError("argmax_index needs a 1-D fp32/bf16/fp16 GPU tensor")
    x = x if x.stride(0) == 1 else x.contiguous()
    if out is None:
        out = torch.empty(1, dtype=torch.int64, device=x.device)
    elif out.dtype != torch.int64 or out.numel() != 1 or not out.is_cuda:
        raise ValueError("argmax_index: out must be an int64 [1] GPU tensor")
    _lib.check(_lib.lib().bb_argmax(_lib.ptr(x), x.shape[0], _ARGMAX_KIND[x.dtype], _lib.ptr(out), _lib.stream_of(x)))
    return out


def _matrix16(x, d):
    """x as [rows, d] with 16-byte aligned rows (a copy only when x's layout does not allow it)."""
    x2 = x.reshape(-1, d)
    if x2.stride(-1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    return x2


def rms_norm(x, weight, eps):
    """transformers' LlamaRMSNorm on a 16-bit GPU tensor [..., D] in one launch (fp32 mean of squares,
    rsqrt(mean + eps), round to x's dtype, times `weight`, round); D % 8 == 0, D <= 8192."""
    if not x.is_cuda or x.dtype not in (torch.bfloat16, torch.float16) or weight.dtype != x.dtype:
        raise ValueError("rms_norm needs bf16/fp16 GPU tensors of one dtype")
    d = x.shape[-1]
    x2 = _matrix16(x, d)
    w = weight.contiguous()
    out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    _lib.check(_lib.lib().bb_rms_norm(_lib.ptr(x2), x2.stride(0), x2.shape[0], d, _lib.ptr(w), float(eps),
                                      int(x.dtype == torch.float16), _lib.ptr(out), d, _lib.stream_of(x)))
    return out


def add_rms_norm(x, res, weight, eps):
    """A decoder layer's residual add and the RMSNorm after it, in one launch: returns (x + res, rms_norm(x + res))
    with the arithmetic of the 16-bit tensor add and of transformers' LlamaRMSNorm (as `rms_norm`)."""
    if (not x.is_cuda or x.dtype not in (torch.bfloat16, torch.float16) or res.dtype != x.dtype
            or weight.dtype != x.dtype):
        raise ValueError("add_rms_norm needs bf16/fp16 GPU tensors of one dtype")
    if res.shape != x.shape:
        raise ValueError("add_rms_norm: x and res must have one shape")
    d = x.shape[-1]
    x2, r2 = _matrix16(x, d), _matrix16(res, d)
    w = weight.contiguous()
    total = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    _lib.check(_lib.lib().bb_add_rms_norm(_lib.ptr(x2), x2.stride(0), _lib.ptr(r2), r2.stride(0), x2.shape[0], d,
                                          _lib.ptr(w), float(eps), int(x.dtype == torch.float16), _lib.ptr(total), d,
                                          _lib.ptr(out), d, _lib.stream_of(x)))
    return total, out


def silu_mul(g, u):
    """F.silu(g) * u on 16-bit GPU tensors of one shape in one launch, with the arithmetic of those two torch ops
    (silu in fp32, rounded; the product in fp32, rounded): the gate of a Llama MLP."""
    if not g.is_cuda or g.dtype not in (torch.bfloat16, torch.float16) or u.dtype != g.dtype or u.shape != g.shape:
        raise ValueError("silu_mul needs bf16/fp16 GPU tensors of one dtype and shape")
    g2, u2 = g.contiguous(), u.contiguous()
    if g2.numel() % 8 or g2.data_ptr() % 16 or u2.data_ptr() % 16:
        raise ValueError("silu_mul: the length must be a multiple of 8 (16-byte aligned buffers)")
    out = torch.empty(g.shape, dtype=g.dtype, device=g.device)
    _lib.check(_lib.lib().bb_silu_mul(_lib.ptr(g2), _lib.ptr(u2), g2.numel(), int(g.dtype == torch.float16),
                                      _lib.ptr(out), _lib.stream_of(g)))
    return out


def gemv_ok(weight, x=None):
    """Whether `linear_vec` can run this weight (16-bit [N, K], K % 8 == 0, K <= 16384, 16-byte aligned rows) and,
    if given, this input's dtype."""
    return (weight.is_cuda and weight.dtype in (torch.bfloat16, torch.float16) and weight.ndim == 2
            and weight.stride(1) == 1 and weight.stride(0) % 8 == 0 and weight.data_ptr() % 16 == 0
            and 0 < weight.shape[1] <= 16384 and weight.shape[1] % 8 == 0 and (x is None or x.dtype == weight.dtype))


def linear_vec(x, weight, glu=False):
    """One token through a bias-free linear layer, y = x W^T (x [..., K] holding K values in all; y [..., M] for W
    [M, K]), as one HBM-streaming HIP launch. glu: W is a fused [gate; up] projection [2M, K] and y = silu(x gate^T) *
    (x up^T) with the rounding of those torch ops on 16-bit tensors (`silu_mul`'s arithmetic): a Llama MLP's
    activation input."""
    m, k = weight.shape
    if not gemv_ok(weight, x) or not x.is_cuda:
        raise ValueError("linear_vec needs a 16-bit GPU weight [N, K] (K % 8 == 0, K <= 16384, aligned rows) "
                         "and an input of its dtype")
    if x.numel() != k:
        raise ValueError("linear_vec takes one token: x must hold K values")
    if glu and m % 2:
        raise ValueError("linear_vec(glu=True) needs a [2N, K] gate / up weight")
    n = m // 2 if glu else m
    x1 = x.reshape(-1)
    if x1.data_ptr() % 16:
        x1 = x1.clone()
    y = torch.empty(x.shape[:-1] + (n,), dtype=x.dtype, device=x.device)
    _lib.check(_lib.lib().bb_gemv(_lib.ptr(weight), weight.stride(0), n, k, _lib.ptr(x1), int(glu),
                                  int(x.dtype == torch.float16), _lib.ptr(y), _lib.stream_of(x)))
    return y


def linear_vec_norm(x, res, norm_weight, eps, weight, glu=False):
    """`linear_vec` on the RMSNorm of one hidden row, in one launch: returns (x + res, linear_vec(rms_norm(x + res)))
    (res None: (x, linear_vec(rms_norm(x)))), bit-identical to add_rms_norm / rms_norm followed by linear_vec."""
    m, k = weight.shape
    if not gemv_ok(weight, x) or not x.is_cuda or k > 8192 or norm_weight.dtype != x.dtype:
        raise ValueError("linear_vec_norm needs a 16-bit GPU weight [N, K] (K % 8 == 0, K <= 8192, aligned rows), "
                         "an input and a norm weight of its dtype")
    if x.numel() != k or norm_weight.numel() != k or (res is not None and (res.numel() != k or res.dtype != x.dtype)):
        raise ValueError("linear_vec_norm takes one token: x, res and the norm weight must hold K values")
    if glu and m % 2:
        raise ValueError("linear_vec_norm(glu=True) needs a [2N, K] gate / up weight")
    n = m // 2 if glu else m

    def flat(t):
        t1 = t.reshape(-1)
        return t1 if t1.data_ptr() % 16 == 0 else t1.clone()

    x1, w1 = flat(x), flat(norm_weight)
    r1 = flat(res) if res is not None else None
    total = torch.empty_like(x) if res is not None else x
    y = torch.empty(x.shape[:-1] + (n,), dtype=x.dtype, device=x.device)
    _lib.check(_lib.lib().bb_gemv_norm(_lib.ptr(weight), weight.stride(0), n, k, _lib.ptr(x1),
                                       _lib.ptr(r1) if r1 is not None else None, _lib.ptr(w1), float(eps), int(glu),
                                       int(x.dtype == torch.float16), _lib.ptr(total) if r1 is not None else None,
                                       _lib.ptr(y), _lib.stream_of(x)))
    return total, y
