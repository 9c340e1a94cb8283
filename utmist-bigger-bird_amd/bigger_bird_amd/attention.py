"""RDAttention on MI355X: Bigger Bird v3 sparse prefill (drop-in for modal_rd/attention.py of the reference).

Same constructor keywords, `forward`/`routes`/`sparse_prefill`/`exact_attention` methods, `last_routes`, `kept` and
`install()` as the reference module; per layer and head the attended keys are
  * sink:       the first `sink` tokens,
  * local:      a causal window of `window` tokens,
  * vertical:   `vertical` key columns per head chosen by the mean (or max) softmax probability of `n_route` route
                queries (the last ones, or evenly spread),
  * exact_tail: the final `exact_tail` queries attend exactly.
Every step on the path runs in the HIP library: in-place RoPE (bb_rope_inplace), routing (bb_routes), the sparse
kernel (bb_sparse_flash, with V^T shared by the main pass and the tail), dense/exact attention through the same
kernel with window = n, and one-token decode (bb_decode, fused over int8 caches through the `attend` hook).
"""
import math

import torch
import torch.nn as nn

from . import _lib
from .decode import gather_rows, topk_columns
from .flash import bigger_bird_flash, exact_attention, transpose_v

ROPE_CHUNK = 8192


def rope_inplace(x, cos, sin, chunk=ROPE_CHUNK):
    """HF `apply_rotary_pos_emb` on x [b, h, t, d] in place, bit-identical (modal_rd/attention.py:51-60).

    One HIP launch over the whole tensor; `chunk` is accepted for signature compatibility (the kernel needs no
    transient buffers). cos/sin are [b, t, d] (or [t, d]) in x's dtype, bf16 or fp16."""
    _lib.require_gpu(x, cos, sin, what="rope_inplace")
    if x.dtype not in (torch.bfloat16, torch.float16) or cos.dtype != x.dtype or sin.dtype != x.dtype:
        raise ValueError("rope_inplace: bf16 or fp16 tensors of one dtype required")
    b, h, t, d = x.shape
    if cos.ndim == 2:
        cos, sin = cos[None], sin[None]
    cos, sin = cos.expand(b, t, d), sin.expand(b, t, d)
    if cos.stride(-1) != 1 or sin.stride(-1) != 1 or cos.stride() != sin.stride():
        cos, sin = cos.contiguous(), sin.contiguous()
    _lib.check(_lib.lib().bb_rope_inplace(_lib.ptr(x), _lib.i64s(*x.stride()[:3]), b, h, t, d, _lib.ptr(cos),
                                          _lib.ptr(sin), _lib.i64s(cos.stride(0), cos.stride(1)),
                                          int(x.dtype == torch.float16), _lib.stream_of(x)))
    return x


def vertical_budget(n, vertical, vertical_sqrt):
    """Fixed budget, or c*sqrt(n) (rounded to 64) when vertical_sqrt=c > 0 (modal_rd/attention.py:63-67)."""
    if vertical_sqrt > 0:
        return int(math.ceil(vertical_sqrt * math.sqrt(n) / 64) * 64)
    return vertical


def forward_pool(score, p, back=0):
    """[H, n] -> [H, n] span pooling of key scores (modal_rd/attention.py:70-75): key j takes the largest score among
    keys j - (p - 1) .. j + back (the row's ends clipped), so the p - 1 keys that continue a high-scoring key (the rest
    of a copied number or span) and the `back` keys leading up to it rank with it. p < 1 counts as 1."""
    before = max(p, 1) - 1
    padded = torch.nn.functional.pad(score[:, None], (before, back), value=-float("inf"))
    return torch.nn.functional.max_pool1d(padded, before + back + 1, stride=1)[:, 0]


def route_positions(n, r, mode, sink, window, device):
    """Absolute positions of the route queries (modal_rd/attention.py:150-155)."""
    if mode == "spread":
        return torch.linspace(sink + window, n - 1, r, device=device).long()
    return torch.arange(n - r, n, device=device)


def _flat_heads(x):
    """[B, Hh, T, d] -> a [B * Hh, T, d] view when the batch stride is Hh head strides (always for B = 1), else
    None."""
    b, hh, t, d = x.shape
    if b > 1 and x.stride(0) != hh * x.stride(1):
        return None
    return x.as_strided((b * hh, t, d), (x.stride(1), x.stride(2), x.stride(3)), x.storage_offset())


def routes(q, k, *, num_heads, num_kv_heads, sink, window, budget, n_route=64, route_pool="mean",
           route_queries="last", scaling, return_pooled=False):
    """Per-head top-`budget` key columns by pooled softmax probability of the route queries.

    q [B, H, n, d], k [B, Hkv, n, d] (strided views are fine; for B > 1 the batch stride must be H head strides).
    Returns int32 [B * H, budget], ascending per head (and the pooled scores [B * H, n] as float probabilities
    when `return_pooled`)."""
    _lib.require_gpu(q, k, what="routes")
    if q.dtype not in (torch.bfloat16, torch.float16) or k.dtype != q.dtype:
        # the reference runs routes() in the model dtype (modal_rd/attention.py:164): bf16 or fp16 scores
        raise ValueError("routes: bf16 or fp16 q and k of one dtype required")
    bsz = q.shape[0]
    n, d = k.shape[-2], k.shape[-1]
    r = min(n_route, n)
    qpos = route_positions(n, r, route_queries, sink, window, q.device).to(torch.int64).contiguous()
    Q, K = _flat_heads(q), _flat_heads(k)
    if Q is None or K is None:
        raise ValueError("routes: batched q / k need a batch stride of H head strides")
    if Q.stride(-1) != 1 or Q.stride(0) % 8 or Q.stride(1) % 8 or Q.data_ptr() % 16:
        Q = Q.contiguous()
    if K.stride(-1) != 1 or K.stride(0) % 8 or K.stride(1) % 8 or K.data_ptr() % 16:
        K = K.contiguous()
    idx = torch.empty(bsz * num_heads, budget, dtype=torch.int32, device=q.device)
    pooled = torch.empty(bsz * num_heads, n, dtype=torch.int64, device=q.device) if return_pooled else None
    L = _lib.lib()
    ws_bytes = L.bb_routes_workspace(n, num_heads, num_kv_heads, bsz, r)
    ws = _lib.workspace(ws_bytes, q.device)
    _lib.check(L.bb_routes(_lib.ptr(Q), _lib.i64s(Q.stride(0), Q.stride(1)), _lib.ptr(K),
                           _lib.i64s(K.stride(0), K.stride(1)), _lib.ptr(qpos), r, bsz, num_heads, num_kv_heads, n, d,
                           int(q.dtype == torch.float16), sink, window, budget, float(scaling), int(route_pool == "max"),
                           _lib.ptr(idx) if budget else None, _lib.ptr(pooled), _lib.ptr(ws), ws_bytes,
                           _lib.stream_of(q)))
    if not return_pooled:
        return idx
    # fixed point (units of 2^-40, summed over r rows for mean pooling) -> probabilities
    prob = pooled.to(torch.float64) * 2.0 ** -40  # values < 2^63: int64 storage is exact
    if route_pool == "mean":
        prob = prob / r
    return idx, prob.to(torch.float32)


class RDAttention(nn.Module):
    def __init__(self, base, *, sink=64, window=4096, vertical=2048, vertical_sqrt=0.0,
                 n_route=64, route_pool="mean", route_queries="last", exact_tail=0,
                 vertical_scope=0, scope_chunk=4096, kv_evict=False, evict_keep=0, evict_pool=0, evict_obs=0,
                 evict_obs_max=False, evict_pool_back=0, evict_window=0, evict_full_layers=0, dense=False,
                 block_m=64, block_n=64, num_warps=4, num_stages=2):
        super().__init__()
        cfg = base.config
        self.layer_idx = base.layer_idx
        self.head_dim = base.head_dim
        self.num_heads = cfg.num_attention_heads
        self.num_kv_heads = cfg.num_key_value_heads
        self.groups = self.num_heads // self.num_kv_heads
        self.scaling = base.scaling
        self.q_proj, self.k_proj, self.v_proj, self.o_proj = base.q_proj, base.k_proj, base.v_proj, base.o_proj
        self.sink, self.window, self.vertical, self.vertical_sqrt = sink, window, vertical, vertical_sqrt
        if route_pool not in ("mean", "max"):
            raise ValueError("route_pool must be mean or max")
        self.n_route, self.route_pool, self.dense, self.block_m, self.block_n = n_route, route_pool, dense, block_m, block_n
        if route_queries not in ("last", "spread"):
            raise ValueError("route_queries must be last or spread")
        if scope_chunk % block_m or scope_chunk & (scope_chunk - 1):
            raise ValueError("scope_chunk must be a power of two multiple of block_m")
        self.exact_tail, self.route_queries = exact_tail, route_queries
        self.vertical_scope, self.scope_chunk = vertical_scope, scope_chunk
        self.num_warps, self.num_stages = num_warps, num_stages
        self.kv_evict = kv_evict
        self.evict_keep, self.evict_pool, self.evict_obs = evict_keep, evict_pool, evict_obs
        self.evict_full_layers, self.evict_window = evict_full_layers, evict_window
        self.evict_obs_max, self.evict_pool_back = evict_obs_max, evict_pool_back
        self.last_routes = None
        self.kept = None  # after kv_evict: int64 [Hkv, m], per KV head the sequence positions of the rows kept
        self._col = None

    def forward(self, hidden_states, position_embeddings=None, attention_mask=None, past_key_values=None, **kwargs):
        b, t, _ = hidden_states.shape
        q = self.q_proj(hidden_states).view(b, t, self.num_heads, self.head_dim).transpose(1, 2)
        k = self.k_proj(hidden_states).view(b, t, self.num_kv_heads, self.head_dim).transpose(1, 2)
        v = self.v_proj(hidden_states).view(b, t, self.num_kv_heads, self.head_dim).transpose(1, 2)
        if torch.is_grad_enabled() and q.requires_grad:
            return self._forward_autograd(q, k, v, position_embeddings, past_key_values)
        q, k = rope_inplace(q, *position_embeddings), rope_inplace(k, *position_embeddings)
        if past_key_values is not None:
            # the cache kwargs tell an Int8KVLayer that this module takes fused decode handles (exact_attention)
            k, v = past_key_values.update(k, v, self.layer_idx, {"bb_attend": True})
        n = k.shape[-2]
        if b != 1:
            raise ValueError("batch size 1 only")
        if self.dense or t < n or n <= self.sink + self.window:
            out = self.exact_attention(q, k, v, t, n)
        else:
            out = self.sparse_prefill(q, k, v)
            if self.kv_evict and past_key_values is not None:
                self.evict(past_key_values, q, k, v)
        out = out.transpose(1, 2).reshape(b, t, -1)
        return self.o_proj(out), None

    def _forward_autograd(self, q, k, v, position_embeddings, past_key_values):
        """forward with autograd on, as the reference takes it (modal_rd/attention.py:118-119, 127-129, 140-141): RoPE
        out of place (HF apply_rotary_pos_emb), and the exact layers (dense, cached decode, short prompts) through
        torch's differentiable SDPA, so they backpropagate. The sparse prefill has no backward here, as the
        reference's Triton kernel has none: it runs the HIP path on detached tensors and its output carries no
        gradient to q, k and v."""
        import torch.nn.functional as F
        from transformers.models.llama.modeling_llama import apply_rotary_pos_emb

        _lib.lib()  # the HIP library is required in every mode
        b, _, t, _ = q.shape
        q, k = apply_rotary_pos_emb(q, k, *position_embeddings)
        if past_key_values is not None:
            k, v = past_key_values.update(k, v, self.layer_idx)
        n = k.shape[-2]
        if b != 1:
            raise ValueError("batch size 1 only")
        if self.dense or t < n or n <= self.sink + self.window:
            out = F.scaled_dot_product_attention(q, k, v, is_causal=t == n and t > 1, scale=self.scaling,
                                                 enable_gqa=True)
        else:
            with torch.no_grad():
                qd, kd, vd = q.detach(), k.detach(), v.detach()
                out = self.sparse_prefill(qd, kd, vd)
                if self.kv_evict and past_key_values is not None:
                    self.evict(past_key_values, qd, kd, vd)
        out = out.transpose(1, 2).reshape(b, t, -1)
        return self.o_proj(out), None

    def exact_attention(self, q, k, v, t, n):
        """Exact attention: t == n causal prefill, or t < n over all n cached keys (modal_rd/attention.py:137-141)."""
        if getattr(k, "turbo", None) is not None:      # compressed KV cache handle, one decode token
            return k.attend(q, self.scaling)
        if t == n:
            none = torch.full((self.num_heads, 1, 1), -1, dtype=torch.int32, device=q.device)
            return bigger_bird_flash(q[0], k[0], v[0], none, front=0, window=n, num_heads=self.num_heads,
                                     kv_groups=self.groups, scale=self.scaling)[None]
        if t == 1 and q.dtype == torch.bfloat16 and self.head_dim in (64, 128) and self.groups in (1, 2, 4, 8):
            from .kv_int8 import decode_bf16
            return decode_bf16(q[0, :, 0], k[0], v[0], self.scaling)[None, :, None]
        # 1 < t < n, or a decode step the decode kernel does not take (head_dim 32, fp16, other group counts): every
        # query attends every cached key (the reference's non-causal SDPA), one launch
        return exact_attention(q[0], k[0], v[0], num_heads=self.num_heads, kv_groups=self.groups,
                               scale=self.scaling)[None]

    def routes(self, q, k):
        """Per-head top-V key columns by mean (or max) softmax prob of the route queries (HIP, deterministic)."""
        n = k.shape[-2]
        budget = min(vertical_budget(n, self.vertical, self.vertical_sqrt), max(0, n - self.sink - self.window))
        res = routes(q, k, num_heads=self.num_heads, num_kv_heads=self.num_kv_heads, sink=self.sink,
                     window=self.window, budget=budget, n_route=self.n_route, route_pool=self.route_pool,
                     route_queries=self.route_queries, scaling=self.scaling, return_pooled=self.kv_evict)
        if self.kv_evict:
            idx, col = res
            col[:, :self.sink] = -1
            col[:, n - self.window:] = -1
            self._col = col
            return idx
        return res

    def sparse_prefill(self, q, k, v):
        """Routes, then the sink + window + routed pass over rows < n - exact_tail and the exact tail written in
        place (modal_rd/attention.py:176-206). B > 1 (BASELINE's short-context arm; the reference reads q[0] only) runs
        as one batch of B * H heads per launch when the batch strides allow it, else one call per element; parity is
        per element, and last_routes is then [B, H, budget]."""
        bsz = q.shape[0]
        Q, K, V = _flat_heads(q), _flat_heads(k), _flat_heads(v)
        if bsz > 1 and (Q is None or K is None or V is None or self.kv_evict):
            outs, routes = [], []
            for i in range(bsz):
                outs.append(self.sparse_prefill(q[i:i + 1], k[i:i + 1], v[i:i + 1]))
                routes.append(self.last_routes)
            self.last_routes = torch.stack(routes)
            return torch.cat(outs)
        n = k.shape[-2]
        idx = self.routes(q, k)
        self.last_routes = idx if bsz == 1 else idx.view(bsz, self.num_heads, -1)
        bh = bsz * self.num_heads
        vt = transpose_v(V)
        flash = dict(num_heads=self.num_heads, kv_groups=self.groups, scale=self.scaling,
                     block_m=self.block_m, block_n=self.block_n, num_warps=self.num_warps, num_stages=self.num_stages)
        if self.vertical_scope:
            chunk = self.scope_chunk
            groups = -(-n // chunk)
            starts = torch.arange(groups, device=q.device) * chunk
            active = (starts + chunk > n - self.vertical_scope)[None, :, None]
            routed = torch.where(active, idx[:, None, :], torch.full_like(idx[:, None, :], -1))
        else:
            chunk, routed = None, idx.view(bh, 1, -1)
        r = min(self.exact_tail, n)
        out = bigger_bird_flash(Q, K, V, routed.contiguous(), front=self.sink, window=self.window, token_mask=None,
                                route_chunk=chunk, row_end=n - r, vt=vt, **flash)
        if r:
            # Final r queries attend exactly (window = n): written straight into the output rows.
            none = torch.full((bh, 1, 1), -1, dtype=torch.int32, device=q.device)
            bigger_bird_flash(Q[:, n - r:], K, V, none, front=0, window=n, token_mask=None, route_chunk=None, vt=vt,
                              out=out[:, n - r:], **flash)
        return out.unflatten(0, (bsz, self.num_heads))

    def evict_scores(self, q, k):
        """[Hkv, n] importance of every key for the last `evict_obs` queries (modal_rd/attention.py:209-224): exact
        fp32 softmax of each of those queries, pooled over the queries by mean (max with `evict_obs_max`), then the
        max over the KV head's query heads."""
        n = k.shape[-2]
        obs = min(self.evict_obs, n)
        pos = torch.arange(n, device=q.device)
        future = pos[None, :] > pos[n - obs:, None]  # [obs, n]: keys after the query
        per_kv = []
        for kvh in range(self.num_kv_heads):
            heads = q[0, kvh * self.groups:(kvh + 1) * self.groups, n - obs:, :]  # [g, obs, d]
            logits = torch.matmul(heads, k[0, kvh].transpose(-1, -2)).float() * self.scaling
            probs = logits.masked_fill(future, -float("inf")).softmax(-1)  # [g, obs, n]
            pooled = probs.amax(1) if self.evict_obs_max else probs.mean(1)
            per_kv.append(pooled.amax(0))
        return torch.stack(per_kv)

    def evict(self, cache, q, k, v):
        """Compact this layer's cache to the keys the sparse pattern can use (modal_rd/attention.py:226-259): the sink,
        the recent window (at least `evict_window`), and per KV head the routed columns of its query heads, topped
        up to `max(evict_keep, g * budget)` middle slots with the best-scoring remaining columns."""
        n, d = k.shape[-2], k.shape[-1]
        hk, g = self.num_kv_heads, self.groups
        routes, pooled = self.last_routes, self._col
        self._col = None
        if self.layer_idx < self.evict_full_layers:
            self.kept = torch.arange(n, device=k.device).expand(hk, n)
            return
        routed = torch.zeros(self.num_heads, n, dtype=torch.bool, device=k.device)
        routed.scatter_(1, routes.long(), True)
        routed = routed.view(hk, g, n).any(1)
        score = self.evict_scores(q, k) if self.evict_obs else pooled.view(hk, g, n).amax(1)
        if self.evict_pool > 1 or self.evict_pool_back:
            score = forward_pool(score, self.evict_pool, self.evict_pool_back)
        recent = min(max(self.window, self.evict_window), n - self.sink)
        priority = routed.float() * 2 + score  # routed columns first, then by score (>= 0 on [sink, n - recent))
        slots = g * routes.shape[-1]
        if self.evict_keep:
            slots = max(self.evict_keep, slots)
        slots = min(slots, n - self.sink - recent)
        # the top-`slots` middle columns, ascending (HIP top-k over [sink, n - recent)), then the HIP row gather
        middle = topk_columns(priority, slots, front=self.sink, tail=recent).long()
        every = torch.arange(n, device=k.device)
        kept = torch.cat([every[:self.sink].expand(hk, -1), middle, every[n - recent:].expand(hk, -1)], dim=1)
        layer = cache.layers[self.layer_idx]
        layer.keys, layer.values = gather_rows(k[0], kept)[None], gather_rows(v[0], kept)[None]
        self.kept = kept


def install(model, arm, dense_layers=(), **kw):
    """Replace every decoder layer's attention by RDAttention (modal_rd/attention.py:262-270). Layers listed in
    `dense_layers`, or all layers for arm "dense_rd", run exact attention. Re-installing reuses the original module."""
    for i, layer in enumerate(model.model.layers):
        original = getattr(layer.self_attn, "_rd_base", layer.self_attn)
        wrapped = RDAttention(original, dense=(arm == "dense_rd" or i in dense_layers), **kw)
        wrapped._rd_base = original
        layer.self_attn = wrapped
    return model
