"""INT8 KV cache and exact decode on MI355X (drop-in for modal_rd/kv_int8.py and kernels/kv_int8_triton.py).

Symmetric per token and KV head: scale = max(absmax / 127, MIN_SCALE) in fp32, q = round_half_even(x / scale)
clamped to [-127, 127], scale stored as fp16 (the reference's format; `scale_dtype=torch.float32` keeps fp32).
Buffers are token-major [capacity, Hkv, d] (scales [capacity, Hkv, 1]) so the valid rows are one contiguous block and
decode appends into spare capacity (GROW rows at a time).

Decode differs from the reference in one place, by design: instead of dequantising the whole cache to bf16 and
running SDPA each step, `update` returns handles whose `attend` runs bb_decode, which reads the int8 rows and their
scales once (no dequantised copy). The math is the same exact attention over the dequantised values.
"""
import torch
from transformers import DynamicCache
from transformers.cache_utils import DynamicLayer

from . import _lib

MIN_SCALE = 1e-4
GROW = 256


def _scale_flag(scale_dtype):
    if scale_dtype == torch.float16:
        return 1
    if scale_dtype == torch.float32:
        return 0
    raise ValueError("scale dtype must be float16 or float32")


def _rows(x):
    """x [..., d] as (tensor, outer, inner, outer stride, inner stride) with 16-byte aligned rows (a copy otherwise)."""
    d = x.shape[-1]
    if x.ndim >= 3 and x.stride(-1) == 1:
        x3 = x.reshape(-1, x.shape[-2], d) if x.ndim > 3 else x
        if x.ndim > 3 and x3.data_ptr() != x.data_ptr():
            x3 = x.contiguous().view(-1, x.shape[-2], d)
        outer, inner = x3.shape[0], x3.shape[1]
        so, si = x3.stride(0), x3.stride(1)
    else:
        x3 = x.reshape(-1, d).contiguous()
        outer, inner, so, si = x3.shape[0], 1, x3.stride(0), 0
    el = x.element_size()
    if x3.data_ptr() % 16 or (so * el) % 16 or (si * el) % 16:
        x3 = x3.contiguous()
        so, si = (x3.stride(0), x3.stride(1)) if x3.ndim == 3 else (x3.stride(0), 0)
    return x3, outer, inner, so, si


def _outputs(x, out, scale_dtype):
    lead = x.shape[:-1]
    if out is None:
        out = (torch.empty(x.shape, device=x.device, dtype=torch.int8),
               torch.empty(*lead, 1, device=x.device, dtype=scale_dtype))
    q, s = out
    if not (q.is_contiguous() and s.is_contiguous()) or q.numel() != x.numel() or s.numel() * x.shape[-1] != x.numel():
        raise ValueError("quantize: out tensors must be contiguous and match x")
    return q, s


def quantize(x, out=None, scale_dtype=torch.float16, min_scale=MIN_SCALE):
    """[..., d] (bf16 or fp32, rows may be strided) -> int8 [..., d], scales [..., 1]; one row per leading index.

    `out` = (q, s): contiguous tensors to write into (e.g. the next rows of a cache buffer)."""
    _lib.require_gpu(x, what="quantize")
    if x.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("quantize: bf16 or fp32 input")
    q, s = _outputs(x, out, scale_dtype)
    x3, outer, inner, so, si = _rows(x)
    _lib.check(_lib.lib().bb_int8_quantize(_lib.ptr(x3), int(x.dtype == torch.float32), outer, so, inner, si,
                                           x.shape[-1], float(min_scale), _lib.ptr(q), _lib.ptr(s),
                                           _scale_flag(s.dtype), _lib.stream_of(x)))
    return q, s


def quantize_pair(xk, xv, out_k, out_v, scale_dtype=torch.float16, min_scale=MIN_SCALE):
    """quantize(xk, out_k) and quantize(xv, out_v) in one launch when the two inputs share shape, dtype and strides
    (a decode step's new K and V rows); two launches otherwise."""
    _lib.require_gpu(xk, xv, what="quantize")
    if xk.dtype not in (torch.bfloat16, torch.float32) or xv.dtype != xk.dtype or xv.shape != xk.shape:
        return quantize(xk, out_k, scale_dtype, min_scale), quantize(xv, out_v, scale_dtype, min_scale)
    (qk, sk), (qv, sv) = _outputs(xk, out_k, scale_dtype), _outputs(xv, out_v, scale_dtype)
    a, b = _rows(xk), _rows(xv)
    if a[1:] != b[1:] or sk.dtype != sv.dtype:
        return quantize(xk, (qk, sk), scale_dtype, min_scale), quantize(xv, (qv, sv), scale_dtype, min_scale)
    _, outer, inner, so, si = a
    _lib.check(_lib.lib().bb_int8_quantize_pair(
        _lib.ptr(a[0]), _lib.ptr(b[0]), int(xk.dtype == torch.float32), outer, so, inner, si, xk.shape[-1],
        float(min_scale), _lib.ptr(qk), _lib.ptr(sk), _lib.ptr(qv), _lib.ptr(sv), _scale_flag(sk.dtype),
        _lib.stream_of(xk)))
    return (qk, sk), (qv, sv)


def dequantize(q, scale, dtype):
    """int8 [..., d] * scale [..., 1] -> dtype (bf16 or fp32)."""
    _lib.require_gpu(q, scale, what="dequantize")
    if dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("dequantize: bf16 or fp32 output")
    q, scale = q.contiguous(), scale.contiguous()
    out = torch.empty(q.shape, device=q.device, dtype=dtype)
    rows = q.numel() // q.shape[-1]
    _lib.check(_lib.lib().bb_int8_dequantize(_lib.ptr(q), _lib.ptr(scale), _scale_flag(scale.dtype), rows, q.shape[-1],
                                             _lib.ptr(out), int(dtype == torch.float32), _lib.stream_of(q)))
    return out


def _decode(q, n, scale, *, k8=None, ks=None, v8=None, vs=None, kb=None, vb=None):
    _lib.require_gpu(q, what="decode")
    if q.dtype != torch.bfloat16:
        raise ValueError("decode: bf16 query")
    q = q.contiguous()
    h, d = q.shape
    hk = (k8 if k8 is not None else kb).shape[1 if k8 is not None else 0]
    out = torch.empty(h, d, dtype=torch.bfloat16, device=q.device)
    L = _lib.lib()
    ws_bytes = L.bb_decode_workspace(n, h, hk, d)
    ws = _lib.workspace(ws_bytes, q.device)
    if k8 is not None:
        args = (_lib.ptr(k8), _lib.ptr(ks), _lib.ptr(v8), _lib.ptr(vs), _scale_flag(ks.dtype), None, None, None, None)
    else:
        args = (None, None, None, None, 0, _lib.ptr(kb), _lib.i64s(kb.stride(0), kb.stride(1)), _lib.ptr(vb),
                _lib.i64s(vb.stride(0), vb.stride(1)))
    _lib.check(L.bb_decode(_lib.ptr(q), q.stride(0), *args, n, h, hk, d, float(scale), _lib.ptr(out), out.stride(0),
                           _lib.ptr(ws), ws_bytes, _lib.stream_of(q)))
    return out


def decode_int8(q, k8, ks, v8, vs, n, scale):
    """q [H, d] bf16 over the first n rows of an int8 cache k8/v8 [cap, Hkv, d] with scales [cap, Hkv, 1]."""
    _lib.require_gpu(k8, ks, v8, vs, what="decode_int8")
    return _decode(q, n, scale, k8=k8, ks=ks, v8=v8, vs=vs)


def decode_bf16(q, k, v, scale):
    """q [H, d] bf16 over k/v [Hkv, n, d] (strided views of a bf16 cache)."""
    _lib.require_gpu(k, v, what="decode_bf16")
    for x in (k, v):
        if x.stride(-1) != 1 or x.stride(0) % 8 or x.stride(1) % 8 or x.data_ptr() % 16:
            raise ValueError("decode_bf16: cache rows must be 16-byte aligned with a contiguous head_dim")
    return _decode(q, k.shape[1], scale, kb=k, vb=v)


class Int8Handle:
    """Stands in for the K / V tensors of one decode step; RDAttention.exact_attention calls `attend` (the same
    protocol as the reference's compressed-cache handle, modal_rd/turbo_kv.py:129-141)."""

    def __init__(self, layer, shape):
        self.turbo, self.shape = layer, shape

    def attend(self, q, scale):
        """q [1, H, 1, d] -> [1, H, 1, d] exact attention over the layer's whole int8 cache."""
        layer = self.turbo
        n = layer.n
        out = decode_int8(q[0, :, 0], layer.qk, layer.sk, layer.qv, layer.sv, n, scale)
        return out[None, :, None]


class Int8KVLayer(DynamicLayer):
    """HF cache layer with int8 storage (modal_rd/kv_int8.py:49-133). Batch size 1 only."""

    scale_dtype = torch.float16
    fused = True

    def lazy_initialization(self, key_states, value_states, *args, **kwargs):
        self.dtype, self.device = key_states.dtype, key_states.device
        self.qk = self.qv = self.sk = self.sv = None
        self.n = 0
        self.is_initialized = True

    def _quantize(self, x):  # [1, Hkv, t, d] -> [t, Hkv, d] int8, [t, Hkv, 1] scales
        if x.shape[0] != 1:
            raise NotImplementedError("Int8KVLayer is batch-size-1 only")
        return quantize(x[0].transpose(0, 1), scale_dtype=self.scale_dtype)

    def _get(self, q, s):  # -> [1, Hkv, n, d] view of the dequantised rows
        if q is None:
            return None
        return dequantize(q[:self.n], s[:self.n], self.dtype).transpose(0, 1)[None]

    @property
    def keys(self):
        return self._get(getattr(self, "qk", None), getattr(self, "sk", None))

    @keys.setter
    def keys(self, x):
        if x is not None and x.numel():
            self.qk, self.sk = self._quantize(x)
            self.n = x.shape[-2]

    @property
    def values(self):
        return self._get(getattr(self, "qv", None), getattr(self, "sv", None))

    @values.setter
    def values(self, x):
        if x is not None and x.numel():
            self.qv, self.sv = self._quantize(x)
            self.n = x.shape[-2]

    def _reserve(self, t):
        if self.n + t <= self.qk.shape[0]:
            return

        def grow(x):
            return torch.cat([x[:self.n], x.new_empty(max(t, GROW), *x.shape[1:])])

        self.qk, self.sk, self.qv, self.sv = map(grow, (self.qk, self.sk, self.qv, self.sv))

    def update(self, key_states, value_states, *args, **kwargs):
        if not self.is_initialized:
            self.lazy_initialization(key_states, value_states)
        t = key_states.shape[-2]
        if self.qk is None:  # prefill: store quantised, attend in full precision
            (self.qk, self.sk), (self.qv, self.sv) = self._quantize(key_states), self._quantize(value_states)
            self.n = t
            return key_states, value_states
        self._reserve(t)
        rows = slice(self.n, self.n + t)
        quantize_pair(key_states[0].transpose(0, 1), value_states[0].transpose(0, 1), (self.qk[rows], self.sk[rows]),
                      (self.qv[rows], self.sv[rows]), scale_dtype=self.scale_dtype)
        self.n += t
        if self.fused and t == 1:
            handle = Int8Handle(self, (1, self.qk.shape[1], self.n, self.qk.shape[2]))
            return handle, handle
        return self.keys, self.values

    def get_seq_length(self, *args, **kwargs):
        return 0 if not self.is_initialized or self.qk is None else self.n

    def crop(self, tokens_to_remove):
        if tokens_to_remove < 0 and self.get_seq_length():
            self.n = max(0, self.n + tokens_to_remove)
        elif tokens_to_remove:
            raise NotImplementedError("Int8KVLayer.crop supports negative token counts only")

    def batch_repeat_interleave(self, repeats):
        raise NotImplementedError("Int8KVLayer is batch-size-1 only")

    batch_select_indices = batch_repeat_interleave

    def nbytes(self):
        """Bytes of the valid rows (spare decode capacity, at most GROW rows, is not counted)."""
        if self.qk is None:
            return 0
        return sum(t[:self.n].numel() * t.element_size() for t in (self.qk, self.sk, self.qv, self.sv))


def make_int8_cache(config, fused=True, scale_dtype=torch.float16):
    cache = DynamicCache(config=config)
    n_layers = config.get_text_config(decoder=True).num_hidden_layers
    layers = []
    for _ in range(n_layers):
        layer = Int8KVLayer()
        layer.fused, layer.scale_dtype = fused, scale_dtype
        layers.append(layer)
    cache.layers = layers
    return cache
