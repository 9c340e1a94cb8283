"""INT8 KV cache and exact decode on MI355X (drop-in for modal_rd/kv_int8.py and kernels/kv_int8_triton.py).

Symmetric per token and KV head: scale = max(absmax / 127, MIN_SCALE) in fp32, q = round_half_even(x / scale)
clamped to [-127, 127], scale stored as fp16 (the reference's format; `scale_dtype=torch.float32` keeps fp32).
Rows are stored token-major [capacity, Hkv, d] (scales [capacity, Hkv, 1]), so the valid rows are one contiguous
block that the decode kernels stream and that a new token is appended to.

Decode differs from the reference in one place, by design. A consumer that opts in (RDAttention passes
`{"bb_attend": True}` as the cache kwargs of its update call) receives handles whose `attend` runs bb_decode over
the int8 rows and their scales, with no dequantised copy. Every other consumer, e.g. a stock HF attention module,
receives dequantised [1, Hkv, n, d] tensors as from the reference's layer. The math is the same exact attention
over the dequantised values.
"""
import torch
from transformers import DynamicCache
from transformers.cache_utils import DynamicLayer

from . import _lib

MIN_SCALE = 1e-4
GROW = 256


_KINDS = {torch.bfloat16: 0, torch.float32: 1, torch.float16: 2}  # element kinds of the quantise / dequantise ABI


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
    """[..., d] (bf16, fp16 or fp32, rows may be strided) -> int8 [..., d], scales [..., 1]; one row per leading
    index (the reference quantises whatever float dtype the model runs in, modal_rd/kv_int8.py:19-22).

    `out` = (q, s): contiguous tensors to write into (e.g. the next rows of a cache buffer)."""
    _lib.require_gpu(x, what="quantize")
    if x.dtype not in _KINDS:
        raise ValueError("quantize: bf16, fp16 or fp32 input")
    q, s = _outputs(x, out, scale_dtype)
    x3, outer, inner, so, si = _rows(x)
    _lib.check(_lib.lib().bb_int8_quantize(_lib.ptr(x3), _KINDS[x.dtype], outer, so, inner, si,
                                           x.shape[-1], float(min_scale), _lib.ptr(q), _lib.ptr(s),
                                           _scale_flag(s.dtype), _lib.stream_of(x)))
    return q, s


def quantize_pair(xk, xv, out_k, out_v, scale_dtype=torch.float16, min_scale=MIN_SCALE):
    """quantize(xk, out_k) and quantize(xv, out_v) in one launch when the two inputs share shape, dtype and strides
    (a decode step's new K and V rows); two launches otherwise."""
    _lib.require_gpu(xk, xv, what="quantize")
    if xk.dtype not in _KINDS or xv.dtype != xk.dtype or xv.shape != xk.shape:
        return quantize(xk, out_k, scale_dtype, min_scale), quantize(xv, out_v, scale_dtype, min_scale)
    (qk, sk), (qv, sv) = _outputs(xk, out_k, scale_dtype), _outputs(xv, out_v, scale_dtype)
    a, b = _rows(xk), _rows(xv)
    if a[1:] != b[1:] or sk.dtype != sv.dtype:
        return quantize(xk, (qk, sk), scale_dtype, min_scale), quantize(xv, (qv, sv), scale_dtype, min_scale)
    _, outer, inner, so, si = a
    _lib.check(_lib.lib().bb_int8_quantize_pair(
        _lib.ptr(a[0]), _lib.ptr(b[0]), _KINDS[xk.dtype], outer, so, inner, si, xk.shape[-1],
        float(min_scale), _lib.ptr(qk), _lib.ptr(sk), _lib.ptr(qv), _lib.ptr(sv), _scale_flag(sk.dtype),
        _lib.stream_of(xk)))
    return (qk, sk), (qv, sv)


def dequantize(q, scale, dtype):
    """int8 [..., d] * scale [..., 1] -> dtype (bf16, fp16 or fp32; the fp32 product rounded to nearest even)."""
    _lib.require_gpu(q, scale, what="dequantize")
    if dtype not in _KINDS:
        raise ValueError("dequantize: bf16, fp16 or fp32 output")
    q, scale = q.contiguous(), scale.contiguous()
    out = torch.empty(q.shape, device=q.device, dtype=dtype)
    rows = q.numel() // q.shape[-1]
    _lib.check(_lib.lib().bb_int8_dequantize(_lib.ptr(q), _lib.ptr(scale), _scale_flag(scale.dtype), rows, q.shape[-1],
                                             _lib.ptr(out), _KINDS[dtype], _lib.stream_of(q)))
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


def decode_int8_append(q, k8, ks, v8, vs, knew, vnew, n, scale, min_scale=MIN_SCALE):
    """One decode step over an int8 cache: the new token's K / V rows knew / vnew (bf16 [Hkv, d], any head stride)
    are quantised into cache row n - 1 (as quantize_pair would) and q [H, d] attends all n rows (as decode_int8).
    One kernel at d = 128 with 4 query heads per KV head (bb_decode_append)."""
    _lib.require_gpu(q, k8, ks, v8, vs, knew, vnew, what="decode_int8_append")
    if q.dtype != torch.bfloat16 or knew.dtype != torch.bfloat16 or vnew.dtype != torch.bfloat16:
        raise ValueError("decode_int8_append: bf16 query and new rows")
    if ks.dtype != vs.dtype or not (k8.is_contiguous() and v8.is_contiguous() and ks.is_contiguous()
                                    and vs.is_contiguous()):
        raise ValueError("decode_int8_append: contiguous int8 rows and scales of one dtype")
    if n > k8.shape[0]:
        raise ValueError("decode_int8_append: row n - 1 is past the cache capacity")
    hk, d = k8.shape[1], k8.shape[2]
    if tuple(knew.shape) != (hk, d) or tuple(vnew.shape) != (hk, d) or knew.stride(-1) != 1 or vnew.stride(-1) != 1:
        raise ValueError("decode_int8_append: new rows must be [Hkv, d] with a contiguous head_dim")
    q = q.contiguous()
    h = q.shape[0]
    out = torch.empty(h, d, dtype=torch.bfloat16, device=q.device)
    L = _lib.lib()
    ws_bytes = L.bb_decode_workspace(n, h, hk, d)
    ws = _lib.workspace(ws_bytes, q.device)
    _lib.check(L.bb_decode_append(_lib.ptr(q), q.stride(0), _lib.ptr(k8), _lib.ptr(ks), _lib.ptr(v8), _lib.ptr(vs),
                                  _scale_flag(ks.dtype), _lib.ptr(knew), knew.stride(0), _lib.ptr(vnew), vnew.stride(0),
                                  float(min_scale), n, h, hk, d, float(scale), _lib.ptr(out), out.stride(0),
                                  _lib.ptr(ws), ws_bytes, _lib.stream_of(q)))
    return out


def decode_bf16(q, k, v, scale):
    """q [H, d] bf16 over k/v [Hkv, n, d] (strided views of a bf16 cache)."""
    _lib.require_gpu(k, v, what="decode_bf16")
    if k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16:
        raise ValueError("decode_bf16: bf16 cache required")
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
        """q [1, H, 1, d] -> [1, H, 1, d] exact attention over the layer's whole int8 cache. The step's new row, when
        the layer still holds it unquantised, is quantised by the same kernel (decode_int8_append)."""
        layer = self.turbo
        k, v = layer.store_k, layer.store_v
        pending = layer._pending
        if pending is not None and pending[2] == layer.n - 1:
            layer._pending = None
            out = decode_int8_append(q[0, :, 0], k.q, k.s, v.q, v.s, pending[0], pending[1], layer.n, scale)
        else:
            layer._flush()
            out = decode_int8(q[0, :, 0], k.q, k.s, v.q, v.s, layer.n, scale)
        return out[None, :, None]


class _Int8Rows:
    """One cached tensor (K or V) as int8 rows [capacity, Hkv, d] plus scales [capacity, Hkv, 1]; rows [0, n) are
    valid (n is kept by the owning layer). Capacity comes in whole GROW-row steps past what is needed."""

    def __init__(self, hkv, d, rows, scale_dtype, device):
        cap = rows + GROW
        self.q = torch.empty(cap, hkv, d, dtype=torch.int8, device=device)
        self.s = torch.empty(cap, hkv, 1, dtype=scale_dtype, device=device)

    @property
    def capacity(self):
        return self.q.shape[0]

    def ensure(self, n, need):
        """Make room for rows [n, need), keeping rows [0, n)."""
        if need <= self.capacity:
            return
        cap = need + GROW
        q = torch.empty(cap, *self.q.shape[1:], dtype=self.q.dtype, device=self.q.device)
        s = torch.empty(cap, *self.s.shape[1:], dtype=self.s.dtype, device=self.s.device)
        q[:n].copy_(self.q[:n])
        s[:n].copy_(self.s[:n])
        self.q, self.s = q, s

    def rows(self, a, b):
        return self.q[a:b], self.s[a:b]

    def dequantized(self, n, dtype):
        """[1, Hkv, n, d] in `dtype` (a fresh tensor, viewed head-major like the reference's cache)."""
        return dequantize(self.q[:n], self.s[:n], dtype).transpose(0, 1)[None]

    def nbytes(self, n):
        return n * (self.q[0].numel() * self.q.element_size() + self.s[0].numel() * self.s.element_size())


class Int8KVLayer(DynamicLayer):
    """HF cache layer with int8 K/V storage (modal_rd/kv_int8.py:49-133), batch size 1.

    * prefill (the first update): the K/V are quantised into fresh row stores and the full-precision inputs are
      returned, so prefill attention is unchanged;
    * later updates quantise the new rows (K and V in one launch) into spare capacity and return the dequantised
      cache, or, for a one-token step whose consumer opts in, Int8Handle stand-ins for the fused decode;
    * assigning `keys` / `values` (kv_evict compacting the cache) re-quantises the given rows;
    * `crop(-r)` drops the last r rows.
    """

    scale_dtype = torch.float16
    fused = True  # hand handles to consumers that ask for them (cache kwargs {"bb_attend": True})

    def __init__(self):
        self._pending = None  # first: DynamicLayer.__init__ assigns keys / values, whose setters flush
        self.store_k = self.store_v = None
        super().__init__()
        self.store_k = self.store_v = None
        self.n = 0

    def lazy_initialization(self, key_states, value_states, *args, **kwargs):
        self.dtype, self.device = key_states.dtype, key_states.device
        self.store_k = self.store_v = None
        self.n = 0
        self._pending = None
        self.is_initialized = True

    def _flush(self):
        """Quantise a one-token step's rows still held for the fused decode (the handle was not attended)."""
        if self._pending is not None:
            kr, vr, row = self._pending
            self._pending = None
            quantize_pair(kr[None], vr[None], self.store_k.rows(row, row + 1),
                          self.store_v.rows(row, row + 1), scale_dtype=self.scale_dtype)

    @staticmethod
    def _token_major(x):
        """[1, Hkv, t, d] -> a [t, Hkv, d] view."""
        if x.ndim != 4 or x.shape[0] != 1:
            raise NotImplementedError("Int8KVLayer is batch-size-1 only")
        return x[0].transpose(0, 1)

    def _fill(self, x):
        """A new row store holding the quantised rows of x [1, Hkv, t, d]."""
        rows = self._token_major(x)
        t, hkv, d = rows.shape
        store = _Int8Rows(hkv, d, t, self.scale_dtype, x.device)
        quantize(rows, out=store.rows(0, t), scale_dtype=self.scale_dtype)
        return store

    # keys / values read back dequantised, as the reference's layer exposes them; assignment re-quantises
    @property
    def keys(self):
        self._flush()
        return None if self.store_k is None else self.store_k.dequantized(self.n, self.dtype)

    @keys.setter
    def keys(self, x):
        self._flush()
        if x is not None and x.numel():
            self.store_k, self.n = self._fill(x), x.shape[-2]

    @property
    def values(self):
        self._flush()
        return None if self.store_v is None else self.store_v.dequantized(self.n, self.dtype)

    @values.setter
    def values(self, x):
        self._flush()
        if x is not None and x.numel():
            self.store_v, self.n = self._fill(x), x.shape[-2]

    def update(self, key_states, value_states, cache_kwargs=None, *args, **kwargs):
        if not self.is_initialized:
            self.lazy_initialization(key_states, value_states)
        self._flush()
        t = key_states.shape[-2]
        if self.store_k is None:
            self.store_k, self.store_v = self._fill(key_states), self._fill(value_states)
            self.n = t
            return key_states, value_states
        start, end = self.n, self.n + t
        self.store_k.ensure(start, end)
        self.store_v.ensure(start, end)
        self.n = end
        wants_handle = isinstance(cache_kwargs, dict) and cache_kwargs.get("bb_attend", False)
        kr, vr = self._token_major(key_states), self._token_major(value_states)
        # the fused decode reads the new rows as 16-byte units: contiguous head_dim, 16-byte aligned rows and a head
        # stride of whole units (bb_decode_append's checks); anything else is quantised here
        if (self.fused and wants_handle and t == 1 and kr.dtype == torch.bfloat16 and vr.dtype == torch.bfloat16
                and all(x[0].stride(-1) == 1 and x[0].stride(0) % 8 == 0 and x[0].data_ptr() % 16 == 0
                        for x in (kr, vr))):
            # the row is quantised by the decode kernel when the handle is attended (or by _flush before any other
            # use of the cache)
            self._pending = (kr[0], vr[0], start)
            handle = Int8Handle(self, (1, self.store_k.q.shape[1], end, self.store_k.q.shape[2]))
            return handle, handle
        quantize_pair(kr, vr, self.store_k.rows(start, end), self.store_v.rows(start, end),
                      scale_dtype=self.scale_dtype)
        return self.keys, self.values

    def get_seq_length(self, *args, **kwargs):
        return self.n if self.is_initialized and self.store_k is not None else 0

    def crop(self, tokens_to_remove):
        self._flush()
        if tokens_to_remove > 0:
            raise NotImplementedError("Int8KVLayer.crop supports negative token counts only")
        if tokens_to_remove < 0 and self.get_seq_length():
            self.n = max(0, self.n + tokens_to_remove)

    def batch_repeat_interleave(self, repeats):
        raise NotImplementedError("Int8KVLayer is batch-size-1 only")

    def batch_select_indices(self, indices):
        raise NotImplementedError("Int8KVLayer is batch-size-1 only")

    def nbytes(self):
        """Bytes held by the valid rows of K and V with their scales; spare capacity is not counted."""
        self._flush()
        if self.store_k is None:
            return 0
        return self.store_k.nbytes(self.n) + self.store_v.nbytes(self.n)


def make_int8_cache(config, fused=True, scale_dtype=torch.float16):
    """A DynamicCache whose layers are Int8KVLayer (modal_rd/kv_int8.py:136-139). `fused=False` never hands out
    decode handles, even to consumers that ask for them."""
    cache = DynamicCache(config=config)
    layers = []
    for _ in range(config.get_text_config(decoder=True).num_hidden_layers):
        layer = Int8KVLayer()
        layer.fused, layer.scale_dtype = fused, scale_dtype
        layers.append(layer)
    cache.layers = layers
    return cache
