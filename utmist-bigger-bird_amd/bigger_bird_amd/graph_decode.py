"""HIP-graph greedy decode for Llama-family models at batch 1 (drop-in for modal_rd/graph_decode.py).

Prefill is an ordinary eager forward through the installed attention modules. Decode is one token step assembled by
hand (embedding -> every decoder layer -> final norm -> lm_head -> greedy choice) over fixed-capacity per-layer K/V
buffers [Hkv, capacity, d]. The cache length, the write slot, the RoPE position, the input token and the step counter
live in GPU tensors, so the step is captured once as a HIP graph (torch.cuda.CUDAGraph) and replayed per token.

* Attention per layer: split-K flash decoding over the filled buffer (bigger_bird_decode with front=0,
  window=capacity and no routes, reading the length on the GPU), as the reference does for its dense / v3 / v3 +
  eviction arms. `sparse_decode={"front", "window", "routed"}` switches the RDAttention layers that are not dense to
  fused decode routing (bigger_bird_route, pooled per KV head) + sparse decode.
* The greedy choice is a one-workgroup HIP argmax and new K/V rows go in with index_copy_ at the device-side slot:
  the captured step holds no multi-workgroup reduction and no memset node.
* On a bf16 model the RMSNorms (`bb_rms_norm`, HF LlamaRMSNorm arithmetic) and RoPE (`bb_rope_inplace`, bit-identical
  to HF apply_rotary_pos_emb) run as one launch each instead of the handful of elementwise launches of the HF
  modules, which at batch 1 cost more than their arithmetic.
* With kv_evict the prefill runs on a DynamicCache (evicted layer by layer) and the kept rows are copied into the
  buffers afterwards; otherwise the prefill writes straight into them (BufferLayer), so there is one cache copy.
* Not supported, as in the reference: the INT8 KV cache, batch > 1, sampling. The reference's compressed-cache
  (turbo) and host-embedding variants are not part of this package.
* Generation runs in blocks of `block` steps and stops after the block that produced an EOS; the cache is rewound to
  just after the input that produced it, so a further turn can be appended (`feed` + `run`).
* The decoder's tensors are ordinary tensors (made outside inference mode) and the step runs and is captured under
  no_grad: a capture under inference mode would leave the CUDA generator's graph state as inference tensors, and any
  later capture outside inference mode would then fail.
"""
import time

import torch
from transformers import DynamicCache
from transformers.cache_utils import DynamicLayer
from transformers.models.llama.modeling_llama import apply_rotary_pos_emb

from .attention import rope_inplace
from .decode import argmax_index, bigger_bird_decode, bigger_bird_route, rms_norm


class BufferLayer(DynamicLayer):
    """Cache layer over preallocated [Hkv, capacity, d] buffers: prefill rows are written in place and `keys` /
    `values` are [1, Hkv, n, d] views of the filled part (modal_rd/graph_decode.py:40-57)."""

    def __init__(self, kb, vb):
        super().__init__()
        self.kb, self.vb, self.n = kb, vb, 0
        self.dtype, self.device, self.is_initialized = kb.dtype, kb.device, True
        self._views()

    def _views(self):
        self.keys, self.values = self.kb[None, :, :self.n], self.vb[None, :, :self.n]

    def update(self, key_states, value_states, *args, **kwargs):
        end = self.n + key_states.shape[-2]
        if end > self.kb.shape[1]:
            raise ValueError("graph decode buffer too small for the prompt")
        self.kb[:, self.n:end].copy_(key_states[0])
        self.vb[:, self.n:end].copy_(value_states[0])
        self.n = end
        self._views()
        return self.keys, self.values


class StaticDecoder:
    """Fixed-shape one-token decoder over per-layer K/V buffers (modal_rd/graph_decode.py:65-269)."""

    _STATE = ("length", "position", "token", "step_i")

    def __init__(self, model, capacity, sparse_decode=None):
        cfg = model.config
        self.model, self.capacity = model, int(capacity)
        self.layers = model.model.layers
        self.h, self.hk = cfg.num_attention_heads, cfg.num_key_value_heads
        self.d = getattr(self.layers[0].self_attn, "head_dim", cfg.hidden_size // self.h)
        w = model.lm_head.weight
        dev = w.device
        dt = w.dtype if w.dtype in (torch.float16, torch.bfloat16) else torch.bfloat16
        with torch.inference_mode(False):
            self.k = [torch.zeros(self.hk, self.capacity, self.d, device=dev, dtype=dt) for _ in self.layers]
            self.v = [torch.zeros_like(x) for x in self.k]
            self.length = torch.zeros(1, dtype=torch.long, device=dev)     # filled cache slots
            self.position = torch.zeros(1, dtype=torch.long, device=dev)   # RoPE position of the next input token
            self.token = torch.zeros(1, 1, dtype=torch.long, device=dev)   # next input token
            self.step_i = torch.zeros(1, dtype=torch.long, device=dev)     # tokens produced since load
            self.out = torch.zeros(self.capacity, dtype=torch.long, device=dev)
            self.no_routes = torch.empty(self.hk, 0, dtype=torch.long, device=dev)
        self.logits = None   # last step's logits [vocab] (inside the graph's memory once captured)
        self.graph = None
        self.sparse_cfg = dict(sparse_decode) if sparse_decode else None
        if self.sparse_cfg and set(self.sparse_cfg) != {"front", "window", "routed"}:
            raise ValueError("sparse_decode takes front, window and routed")
        self.sparse = [bool(self.sparse_cfg) and not getattr(layer.self_attn, "dense", True) for layer in self.layers]

    def buffer_cache(self):
        """A DynamicCache whose layers write the prefill's K/V straight into this decoder's buffers."""
        cache = DynamicCache(config=self.model.config)
        cache.layers = [BufferLayer(k, v) for k, v in zip(self.k, self.v)]
        return cache

    @torch.no_grad()
    def load(self, cache, prompt_len, first_token):
        """Take a prefilled cache (a `buffer_cache()` or a DynamicCache, e.g. after eviction) and set the first
        input token; `prompt_len` is the RoPE position of that token."""
        layers = getattr(cache, "layers", None)
        if not layers or not all(isinstance(x, DynamicLayer) and torch.is_tensor(x.keys) for x in layers) \
                or layers[0].keys.dtype != self.k[0].dtype:
            raise ValueError("graph decode needs a BF16/FP16 DynamicCache (INT8 KV cache is not supported)")
        m = layers[0].keys.shape[-2]
        if m >= self.capacity:
            raise ValueError("graph decode buffer too small")
        for i, layer in enumerate(layers):
            if layer.keys.shape[-2] != m:
                raise ValueError("all layers must hold the same number of cached keys")
            if layer.keys.data_ptr() != self.k[i].data_ptr():
                self.k[i][:, :m].copy_(layer.keys[0])
                self.v[i][:, :m].copy_(layer.values[0])
        self.length.fill_(m)
        self.position.fill_(prompt_len)
        self.step_i.zero_()
        self.feed(first_token)

    @torch.no_grad()
    def feed(self, token):
        """Set the next input token (a prompt continuation or a generated token)."""
        self.token.fill_(int(token))

    def attention(self, i, attn, q):
        """q [H, d] of the new token, whose K/V row is already in the buffers -> [H, d]."""
        K, V = self.k[i], self.v[i]
        if not self.sparse[i]:
            return bigger_bird_decode(q, K, V, self.no_routes, front=0, window=self.capacity, scale=attn.scaling,
                                      n=self.length)
        c = self.sparse_cfg
        idx = bigger_bird_route(q, K, c["routed"], front=c["front"], window=c["window"], scale=attn.scaling,
                                n=self.length)
        return bigger_bird_decode(q, K, V, idx, front=c["front"], window=c["window"], scale=attn.scaling,
                                  n=self.length)

    @staticmethod
    def _norm(module, x):
        """A Llama RMSNorm module applied to x, in one launch when it is the plain bf16/fp16 module."""
        w, eps = getattr(module, "weight", None), getattr(module, "variance_epsilon", None)
        if type(module).__name__.endswith("RMSNorm") and w is not None and eps is not None and w.dtype == x.dtype \
                and x.dtype in (torch.bfloat16, torch.float16) and x.shape[-1] % 8 == 0 and x.shape[-1] <= 8192:
            return rms_norm(x, w, eps)
        return module(x)

    def step(self):
        """One greedy token. Every shape is fixed and all state lives in GPU tensors (capturable)."""
        core = self.model.model
        hid = core.embed_tokens(self.token)
        cos, sin = core.rotary_emb(hid, self.position[None])
        slot = self.length.clone()
        self.length.add_(1)
        for i, layer in enumerate(self.layers):
            attn = layer.self_attn
            base = getattr(attn, "_rd_base", attn)
            x = self._norm(layer.input_layernorm, hid)
            q = base.q_proj(x).view(1, 1, self.h, self.d).transpose(1, 2)
            k = base.k_proj(x).view(1, 1, self.hk, self.d).transpose(1, 2)
            v = base.v_proj(x).view(1, 1, self.hk, self.d).transpose(1, 2)
            if q.dtype == torch.bfloat16 and cos.dtype == torch.bfloat16:
                rope_inplace(q, cos, sin)
                rope_inplace(k, cos, sin)
            else:
                q, k = apply_rotary_pos_emb(q, k, cos, sin)
            self.k[i].index_copy_(1, slot, k[0])
            self.v[i].index_copy_(1, slot, v[0])
            o = self.attention(i, attn, q[0, :, 0])
            hid = hid + base.o_proj(o.reshape(1, 1, -1))
            hid = hid + layer.mlp(self._norm(layer.post_attention_layernorm, hid))
        self.logits = self.model.lm_head(self._norm(core.norm, hid))[0, -1]
        nxt = argmax_index(self.logits)
        self.out.index_copy_(0, self.step_i, nxt)
        self.token.copy_(nxt.view(1, 1))
        self.position.add_(1)
        self.step_i.add_(1)

    def _state(self):
        return [getattr(self, n).clone() for n in self._STATE]

    def _restore(self, saved):
        for n, x in zip(self._STATE, saved):
            getattr(self, n).copy_(x)

    def capture(self):
        """Record `step` as a HIP graph; the decoder state is restored around the warm-up and capture runs. Runs
        outside inference mode (even when called inside it), under no_grad."""
        with torch.inference_mode(False), torch.no_grad():
            saved = self._state()
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                for _ in range(2):  # library handles and allocator pools warmed outside the capture
                    self.step()
                    self._restore(saved)
            torch.cuda.current_stream().wait_stream(side)
            self.graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(self.graph):
                self.step()
            self._restore(saved)

    @torch.no_grad()
    def run(self, steps, graph=True):
        """Advance `steps` tokens, each consuming the current input token and producing the next. Raises ValueError
        (one host read of the length) when the buffers cannot hold `steps` more rows."""
        if int(self.length) + steps > self.capacity:
            raise ValueError("graph decode buffer full: build the decoder with a larger capacity")
        if graph and self.graph is None:
            self.capture()
        for _ in range(steps):
            if graph:
                self.graph.replay()
            else:
                self.step()

    def generated(self):
        """Every token produced since `load`, as a Python list."""
        return self.out[:int(self.step_i)].tolist()

    @torch.no_grad()
    def rewind(self, r):
        """Drop the last `r` consumed tokens from the cache (steps run past an EOS)."""
        for t in (self.length, self.position, self.step_i):
            t.sub_(r)

    @torch.no_grad()
    def generate(self, max_steps, eos=(), block=8, graph=True):
        """Greedy steps until a produced token is in `eos` (kept) or `max_steps`; returns (tokens, steps run). The
        cache is rewound to end right after the input that produced the EOS, which becomes the next input."""
        eos = set(eos)
        start, steps, toks = int(self.step_i), 0, []
        while steps < max_steps:
            b = min(block, max_steps - steps)
            self.run(b, graph)
            new = self.out[start + steps:start + steps + b].tolist()
            steps += b
            toks += new
            if eos.intersection(new):
                break
        cut = next((j + 1 for j, t in enumerate(toks) if t in eos), len(toks))
        if steps > cut:
            self.rewind(steps - cut)
            self.feed(toks[cut - 1])
        return toks[:cut], steps


_DECODERS = {}


def _evicting(model):
    return any(getattr(layer.self_attn, "kv_evict", False) for layer in model.model.layers)


def _key(model, sparse_decode=None):
    sd = tuple(sorted(sparse_decode.items())) if sparse_decode else ()
    return tuple(id(layer.self_attn) for layer in model.model.layers) + (sd,)


def decoder_for(model, capacity, sparse_decode=None):
    """The cached decoder of the installed attention modules, rebuilt when it is too small."""
    key = _key(model, sparse_decode)
    dec = _DECODERS.get(key)
    if dec is None or dec.capacity < capacity:
        _DECODERS.clear()
        dec = None
        torch.cuda.empty_cache()
        dec = _DECODERS[key] = StaticDecoder(model, capacity, sparse_decode)
    return dec


@torch.inference_mode()
def graph_prefill(model, input_ids, max_new, headroom=4096, position_offset=0, sparse_decode=None):
    """Eager prefill of input_ids [1, n], loaded into a (cached) StaticDecoder. Returns (decoder, prefill output,
    prefill seconds); the argmax of the output's last logits is already the decoder's next input. The capacity
    covers the kept cache plus `max_new` tokens; `headroom` extra slots let slightly longer prompts reuse the graph."""
    n = input_ids.shape[1]
    key = _key(model, sparse_decode)
    if _DECODERS and key not in _DECODERS:  # another arm's buffers: free them before this prefill
        _DECODERS.clear()
        torch.cuda.empty_cache()
    if _evicting(model):
        dec, cache = None, DynamicCache(config=model.config)
    else:
        dec = decoder_for(model, n + max_new + 8, sparse_decode)
        cache = dec.buffer_cache()
    pos = torch.arange(position_offset, position_offset + n, device=input_ids.device)[None]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    out = model(input_ids=input_ids, position_ids=pos, past_key_values=cache, use_cache=True, logits_to_keep=1)
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - t0
    if dec is None:
        m = cache.layers[0].keys.shape[-2]
        dec = _DECODERS.get(key)
        if dec is None or dec.capacity < m + max_new + 8:
            dec = decoder_for(model, m + max_new + 8 + headroom, sparse_decode)
    dec.load(cache, position_offset + n, out.logits[0, -1].argmax().item())
    del cache
    return dec, out, prefill_s


@torch.inference_mode()
def graph_generate(model, input_ids, max_new, eos=(), block=8, sparse_decode=None):
    """Greedy generation (like model.generate(do_sample=False, max_new_tokens=max_new)) with a HIP-graph decode.
    Returns (token ids incl. a final EOS, prefill seconds, decode seconds, decode steps run)."""
    dec, out, prefill_s = graph_prefill(model, input_ids, max_new, sparse_decode=sparse_decode)
    first = out.logits[0, -1].argmax().item()
    del out
    if first in set(eos) or max_new <= 1:
        return [first], prefill_s, 0.0, 0
    if dec.graph is None:
        dec.capture()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    toks, steps = dec.generate(max_new - 1, eos, block)
    torch.cuda.synchronize()
    return [first] + toks, prefill_s, time.perf_counter() - t0, steps
