"""Greedy batch-1 decode of Llama-family models as a replayed HIP graph (drop-in for modal_rd/graph_decode.py).

Public surface kept from the reference: `StaticDecoder` (buffer_cache / load / feed / step / capture / run /
generated / rewind / generate), `BufferLayer`, `decoder_for`, `graph_prefill` and `graph_generate`, with the same
generate / EOS / rewind / feed protocol. The design is this package's own:

* Memory. Every layer's K and V live in one arena [layers, 2, Hkv, capacity, d] (one allocation, sized once for the
  prompt plus the tokens to generate). Without kv_evict the prefill writes its K/V rows straight into the arena
  through `BufferLayer`; with kv_evict the prefill runs on a DynamicCache (each layer evicts right after its prefill)
  and `load` copies the kept rows in.
* State. A 5-slot int64 control block on the GPU holds (n, position, token, produced, slot): the filled cache rows,
  the RoPE position and id of the next input token, the number of tokens produced since `load`, and the cache row
  the next token's K/V go to. A step advances the block with two vector adds, so every launch in it has a fixed
  shape and reads its varying values from device memory: the step is captured once and replayed per token.
* Step (one token through the model): embedding; per layer RMSNorm -> one fused QKV projection (the q, k and v
  weights concatenated once at construction when they are plain bias-free Linear layers of one dtype) -> RoPE on q and
  k in place (one launch over both) -> attention, which also writes the new K and V row into the arena at `slot` =
  n - 1 -> o_proj, residual + RMSNorm (one launch) -> MLP (gate and up as one fused projection whose launch also
  applies SiLU(gate) * up, then down), residual + the next RMSNorm (one launch); final norm, lm_head, greedy token
  by a one-workgroup HIP argmax written straight into the control block. The projections run as bb_gemv (one token:
  a matrix-vector product streaming the weight once, faster at batch 1 than the vendor GEMM) where the weight is a
  16-bit bias-free Linear with K <= 16384, and each residual add and RMSNorm rides in the launch of the projection
  that follows it (bb_gemv_norm): 7 launches per Llama layer (q/k/v, RoPE, decode, merge, o, gate / up, down).
* Attention per layer: one bb_decode_step. Dense layers run split-K flash decoding over the filled rows (front 0,
  window = capacity, no routes, length read on the GPU); `sparse_decode={"front", "window", "routed"}` switches the
  non-dense RDAttention layers to fused decode routing (pooled per KV head) + sparse decode. The first kernel that
  reads the cache takes the new row from the projection output and stores it in the arena, so the append needs no
  launch of its own (bit-identical to bb_kv_append followed by bigger_bird_decode / bigger_bird_route).
* On bf16 / fp16 models the RMSNorms run as one bb_rms_norm launch each (bb_add_rms_norm with the residual add before
  them), RoPE as bb_rope_inplace (bit-identical to HF apply_rotary_pos_emb) and the MLP's activation as bb_silu_mul:
  at batch 1 the HF modules' elementwise launches cost more than their arithmetic. Modules of other types run as
  they are.
* A captured step holds no memset node and no multi-workgroup reduction of torch's (those have given wrong results
  on replays after the first on these boxes).
* Not supported: the INT8 KV cache, batch > 1, sampling (as in the reference).
"""
import time

import torch
from transformers import DynamicCache
from transformers.cache_utils import DynamicLayer
from transformers.models.llama.modeling_llama import apply_rotary_pos_emb

from .attention import rope_inplace
from .decode import (add_rms_norm, argmax_index, decode_step, gemv_ok, linear_vec, linear_vec_norm, rms_norm,
                     silu_mul)

# Control block: slot indices and the per-step / per-token increments.
N, POS, TOK, MADE, SLOT = range(5)
_CLAIM = (1, 0, 0, 0, 0)    # a step first grows the cache by the row it is about to write (at SLOT)
_ADVANCE = (0, 1, 0, 1, 1)  # ... and ends one position further, with one more token produced and the next free row
_UNDO = (1, 1, 0, 1, 1)     # one consumed token taken back (rewind)


class BufferLayer(DynamicLayer):
    """Cache layer over decoder-owned buffers kb / vb [Hkv, capacity, d]: update writes the new rows in place and
    keys / values are [1, Hkv, filled, d] views (modal_rd/graph_decode.py:40-57)."""

    def __init__(self, kb, vb):
        super().__init__()
        self._kb, self._vb = kb, vb
        self.dtype, self.device = kb.dtype, kb.device
        self.is_initialized = True
        self._expose(0)

    def _expose(self, filled):
        self.filled = filled
        self.keys = self._kb.narrow(1, 0, filled).unsqueeze(0)
        self.values = self._vb.narrow(1, 0, filled).unsqueeze(0)

    def lazy_initialization(self, key_states, value_states, *args, **kwargs):
        pass

    def update(self, key_states, value_states, *args, **kwargs):
        t = key_states.shape[-2]
        if self.filled + t > self._kb.shape[1]:
            raise ValueError("graph decode buffer too small for the prompt")
        self._kb.narrow(1, self.filled, t).copy_(key_states[0])
        self._vb.narrow(1, self.filled, t).copy_(value_states[0])
        self._expose(self.filled + t)
        return self.keys, self.values


def _plain_linear(m):
    return isinstance(m, torch.nn.Linear) and m.bias is None


class _LayerPlan:
    """What a decode step needs of one decoder layer, resolved once."""

    def __init__(self, layer, attn, sparse):
        base = getattr(attn, "_rd_base", attn)
        self.layer, self.base, self.sparse = layer, base, sparse
        self.scaling = getattr(attn, "scaling", None) or base.scaling
        projs = (base.q_proj, base.k_proj, base.v_proj)
        self.qkv_w = None
        if all(_plain_linear(p) for p in projs) and len({p.weight.dtype for p in projs}) == 1:
            with torch.inference_mode(False), torch.no_grad():
                self.qkv_w = _fuse_rows([p.weight for p in projs])
        # a Llama MLP (down(silu(gate(x)) * up(x)), plain 16-bit Linear layers): gate and up as one projection
        mlp = layer.mlp
        self.gate_up_w, self.inter = None, 0
        lin = [getattr(mlp, n, None) for n in ("gate_proj", "up_proj", "down_proj")]
        silu = type(getattr(mlp, "act_fn", None)).__name__ in ("SiLU", "SiLUActivation")  # torch's or HF's F.silu
        if (silu and all(_plain_linear(m) for m in lin)
                and len({m.weight.dtype for m in lin}) == 1 and lin[0].weight.dtype in (torch.bfloat16, torch.float16)
                and lin[0].weight.shape == lin[1].weight.shape and lin[0].weight.shape[0] % 8 == 0):
            with torch.inference_mode(False), torch.no_grad():
                self.gate_up_w = _fuse_rows([lin[0].weight, lin[1].weight])
            self.inter = lin[0].weight.shape[0]
        # one-token projections on the HIP GEMV where the weight allows it (else nn.Linear / F.linear)
        self.qkv_vec = self.qkv_w is not None and gemv_ok(self.qkv_w)
        o = base.o_proj
        self.o_vec = _plain_linear(o) and gemv_ok(o.weight)
        self.mlp_vec = (self.gate_up_w is not None and gemv_ok(self.gate_up_w)
                        and gemv_ok(layer.mlp.down_proj.weight))


def _fuse_rows(weights):
    """One [sum of rows, cols] matrix whose row blocks are the given weights, without a second copy of them: the
    weights are moved into the fused buffer once (each parameter then holds a view of its block, same values), and
    weights that already are adjacent blocks of one buffer are viewed as it directly."""
    first = weights[0]
    rows, cols = sum(w.shape[0] for w in weights), first.shape[1]
    adjacent = all(w.is_contiguous() and w.shape[1] == cols for w in weights)
    offset = first.storage_offset()
    for w in weights:
        adjacent = adjacent and w.untyped_storage().data_ptr() == first.untyped_storage().data_ptr()
        adjacent = adjacent and w.storage_offset() == offset
        offset += w.numel()
    if adjacent:
        return first.new_empty(0).set_(first.untyped_storage(), first.storage_offset(), (rows, cols), (cols, 1))
    fused = torch.cat([w.detach() for w in weights], 0)
    start = 0
    for w in weights:
        w.data = fused[start:start + w.shape[0]]
        start += w.shape[0]
    return fused


class StaticDecoder:
    """Fixed-shape one-token decoder over one K/V arena, capturable as a HIP graph (modal_rd/graph_decode.py:65-269).

    Attributes: `length`, `position`, `token` ([1, 1]) and `step_i` are views of the control block; `logits` is the
    last step's logits [vocab]; `k[i]` / `v[i]` are layer i's [Hkv, capacity, d] buffers; `sparse[i]` tells whether
    layer i decodes sparsely."""

    def __init__(self, model, capacity, sparse_decode=None):
        if sparse_decode is not None and set(sparse_decode) != {"front", "window", "routed"}:
            raise ValueError("sparse_decode takes front, window and routed")
        cfg = model.config
        self.model, self.capacity = model, int(capacity)
        self.core = model.model
        self.h, self.hk = cfg.num_attention_heads, cfg.num_key_value_heads
        first = self.core.layers[0].self_attn
        self.d = getattr(first, "head_dim", cfg.hidden_size // self.h)
        w = model.lm_head.weight
        dev = w.device
        dt = w.dtype if w.dtype in (torch.float16, torch.bfloat16) else torch.bfloat16
        self.sparse_cfg = dict(sparse_decode) if sparse_decode else None
        layers = list(self.core.layers)
        with torch.inference_mode(False):
            self.arena = torch.zeros(len(layers), 2, self.hk, self.capacity, self.d, device=dev, dtype=dt)
            self.ctl = torch.zeros(5, dtype=torch.int64, device=dev)
            self._claim, self._advance, self._undo = (torch.tensor(v, dtype=torch.int64, device=dev)
                                                      for v in (_CLAIM, _ADVANCE, _UNDO))
            self.out = torch.zeros(self.capacity, dtype=torch.int64, device=dev)
            self.no_routes = torch.empty(self.hk, 0, dtype=torch.int32, device=dev)
            # views made here, outside inference mode, so that later in-place updates are allowed in either mode
            self.k = [self.arena[i, 0] for i in range(len(layers))]
            self.v = [self.arena[i, 1] for i in range(len(layers))]
            self.length, self.position = self.ctl[N:N + 1], self.ctl[POS:POS + 1]
            self.step_i = self.ctl[MADE:MADE + 1]
            self.token = self.ctl[TOK:TOK + 1].view(1, 1)
            self._token_flat = self.ctl[TOK:TOK + 1]
        self.plans = [_LayerPlan(layer, layer.self_attn,
                                 bool(self.sparse_cfg) and not getattr(layer.self_attn, "dense", True))
                      for layer in layers]
        self.sparse = [p.sparse for p in self.plans]
        self.logits = None
        self.graph = None

    # ---- loading a prefilled cache ----
    def buffer_cache(self):
        """A DynamicCache whose layers write the prefill's K/V straight into this decoder's arena."""
        cache = DynamicCache(config=self.model.config)
        cache.layers = [BufferLayer(kb, vb) for kb, vb in zip(self.k, self.v)]
        return cache

    @torch.no_grad()
    def load(self, cache, prompt_len, first_token):
        """Take a prefilled cache (this decoder's `buffer_cache()`, or a bf16/fp16 DynamicCache, e.g. after kv_evict)
        and make `first_token` the next input at RoPE position `prompt_len`."""
        layers = list(getattr(cache, "layers", None) or [])
        tensors = all(isinstance(x, DynamicLayer) and torch.is_tensor(x.keys) for x in layers)
        if len(layers) != len(self.plans) or not tensors or layers[0].keys.dtype != self.arena.dtype:
            raise ValueError("graph decode needs a BF16/FP16 DynamicCache (INT8 KV cache is not supported)")
        rows = {x.keys.shape[-2] for x in layers}
        if len(rows) != 1:
            raise ValueError("all layers must hold the same number of cached keys")
        m = rows.pop()
        if m >= self.capacity:
            raise ValueError("graph decode buffer too small")
        for i, x in enumerate(layers):
            if x.keys.data_ptr() == self.k[i].data_ptr() and x.values.data_ptr() == self.v[i].data_ptr():
                continue  # already in the arena (BufferLayer)
            self.k[i].narrow(1, 0, m).copy_(x.keys[0])
            self.v[i].narrow(1, 0, m).copy_(x.values[0])
        state = torch.tensor([m, int(prompt_len), int(first_token), 0, m], dtype=torch.int64)
        self.ctl.copy_(state)

    @torch.no_grad()
    def feed(self, token):
        """Make `token` the next input (a prompt continuation or a token already produced)."""
        self.token.fill_(int(token))

    # ---- the step ----
    @staticmethod
    def _fast_norm(module, x):
        """(weight, eps) of a plain bf16/fp16 Llama RMSNorm module that the HIP norm can run on x, else None."""
        w, eps = getattr(module, "weight", None), getattr(module, "variance_epsilon", None)
        fast = (type(module).__name__.endswith("RMSNorm") and w is not None and eps is not None
                and w.dtype == x.dtype and x.dtype in (torch.bfloat16, torch.float16)
                and x.shape[-1] % 8 == 0 and x.shape[-1] <= 8192)
        return (w, eps) if fast else None

    def _norm(self, module, x):
        """An RMSNorm module on x: one bb_rms_norm launch for the plain bf16/fp16 Llama module, else the module."""
        f = self._fast_norm(module, x)
        return rms_norm(x, *f) if f else module(x)

    def _add_norm(self, module, hid, res):
        """(hid + res, module(hid + res)); one bb_add_rms_norm launch where the module allows (res None: no add)."""
        if res is None:
            return hid, self._norm(module, hid)
        f = self._fast_norm(module, hid)
        if f and res.dtype == hid.dtype and res.shape == hid.shape:
            return add_rms_norm(hid, res, *f)
        hid = hid + res
        return hid, module(hid)

    @staticmethod
    def _mlp(plan, x):
        """The layer's MLP on the normed x: two HIP GEMVs (the fused gate / up projection with the SiLU gate, then
        down) where the weights allow; else the fused projection, bb_silu_mul and down_proj; else the module."""
        mlp = plan.layer.mlp
        if plan.mlp_vec:
            return linear_vec(linear_vec(x, plan.gate_up_w, glu=True), mlp.down_proj.weight)
        if plan.gate_up_w is None:
            return mlp(x)
        y = torch.nn.functional.linear(x, plan.gate_up_w)
        return mlp.down_proj(silu_mul(y[..., :plan.inter], y[..., plan.inter:]))

    @staticmethod
    def _o_proj(plan, o):
        """o_proj on the attention output [H, d] of one token -> [1, 1, hidden]."""
        o = o.reshape(1, 1, -1)
        return linear_vec(o, plan.base.o_proj.weight) if plan.o_vec else plan.base.o_proj(o)

    def _norm_qkv(self, plan, module, hid, res):
        """The layer's input: hid + res (res None: hid), its norm and the q/k/v projections, as one bb_gemv_norm
        launch where the modules allow. Returns the new hid and q [1, H, 1, d], k and v [1, Hkv, 1, d], and, with the
        fused projection, the [2, Hkv, 1, d] view of its K and V part (so RoPE on k in place also lands there) and the
        [1, H + Hkv, 1, d] view of q and k together (one RoPE launch for both)."""
        h, hk, d = self.h, self.hk, self.d
        f = self._fast_norm(module, hid)
        if plan.qkv_vec and f and hid.shape[-1] <= 8192 and (res is None or res.dtype == hid.dtype):
            hid, y = linear_vec_norm(hid, res, *f, plan.qkv_w)
            y = y[0, 0]
        else:
            hid, x = self._add_norm(module, hid, res)
            if plan.qkv_w is None:
                q, k, v = (p(x)[0, 0] for p in (plan.base.q_proj, plan.base.k_proj, plan.base.v_proj))
                return hid, q.view(1, h, 1, d), k.view(1, hk, 1, d), v.view(1, hk, 1, d), None, None
            y = (linear_vec(x, plan.qkv_w) if plan.qkv_vec else torch.nn.functional.linear(x, plan.qkv_w))[0, 0]
        q, k, v = y.split((h * d, hk * d, hk * d))
        kv = y[h * d:].view(2, hk, 1, d)
        qk = y[:(h + hk) * d].view(1, h + hk, 1, d)
        return hid, q.view(1, h, 1, d), k.view(1, hk, 1, d), v.view(1, hk, 1, d), kv, qk

    def _norm_mlp(self, plan, module, hid, res):
        """hid + res, its norm and the MLP: returns the new hid and the MLP's output. With the HIP GEMVs the norm
        rides in the gate / up launch (bb_gemv_norm with the SiLU gate), then the down GEMV: two launches."""
        f = self._fast_norm(module, hid)
        if plan.mlp_vec and f and hid.shape[-1] <= 8192 and res.dtype == hid.dtype and res.numel() == hid.numel():
            hid, g = linear_vec_norm(hid, res, *f, plan.gate_up_w, glu=True)
            return hid, linear_vec(g, plan.layer.mlp.down_proj.weight)
        hid, x = self._add_norm(module, hid, res)
        return hid, self._mlp(plan, x)

    def _attend(self, i, plan, q, kn, vn):
        """q [H, d] of the new token, its K / V rows kn / vn [Hkv, d] -> [H, d]. The rows become arena row
        length - 1 (the write slot: the step's claim has already counted them) inside the step's first kernel."""
        K, V = self.k[i], self.v[i]
        if not plan.sparse:
            return decode_step(q, K, V, kn, vn, self.length, routed=0, scale=plan.scaling)
        c = self.sparse_cfg
        return decode_step(q, K, V, kn, vn, self.length, routed=c["routed"], front=c["front"], window=c["window"],
                           scale=plan.scaling)[0]

    def step(self):
        """One greedy token: fixed shapes, all varying state read from the control block (capturable)."""
        hid = self.core.embed_tokens(self.token)
        cos, sin = self.core.rotary_emb(hid, self.position.view(1, 1))
        self.ctl.add_(self._claim)
        pending = None  # the last MLP's output, added to hid together with the next norm
        for i, plan in enumerate(self.plans):
            layer = plan.layer
            hid, q, k, v, kv, qk = self._norm_qkv(plan, layer.input_layernorm, hid, pending)
            if q.dtype == torch.bfloat16 and cos.dtype == torch.bfloat16:
                if qk is not None:
                    rope_inplace(qk, cos, sin)
                else:
                    rope_inplace(q, cos, sin)
                    rope_inplace(k, cos, sin)
            else:
                q, k = apply_rotary_pos_emb(q, k, cos, sin)
                kv = None
            if kv is None:
                kv = torch.stack((k[0], v[0]))
            o = self._attend(i, plan, q[0, :, 0], kv[0, :, 0], kv[1, :, 0])
            hid, pending = self._norm_mlp(plan, layer.post_attention_layernorm, hid, self._o_proj(plan, o))
        hid, x = self._add_norm(self.core.norm, hid, pending)
        self.logits = self.model.lm_head(x)[0, -1]
        argmax_index(self.logits, out=self._token_flat)
        self.out.index_copy_(0, self.step_i, self._token_flat)
        self.ctl.add_(self._advance)

    # ---- graph capture and running ----
    def capture(self):
        """Record `step` as a HIP graph. Two warm-up steps run first on a side stream (allocator pools and library
        handles settle outside the capture); the control block is put back after them and after the capture. Runs
        outside inference mode, under no_grad: a capture under inference mode leaves the CUDA generator's graph
        state as inference tensors, and every later capture outside it would fail."""
        with torch.inference_mode(False), torch.no_grad():
            before = self.ctl.clone()
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                for _ in range(2):
                    self.step()
                    self.ctl.copy_(before)
            torch.cuda.current_stream().wait_stream(side)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                self.step()
            self.ctl.copy_(before)
            self.graph = graph

    @torch.no_grad()
    def run(self, steps, graph=True):
        """Advance `steps` tokens (each consumes the next input and produces the one after). Raises ValueError (one
        host read of the length) when the arena cannot hold `steps` more rows."""
        if int(self.length) + steps > self.capacity:
            raise ValueError("graph decode buffer full: build the decoder with a larger capacity")
        if graph and self.graph is None:
            self.capture()
        go = self.graph.replay if graph else self.step
        for _ in range(steps):
            go()

    def generated(self):
        """The tokens produced since `load`, as a list."""
        return self.out[:int(self.step_i)].tolist()

    @torch.no_grad()
    def rewind(self, r):
        """Take back the last `r` consumed tokens (their cache rows, positions and produced tokens)."""
        self.ctl.sub_(self._undo * int(r))

    @torch.no_grad()
    def generate(self, max_steps, eos=(), block=8, graph=True):
        """Greedy steps, `block` at a time, until a produced token is in `eos` or `max_steps` ran; returns
        (tokens through the first EOS, steps run). Steps run past that EOS are taken back, and the EOS becomes the
        next input, so the cache ends right after the input that produced it (as eager decoding stopping on EOS)."""
        stop = frozenset(int(t) for t in eos)
        first = int(self.step_i)
        ran = 0
        while ran < max_steps:
            b = min(block, max_steps - ran)
            self.run(b, graph)
            ran += b
            if stop and not stop.isdisjoint(self.out[first + ran - b:first + ran].tolist()):
                break
        made = self.out[first:first + ran].tolist()
        keep = next((j + 1 for j, t in enumerate(made) if t in stop), ran)
        if keep < ran:
            self.rewind(ran - keep)
            self.feed(made[keep - 1])
        return made[:keep], ran


class _Cache:
    """At most one live decoder, reused while the installed attention modules and the sparse config stay the same
    and its capacity suffices (graph capture is the expensive part to keep)."""

    def __init__(self):
        self.key, self.dec = None, None

    @staticmethod
    def key_of(model, sparse_decode):
        modules = tuple(id(layer.self_attn) for layer in model.model.layers)
        return modules, tuple(sorted(sparse_decode.items())) if sparse_decode else ()

    def release(self):
        if self.dec is not None:
            self.key, self.dec = None, None
            torch.cuda.empty_cache()

    def get(self, model, capacity, sparse_decode):
        key = self.key_of(model, sparse_decode)
        if self.dec is not None and (self.key != key or self.dec.capacity < capacity):
            self.release()
        if self.dec is None:
            self.key, self.dec = key, StaticDecoder(model, capacity, sparse_decode)
        return self.dec

    def holds(self, model, sparse_decode):
        return self.dec is not None and self.key == self.key_of(model, sparse_decode)


_CACHE = _Cache()


def release():
    """Drop the cached decoder (its arena and graph) and return the memory to the allocator."""
    _CACHE.release()


def decoder_for(model, capacity, sparse_decode=None):
    """The cached decoder for the installed attention modules, rebuilt when it is too small or for other modules."""
    return _CACHE.get(model, int(capacity), sparse_decode)


@torch.inference_mode()
def graph_prefill(model, input_ids, max_new, headroom=4096, position_offset=0, sparse_decode=None):
    """Eager prefill of input_ids [1, n] loaded into the cached decoder; returns (decoder, prefill output, prefill
    seconds). The argmax of the output's last logits is already the decoder's next input. The decoder holds the
    kept cache rows plus `max_new` tokens and `headroom` spare rows (so slightly longer prompts reuse the graph)."""
    n = input_ids.shape[1]
    if not _CACHE.holds(model, sparse_decode):
        release()  # another arm's arena: free it before this prefill
    evicting = any(getattr(layer.self_attn, "kv_evict", False) for layer in model.model.layers)
    spare = max_new + 8 + headroom
    if evicting:
        dec, cache = None, DynamicCache(config=model.config)
    else:
        dec = decoder_for(model, n + spare, sparse_decode)
        cache = dec.buffer_cache()
    pos = torch.arange(position_offset, position_offset + n, device=input_ids.device)[None]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    out = model(input_ids=input_ids, position_ids=pos, past_key_values=cache, use_cache=True, logits_to_keep=1)
    torch.cuda.synchronize()
    seconds = time.perf_counter() - t0
    if dec is None:
        dec = decoder_for(model, cache.layers[0].keys.shape[-2] + spare, sparse_decode)
    dec.load(cache, position_offset + n, out.logits[0, -1].argmax().item())
    return dec, out, seconds


@torch.inference_mode()
def graph_generate(model, input_ids, max_new, eos=(), block=8, sparse_decode=None):
    """Greedy generation (as model.generate(do_sample=False, max_new_tokens=max_new)) with the graph decode. Returns
    (token ids through a final EOS, prefill seconds, decode seconds, decode steps run)."""
    dec, out, prefill_s = graph_prefill(model, input_ids, max_new, sparse_decode=sparse_decode)
    first = int(dec.token)
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
