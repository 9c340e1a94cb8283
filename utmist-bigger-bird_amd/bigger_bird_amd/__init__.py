"""bigger_bird_amd -- MI355X-native Bigger Bird v3 sparse prefill attention (gfx950 HIP kernels behind a C ABI).

Public surface (mirrors the reference's modal_rd.attention / kernels.bigger_bird_flash / modal_rd.kv_int8):
  RDAttention, install, rope_inplace, vertical_budget, routes,       -- attention module, routing and the kv_evict
  forward_pool                                                           span pooling
  bigger_bird_flash, transpose_v                                      -- the sparse attention operator
  quantize, dequantize, Int8KVLayer, make_int8_cache, decode_int8     -- INT8 KV cache and exact decode
  bigger_bird_decode, bigger_bird_route, pooled_probs                 -- split-K sparse decode and decode routing
  StaticDecoder, graph_prefill, graph_generate                        -- HIP-graph greedy decode (modal_rd.graph_decode)
"""
from .attention import RDAttention, forward_pool, install, rope_inplace, routes, vertical_budget
from .decode import bigger_bird_decode, bigger_bird_route, pooled_probs
from .flash import bigger_bird_flash, exact_attention, transpose_v
from .graph_decode import StaticDecoder, graph_generate, graph_prefill
from .kv_int8 import (Int8KVLayer, decode_bf16, decode_int8, decode_int8_append, dequantize, make_int8_cache,
                      quantize)

__all__ = ["RDAttention", "forward_pool", "install", "rope_inplace", "routes", "vertical_budget", "bigger_bird_flash", "exact_attention", "transpose_v",
           "Int8KVLayer", "decode_bf16", "decode_int8", "decode_int8_append", "dequantize", "make_int8_cache", "quantize",
           "bigger_bird_decode", "bigger_bird_route", "pooled_probs", "StaticDecoder", "graph_prefill",
           "graph_generate"]
