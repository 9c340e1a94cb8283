"""The C-ABI library without a GPU: it loads, exports every function include/bb_attn.h declares, and its host-side
argument checks return the reference's error texts (kernels/bigger_bird_flash.py:110-130) before any launch.
Also the Python surface's own argument errors (modal_rd/attention.py:94-100) and the FLOP-count helper."""
import ctypes
import re
from pathlib import Path

import pytest
import torch

from bigger_bird_amd import RDAttention, _lib, bigger_bird_flash
from bigger_bird_amd.synth import attended_pairs

HEADER = Path(__file__).resolve().parents[1] / "include" / "bb_attn.h"


def _declared():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(bb_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_function():
    L = _lib.lib()
    names = _declared()
    assert len(names) >= 12
    for name in names:
        assert hasattr(L, name), name
    assert set(names) <= set(_lib.SIGNATURES), "ctypes signatures missing for some declared functions"


def test_version_and_sizes():
    L = _lib.lib()
    assert L.bb_version() == 203  # the parameter lists of include/bb_attn.h (BB_ABI_VERSION)
    assert L.bb_transpose_v_cols(1) == 64 and L.bb_transpose_v_cols(64) == 64 and L.bb_transpose_v_cols(65) == 128
    assert L.bb_routes_workspace(131072, 32, 8, 1, 64) > 32 * 131072 * 8
    assert L.bb_decode_workspace(131072, 32, 8, 128) > 0
    # tail shape: few row tiles, no routes -> the split-key schedule asks for partials
    tail = L.bb_sparse_flash_workspace(32, 256, 131072, 128, 32, 4, 0, 131072, 0, 1, 256, 1, 0)
    main = L.bb_sparse_flash_workspace(32, 131072, 131072, 128, 32, 4, 64, 16384, 512, 1, 131072 - 256, 1, 0)
    # main pass: only the routed tiles pre-gathered per head (512 slots = 8 batches of a 16 KB K and V^T tile each)
    assert tail > 0 and main == 32 * 8 * 2 * 64 * 128 * 2
    # the module's default budget (2048 slots) pre-gathers 32 batches per head
    assert L.bb_sparse_flash_workspace(32, 131072, 131072, 128, 32, 4, 64, 4096, 2048, 1, 131072, 1, 0) == \
        32 * 32 * 2 * 64 * 128 * 2
    # vertical_scope (modal_rd/results/b7_v2k_scope8k.json: vertical 2048, scope_chunk 4096 -> 32 route groups at
    # 128K): the kernel gathers the used batches itself, so nothing is reserved for routed tiles (1 GiB otherwise)
    assert L.bb_sparse_flash_workspace(32, 131072, 131072, 128, 32, 4, 64, 4096, 2048, 32, 131072, 1, 0) == 0
    # a key mask leaves the pipelined kernel: no routed tiles either
    assert L.bb_sparse_flash_workspace(32, 131072, 131072, 128, 32, 4, 64, 16384, 512, 1, 131072, 1, 1) == 0


def _flash_call(**over):
    L = _lib.lib()
    s3 = _lib.i64s(4096, 128, 1)
    a = dict(q=ctypes.c_void_p(16), sq=s3, k=ctypes.c_void_p(16), sk=s3, v=ctypes.c_void_p(16), sv=s3, vt=None,
             idx=None, si=_lib.i64s(1, 1, 1), n_groups=1, route_k=0, key_mask=None, smb=0, out=ctypes.c_void_p(16),
             so=s3, BH=32, T=64, N=64, D=128, is_f16=0, num_heads=32, kv_groups=4, front=0, window=8, route_chunk=64,
             scale=1.0, row_end=64, ws=None, ws_bytes=0, stream=None)
    a.update(over)
    rc = L.bb_sparse_flash(*a.values())
    return rc, L.bb_last_error().decode()


@pytest.mark.parametrize("over,msg", [
    (dict(front=-1), "front >= 0 and window >= 1 required"),
    (dict(window=0), "front >= 0 and window >= 1 required"),
    (dict(kv_groups=3), "must have matching heads"),
    (dict(T=65), "Key sequence must be at least as long as query sequence"),
    (dict(route_k=4, idx=ctypes.c_void_p(16), n_groups=2), "Routing groups must cover the sequence"),
    (dict(D=96), "head_dim 96 unsupported"),
    (dict(scale=0.0), "scale must be positive"),
    (dict(sq=_lib.i64s(4096, 129, 1)), "16-byte aligned rows"),
])
def test_flash_argument_errors(over, msg):
    rc, err = _flash_call(**over)
    assert rc == -1 and msg in err


def test_routes_argument_errors():
    L = _lib.lib()
    s2 = _lib.i64s(128 * 1000, 128)
    rc = L.bb_routes(ctypes.c_void_p(16), s2, ctypes.c_void_p(16), s2, ctypes.c_void_p(16), 64, 1, 32, 8, 1000, 128,
                     0, 64, 512, 600, 0.1, 0, ctypes.c_void_p(16), None, ctypes.c_void_p(16), 1 << 30, None)
    assert rc == -1 and "exceeds" in L.bb_last_error().decode()


def test_python_surface_errors_without_gpu():
    base = type("B", (), {})()
    base.config = type("C", (), {"num_attention_heads": 32, "num_key_value_heads": 8})()
    base.layer_idx, base.head_dim, base.scaling = 0, 128, 128 ** -0.5
    base.q_proj = base.k_proj = base.v_proj = base.o_proj = None
    with pytest.raises(ValueError, match="route_pool"):
        RDAttention(base, route_pool="median")
    with pytest.raises(ValueError, match="route_queries"):
        RDAttention(base, route_queries="first")
    with pytest.raises(ValueError, match="scope_chunk"):
        RDAttention(base, scope_chunk=96)
    q = torch.zeros(8, 64, 32, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="ROCm FP16/BF16"):  # no silent CPU path
        bigger_bird_flash(q, q[:2], q[:2], torch.zeros(8, 1, 4, dtype=torch.int32), num_heads=8, kv_groups=4)


def test_attended_pairs_matches_brute_force():
    T, H, sink, window, tail = 300, 4, 7, 50, 20
    g = torch.Generator().manual_seed(0)
    routes = torch.stack([(torch.randperm(T - window - sink, generator=g)[:15] + sink).sort().values
                          for _ in range(H)]).to(torch.int32)
    q = torch.arange(T)[:, None]
    kk = torch.arange(T)[None, :]
    total = 0
    for h in range(H):
        allowed = (kk <= q) & ((kk < sink) | (kk > q - window))
        member = torch.zeros(T, dtype=torch.bool)
        member[routes[h].long()] = True
        allowed |= member[None, :] & (kk <= q - window) & (kk >= sink)
        allowed[T - tail:] = kk <= q[T - tail:]
        total += int(allowed.sum())
    assert attended_pairs(T, H, sink, window, routes, tail) == total


def test_argmax_argument_checks():
    L = _lib.lib()
    out = ctypes.c_void_p(16)
    assert L.bb_argmax(ctypes.c_void_p(16), 0, 1, out, None) != 0
    assert "row length" in L.bb_last_error().decode()
    assert L.bb_argmax(ctypes.c_void_p(16), 10, 3, out, None) != 0
    assert "dtype must be" in L.bb_last_error().decode()
    assert L.bb_argmax(None, 10, 1, out, None) != 0


def test_decode_step_op_argument_checks():
    """The decode step's fused residual-add + RMSNorm, SiLU-gate and one-token GEMV entry points refuse bad shapes
    and alignment before touching the GPU."""
    L = _lib.lib()
    p, q = ctypes.c_void_p(256), ctypes.c_void_p(8)
    assert L.bb_add_rms_norm(p, 4096, p, 4096, 1, 4100, p, 1e-5, 0, p, 4096, p, 4096, None) != 0
    assert "hidden size" in L.bb_last_error().decode()
    assert L.bb_add_rms_norm(p, 4096, q, 4096, 1, 4096, p, 1e-5, 0, p, 4096, p, 4096, None) != 0
    assert "16-byte aligned" in L.bb_last_error().decode()
    assert L.bb_add_rms_norm(p, 4096, None, 4096, 1, 4096, p, 1e-5, 0, p, 4096, p, 4096, None) != 0
    assert "null" in L.bb_last_error().decode()
    assert L.bb_silu_mul(p, p, 14340, 0, p, None) != 0
    assert "multiple of 8" in L.bb_last_error().decode()
    assert L.bb_silu_mul(p, q, 14336, 0, p, None) != 0
    assert "aligned" in L.bb_last_error().decode()
    assert L.bb_gemv(p, 16392, 4096, 16392, p, 0, 0, p, None) != 0  # K above 16384
    assert "K = 16392" in L.bb_last_error().decode()
    assert L.bb_gemv(p, 4100, 4096, 4096, p, 0, 0, p, None) != 0  # row stride not 16-byte aligned
    assert "16-byte aligned" in L.bb_last_error().decode()
    assert L.bb_gemv(p, 4096, 4096, 4096, None, 1, 0, p, None) != 0
    assert "null" in L.bb_last_error().decode()


def test_int8_layer_host_state_without_gpu():
    """Int8KVLayer's host-side state: construction (HF's DynamicLayer assigns keys / values in its constructor),
    the empty-cache queries, crop on an empty layer and make_int8_cache's per-layer settings need no GPU."""
    from bigger_bird_amd.kv_int8 import Int8KVLayer, make_int8_cache

    layer = Int8KVLayer()
    assert layer._pending is None and layer.keys is None and layer.values is None
    assert layer.get_seq_length() == 0 and layer.nbytes() == 0
    layer.crop(-3)
    assert layer.get_seq_length() == 0
    with pytest.raises(NotImplementedError):
        layer.batch_repeat_interleave(2)
    from transformers import LlamaConfig

    cfg = LlamaConfig(num_hidden_layers=3, hidden_size=64, num_attention_heads=4, num_key_value_heads=2,
                      intermediate_size=128, vocab_size=32)
    cache = make_int8_cache(cfg, fused=False, scale_dtype=torch.float32)
    assert len(cache.layers) == 3
    assert all(isinstance(x, Int8KVLayer) and not x.fused and x.scale_dtype == torch.float32 for x in cache.layers)


def test_decode_append_and_kv_append_argument_errors():
    """Argument checks of the decode-step entry points run before any launch (no GPU needed)."""
    L = _lib.lib()
    p = ctypes.c_void_p(256)
    # bb_decode_append: a missing new row, then a misaligned one, then a non-positive min_scale
    rc = L.bb_decode_append(p, 128, p, p, p, p, 0, None, 128, p, 128, 1e-4, 100, 32, 8, 128, 0.1, p, 128, p, 1 << 30,
                            None)
    assert rc == -1 and "null argument" in L.bb_last_error().decode()
    rc = L.bb_decode_append(p, 128, p, p, p, p, 0, ctypes.c_void_p(258), 128, p, 128, 1e-4, 100, 32, 8, 128, 0.1, p,
                            128, p, 1 << 30, None)
    assert rc == -1 and "16-byte aligned" in L.bb_last_error().decode()
    rc = L.bb_decode_append(p, 128, p, p, p, p, 0, p, 128, p, 128, 0.0, 100, 32, 8, 128, 0.1, p, 128, p, 1 << 30, None)
    assert rc == -1 and "min_scale" in L.bb_last_error().decode()
    rc = L.bb_decode_append(p, 128, p, p, p, p, 0, p, 128, p, 128, 1e-4, 100, 32, 8, 128, 0.1, p, 128, p, 16, None)
    assert rc == -1 and "workspace" in L.bb_last_error().decode()
    # bb_kv_append
    s2 = _lib.i64s(128 * 64, 128)
    rc = L.bb_kv_append(p, s2, p, s2, p, 128, p, 128, 8, 128, 64, None, 1, None)
    assert rc == -1 and "null argument" in L.bb_last_error().decode()
    rc = L.bb_kv_append(p, s2, p, s2, p, 128, p, 128, 8, 100, 64, p, 1, None)
    assert rc == -1 and "16-byte units" in L.bb_last_error().decode()
    rc = L.bb_kv_append(p, _lib.i64s(128 * 64, 129), p, s2, p, 128, p, 128, 8, 128, 64, p, 1, None)
    assert rc == -1 and "16-byte aligned" in L.bb_last_error().decode()
    # bb_decode_step: q, sq, k, sk, v, sv, knew, skn, vnew, svn, n_dev, advance, cap, H, Hkv, D, front, window,
    # routed, scale, is_f16, idx_out, out, so, ws, ws_bytes, stream
    def step(**over):
        a = dict(q=p, sq=128, k=p, sk=s2, v=p, sv=s2, knew=p, skn=128, vnew=p, svn=128, n_dev=p, advance=1, cap=64,
                 H=32, Hkv=8, D=128, front=4, window=16, routed=8, scale=0.1, is_f16=0, idx=p, out=p, so=128, ws=p,
                 ws_bytes=1 << 30, stream=None)
        a.update(over)
        return L.bb_decode_step(*a.values()), L.bb_last_error().decode()
    assert step(knew=None) == (-1, "decode step: null argument")
    rc, msg = step(H=24)
    assert rc == -1 and "groups 3 unsupported" in msg
    rc, msg = step(D=96)
    assert rc == -1 and "head_dim 96 unsupported" in msg
    rc, msg = step(idx=None)
    assert rc == -1 and "index output" in msg
    rc, msg = step(advance=-1)
    assert rc == -1 and "advance" in msg
    rc, msg = step(skn=129)
    assert rc == -1 and "16-byte aligned" in msg
    rc, msg = step(ws_bytes=16)
    assert rc == -1 and "workspace" in msg
    # dense (routed 0) needs no routing workspace; routed adds the routing workspace and the probabilities
    dense = L.bb_decode_step_workspace(131072, 32, 8, 128, 64, 16384, 0)
    routed = L.bb_decode_step_workspace(131072, 32, 8, 128, 64, 16384, 512)
    assert 0 < dense < routed
    assert routed >= L.bb_decode_route_workspace(131072, 32, 8, 0, 512) + 8 * 131072 * 4
