"""bb_decode_noalloc (static device scratch, no workspace argument, no allocation) against bb_decode (caller
workspace) through the C ABI: same kernels, so the outputs must be bitwise equal. Two calls in a row, the second
over a smaller cache (fewer splits), so a stale partial left by the first call would show; plus the size limit."""
import pytest
import torch

from bigger_bird_amd import _lib, quantize

pytestmark = pytest.mark.gpu


def _call(L, noalloc, q, k8, ks, v8, vs, n, H, Hkv, d, out, ws=None):
    f16 = int(ks.dtype == torch.float16)
    common = (_lib.ptr(q), q.stride(0), _lib.ptr(k8), _lib.ptr(ks), _lib.ptr(v8), _lib.ptr(vs), f16, None, None, None,
              None, n, H, Hkv, d, float(d ** -0.5), _lib.ptr(out), out.stride(0))
    if noalloc:
        return L.bb_decode_noalloc(*common, _lib.stream_of(q))
    return L.bb_decode(*common, _lib.ptr(ws), ws.numel(), _lib.stream_of(q))


def _cache(n, Hkv, d, seed, dev, f16):
    g = torch.Generator(device=dev).manual_seed(seed)
    k = torch.randn(n, Hkv, d, device=dev, generator=g).to(torch.bfloat16)
    v = torch.randn(n, Hkv, d, device=dev, generator=g).to(torch.bfloat16)
    sd = torch.float16 if f16 else torch.float32
    return (*quantize(k, scale_dtype=sd), *quantize(v, scale_dtype=sd))


@pytest.mark.parametrize("H,Hkv,d,f16,sizes", [(32, 8, 128, True, (131072, 3000)), (16, 2, 64, False, (20000, 700))])
def test_noalloc_matches_workspace_decode(H, Hkv, d, f16, sizes, dev):
    L = _lib.lib()
    assert L.bb_decode_noalloc_max_bytes() == 2 << 20
    for i, n in enumerate(sizes):
        print(f"case decode_noalloc call {i} n={n} H={H}/{Hkv} d={d} f16={f16}", flush=True)
        k8, ks, v8, vs = _cache(n, Hkv, d, 11 + i, dev, f16)
        g = torch.Generator(device=dev).manual_seed(100 + i)
        q = torch.randn(H, d, device=dev, generator=g).to(torch.bfloat16)
        need = L.bb_decode_workspace(n, H, Hkv, d)
        assert 0 < need <= L.bb_decode_noalloc_max_bytes()
        ws = torch.empty(need, dtype=torch.uint8, device=dev)
        want = torch.empty(H, d, dtype=torch.bfloat16, device=dev)
        got = torch.full((H, d), float("nan"), dtype=torch.bfloat16, device=dev)
        _lib.check(_call(L, False, q, k8, ks, v8, vs, n, H, Hkv, d, want, ws))
        _lib.check(_call(L, True, q, k8, ks, v8, vs, n, H, Hkv, d, got))
        torch.cuda.synchronize()
        assert torch.isfinite(want.float()).all()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"call {i} (n={n}) differs"


def test_noalloc_rejects_partials_beyond_the_scratch(dev):
    """16 query heads over 2 KV heads at 128K keys need 256 splits * 16 heads * 130 floats = 2.13 MB > 2 MiB."""
    print("case decode_noalloc size limit", flush=True)
    L = _lib.lib()
    H, Hkv, d, n = 16, 2, 128, 131072
    assert L.bb_decode_workspace(n, H, Hkv, d) > L.bb_decode_noalloc_max_bytes()
    k8 = torch.zeros(n, Hkv, d, dtype=torch.int8, device=dev)
    ks = torch.ones(n, Hkv, 1, dtype=torch.float16, device=dev)
    q = torch.zeros(H, d, dtype=torch.bfloat16, device=dev)
    out = torch.empty(H, d, dtype=torch.bfloat16, device=dev)
    rc = _call(L, True, q, k8, ks, k8, ks, n, H, Hkv, d, out)
    assert rc == -1 and "exceed the static scratch" in L.bb_last_error().decode()
    with pytest.raises(ValueError, match="static scratch"):
        _lib.check(rc)


def test_noalloc_in_captured_graph(dev):
    """bb_decode_noalloc captured into a HIP graph (its scratch address is resolved when the library is loaded, before
    any capture): every replay, with eager work between replays, equals bb_decode bitwise."""
    print("case decode_noalloc graph capture", flush=True)
    L = _lib.lib()
    H, Hkv, d, n = 32, 8, 128, 40000
    k8, ks, v8, vs = _cache(n, Hkv, d, 21, dev, True)
    g = torch.Generator(device=dev).manual_seed(22)
    q = torch.randn(H, d, device=dev, generator=g).to(torch.bfloat16)
    ws = torch.empty(L.bb_decode_workspace(n, H, Hkv, d), dtype=torch.uint8, device=dev)
    want = torch.empty(H, d, dtype=torch.bfloat16, device=dev)
    _lib.check(_call(L, False, q, k8, ks, v8, vs, n, H, Hkv, d, want, ws))
    out = torch.empty(H, d, dtype=torch.bfloat16, device=dev)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up outside the capture
        _lib.check(_call(L, True, q, k8, ks, v8, vs, n, H, Hkv, d, out))
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _lib.check(_call(L, True, q, k8, ks, v8, vs, n, H, Hkv, d, out))
    for i in range(3):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), want.view(torch.int16)), f"replay {i} differs"
