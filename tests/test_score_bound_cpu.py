"""The certification bound of the route scorer (scores_mfma_kernel, csrc/bb_routes.hip) checked on the CPU.

The scorer computes every route score s = q . k (d = 128, bf16 inputs) on MFMA and keeps its bf16 rounding only when
[s - B, s + B] rounds to one bf16 value; B must bound |reference-order result - MFMA result|. The reference order is
torch's CPU bf16 matmul (modal_rd/attention.py:164): per 32-element block, sequential fp32 chains over the even and
the odd elements, then acc = acc + (even + odd) (oracle/bb_oracle.c amx_dot). The MFMA path sums each 16-element
slice with one instruction whose error model (measured on the hardware: products aligned to the largest and
truncated below 2^-23 of it, then one rounding) is restated here, and adds the 8 slice partials in order.

B = u (sum_d c_d |q_d k_d| + 32 sum_s max_s|q| max_s|k|), u = 2^-24, with c_d the rounding count of product d on
both paths. The checks: the reference chain alone stays within u sum_d w_ref(d) |p_d| of the exact sum, the MFMA
model within the rest, and |ref - mfma| <= B, on random, wide-range, cancelling, sorted, one-dominant, truncating and
tie-rounding inputs; two
planted mistakes (no per-slice maximum term; reference weights counted from the wrong end of the chain) each fail
on the inputs built to expose them.
"""
import numpy as np
import pytest
import torch

U = 2.0 ** -24
D = 128


def _weights():
    d = np.arange(D)
    c, t, s = d >> 5, (d & 31) >> 1, d >> 4
    w_ref = (16 - np.maximum(t, 1)) + 1 + (4 - np.maximum(c, 1))
    w_mfma = 10 - np.maximum(s, 1)
    return w_ref.astype(np.float64), w_mfma.astype(np.float64)


def _bf16(x):
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16).float().numpy()


def _ref_order(q, k):
    """torch CPU AMX order in fp32 (numpy float32 adds round to nearest even; bf16 products are exact)."""
    p = (q * k).astype(np.float32)
    acc = np.zeros(q.shape[0], np.float32)
    for b in range(D // 32):
        ev = np.zeros_like(acc)
        od = np.zeros_like(acc)
        for t in range(16):
            ev = ev + p[:, 32 * b + 2 * t]
            od = od + p[:, 32 * b + 2 * t + 1]
        acc = acc + (ev + od)
    return acc.astype(np.float64)


def _mfma_model(q, k, final="nearest"):
    """Eight 16-element slices: products aligned to the slice's largest and truncated below 2^-23 of it, summed
    exactly, rounded once to fp32; slice partials added in order in fp32."""
    p = q.astype(np.float64) * k.astype(np.float64)
    acc = None
    for s in range(D // 16):
        ps = p[:, 16 * s:16 * s + 16]
        mx = np.abs(ps).max(1, keepdims=True)
        e = np.floor(np.log2(np.where(mx > 0, mx, 1.0)))
        quantum = np.exp2(e - 23)
        tr = np.trunc(ps / quantum) * quantum
        tot = tr.sum(1)  # exact: every term a multiple of quantum below 2^(e + 1)
        part = tot.astype(np.float32)
        if final == "truncate":  # round toward zero instead of to nearest (the bound allows 2 u per slice)
            over = np.abs(part.astype(np.float64)) > np.abs(tot)
            part = np.where(over, np.nextafter(part, np.float32(0)), part)
        acc = part if acc is None else (acc + part).astype(np.float32)
    return acc.astype(np.float64)


def _bound(q, k, max_term=True, w_ref=None):
    wr, wm = _weights()
    if w_ref is not None:
        wr = w_ref
    a = np.abs(q.astype(np.float64) * k.astype(np.float64))
    b = (a * (wr + wm)).sum(1)
    if max_term:
        qm = np.abs(q).reshape(-1, 8, 16).max(2)
        km = np.abs(k).reshape(-1, 8, 16).max(2)
        b = b + 32.0 * (qm.astype(np.float64) * km.astype(np.float64)).sum(1)
    return U * b


def _inputs(kind, n, seed):
    g = np.random.default_rng(seed)
    if kind == "normal":
        q, k = g.standard_normal((n, D)), g.standard_normal((n, D))
    elif kind == "wide":  # every element its own binade in 2^-20 .. 2^20
        q = g.standard_normal((n, D)) * np.exp2(g.integers(-20, 21, (n, D)))
        k = g.standard_normal((n, D)) * np.exp2(g.integers(-20, 21, (n, D)))
    elif kind == "cancel":  # large partial sums that cancel: k = +q then -q within every block
        q = g.standard_normal((n, D)) * np.exp2(g.integers(-4, 5, (n, 1)))
        sign = np.where((np.arange(D) % 32) < 16, 1.0, -1.0)
        k = q * sign * (1 + g.standard_normal((n, D)) * 2.0 ** -6)
    elif kind == "sorted":  # chains that start with their largest products
        q = np.sort(np.abs(g.standard_normal((n, D))), 1)[:, ::-1] * np.exp2(-np.arange(D) / 8.0)
        k = np.abs(g.standard_normal((n, D)))
    elif kind == "dominant":  # one huge product per slice, the rest just above its truncation point
        q = g.standard_normal((n, D)) * 2.0 ** -10
        k = g.standard_normal((n, D))
        q[:, ::16] = 1.0 + g.random((n, D // 16))
        k[:, ::16] = 1.0 + g.random((n, D // 16))
    elif kind == "truncation":  # one product of 2.25 per slice, 15 same-sign products just under its 2^-23 quantum
        q = np.full((n, D), 2.0 ** -11)
        k = np.full((n, D), 2.0 ** -11) * (0.98 + 0.015 * g.random((n, D)))
        q[:, ::16], k[:, ::16] = 1.5, 1.5
    elif kind == "ties":  # every chain starts at 1 and then adds half an ulp of it 15 times (each add rounds away)
        scale = np.exp2(g.integers(-6, 7, (n, 1)))
        q = np.full((n, D), 2.0 ** -12) * scale
        k = np.full((n, D), 2.0 ** -12)
        first = (np.arange(D) % 32) < 2
        q[:, first], k[:, first] = scale, 1.0
    else:
        raise ValueError(kind)
    return _bf16(q), _bf16(k)


KINDS = ["normal", "wide", "cancel", "sorted", "dominant", "truncation", "ties"]


@pytest.mark.parametrize("kind", KINDS)
def test_bound_covers_reference_and_mfma_model(kind):
    q, k = _inputs(kind, 40000, KINDS.index(kind))
    exact = (q.astype(np.float64) * k.astype(np.float64)).sum(1)  # products exact, sum rounded at 2^-53
    ref = _ref_order(q, k)
    wr, wm = _weights()
    a = np.abs(q.astype(np.float64) * k.astype(np.float64))
    slack = 1 + 2.0 ** -10
    assert (np.abs(ref - exact) <= U * (a * wr).sum(1) * slack + 1e-30).all(), "reference chain exceeds its part"
    for final in ("nearest", "truncate"):
        mf = _mfma_model(q, k, final)
        qm, km = np.abs(q).reshape(-1, 8, 16).max(2), np.abs(k).reshape(-1, 8, 16).max(2)
        mpart = U * ((a * wm).sum(1) + 32.0 * (qm.astype(np.float64) * km.astype(np.float64)).sum(1))
        assert (np.abs(mf - exact) <= mpart * slack + 1e-30).all(), f"MFMA model exceeds its part ({final})"
        b = _bound(q, k)
        ratio = np.abs(ref - mf) / np.maximum(b, 1e-300)
        print(f"{kind} {final}: max |ref - mfma| / B = {ratio.max():.3f}", flush=True)
        assert (np.abs(ref - mf) <= b * slack + 1e-30).all()


def test_bound_is_tighter_than_uniform():
    """On N(0,1) inputs the weighted bound is well under the former uniform 67 u sum|p| (fewer fix-ups)."""
    q, k = _inputs("normal", 20000, 9)
    a = np.abs(q.astype(np.float64) * k.astype(np.float64)).sum(1)
    ratio = _bound(q, k) / (67 * U * a)
    print(f"weighted / uniform bound: mean {ratio.mean():.3f}", flush=True)
    assert ratio.mean() < 0.5 and ratio.max() < 1.0


def test_planted_mistakes_fail():
    """Without the per-slice maximum term the MFMA truncation of slices with one large product escapes the bound; with the
    reference weights reversed (the first products of a chain counted once) chains that round at every step escape it."""
    q, k = _inputs("truncation", 4000, 3)
    mf = _mfma_model(q, k)
    exact = (q.astype(np.float64) * k.astype(np.float64)).sum(1)
    wr, wm = _weights()
    a = np.abs(q.astype(np.float64) * k.astype(np.float64))
    assert (np.abs(mf - exact) > U * (a * wm).sum(1)).any(), "dropping the max term should be caught"
    q, k = _inputs("ties", 4000, 4)
    ref = _ref_order(q, k)
    exact = (q.astype(np.float64) * k.astype(np.float64)).sum(1)
    a = np.abs(q.astype(np.float64) * k.astype(np.float64))
    d = np.arange(D)
    wrong = (np.maximum((d & 31) >> 1, 1) + 1 + np.maximum(d >> 5, 1)).astype(np.float64)
    assert (np.abs(ref - exact) > U * (a * wrong).sum(1)).any(), "reversed chain weights should be caught"
