"""Loader for tests/golden/routes_golden.npz (the reference's own routes() indices, see golden/make_golden.py).

Inputs are regenerated from the recorded seeds with the host RNG and checked against the recorded SHA-256 of their
bytes, so a comparison never runs on inputs other than the ones the reference saw.
"""
import hashlib
import json
from pathlib import Path

import numpy as np
import torch

from bigger_bird_amd.attention import vertical_budget
from bigger_bird_amd.synth import make_inputs

PATH = Path(__file__).resolve().parent / "golden" / "routes_golden.npz"


def load():
    z = np.load(PATH)  # allow_pickle=False (default): plain arrays only
    meta = json.loads(bytes(z["meta"]).decode())
    return z, meta


def case_names():
    return [c["name"] for c in load()[1]["cases"]]


def _sha(x):
    return hashlib.sha256(x.contiguous().view(torch.int16).numpy().tobytes()).hexdigest()


def case(name):
    """dict(q, k [1,H,T,d] bf16 CPU, routes int32 [H, budget], kth, kth1, params) for one golden case."""
    z, meta = load()
    c = next(c for c in meta["cases"] if c["name"] == name)
    cfg = c["cfg"]
    inp = make_inputs(c["T"], c["H"], c["Hkv"], c["d"], seed=c["seed"], planted=c["planted"], sink=cfg["sink"],
                      window=cfg["window"], dtype=getattr(torch, c.get("dtype", "bfloat16")))
    if _sha(inp["q"]) != c["q_sha256"] or _sha(inp["k"]) != c["k_sha256"]:
        raise AssertionError(f"{name}: regenerated inputs differ from the ones the reference saw (RNG drift)")
    T = c["T"]
    budget = min(vertical_budget(T, cfg.get("vertical", 2048), cfg.get("vertical_sqrt", 0.0)),
                 max(0, T - cfg["sink"] - cfg["window"]))
    n_route = cfg.get("n_route", 64)
    r = min(n_route, T)
    spread = cfg.get("route_queries", "last") == "spread"
    qpos = torch.linspace(cfg["sink"] + cfg["window"], T - 1, r).long() if spread else torch.arange(T - r, T)
    out = dict(q=inp["q"], k=inp["k"], routes=torch.from_numpy(z[f"{name}/routes"]),
               kth=torch.from_numpy(z[f"{name}/kth"]), kth1=torch.from_numpy(z[f"{name}/kth1"]),
               planted=inp["planted_pos"], budget=budget, n_route=n_route, qpos=qpos,
               route_pool=cfg.get("route_pool", "mean"), route_queries=cfg.get("route_queries", "last"),
               sink=cfg["sink"], window=cfg["window"], scaling=c["scaling"], H=c["H"], Hkv=c["Hkv"], T=T, d=c["d"])
    if f"{name}/col" in z.files:
        out["col"] = torch.from_numpy(z[f"{name}/col"])
    return out


def check_against_golden(got, g, pooled=None, what=""):
    """Set-exact per head, except at a boundary where the reference's own pooled values tie exactly (kth == kth1):
    there torch.topk's pick among equal values is implementation-defined, while this build takes the lower index.
    In that case the heads must agree outside the tied group and `pooled` (this build's scores, [H, n]) must show
    every differing column tied with the boundary. Returns the number of heads compared under the tie rule."""
    want = g["routes"]
    assert got.shape == want.shape, f"{what}: shape {tuple(got.shape)} vs {tuple(want.shape)}"
    tied_heads = 0
    for h in range(want.shape[0]):
        a, b = set(want[h].tolist()), set(got[h].tolist())
        if a == b:
            continue
        assert g["kth"][h] == g["kth1"][h], f"{what}: head {h} differs from the reference without a boundary tie"
        assert pooled is not None, f"{what}: head {h} tie needs pooled scores"
        diff = sorted(a ^ b)
        vals = {pooled[h, j].item() for j in diff}
        boundary = min(pooled[h, j].item() for j in b)
        assert vals == {boundary}, f"{what}: head {h} differing columns {diff} are not a tie in this build"
        tied_heads += 1
    return tied_heads
