"""Shared helpers for the parity tests: run a catalog group on the GPU and
through the CPU oracle on the same inputs."""
import numpy as np

import hfusion_mi355x as hf
from oracle import interp


def np_of(elem):
    return interp.NP[elem]


def empty_like_param(p):
    return np.zeros(p["shape"], dtype=np_of(p["elem"]))


def to_dev(a, elem, device):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a))
    if elem in ("bf16", "f16"):
        t = t.view(torch.bfloat16 if elem == "bf16" else torch.float16)
    if elem in ("f8E4M3FN", "f8E5M2"):
        t = t.view(torch.uint8).view(torch.float8_e4m3fn if elem == "f8E4M3FN" else torch.float8_e5m2)
    return t.to(device)


def to_host(t, elem):
    import torch
    if elem in ("bf16", "f16"):
        t = t.view(torch.int16)
        return t.cpu().numpy().view(np.uint16)
    if elem in ("f8E4M3FN", "f8E5M2"):
        return t.view(torch.uint8).cpu().numpy()
    if elem == "i1":
        return t.cpu().numpy().astype(np.bool_)
    return t.cpu().numpy()


def run_gpu(name, inputs, device, func=None):
    """Runs prebuilt catalog group `name` on the GPU; `inputs` holds one numpy
    array per group argument (outputs' initial contents included)."""
    art = hf.compile(hf.catalog.get(name), require_cached=True)
    grp = art.load(func)
    params = grp.meta["params"]
    devs = []
    for a, p in zip(inputs, params):
        devs.append(a if p["role"] == "scalar" else to_dev(a, p["elem"], device))
    out = grp(*devs)
    outs = out if isinstance(out, tuple) else (out,)
    import torch
    torch.cuda.synchronize()
    return [to_host(t, r["elem"]) for t, r in zip(outs, grp.meta["results"])]


def run_oracle(name, inputs, func=None, cast_semantics="declared"):
    return interp.run(hf.catalog.get(name), *inputs, func=func, cast_semantics=cast_semantics)


def bf16_ulp_diff(a, b):
    """|a - b| in bf16 units in the last place (same-sign finite values)."""
    ia = np.asarray(a, np.uint16).astype(np.int32)
    ib = np.asarray(b, np.uint16).astype(np.int32)
    # map sign-magnitude to a monotonic integer line
    ma = np.where(ia & 0x8000, -(ia & 0x7FFF), ia & 0x7FFF)
    mb = np.where(ib & 0x8000, -(ib & 0x7FFF), ib & 0x7FFF)
    return np.abs(ma - mb)
