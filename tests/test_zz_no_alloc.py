"""hfr_group_launch_noalloc: the same results as hfr_group_launch, with the
library's static per-device scratch in place of the group's workspace.

Two calls in a row, the second on a smaller input, for each kind of kernel
that takes a workspace: split-row reduce_with_index (per-segment records and
arrival counters) and histogram (u64 bins, zeroed before the call).  Each
output is compared bit-exactly with hfr_group_launch on the same inputs."""
import numpy as np
import pytest

import hfusion_mi355x as hf
import group_catalog as cat
from hfusion_mi355x import native
from helpers import misc_inputs, to_dev, to_host

pytestmark = pytest.mark.gpu
I = hf.inputs


def note(msg):
    print(f"[case] {msg}", flush=True)


def _run(name, inputs, device, func=None, noalloc=False):
    import torch
    grp = hf.compile(cat.get(name), require_cached=True).load(func)
    devs = [a if p["role"] == "scalar" else to_dev(a, p["elem"], device) for a, p in zip(inputs, grp.meta["params"])]
    out = grp(*devs, noalloc=noalloc)
    torch.cuda.synchronize()
    outs = out if isinstance(out, tuple) else (out,)
    return [to_host(t, r["elem"]) for t, r in zip(outs, grp.meta["results"])], grp


def _same(a, b):
    assert len(a) == len(b)
    for x, y in zip(a, b):
        assert x.dtype == y.dtype and x.shape == y.shape
        assert np.array_equal(np.asarray(x).view(np.uint8), np.asarray(y).view(np.uint8))


@pytest.mark.parametrize("big,small", [(("argmax_16", 16, 152064), ("argmax_ragged", 5, 1001)),
                                       (("argmin_ragged", 9, 5001), ("argmax_ragged", 5, 1001))])
def test_noalloc_argreduce_matches(gpu, big, small):
    for name, rows, cols in (big, small):
        note(f"noalloc {name} {rows}x{cols}")
        x = I.argmax_logits(I.SEED_BASE + 40 + rows, rows, cols, dup_every=1)
        if name.startswith("argmin"):
            x = -x
        x[rows // 2, cols // 3] = np.nan
        args = [x, np.zeros(rows, np.float32), np.zeros(rows, np.int32)]
        ref, grp = _run(name, args, gpu)
        assert 0 < grp.info.workspace_bytes <= native.hfr().hfr_scratch_bytes()
        got, _ = _run(name, args, gpu, noalloc=True)
        _same(got, ref)


def test_noalloc_histogram_matches(gpu):
    native_bytes = native.hfr().hfr_scratch_bytes()
    for name in ("hist_mask_i64", "hist_i8_wrap"):  # the second is the smaller input
        note(f"noalloc {name}")
        args = misc_inputs(name)
        ref, grp = _run("misc_ops", args, gpu, func=name)
        assert 0 < grp.info.workspace_bytes <= native_bytes
        got, _ = _run("misc_ops", args, gpu, func=name, noalloc=True)
        _same(got, ref)


def test_noalloc_without_workspace(gpu):
    """A group without a workspace launches as usual."""
    note("noalloc vec_add_ragged")
    a, b = I.config_inputs("vec_add", n=1001)
    ref, grp = _run("vec_add_ragged", [a, b, np.zeros(1001, np.float32)], gpu)
    got, _ = _run("vec_add_ragged", [a, b, np.zeros(1001, np.float32)], gpu, noalloc=True)
    _same(got, ref)
