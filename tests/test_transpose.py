"""linalg.transpose inside elementwise groups (catalog module transpose_ops
and the benchmarked transpose_cast group): the oracle against numpy closed
forms (CPU), then the LDS-tiled HIP kernels against the oracle, bit-exact
(GPU).  Meaning: out dim k is in dim perm[k] (linalg.transpose), and
elementwise ops commute with the permutation."""
import os

import numpy as np
import pytest

import hfusion_mi355x as hf
import group_catalog as cat
from helpers import run_gpu, run_oracle

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def note(msg):
    print(f"[case] {msg}", flush=True)


def bf16_bits_to_f32(b):
    return (np.asarray(b, np.uint32) << 16).view(np.float32)


def f32_to_bf16_rne(x):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def inputs(name, seed=0x5452):
    rng = np.random.default_rng(seed + sum(map(ord, name)))
    if name == "tr2d_cast":
        return [rng.integers(0, 65536, (300, 200)).astype(np.uint16) & 0xBFFF, np.zeros((200, 300), np.float32)]
    if name == "tr3d_add":
        return [np.abs(rng.normal(0, 3, (8, 96, 130))).astype(np.float32), rng.normal(0, 1, (8, 130, 96)).astype(np.float32),
                np.zeros((8, 130, 96), np.uint16)]
    if name == "tr3d_rot_i8":
        return [rng.integers(-128, 128, (16, 33, 64)).astype(np.int8), np.zeros((64, 16, 33), np.int32)]
    if name == "tr_unit":
        return [rng.normal(0, 1, (4, 1, 100)).astype(np.float32), np.zeros((4, 100, 1), np.float32)]
    raise KeyError(name)


def closed_form(name, args):
    if name == "tr2d_cast":
        return bf16_bits_to_f32(args[0]).T
    if name == "tr3d_add":
        t = np.transpose(np.sqrt(args[0]), (0, 2, 1)) + args[1]
        return f32_to_bf16_rne(t)
    if name == "tr3d_rot_i8":
        return np.transpose(args[0], (2, 0, 1)).astype(np.int32)
    if name == "tr_unit":
        return np.abs(args[0]).reshape(4, 100, 1)


@pytest.mark.parametrize("name", cat.TRANSPOSE_OPS)
def test_oracle_transpose(name):
    args = inputs(name)
    ref, = run_oracle("transpose_ops", args, func=name)
    want = closed_form(name, args)
    assert ref.shape == want.shape and np.array_equal(ref, want)


def test_reference_foldable_transpose_lowers(tmp_path):
    """compile-pure-elemwise-with-foldable-transpose.mlir:5-12: a transpose
    that only moves a unit dim, between an expand and a collapse, fused with a
    cast: one streaming kernel."""
    src = "/root/reference/bishengir/test/bishengir-compile/hfusion/compile-pure-elemwise-with-foldable-transpose.mlir"
    if not os.path.exists(src):
        pytest.skip("reference tree not present")
    art = hf.compile(open(src).read())
    assert art.blocks[0]["kind"] == "PURE_ELEMWISE"


def test_lowering_stages_transposed_inputs():
    kinds = {b["func"]: b.get("variant", "") for b in hf.compile(cat.get("transpose_ops")).blocks}
    assert "LDS-staged" in kinds["tr2d_cast"] and "LDS-staged" in kinds["tr3d_rot_i8"]
    assert kinds["tr_unit"] == "streaming"


@pytest.mark.gpu
@pytest.mark.parametrize("name", cat.TRANSPOSE_OPS)
def test_gpu_transpose(gpu, name):
    note(f"transpose_ops {name}")
    args = inputs(name)
    out, = run_gpu("transpose_ops", args, gpu, func=name)
    ref, = run_oracle("transpose_ops", args, func=name)
    assert np.array_equal(np.asarray(out).view(np.uint8), np.asarray(ref).view(np.uint8))


@pytest.mark.gpu
def test_gpu_transpose_cast_full(gpu):
    """The benchmarked group at its full shape, bf16 [4096, 8192] -> f32
    [8192, 4096]: bit-exact against the closed form (the cast is exact)."""
    note("transpose_cast 4096x8192")
    rng = np.random.default_rng(7)
    x = rng.integers(0, 65536, (4096, 8192), dtype=np.uint32).astype(np.uint16) & 0xBFFF
    out, = run_gpu("transpose_cast", [x, np.zeros((8192, 4096), np.float32)], gpu)
    assert np.array_equal(out, bf16_bits_to_f32(x).T)
