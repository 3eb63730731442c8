"""The device runner behind `bishengir-compile --enable-cpu-runner*`: input
generation (the reference runner's std::mt19937(1) per element type,
BiShengIRRunnerUtils.cpp:62-68, 103-125), the printData text format and the
option checks.  CPU only; the GPU run is in test_gpu_runner.py."""
import os
import subprocess

import numpy as np
import pytest

import hfusion_mi355x as hf
from hfusion_mi355x import native
from helpers import parse_data_file, print_data

CLI = os.path.join(native.BIN_DIR, "bishengir-compile")


def mt19937_seed1(n):
    """The first n outputs of std::mt19937(1): numpy's legacy RandomState
    seeds MT19937 with the same init_genrand(1)."""
    u = np.random.RandomState(1).randint(0, 2 ** 32, size=n, dtype=np.uint64).astype(np.uint32)
    assert u[0] == 1791095845  # the published first output for seed 1
    return u


def uniform_float(u, lo, hi):
    """libstdc++ uniform_real_distribution<float>: generate_canonical<float, 24>
    takes one 32-bit draw, float(u) / 2^32 (clamped below 1), then
    r * (hi - lo) + lo in float."""
    r = u.astype(np.float32) / np.float32(2 ** 32)
    r = np.where(r >= 1, np.nextafter(np.float32(1), np.float32(0)), r).astype(np.float32)
    return (r * np.float32(hi - lo) + np.float32(lo)).astype(np.float32)


def bf16_rne(f):
    u = f.astype(np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def run_cli(args, tmp_path):
    return subprocess.run([CLI] + args, capture_output=True, text=True, cwd=tmp_path)


def test_inputs_follow_the_reference_generator(tmp_path):
    """Two f32 arguments continue one f32 stream; a bf16 argument has a stream
    of its own (function-local static generator per element type)."""
    X, G = "tensor<7x5xf32>", "tensor<5xbf16>"
    ir = f"""module {{
  func.func @k(%a: {X}, %g: {G}, %b: {X}) -> {X} attributes {{hacc.function_kind = #hacc.function_kind<HOST>}} {{
    %e = tensor.empty() : tensor<5xf32>
    %gf = hfusion.cast {{round_mode = #hfusion.round_mode<rint>}} ins(%g : {G}) outs(%e : tensor<5xf32>) -> tensor<5xf32>
    %e1 = tensor.empty() : {X}
    %bg = linalg.broadcast ins(%gf : tensor<5xf32>) outs(%e1 : {X}) dimensions = [0]
    %e2 = tensor.empty() : {X}
    %m = linalg.elemwise_binary {{fun = #linalg.binary_fn<mul>}} ins(%a, %bg : {X}, {X}) outs(%e2 : {X}) -> {X}
    %o = linalg.elemwise_binary {{fun = #linalg.binary_fn<add>}} ins(%m, %b : {X}, {X}) outs(%b : {X}) -> {X}
    return %o : {X}
  }}
}}
"""
    (tmp_path / "k.mlir").write_text(ir)
    r = run_cli(["k.mlir", "-o", "k", "--enable-cpu-runner-after=hfusion-fuse-ops,1,wrapper-name=main_wrapper"],
                tmp_path)
    raw = (tmp_path / "k.runner_inputs.txt").read_bytes()
    a, g, b = parse_data_file(raw, ["f32", "bf16", "f32"], [(7, 5), (5,), (7, 5)])
    u = mt19937_seed1(70)
    assert np.array_equal(a.reshape(-1).view(np.uint32), uniform_float(u[:35], -1000, 1000).view(np.uint32))
    assert np.array_equal(b.reshape(-1).view(np.uint32), uniform_float(u[35:70], -1000, 1000).view(np.uint32))
    assert np.array_equal(g, bf16_rne(uniform_float(u[:5], -100, 100)))
    # the text is exactly what printData writes for these values
    assert raw == print_data(a, "f32") + print_data(g, "bf16") + print_data(b, "f32")
    # without a GPU the run stops at the first device call, after the inputs
    assert r.returncode == 0 or "[Runner]" in r.stderr


def test_print_data_int8_is_raw_bytes():
    out = print_data(np.array([[65, -1]], np.int8), "i8")
    assert out == b"2\n1 2\nA \xff\n"
    (back,) = parse_data_file(out, ["i8"], [(1, 2)])
    assert back.tolist() == [[65, -1]]


@pytest.mark.parametrize("flags,msg", [
    (["--enable-cpu-runner", "--enable-cpu-runner-after=cse"], "Cannot combine"),
    (["--enable-cpu-runner-before=cse,0"], "positive non-zero"),
    (["--enable-cpu-runner-after="], "pass name"),
    (["--enable-cpu-runner-after=not a pass"], "is not a pass"),
])
def test_runner_option_errors(flags, msg, tmp_path):
    (tmp_path / "v.mlir").write_text(hf.groups.vec_add(8))
    r = run_cli(["v.mlir", "-o", "v"] + flags, tmp_path)
    assert r.returncode != 0 and "[ERROR]" in r.stderr and msg in r.stderr
