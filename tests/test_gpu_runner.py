"""`bishengir-compile --enable-cpu-runner` on the MI355X: the runner's output
file must equal, byte for byte, the printData text of the oracle's results on
the inputs the runner wrote."""
import os
import subprocess

import numpy as np
import pytest

import hfusion_mi355x as hf
import group_catalog as cat
from hfusion_mi355x import native
from helpers import parse_data_file, print_data
from oracle import interp

pytestmark = pytest.mark.gpu
CLI = os.path.join(native.BIN_DIR, "bishengir-compile")


@pytest.mark.parametrize("name", ["vec_add_ragged", "prog_gemm_rmsnorm_quant_ragged"])
def test_runner_matches_oracle(name, tmp_path, gpu):
    print(f"[case] runner {name}", flush=True)
    ir = cat.get(name)
    (tmp_path / "m.mlir").write_text(ir)
    r = subprocess.run([CLI, "m.mlir", "-o", "m", "--enable-cpu-runner"], capture_output=True, text=True,
                       cwd=tmp_path, timeout=300)
    assert r.returncode == 0, r.stderr
    art = hf.compile(ir, require_cached=True)
    meta = art.programs[0] if art.programs else art.blocks[0]
    params, results = meta["params"], meta["results"]
    inputs = parse_data_file((tmp_path / "m.runner_inputs.txt").read_bytes(), [p["elem"] for p in params],
                             [p["shape"] for p in params])
    ref = interp.run(ir, *inputs)
    ref = ref if isinstance(ref, (list, tuple)) else [ref]
    expect = b"".join(print_data(o, res["elem"]) for o, res in zip(ref, results))
    assert (tmp_path / "m.runner_outputs.txt").read_bytes() == expect
