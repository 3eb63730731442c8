"""Dynamic dims (`?` in the group's types): shape specialisation.

The compiler makes every type static from the sizes of the function's
dynamic argument dims (option dyn=<func>:<arg>.<dim>=<size>,...); the host's
DynamicGroup reads those sizes from each call's tensors and compiles one code
object per size set.  CPU: the specialised group lowers to exactly the kernel
of the same group written with static types; missing or disagreeing sizes
are errors; the oracle runs the dynamic IR directly.  GPU: the dynamic groups
at several row counts against the oracle (through prebuilt code objects)."""
import ctypes
import os

import numpy as np
import pytest

import hfusion_mi355x as hf
import group_catalog as cat
from hfusion_mi355x.runtime import dynamic_dims
from helpers import bf16_ulp_diff, run_oracle, to_dev

G = hf.groups


def note(msg):
    print(f"[case] {msg}", flush=True)


def emit_hip(ir, options, tmp_path):
    """The generated HIP source (no hipcc), or the error."""
    err = ctypes.create_string_buffer(8192)
    os.makedirs(tmp_path, exist_ok=True)
    prefix = str(tmp_path / "g")
    rc = hf.native.hfc().hfc_compile(ir.encode(), prefix.encode(), ("emit=hip;" + options).encode(), err, len(err))
    if rc:
        return None, err.value.decode()
    return open(prefix + ".hip").read(), ""


@pytest.mark.parametrize("rows", [1, 37, 8192])
def test_specialised_equals_static(rows, tmp_path):
    dyn = cat.get("rmsnorm_quant_dyn")
    a, err = emit_hip(dyn, cat.dyn_options("rmsnorm_quant_dyn", rows), tmp_path / "a")
    assert a is not None, err
    b, err = emit_hip(G.rmsnorm_quant(rows, 4096), "", tmp_path / "b")
    assert a == b


def test_dynamic_dims_and_errors(tmp_path):
    dyn = cat.get("rmsnorm_quant_dyn")
    assert dynamic_dims(dyn) == [("rmsnorm_quant", 0, 0), ("rmsnorm_quant", 2, 0), ("rmsnorm_quant", 3, 0)]
    src, err = emit_hip(dyn, "", tmp_path)
    assert src is None and "has no size (compile with dyn=rmsnorm_quant:0.0=<size>)" in err
    src, err = emit_hip(dyn, "dyn=rmsnorm_quant:0.0=5,rmsnorm_quant:2.0=6,rmsnorm_quant:3.0=5", tmp_path)
    assert src is None and "disagree" in err
    src, err = emit_hip(dyn, "dyn=rmsnorm_quant:0.0", tmp_path)
    assert src is None and "bad dyn entry" in err
    # a dynamic host function the fusion front-end would split
    host = """func.func @h(%a: tensor<?x8xf32>, %o: tensor<?xf32>) -> tensor<?xf32>
    attributes {hacc.function_kind = #hacc.function_kind<HOST>} {
  %c0 = arith.constant 0 : index
  %d = tensor.dim %a, %c0 : tensor<?x8xf32>
  %z = arith.constant 0.0 : f32
  %e = tensor.empty(%d) : tensor<?x8xf32>
  %x = hfusion.elemwise_unary {fun = #hfusion.unary_fn<sqrt>} ins(%a : tensor<?x8xf32>) outs(%e : tensor<?x8xf32>) -> tensor<?x8xf32>
  %i = linalg.fill ins(%z : f32) outs(%o : tensor<?xf32>) -> tensor<?xf32>
  %s = linalg.reduce {arith.addf} ins(%x : tensor<?x8xf32>) outs(%i : tensor<?xf32>) dimensions = [1]
  %f = tensor.empty(%d) : tensor<?x8xf32>
  %c = hfusion.cast {round_mode = #hfusion.round_mode<rint>} ins(%s : tensor<?xf32>) outs(%o : tensor<?xf32>) -> tensor<?xf32>
  return %c : tensor<?xf32>
}"""
    src, err = emit_hip(host, "dyn=h:0.0=4,h:1.0=4", tmp_path)
    assert src is None and "must be one group" in err


def test_oracle_runs_dynamic_ir():
    rng = np.random.default_rng(5)
    for rows in (1, 37):
        x = (rng.standard_normal((rows, 4096)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
        g = (rng.uniform(0.5, 1.5, 4096).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
        args = [x, g, np.zeros((rows, 4096), np.int8), np.zeros(rows, np.float32)]
        q, s = run_oracle("rmsnorm_quant_dyn", args)
        from oracle import interp
        q2, s2 = interp.run(G.rmsnorm_quant(rows, 4096), *args)
        assert np.array_equal(q, q2) and np.array_equal(s.view(np.uint32), s2.view(np.uint32))


def _call(name, args, gpu):
    import torch
    dg = hf.DynamicGroup(cat.get(name), require_cached=True)
    g = dg.specialise(dg.sizes_of(args))
    devs = [to_dev(a, p["elem"], gpu) for a, p in zip(args, g.meta["params"])]
    out = dg(*devs)
    torch.cuda.synchronize()
    outs = out if isinstance(out, (list, tuple)) else [out]
    res = []
    for t in outs:
        if t.dtype == torch.bfloat16:
            t = t.view(torch.int16)
        res.append(t.cpu().numpy())
    return res


@pytest.mark.gpu
@pytest.mark.parametrize("rows", cat.DYN_ROWS["rmsnorm_quant_dyn"])
def test_gpu_rmsnorm_quant_dynamic(gpu, rows):
    note(f"rmsnorm_quant_dyn rows={rows}")
    rng = np.random.default_rng(rows)
    x = (rng.standard_normal((rows, 4096)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    g = (rng.uniform(0.5, 1.5, 4096).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    args = [x, g, np.zeros((rows, 4096), np.int8), np.zeros(rows, np.float32)]
    q, s = _call("rmsnorm_quant_dyn", args, gpu)
    rq, rs = run_oracle("rmsnorm_quant_dyn", args)
    assert np.array_equal(q, rq) and np.array_equal(s.view(np.uint32), rs.view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("rows", cat.DYN_ROWS["softmax_dyn"])
def test_gpu_softmax_dynamic(gpu, rows):
    note(f"softmax_dyn rows={rows}")
    x = np.random.default_rng(rows).normal(0, 2, (rows, 1000)).astype(np.float32)
    out, = _call("softmax_dyn", [x, np.zeros((rows, 1000), np.uint16)], gpu)
    ref, = run_oracle("softmax_dyn", [x, np.zeros((rows, 1000), np.uint16)])
    assert bf16_ulp_diff(out.view(np.uint16), ref).max() <= 1


@pytest.mark.gpu
@pytest.mark.parametrize("n", cat.DYN_ROWS["vec_add_dyn"])
def test_gpu_vec_add_dynamic(gpu, n):
    note(f"vec_add_dyn n={n}")
    rng = np.random.default_rng(n)
    a, b = rng.standard_normal(n).astype(np.float32), rng.standard_normal(n).astype(np.float32)
    out, = _call("vec_add_dyn", [a, b, np.zeros(n, np.float32)], gpu)
    assert np.array_equal(out, a + b)


def _half_ir(div):
    """A result of ceil(d / 2) (floordivsi) or floor(d / 2) (ceildivsi)
    elements, computed through a negative intermediate: 0 - div(0 - d, 2)."""
    return f"""module {{
  func.func @half(%x: tensor<?xf32>) -> tensor<?xf32>
      attributes {{hacc.entry, hfusion.fusion_kind = #hfusion.fusion_kind<PURE_ELEMWISE>}} {{
    %c0 = arith.constant 0 : index
    %c2 = arith.constant 2 : index
    %one = arith.constant 1.000000e+00 : f32
    %d = tensor.dim %x, %c0 : tensor<?xf32>
    %m = arith.subi %c0, %d : index
    %q = arith.{div} %m, %c2 : index
    %n = arith.subi %c0, %q : index
    %e = tensor.empty(%n) : tensor<?xf32>
    %r = linalg.fill ins(%one : f32) outs(%e : tensor<?xf32>) -> tensor<?xf32>
    return %r : tensor<?xf32>
  }}
}}
"""


@pytest.mark.parametrize("div,size", [("floordivsi", 4), ("ceildivsi", 3)])
def test_signed_division_folds_round_toward_minus_or_plus_infinity(div, size, tmp_path):
    """floordivsi(-7, 2) = -4 and ceildivsi(-7, 2) = -3 (arith's semantics,
    not C++'s truncation).  The folded size shows in the shape error the
    group then raises (its result and argument differ in length)."""
    hip, err = emit_hip(_half_ir(div), "dyn=half:0.0=7", tmp_path)
    assert hip is None and f"tensor<{size}xf32>" in err


@pytest.mark.parametrize("spec,msg", [("dyn=halff:0.0=7", "not a function"),
                                      ("dyn=half:0.1=7", "names no dynamic dim"),
                                      ("dyn=half:1.0=7", "names no dynamic dim")])
def test_dyn_entries_that_name_nothing_are_refused(spec, msg, tmp_path):
    hip, err = emit_hip(_half_ir("floordivsi"), spec, tmp_path)
    assert hip is None and msg in err
