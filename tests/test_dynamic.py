"""Dynamic dims (`?` in the group's types): shape specialisation.

The compiler makes every type static from the sizes of the function's
dynamic argument dims (option dyn=<func>:<arg>.<dim>=<size>,...); the host's
DynamicGroup reads those sizes from each call's tensors and compiles one code
object per size set.  CPU: the specialised group lowers to exactly the kernel
of the same group written with static types; missing or disagreeing sizes
are errors; the oracle runs the dynamic IR directly.  GPU: the dynamic groups
at several row counts against the oracle (through prebuilt code objects).

Runtime row counts (option dyn=runtime, catalog names ending in _rt): one
kernel for every row count, the count passed at launch
(hfr_group_launch_rows, or read from memref descriptors).  CPU: the
manifest marks the row dims and the launch rule, the kernel source holds no
row count, and groups whose kernels cannot take one are refused.  GPU: each
such group at several row counts, through the same code object, against the
oracle."""
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
    dg = hf.DynamicGroup(cat.get(name), require_cached=True, runtime=name.endswith("_rt"))
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


# ------------------------------------------------------------- runtime rows
RT = ["rmsnorm_quant_dyn_rt", "softmax_dyn_rt", "eltwise_mix_dyn_rt", "w8a8_dyn_rt", "argmax_dyn_rt", "mx_fp4_dyn_rt"]


@pytest.mark.parametrize("name", RT)
def test_runtime_rows_manifest(name, tmp_path):
    art = hf.compile(cat.get(name), options=cat.options(name))
    b = art.blocks[0]
    assert "rows_dyn" in b and b["kargs"][-1] == "rows", b
    for p in b["params"] + b["results"]:
        assert p["shape"].count(-1) <= 1 and (-1 not in p["shape"] or p["shape"][0] == -1), p
    assert any(-1 in p["shape"] for p in b["params"])
    src, err = emit_hip(cat.get(name), cat.options(name), tmp_path)
    assert src is not None, err
    from hfusion_mi355x import native  # noqa: F401
    assert str(1 << 30) not in src and str((1 << 30) - 1) not in src
    assert "hf_rows" in src
    if b["rows_dyn"][0] > 0:
        assert b["grid"][0] == 1  # set at launch from the row count


def test_runtime_rows_refusals(tmp_path):
    # a rank-1 streaming group: its vector chunks would straddle the end
    _, err = emit_hip(cat.get("vec_add_dyn"), "dyn=runtime", tmp_path / "a")
    assert "compiled per size" in err, err
    # a dynamic dim other than dim 0
    ir = """module {
  func.func @f(%x: tensor<4x?xf32>, %y: tensor<4x?xf32>) -> tensor<4x?xf32>
      attributes {hacc.entry, hfusion.fusion_kind = #hfusion.fusion_kind<PURE_ELEMWISE>} {
    %r = linalg.elemwise_unary {fun = #linalg.unary_fn<exp>} ins(%x : tensor<4x?xf32>) outs(%y : tensor<4x?xf32>) -> tensor<4x?xf32>
    return %r : tensor<4x?xf32>
  }
}
"""
    _, err = emit_hip(ir, "dyn=runtime", tmp_path / "b")
    assert "is not dim 0" in err, err
    # a size derived from the row count, not the count itself
    ir2 = """module {
  func.func @g(%x: tensor<?x8xf32>) -> tensor<?xf32>
      attributes {hacc.entry, hfusion.fusion_kind = #hfusion.fusion_kind<PURE_ELEMWISE>} {
    %c = tensor.collapse_shape %x [[0, 1]] : tensor<?x8xf32> into tensor<?xf32>
    return %c : tensor<?xf32>
  }
}
"""
    _, err = emit_hip(ir2, "dyn=runtime", tmp_path / "c")
    assert err and ("derived from the row count" in err or "compiled per size" in err), err


@pytest.mark.gpu
@pytest.mark.parametrize("rows", [1, 37, 300, 4100])
def test_gpu_runtime_rows_rmsnorm_quant(gpu, rows):
    note(f"rmsnorm_quant_dyn_rt rows={rows}")
    rng = np.random.default_rng(1000 + rows)
    x = (rng.standard_normal((rows, 4096)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    g = (rng.uniform(0.5, 1.5, 4096).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    args = [x, g, np.zeros((rows, 4096), np.int8), np.zeros(rows, np.float32)]
    q, s = _call("rmsnorm_quant_dyn_rt", args, gpu)
    rq, rs = run_oracle("rmsnorm_quant_dyn", args)
    assert np.array_equal(q, rq) and np.array_equal(s.view(np.uint32), rs.view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("rows", [1, 5, 129, 1000])
def test_gpu_runtime_rows_softmax(gpu, rows):
    note(f"softmax_dyn_rt rows={rows}")
    x = np.random.default_rng(2000 + rows).normal(0, 2, (rows, 1000)).astype(np.float32)
    out, = _call("softmax_dyn_rt", [x, np.zeros((rows, 1000), np.uint16)], gpu)
    ref, = run_oracle("softmax_dyn", [x, np.zeros((rows, 1000), np.uint16)])
    assert bf16_ulp_diff(out.view(np.uint16), ref).max() <= 1


@pytest.mark.gpu
@pytest.mark.parametrize("rows", [1, 67, 333])
def test_gpu_runtime_rows_eltwise(gpu, rows):
    """Row and column broadcasts through the streaming kernel with a runtime
    row count (bf16 out within 1 ulp: exp; the i1 mask bit-exact)."""
    note(f"eltwise_mix_dyn_rt rows={rows}")
    I = hf.inputs
    s = I.SEED_BASE + 3000 + rows
    x, b, sc = I.normal_f32(s, (rows, 1000)), I.normal_f32(s + 1, (1000,)), I.uniform_f32(s + 2, (rows,), 0.5, 2.0)
    args = [x, b, sc, np.zeros((rows, 1000), np.uint16), np.zeros((rows, 1000), np.bool_)]
    y, mask = _call("eltwise_mix_dyn_rt", args, gpu)
    ry, rmask = run_oracle("eltwise_mix_dyn_rt", args)
    assert np.array_equal(mask.astype(bool), rmask.astype(bool))
    assert bf16_ulp_diff(y.view(np.uint16), ry).max() <= 1


@pytest.mark.gpu
def test_gpu_runtime_rows_memref_and_errors(gpu):
    """The memref entry reads the row count from the descriptors; a launch
    whose arguments disagree on it, hfr_group_launch on a runtime-rows group
    and a negative count are refused."""
    import torch
    from hfusion_mi355x import native
    note("softmax_dyn_rt memref rows=77")
    rows = 77
    art = hf.compile(cat.get("softmax_dyn_rt"), options=cat.options("softmax_dyn_rt"), require_cached=True)
    grp = art.load()
    x = np.random.default_rng(7).normal(0, 2, (rows, 1000)).astype(np.float32)
    xd = torch.from_numpy(x).to(gpu)
    od = torch.zeros((rows, 1000), dtype=torch.int16, device=gpu)

    class Desc(ctypes.Structure):
        _fields_ = [("allocated", ctypes.c_void_p), ("aligned", ctypes.c_void_p), ("offset", ctypes.c_int64),
                    ("sizes", ctypes.c_int64 * 2), ("strides", ctypes.c_int64 * 2)]
    dx = Desc(xd.data_ptr(), xd.data_ptr(), 0, (rows, 1000), (1000, 1))
    do = Desc(od.data_ptr(), od.data_ptr(), 0, (rows, 1000), (1000, 1))
    descs = (ctypes.c_void_p * 2)(ctypes.addressof(dx), ctypes.addressof(do))
    lib = native.hfr()
    stream = torch.cuda.current_stream(gpu).cuda_stream
    native.check(lib.hfr_group_launch_memref(grp._h, descs, 2, stream))
    torch.cuda.synchronize()
    ref, = run_oracle("softmax_dyn", [x, np.zeros((rows, 1000), np.uint16)])
    assert bf16_ulp_diff(od.cpu().numpy().view(np.uint16), ref).max() <= 1
    # disagreeing row counts
    do2 = Desc(od.data_ptr(), od.data_ptr(), 0, (rows - 1, 1000), (1000, 1))
    descs2 = (ctypes.c_void_p * 2)(ctypes.addressof(dx), ctypes.addressof(do2))
    assert lib.hfr_group_launch_memref(grp._h, descs2, 2, stream) == -1
    assert b"rows" in lib.hfr_last_error()
    slots = (ctypes.c_uint64 * 2)(xd.data_ptr(), od.data_ptr())
    res = (ctypes.c_void_p * 1)(None)
    assert lib.hfr_group_launch(grp._h, slots, 2, res, 1, None, stream) != 0
    assert b"row count at launch" in lib.hfr_last_error()
    assert lib.hfr_group_launch_rows(grp._h, slots, 2, res, 1, -5, None, stream) != 0
    # the Python launch refuses arguments that disagree
    with pytest.raises(ValueError):
        grp(xd, torch.zeros((rows + 1, 1000), dtype=torch.bfloat16, device=gpu))
    torch.cuda.synchronize()


@pytest.mark.gpu
@pytest.mark.parametrize("rows", [1, 100, 333, 1000])
def test_gpu_runtime_rows_w8a8(gpu, rows):
    """W8A8 with the token count M at launch (B [N, K] weights, K = N = 512):
    bit-exact bf16 against the oracle for ragged and multiple-of-tile M."""
    note(f"w8a8_dyn_rt M={rows}")
    rng = np.random.default_rng(4000 + rows)
    a = rng.integers(-127, 128, (rows, 512), dtype=np.int8)
    b = rng.integers(-127, 128, (512, 512), dtype=np.int8)
    st = rng.uniform(0.001, 0.02, rows).astype(np.float32)
    sc = rng.uniform(0.001, 0.02, 512).astype(np.float32)
    args = [a, b, st, sc, np.zeros((rows, 512), np.uint16)]
    out, = _call("w8a8_dyn_rt", args, gpu)
    ref, = run_oracle("w8a8_dyn_rt", args)
    assert np.array_equal(out.view(np.uint16), ref.view(np.uint16))


@pytest.mark.gpu
@pytest.mark.parametrize("rows", [1, 100, 333, 600])
def test_gpu_runtime_rows_mx_fp4(gpu, rows):
    """Block-scaled fp4 with the row count M at launch (A [M, K/2] bytes, its
    scales [M, K/32], C [M, N]); against the oracle at the fp4 bar."""
    note(f"mx_fp4_dyn_rt M={rows}")
    from test_matmul_mx import fp4_case, fp4_products, TOL_FP4
    rng = np.random.default_rng(6000 + rows)
    a, b, sa, sb, ca, cb = fp4_case(rng, rows, 256, 512)
    out, = _call("mx_fp4_dyn_rt", [a, b, sa, sb], gpu)
    ref, = run_oracle("mx_fp4_dyn_rt", [a, b, sa, sb])
    mag, _ = fp4_products(ca, cb, sa, sb)
    assert np.all(np.abs(out.astype(np.float64) - ref) <= TOL_FP4 * mag + 1e-30)


@pytest.mark.gpu
@pytest.mark.parametrize("rows", [1, 7, 255, 256, 600])
def test_gpu_runtime_rows_argmax(gpu, rows):
    """argmax over [rows, 50000] logits with the row count at launch: split
    rows below one row per CU, a workgroup per row from 256 rows on; values
    and first-index ties bit-exact (a NaN row and an all -inf row included)."""
    note(f"argmax_dyn_rt rows={rows}")
    x = hf.inputs.argmax_logits(hf.inputs.SEED_BASE + 5000 + rows, rows, 50000, dup_every=3)
    if rows >= 7:
        x[5, 1234] = np.nan
        x[6, :] = -np.inf
    args = [x, np.zeros(rows, np.float32), np.zeros(rows, np.int32)]
    v, i = _call("argmax_dyn_rt", args, gpu)
    rv, ri = run_oracle("argmax_dyn_rt", args)
    assert np.array_equal(v.view(np.uint32), rv.view(np.uint32)) or \
        (np.array_equal(np.isnan(v), np.isnan(rv)) and np.array_equal(v[~np.isnan(v)], rv[~np.isnan(rv)]))
    assert np.array_equal(i, ri)
