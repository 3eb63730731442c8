"""CPU-side tests of the compiler (libhfc / bishengir-compile) and of the
C-ABI libraries: IR reading, group classification, manifests, error paths,
exported symbols.  No GPU calls."""
import ctypes
import os
import re
import subprocess

import pytest

import hfusion_mi355x as hf
import group_catalog as cat
from hfusion_mi355x import native

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLI = os.path.join(native.BIN_DIR, "bishengir-compile")


def emit(ir, tmp_path, name="g", options=""):
    prefix = str(tmp_path / name)
    err = ctypes.create_string_buffer(8192)
    rc = native.hfc().hfc_compile(ir.encode(), prefix.encode(), ("emit=hip;" + options).encode(), err, len(err))
    return rc, err.value.decode(), prefix


def header_symbols(path):
    txt = open(path).read()
    return set(re.findall(r"^\s*(?:const\s+)?[\w\s\*]+?\b(hf[cr]_\w+)\s*\(", txt, re.M))


@pytest.mark.parametrize("lib,header", [("libhfr.so", "hfr.h"), ("libhfc.so", "hfc.h")])
def test_library_exports_every_declared_symbol(lib, header):
    syms = header_symbols(os.path.join(REPO, "include", header))
    assert syms, header
    L = ctypes.CDLL(os.path.join(native.LIB_DIR, lib))
    for s in syms:
        assert hasattr(L, s), f"{lib} does not export {s}"


def test_runtime_error_paths_without_gpu():
    r = native.hfr()
    h = ctypes.c_void_p()
    assert r.hfr_group_load(b"/nonexistent.manifest", None, ctypes.byref(h)) == -3
    assert b"cannot open" in r.hfr_last_error()
    assert r.hfr_group_launch(None, None, 0, None, 0, None, None) == -1
    assert r.hfr_module_load(None, ctypes.byref(h)) == -1


def test_manifest_rejects_garbage(tmp_path):
    p = tmp_path / "bad.manifest"
    p.write_text("not a manifest\n")
    h = ctypes.c_void_p()
    assert native.hfr().hfr_group_load(str(p).encode(), None, ctypes.byref(h)) == -4


@pytest.mark.parametrize("name", sorted(cat.entries()))
def test_every_catalog_group_lowers(name, tmp_path):
    rc, err, prefix = emit(cat.get(name), tmp_path, options=cat.options(name))
    assert rc == 0, err
    blocks = hf.parse_manifest(prefix + ".manifest")
    for b in blocks:
        assert b["kernel"].startswith("hf_")
        assert b["grid"][0] >= 1 and b["block"][0] in (64, 128, 256, 512, 1024) or b["block"][0] % 64 == 0
        # every result is either written into an argument or has its own karg
        for j, r in enumerate(b["results"]):
            assert r["tied"] >= 0 or f"result:{j}" in b["kargs"]


def test_classification_and_ties(tmp_path):
    expect = {"vec_add": "PURE_ELEMWISE", "eltwise_mix": "ANY_PB", "rmsnorm_quant": "LAST_AXIS_PBR",
              "safe_softmax": "LAST_AXIS_PBR", "argmax": "REDUCE_WITH_INDEX", "w8a8_dequant": "SINGLE_CUBE"}
    for name, kind in expect.items():
        rc, err, prefix = emit(cat.get(name), tmp_path, name)
        assert rc == 0, err
        b = hf.parse_manifest(prefix + ".manifest")[0]
        assert b["kind"] == kind, name
    b = hf.parse_manifest(str(tmp_path / "rmsnorm_quant") + ".manifest")[0]
    assert [r["tied"] for r in b["results"]] == [2, 3]
    assert "binade-run exact serial sum" in b["variant"]
    assert b["algo_bytes"] == 100704256
    b = hf.parse_manifest(str(tmp_path / "w8a8_dequant") + ".manifest")[0]
    assert b["algo_ops"] == 2 * 4096 ** 3
    b = hf.parse_manifest(str(tmp_path / "argmax") + ".manifest")[0]
    assert b["workspace"] > 0 and b["workspace_zero"] and b["kargs"][-1] == "ws"


def test_untied_result_gets_its_own_buffer(tmp_path):
    T = "tensor<128xf32>"
    ir = f"""func.func @f(%a: {T}) -> {T} attributes {{hacc.entry}} {{
  %e = tensor.empty() : {T}
  %r = hfusion.elemwise_unary {{fun = #hfusion.unary_fn<sqrt>}} ins(%a : {T}) outs(%e : {T}) -> {T}
  return %r : {T}
}}"""
    rc, err, prefix = emit(ir, tmp_path)
    assert rc == 0, err
    b = hf.parse_manifest(prefix + ".manifest")[0]
    assert b["results"][0]["tied"] == -1 and b["kargs"] == ["param:0", "result:0"]


def test_reference_rms_norm_test_ir_lowers(tmp_path):
    """The reference's own fused RMSNorm group (compile-rms-norm-fp32-split-n.mlir,
    restated here: tensor.dim/index_castui/uitofp/divf scalar folding,
    `__N__` unit attributes, `tensor<256 x128xf32>` spelling)."""
    ir = """#map = affine_map<(d0) -> (d0)>
module {
func.func @rms_norm_f32(%x: tensor<256x128xf32>, %gamma: tensor<128xf32>, %out0: tensor<256x128xf32>, %out1: tensor<256xf32>) -> (tensor<256x128xf32>, tensor<256xf32>)
   attributes {hacc.entry, hacc.function_kind = #hacc.function_kind<DEVICE>, hfusion.fusion_kind = #hfusion.fusion_kind<LAST_AXIS_PBR>} {
      %c0 = arith.constant 0 : index
      %c1 = arith.constant 1 : index
      %dim0 = tensor.dim %x, %c0 : tensor<256x128xf32>
      %dim1 = tensor.dim %x, %c1 : tensor<256x128xf32>
      %epsilon = arith.constant 1.000000e-01 : f32
      %empty0 = tensor.empty() : tensor<256x128xf32>
      %squrare = linalg.elemwise_binary {__1__, fun = #linalg.binary_fn<mul>} ins(%x, %x : tensor<256x128xf32>, tensor<256x128xf32>) outs(%empty0 : tensor<256x128xf32>) -> tensor<256x128xf32>
      %empty1 = tensor.empty() : tensor<256xf32>
      %sum0 = linalg.reduce {arith.addf} ins(%squrare : tensor<256x128xf32>) outs(%empty1 : tensor<256xf32>) dimensions = [1] {__2__}
      %empty2 = tensor.empty() : tensor<256xf32>
      %c1f = arith.constant 1.0 : f32
      %dim1ui = arith.index_castui %dim1 : index to i32
      %dim1f = arith.uitofp %dim1ui : i32 to f32
      %avg_factor = arith.divf %c1f, %dim1f : f32
      %mean = linalg.elemwise_binary {fun = #linalg.binary_fn<mul>, __3__} ins(%sum0, %avg_factor : tensor<256xf32>, f32) outs(%empty2 : tensor<256xf32>) -> tensor<256xf32>
      %empty3 = tensor.empty() : tensor<256xf32>
      %sum1 = linalg.elemwise_binary {fun = #linalg.binary_fn<add>, __4__} ins(%mean, %epsilon : tensor<256xf32>, f32) outs(%empty3 : tensor<256xf32>) -> tensor<256xf32>
      %empty4 = tensor.empty() : tensor<256xf32>
      %sqrt = hfusion.elemwise_unary {fun = #hfusion.unary_fn<sqrt>, __5__} ins(%sum1 : tensor<256xf32>) outs(%empty4 : tensor<256xf32>) -> tensor<256xf32>
      %rsqrt = hfusion.elemwise_unary {fun = #hfusion.unary_fn<rec>, __6__} ins(%sqrt : tensor<256xf32>) outs(%out1 : tensor<256xf32>) -> tensor<256xf32>
      %empty6 = tensor.empty() : tensor<256 x128xf32>
      %brc_rsqrt = linalg.broadcast ins(%rsqrt : tensor<256xf32>) outs(%empty6 : tensor<256x128xf32>) dimensions = [1] {__7__}
      %empty7 = tensor.empty() : tensor<256x128xf32>
      %mul0 = linalg.elemwise_binary {fun = #linalg.binary_fn<mul>, __8__} ins(%brc_rsqrt, %x : tensor<256x128xf32>, tensor<256x128xf32>) outs(%empty7 : tensor<256x128xf32>) -> tensor<256x128xf32>
      %empty8 = tensor.empty() : tensor<256x128xf32>
      %brc_gamma = linalg.broadcast ins(%gamma : tensor<128xf32>) outs(%empty8 : tensor<256x128xf32>) dimensions = [0] {__9__}
      %mul1 = linalg.elemwise_binary {fun = #linalg.binary_fn<mul>, __10__} ins(%brc_gamma, %mul0 : tensor<256x128xf32>, tensor<256x128xf32>) outs(%out0 : tensor<256x128xf32>) -> tensor<256x128xf32>
      return %mul1, %rsqrt : tensor<256x128xf32>, tensor<256xf32>
   }
}"""
    rc, err, prefix = emit(ir, tmp_path)
    assert rc == 0, err
    b = hf.parse_manifest(prefix + ".manifest")[0]
    assert b["kind"] == "LAST_AXIS_PBR" and [r["tied"] for r in b["results"]] == [2, 3]
    src = open(prefix + ".hip").read()
    assert "0x1p-7f" in src  # 1/128 folded from tensor.dim -> uitofp -> divf


HIVM_OPS_MLIR = """// hivm.hir.matmul as written in bishengir/test/Dialect/HIVM/IR/ops.mlir:135-149
func.func @test_matmul_descale_perchannel(%A_gm : memref<16x16xf16, #hivm.address_space<gm>>,
                               %B_gm :  memref<16x16xf16, #hivm.address_space<gm>>,
                               %bias_gm : memref<16xf16, #hivm.address_space<gm>>,
                               %descale_perchannel_gm :  memref<16xf16, #hivm.address_space<gm>>,
                               %res_gm :memref<16x16xf16, #hivm.address_space<gm>> ) {
  hivm.hir.matmul
       ins(%A_gm, %B_gm:
           memref<16x16xf16, #hivm.address_space<gm>>, memref<16x16xf16, #hivm.address_space<gm>>)
       outs(%res_gm : memref<16x16xf16, #hivm.address_space<gm>>)
       bias = %bias_gm : memref<16xf16, #hivm.address_space<gm>>
       descale = %descale_perchannel_gm :  memref<16xf16, #hivm.address_space<gm>>
       descale_mode = #hivm.descale_mode<DescalePerChannel>
  return
}
"""


def test_hivm_matmul_reference_form_lowers(tmp_path):
    """The destination-style op on memrefs: the `outs` argument is the written
    result (tied), bias and descale are per-column loads of the epilogue."""
    rc, err, prefix = emit(HIVM_OPS_MLIR, tmp_path)
    assert rc == 0, err
    b = hf.parse_manifest(prefix + ".manifest")[0]
    assert b["kind"] == "SINGLE_CUBE" and "f16" in b["variant"]
    assert [p["role"] for p in b["params"]] == ["in", "in", "in", "in", "out"]
    assert [r["tied"] for r in b["results"]] == [4]
    src = open(prefix + ".hip").read()
    assert "Cv.bias" in src and "Cv.descale" in src and "hf::f32_to_f16<0>(t)" in src


@pytest.mark.parametrize("ir,code,msg", [
    (HIVM_OPS_MLIR.replace("       descale = %descale_perchannel_gm :  memref<16xf16, #hivm.address_space<gm>>\n", ""), -2,
     "descale operand and descale_mode disagree"),
    (HIVM_OPS_MLIR.replace("xf16", "xf64"), -2, "matmul element types"),
    ("func.func @f(%a: tensor<?xf32>) -> tensor<?xf32> { return %a : tensor<?xf32> }", -1, "dynamic shapes"),
    ("module { }", -1, "no func.func"),
    ("""func.func @test_isfinite() -> tensor<8192xi1> {
  %0 = tensor.empty() : tensor<8192xf32>
  %2 = hfusion.isfinite %0 : tensor<8192xf32> -> tensor<8192xi1>
  return %2 : tensor<8192xi1>
}""", -2, "uninitialised contents of tensor.empty"),
    ("""func.func @f(%a: tensor<4x8xf32>, %o: tensor<8xf32>, %p: tensor<4xf32>) -> (tensor<8xf32>, tensor<4xf32>)
    attributes {hacc.entry, hfusion.fusion_kind = #hfusion.fusion_kind<ANY_PBR>} {
  %r = linalg.reduce {arith.addf} ins(%a : tensor<4x8xf32>) outs(%o : tensor<8xf32>) dimensions = [0]
  %s = linalg.reduce {arith.addf} ins(%a : tensor<4x8xf32>) outs(%p : tensor<4xf32>) dimensions = [1]
  return %r, %s : tensor<8xf32>, tensor<4xf32>
}""", -2, "different dimensions"),
    ("""func.func @f(%a: tensor<4xi32>, %o: tensor<4xi32>) -> tensor<4xi32> {
  %r = hfusion.elemwise_unary {fun = #hfusion.unary_fn<lgamma>} ins(%a : tensor<4xi32>) outs(%o : tensor<4xi32>) -> tensor<4xi32>
  return %r : tensor<4xi32>
}""", -2, "lgamma"),
    ("""func.func @f(%a: tensor<4xi32>, %o: tensor<4xf64>) -> tensor<4xf64> {
  %r = hfusion.elemwise_unary {fun = #hfusion.unary_fn<tan>, cast = #hfusion.type_fn<bitcast>} ins(%a : tensor<4xi32>) outs(%o : tensor<4xf64>) -> tensor<4xf64>
  return %r : tensor<4xf64>
}""", -2, "bitcast"),
    ("""func.func @f(%a: tensor<4xf32>) -> tensor<4xf32> {
  return %b : tensor<4xf32>
}""", -1, "undefined value"),
    ("""func.func @deinterleave_rank0(%arg0: tensor<f32>) -> tensor<f32> {
  %res = hfusion.deinterleave %arg0 channel<0> : tensor<f32> -> tensor<f32>
  return %res : tensor<f32>
}""", -2, "rank-0"),
])
def test_compile_errors(ir, code, msg, tmp_path):
    rc, err, _ = emit(ir, tmp_path)
    assert rc == code and msg in err, (rc, err)


def test_cli_contract(tmp_path):
    src = tmp_path / "add.mlir"
    src.write_text(hf.groups.vec_add(4096))
    out = tmp_path / "add"
    r = subprocess.run([CLI, str(src), "-enable-hfusion-compile", "-block-dim=40", "--target=mi355x", "--emit=hip",
                        "-o", str(out)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    assert (tmp_path / "add.manifest").exists() and (tmp_path / "add.hip").exists()
    bad = subprocess.run([CLI, str(tmp_path / "missing.mlir")], capture_output=True, text=True)
    assert bad.returncode != 0 and bad.stderr.startswith("[ERROR]")
    unk = subprocess.run([CLI, str(src), "--frobnicate"], capture_output=True, text=True)
    assert unk.returncode != 0 and "[ERROR] unknown option" in unk.stderr
    tgt = subprocess.run([CLI, str(src), "--target=ascend910b"], capture_output=True, text=True)
    assert tgt.returncode != 0 and "unsupported target" in tgt.stderr


def test_cli_builds_code_object(tmp_path):
    """Full path through hipcc (cross-compiles for gfx950 without a GPU)."""
    src = tmp_path / "add.mlir"
    src.write_text(hf.groups.vec_add(4096))
    r = subprocess.run([CLI, str(src), "-o", str(tmp_path / "add")], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    assert (tmp_path / "add.hsaco").stat().st_size > 1000


def test_host_api_validates_before_launch():
    """Shape/dtype mismatches are rejected on the host, before any GPU call."""
    import torch
    art = hf.compile(cat.get("vec_add_ragged"))
    meta = art.blocks[0]
    assert meta["params"][0]["shape"] == (1001,)
    g = object.__new__(hf.Group)
    g.meta, g.func = meta, "vec_add"
    with pytest.raises(TypeError):
        g(torch.zeros(1001), torch.zeros(1001))
    with pytest.raises(TypeError):  # host tensors are refused
        g(torch.zeros(1001), torch.zeros(1001), torch.zeros(1001))


def test_memref_form_groups_compile(tmp_path):
    """Destination-style ops on memrefs with a bare `return` (no SSA results):
    each written buffer becomes a result tied to its argument, and a later
    read of a buffer sees the value written to it."""
    ir = """func.func @f(%src : memref<6xf32>, %dst : memref<6xi32>) {
  hfusion.bitcast ins(%src : memref<6xf32>) outs(%dst : memref<6xi32>)
  return
}"""
    rc, err, prefix = emit(ir, tmp_path)
    assert rc == 0, err
    man = open(prefix + ".manifest").read()
    assert "result 0 1 i32 1 6" in man, man
    rc, err, prefix = emit(cat.get("memref_chain"), tmp_path, "chain")
    assert rc == 0, err
    man = open(prefix + ".manifest").read()
    assert "result 0 1 f32" in man and "result 1 2 f32" in man, man


def test_generic_after_reshape_does_not_crash(tmp_path):
    """A linalg.generic fed by an expand_shape, with scalar operands mapped by
    `() ` maps: compiled or rejected with an error code, never a crash."""
    ir = """#map = affine_map<(d0, d1) -> (d0, d1)>
#scalar_map = affine_map<(d0, d1) -> ()>
func.func @f(%arg0: tensor<64xi1>) -> tensor<64x1xf32> {
  %t = arith.constant 1.000000e+00 : f32
  %f = arith.constant 0.000000e+00 : f32
  %x = tensor.expand_shape %arg0 [[0, 1]] output_shape [64, 1] : tensor<64xi1> into tensor<64x1xi1>
  %e = tensor.empty() : tensor<64x1xf32>
  %r = linalg.generic {indexing_maps = [#map, #scalar_map, #scalar_map, #map], iterator_types = ["parallel", "parallel"]}
      ins(%x, %t, %f : tensor<64x1xi1>, f32, f32) outs(%e : tensor<64x1xf32>) {
  ^bb0(%in: i1, %a: f32, %b: f32, %out: f32):
    %s = arith.select %in, %a, %b : f32
    linalg.yield %s : f32
  } -> tensor<64x1xf32>
  return %r : tensor<64x1xf32>
}"""
    rc, err, _ = emit(ir, tmp_path)
    assert rc in (0, -1, -2), (rc, err)


@pytest.mark.parametrize("decl", [
    'func.func private @triton_print(f32) -> f32 attributes {msg = "x", hex = false}',
    "func.func private @g(tensor<4xf32>, i32) attributes {llvm.emit_c_interface}",
    "func.func private @h() -> (f32, i32)",
    "func.func private @k(%a: f32) -> f32 attributes {msg = \"named\"}",
])
def test_external_declarations_are_skipped(decl, tmp_path):
    """External declarations (with or without an attributes dict, with named,
    unnamed or no arguments) carry no body and lower to nothing."""
    ir = "module {\n  " + decl + "\n" + hf.groups.vec_add(64).split("module {", 1)[1]
    rc, err, prefix = emit(ir, tmp_path)
    assert rc == 0, err
    assert [b["func"] for b in hf.parse_manifest(prefix + ".manifest")] == ["vec_add"]
