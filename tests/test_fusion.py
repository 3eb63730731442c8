"""CPU tests of the fusion front-end (libhfc: InferFuncFusionKind +
HFusionOpFusion + OutlineSingleOp as one pass) and of the launch programs it
plans.  No GPU calls.

Grouping decisions are pinned against the expectations of the reference's
own lit tests (bishengir/test/Dialect/HFusion/OpFusion/*.mlir): each case
below restates one of their inputs (static shapes) and the groups their CHECK
lines require.  The programs are pinned semantically: the oracle run over the
outlined groups in program order, with the planned buffers, must give the same
bytes as the oracle run over the un-fused function."""
import ctypes
import os
import re

import numpy as np
import pytest

import hfusion_mi355x as hf
import group_catalog as cat
from hfusion_mi355x import inputs as I
from hfusion_mi355x import native
from oracle import interp


# --------------------------------------------------------------- IR builder
class Host:
    """Builds an un-fused `func.func` in destination-passing form."""

    def __init__(self, name, args, host=True):
        self.name, self.args, self.host = name, args, host
        self.types = {a: t for a, t in args}
        self.lines, self.n = [], 0

    @staticmethod
    def T(shape, dt="f32"):
        return "tensor<" + "".join(f"{d}x" for d in shape) + dt + ">"

    def _out(self, t):
        self.n += 1
        e = f"e{self.n}"
        self.lines.append(f"%{e} = tensor.empty() : {t}")
        return e

    def unary(self, r, fn, x, ns="linalg"):
        t = self.types[x]
        e = self._out(t)
        self.lines.append(f"%{r} = {ns}.elemwise_unary {{fun = #{ns}.unary_fn<{fn}>}} ins(%{x} : {t}) "
                          f"outs(%{e} : {t}) -> {t}")
        self.types[r] = t
        return r

    def binary(self, r, fn, x, y, ns="linalg"):
        t = self.types[x]
        e = self._out(t)
        self.lines.append(f"%{r} = {ns}.elemwise_binary {{fun = #{ns}.binary_fn<{fn}>}} ins(%{x}, %{y} : {t}, "
                          f"{self.types[y]}) outs(%{e} : {t}) -> {t}")
        self.types[r] = t
        return r

    def reduce(self, r, x, dim):
        t = self.types[x]
        shape = [int(d) for d in re.findall(r"(\d+)x", t)]
        rt = self.T(shape[:dim] + shape[dim + 1:])
        e = self._out(rt)
        self.lines.append(f"%{r} = linalg.reduce {{arith.addf}} ins(%{x} : {t}) outs(%{e} : {rt}) dimensions = [{dim}]")
        self.types[r] = rt
        return r

    def bcast(self, r, x, dim, size=7):
        t = self.types[x]
        shape = [int(d) for d in re.findall(r"(\d+)x", t)]
        rt = self.T(shape[:dim] + [size] + shape[dim:])
        e = self._out(rt)
        self.lines.append(f"%{r} = linalg.broadcast ins(%{x} : {t}) outs(%{e} : {rt}) dimensions = [{dim}]")
        self.types[r] = rt
        return r

    def matmul(self, r, a, b, shape):
        rt = self.T(shape)
        e = self._out(rt)
        self.lines.append(f"%{r} = linalg.matmul ins(%{a}, %{b} : {self.types[a]}, {self.types[b]}) "
                          f"outs(%{e} : {rt}) -> {rt}")
        self.types[r] = rt
        return r

    def text(self, rets):
        sig = ", ".join(f"%{a}: {t}" for a, t in self.args)
        rt = ", ".join(self.types[r] for r in rets)
        attrs = " attributes {hacc.function_kind = #hacc.function_kind<HOST>}" if self.host else ""
        body = "\n    ".join(self.lines)
        return (f"module {{\n  func.func @{self.name}({sig}) -> ({rt}){attrs} {{\n    {body}\n"
                f"    return {', '.join('%' + r for r in rets)} : {rt}\n  }}\n}}\n")


def outline(ir, tmp_path, kind=None):
    """Runs the front-end only (emit=outlined); returns (groups, programs):
    groups = [(name, fusion kind, [op names])] in module order."""
    prefix = str(tmp_path / "o")
    err = ctypes.create_string_buffer(8192)
    opts = "emit=outlined" + (f";fusion_kind={kind}" if kind else "")
    rc = native.hfc().hfc_compile(ir.encode(), prefix.encode(), opts.encode(), err, len(err))
    assert rc == 0, err.value.decode()
    text = open(prefix + ".outlined.mlir").read()
    groups = []
    for m in re.finditer(r"func\.func @(\S+)\((.*?)\n  \}", text, re.S):
        k = re.search(r"fusion_kind<(\w+)>", m.group(2))
        ops = [o.split(".", 1)[1] for o in re.findall(r"= ((?:linalg|hfusion)\.\w+)", m.group(2))]
        groups.append((m.group(1), k.group(1) if k else None, ops))
    progs = hf.parse_manifest(prefix + ".programs", with_programs=True)[1] if os.path.getsize(
        prefix + ".programs") else []
    return groups, progs, text


def fused(groups):
    """name -> op list of the multi-op groups (single-op outlines dropped)."""
    return {n: ops for n, _, ops in groups if "_single_outlined_" not in n}


# ---------------------------------------------- reference lit-test pins
def chain_a():
    # test_static_chaincase.mlir:24-48 (testCaseChainA)
    h = Host("testCaseChainA", [("arg0", Host.T([7, 7, 7]))])
    h.unary("c", "ceil", "arg0"); h.unary("x", "exp", "c"); h.bcast("b", "x", 3)
    h.unary("f", "floor", "b"); h.unary("l", "log", "f"); h.reduce("r", "l", 3); h.unary("o", "log", "r")
    return h.text(["o"])


def chain_b():
    # test_static_chaincase.mlir:65-83 (testCaseChainB)
    h = Host("testCaseChainB", [("arg0", Host.T([7, 7, 7]))])
    h.reduce("r", "arg0", 2); h.unary("f", "floor", "r"); h.unary("n", "negf", "f")
    h.reduce("r2", "n", 1); h.unary("o", "ceil", "r2")
    return h.text(["o"])


def chain_c():
    # test_static_chaincase.mlir:100-119 (testCaseChainC)
    h = Host("testCaseChainC", [("arg0", Host.T([7, 7, 7]))])
    h.bcast("b", "arg0", 3); h.unary("c", "ceil", "b"); h.unary("f", "floor", "c")
    h.bcast("b2", "f", 4); h.unary("o", "log", "b2")
    return h.text(["o"])


def chain_d():
    # test_static_chaincase.mlir:148-183 (testCaseChainD)
    h = Host("testCaseChainD", [("arg0", Host.T([7, 7, 7]))])
    h.reduce("r", "arg0", 2); h.unary("l", "log", "r"); h.unary("n", "negf", "l"); h.bcast("b", "n", 2)
    h.unary("x", "exp", "b"); h.unary("n2", "negf", "x"); h.reduce("r2", "n2", 2); h.bcast("b2", "r2", 2)
    h.unary("c", "ceil", "b2"); h.unary("c2", "ceil", "c"); h.reduce("o", "c2", 2)
    return h.text(["o"])


U, B, R = "elemwise_unary", "broadcast", "reduce"


@pytest.mark.parametrize("ir,kind,expect", [
    # LASTAXIS / ELEMWISE prefixes of test_static_chaincase.mlir:6-19, 52-61, 88-96, 124-144
    (chain_a, "LAST_AXIS_PBR", {"testCaseChainA_0": [U, U, B, U, U, R, U]}),
    (chain_a, "PURE_ELEMWISE", {"testCaseChainA_0": [U, U], "testCaseChainA_1": [U, U]}),
    (chain_b, "LAST_AXIS_PBR", {"testCaseChainB_0": [R, U, U], "testCaseChainB_1": [R, U]}),
    (chain_b, "PURE_ELEMWISE", {"testCaseChainB_0": [U, U]}),
    (chain_c, "LAST_AXIS_PBR", {"testCaseChainC_0": [B, U, U, B, U]}),
    (chain_c, "PURE_ELEMWISE", {"testCaseChainC_0": [U, U]}),
    (chain_d, "LAST_AXIS_PBR", {"testCaseChainD_0": [R, U, U, B, U, U, R, B, U, U, R]}),
    (chain_d, "PURE_ELEMWISE", {"testCaseChainD_0": [U, U], "testCaseChainD_1": [U, U], "testCaseChainD_2": [U, U]}),
])
def test_chain_cases_match_reference(ir, kind, expect, tmp_path):
    groups, _, _ = outline(ir(), tmp_path, kind)
    assert fused(groups) == expect


def pp_case(name, second, dim):
    # test_static_reduce_broadcast.mlir testCasePPtoPR / PPtoRP / PPtoBP
    t = Host.T([7, 7, 7])
    h = Host(name, [("arg0", t), ("arg1", t), ("arg2", t)])
    h.binary("m", "mul", "arg0", "arg1")
    (h.reduce if second == "r" else h.bcast)("o", "m", dim)
    return h.text(["o"])


def rb_case(name, first, d1, second, d2, shape=(7, 7, 7)):
    # test_static_reduce_broadcast.mlir testCasePRtoPB / RPtoBP / PBtoPR / BPtoBP ...
    t = Host.T(list(shape))
    h = Host(name, [("arg0", t), ("arg1", t)])
    (h.reduce if first == "r" else h.bcast)("x", "arg0", d1)
    (h.reduce if second == "r" else h.bcast)("o", "x", d2)
    return h.text(["o"])


EB = "elemwise_binary"


@pytest.mark.parametrize("ir,expect", [
    # CHECK lines of test_static_reduce_broadcast.mlir (LAST_AXIS_PBR run)
    (lambda: pp_case("testCasePPtoPR", "r", 2), {"testCasePPtoPR_0": [EB, R]}),
    (lambda: pp_case("testCasePPtoRP", "r", 0), {}),          # CHECK-NOT @testCasePPtoRP_0
    (lambda: pp_case("testCasePPtoBP", "b", 0), {"testCasePPtoBP_0": [EB, B]}),
    (lambda: rb_case("testCasePRtoPB", "r", 2, "b", 2), {"testCasePRtoPB_0": [R, B]}),
    (lambda: rb_case("testCasePRtoBP", "r", 2, "b", 0), {"testCasePRtoBP_0": [R, B]}),
    (lambda: rb_case("testCaseRPtoBP", "r", 0, "b", 0), {}),   # CHECK-NOT @testCaseRPtoBP_0
    (lambda: rb_case("testCaseBPtoPR", "b", 0, "r", 3), {}),   # CHECK-NOT @testCaseBPtoPR_0
    (lambda: rb_case("testCaseBPtoBP", "b", 0, "b", 0), {"testCaseBPtoBP_0": [B, B]}),
    (lambda: rb_case("testCasePBtoBP", "b", 3, "b", 0), {"testCasePBtoBP_0": [B, B]}),
])
def test_reduce_broadcast_cases_match_reference(ir, expect, tmp_path):
    groups, _, _ = outline(ir(), tmp_path, "LAST_AXIS_PBR")
    assert fused(groups) == expect


def test_simple_case_single_group_two_outputs(tmp_path):
    # testCaseSimple: mul, add, sub, reduce[2], broadcast[2] -> one group
    # returning (reduce, broadcast) (test_static_reduce_broadcast.mlir:1-30)
    t = Host.T([7, 7, 7])
    h = Host("testCaseSimple", [("arg0", t), ("arg1", t), ("arg2", t)])
    h.binary("m", "mul", "arg0", "arg1"); h.binary("a", "add", "m", "arg2"); h.binary("s", "sub", "m", "a")
    h.reduce("r", "s", 2); h.bcast("b", "r", 2)
    groups, progs, text = outline(h.text(["r", "b"]), tmp_path, "LAST_AXIS_PBR")
    assert fused(groups) == {"testCaseSimple_0": [EB, EB, EB, R, B]}
    assert re.search(r"return %r, %b : tensor<7x7xf32>, tensor<7x7x7xf32>", text)
    (p,) = progs
    assert [s["group"] for s in p["steps"]] == ["testCaseSimple_0"]
    assert [r["tied"] for r in p["results"]] == [-1, -1] and p["workspace"] == 0


def test_mix_cv_single_output_split(tmp_path):
    """Multi-kernel order with MIX_CV split to single outputs: the matmul and
    the add it feeds form one group, the add's other consumers another
    (test_opfusion_multi_kernel.mlir main_mix_cv: MIX_CV_0 = matmul_transpose_b
    + elemwise_binary, MIX_CV_1 = hfusion.elemwise_binary + hfusion.cast)."""
    F16, F32 = Host.T([64, 256], "f16"), Host.T([64, 256], "f32")
    W = Host.T([256, 256], "f16")
    ir = f"""module {{
  func.func @main_mix_cv(%arg0: {F16}, %arg2: {F16}, %arg3: {W}) -> ({F16}, {F32})
      attributes {{hacc.entry, hacc.function_kind = #hacc.function_kind<HOST>}} {{
    %cst = arith.constant 2.000000e+00 : f16
    %0 = tensor.empty() : {F16}
    %1 = tensor.empty() : {F16}
    %2 = linalg.matmul_transpose_b ins(%arg2, %arg3 : {F16}, {W}) outs(%1 : {F16}) -> {F16}
    %3 = linalg.elemwise_binary {{fun = #linalg.binary_fn<add>}} ins(%arg0, %2 : {F16}, {F16}) outs(%0 : {F16}) -> {F16}
    %4 = hfusion.elemwise_binary {{fun = #hfusion.binary_fn<powf>}} ins(%3, %cst : {F16}, f16) outs(%0 : {F16}) -> {F16}
    %5 = tensor.empty() : {F32}
    %6 = hfusion.cast {{round_mode = #hfusion.round_mode<rint>}} ins(%4 : {F16}) outs(%5 : {F32}) -> {F32}
    return %3, %6 : {F16}, {F32}
  }}
}}
"""
    groups, progs, _ = outline(ir, tmp_path)
    assert fused(groups) == {"main_mix_cv_multi_MIX_CV_0": ["matmul_transpose_b", EB],
                             "main_mix_cv_multi_MIX_CV_1": [EB, "cast"]}
    assert {k for _, k, _ in groups} == {"MIX_CV"}


def test_zero_rank_group(tmp_path):
    """Zero-rank elementwise ops fuse with their producers
    (test_zero_rank_elemwise.mlir:1-30: cast, binary, fill, reduce, cast)."""
    X, S, SI = Host.T([16], "i32"), "tensor<f32>", "tensor<f32>"
    ir = f"""module {{
  func.func @zr(%x: {X}) -> tensor<f32> attributes {{hacc.function_kind = #hacc.function_kind<HOST>}} {{
    %zero = arith.constant 0.000000e+00 : f32
    %two = arith.constant 2.000000e+00 : f32
    %e0 = tensor.empty() : {Host.T([16])}
    %xf = hfusion.cast {{round_mode = #hfusion.round_mode<rint>}} ins(%x : {X}) outs(%e0 : {Host.T([16])}) -> {Host.T([16])}
    %e1 = tensor.empty() : {Host.T([16])}
    %m = linalg.elemwise_binary {{fun = #linalg.binary_fn<mul>}} ins(%xf, %two : {Host.T([16])}, f32) outs(%e1 : {Host.T([16])}) -> {Host.T([16])}
    %e2 = tensor.empty() : {S}
    %i = linalg.fill ins(%zero : f32) outs(%e2 : {S}) -> {S}
    %r = linalg.reduce {{arith.addf}} ins(%m : {Host.T([16])}) outs(%i : {S}) dimensions = [0]
    %e3 = tensor.empty() : {SI}
    %o = linalg.elemwise_unary {{fun = #linalg.unary_fn<exp>}} ins(%r : {S}) outs(%e3 : {SI}) -> {SI}
    return %o : tensor<f32>
  }}
}}
"""
    groups, _, _ = outline(ir, tmp_path)
    (ops,) = fused(groups).values()
    assert ops == ["cast", EB, "fill", R, U]


def test_inference_keeps_declared_groups(tmp_path):
    """A function that already carries hfusion.fusion_kind is one kernel: the
    front-end leaves the module untouched and plans no program."""
    groups, progs, text = outline(cat.get("rmsnorm_quant_256"), tmp_path)
    assert progs == [] and [g[0] for g in groups] == ["rmsnorm_quant"]


def test_single_kind_host_function_is_one_group(tmp_path):
    """InferFuncFusionKind: a host function whose ops fit one kind becomes one
    group named <func>_0 (test_pure_elemwise.mlir model_0)."""
    h = Host("model_0", [("arg0", Host.T([5, 1]))])
    h.unary("n", "negf", "arg0"); h.unary("x", "exp", "n"); h.binary("o", "add", "x", "arg0")
    groups, progs, _ = outline(h.text(["o"]), tmp_path)
    assert groups == [("model_0_0", "PURE_ELEMWISE", [U, U, EB])]
    assert [s["group"] for s in progs[0]["steps"]] == ["model_0_0"]


# ------------------------------------------------------------- programs
def test_program_plan_of_gemm_rmsnorm_quant(tmp_path):
    groups, progs, text = outline(cat.get("prog_gemm_rmsnorm_quant"), tmp_path)
    assert [(n, k) for n, k, _ in groups] == [("gemm_rmsnorm_quant_multi_MIX_CV_0", "MIX_CV"),
                                            ("gemm_rmsnorm_quant_multi_LAST_AXIS_PBR_0", "LAST_AXIS_PBR")]
    # the zero fill of the accumulator is emitted inside the contraction's
    # group, not as a kernel of its own
    assert groups[0][2] == ["fill", "matmul_transpose_b", "cast", EB]
    (p,) = progs
    assert p["workspace"] == 256 * 512 * 4
    assert [t["shape"] for t in p["temps"]] == [(256, 512)]
    s0, s1 = p["steps"]
    assert s0["args"] == ["p0", "p1"] and s0["results"] == ["t0"]
    assert "t0" in s1["args"] and sorted(s1["results"]) == ["p3", "p4"]
    assert [r["tied"] for r in p["results"]] == [3, 4]


def run_program_on_oracle(ir, args, tmp_path):
    """Executes the planned program with the oracle group by group."""
    groups, progs, text = outline(ir, tmp_path)
    (p,) = progs
    bufs = {f"p{i}": a.copy() for i, a in enumerate(args)}
    for j, t in enumerate(p["temps"]):
        bufs[f"t{j}"] = None
    for j, r in enumerate(p["results"]):
        if r["tied"] < 0:
            bufs[f"r{j}"] = None
    for st in p["steps"]:
        outs = interp.run(text, *[bufs[a] for a in st["args"]], func=st["group"])
        outs = outs if isinstance(outs, (list, tuple)) else [outs]
        for b, o in zip(st["results"], outs):
            bufs[b] = np.asarray(o)
    return [bufs[f"p{r['tied']}"] if r["tied"] >= 0 else bufs[f"r{j}"] for j, r in enumerate(p["results"])]


def gemm_args(m, n, k):
    s = I.SEED_BASE + 70
    return [I.int8_uniform(s, (m, k)), I.int8_uniform(s + 1, (n, k)), I.uniform_bf16(s + 2, (n,), 0.5, 1.5),
            np.zeros((m, n), np.int8), np.zeros(m, np.float32)]


def scores_args(m, n, k):
    s = I.SEED_BASE + 80
    return [I.normal_bf16(s, (m, k)), I.normal_bf16(s + 1, (n, k)), np.zeros((m, n), np.uint16)]


@pytest.mark.parametrize("name,make,shape", [
    ("prog_gemm_rmsnorm_quant", gemm_args, (256, 512, 256)),
    ("prog_gemm_rmsnorm_quant_ragged", gemm_args, (100, 320, 192)),
    ("prog_scores_softmax", scores_args, (128, 1024, 128)),
    ("prog_scores_softmax_ragged", scores_args, (72, 1000, 64)),
])
def test_program_equals_unfused_function_on_oracle(name, make, shape, tmp_path):
    ir = cat.get(name)
    args = make(*shape)
    whole = interp.run(ir, *[a.copy() for a in args])
    whole = whole if isinstance(whole, (list, tuple)) else [whole]
    split = run_program_on_oracle(ir, args, tmp_path)
    for w, s in zip(whole, split):
        assert w.dtype == s.dtype and np.array_equal(w.view(np.uint8), s.view(np.uint8))


# ---------------------------------------------------------------- errors
def test_in_place_update_read_later_is_rejected(tmp_path):
    """A group that writes into a tensor a later group still reads would
    clobber it: the front-end refuses instead of miscompiling."""
    t = Host.T([64, 64])
    R1 = Host.T([64])
    ir = f"""module {{
  func.func @clobber(%x: {t}, %r: {R1}) -> ({t}, {R1}) attributes {{hacc.function_kind = #hacc.function_kind<HOST>}} {{
    %a = linalg.elemwise_unary {{fun = #linalg.unary_fn<exp>}} ins(%x : {t}) outs(%x : {t}) -> {t}
    %e = tensor.empty() : {t}
    %m = linalg.matmul ins(%x, %a : {t}, {t}) outs(%e : {t}) -> {t}
    %s = linalg.reduce {{arith.addf}} ins(%x : {t}) outs(%r : {R1}) dimensions = [1]
    return %m, %s : {t}, {R1}
  }}
}}
"""
    prefix = str(tmp_path / "c")
    err = ctypes.create_string_buffer(8192)
    rc = native.hfc().hfc_compile(ir.encode(), prefix.encode(), b"emit=outlined", err, len(err))
    assert rc == -2 and b"updated in place" in err.value


def test_unplaceable_op_is_rejected(tmp_path):
    t = Host.T([8, 8])
    ir = f"""module {{
  func.func @f(%x: {t}) -> {t} attributes {{hacc.function_kind = #hacc.function_kind<HOST>}} {{
    %a = linalg.elemwise_unary {{fun = #linalg.unary_fn<exp>}} ins(%x : {t}) outs(%x : {t}) -> {t}
    %b = "some.op"(%a) : ({t}) -> {t}
    return %b : {t}
  }}
}}
"""
    prefix = str(tmp_path / "u")
    err = ctypes.create_string_buffer(8192)
    rc = native.hfc().hfc_compile(ir.encode(), prefix.encode(), b"emit=outlined", err, len(err))
    assert rc != 0
