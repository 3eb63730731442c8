"""HFusion group IR for the workloads this backend is measured on.

Each function returns the textual MLIR of one outlined, already-fused HFusion
group (``func.func`` tagged ``hacc.entry`` and ``hfusion.fusion_kind``), in the
form the reference's fusion stage hands to its device compiler
(``bishengir/test/bishengir-compile/hfusion/compile-rms-norm-fp32-split-n.mlir:5-47``
for a LAST_AXIS_PBR group).  The IR is the contract: the CPU oracle and the
GPU kernel both execute exactly these ops.
"""

_ATTRS = ("attributes {{hacc.entry, hacc.function_kind = #hacc.function_kind<DEVICE>, "
          "hfusion.fusion_kind = #hfusion.fusion_kind<{kind}>}}")


def _t(shape, dt):
    return "tensor<" + "".join(f"{d}x" for d in shape) + dt + ">"


def vec_add(n=1 << 24, dtype="f32"):
    """HIVM VecAdd (bishengir/test/Integration/HIVM/VecAdd/add.mlir) as the
    HFusion elementwise group `out = a + b`."""
    t = _t([n], dtype)
    return f"""module {{
  func.func @vec_add(%a: {t}, %b: {t}, %out: {t}) -> {t}
      {_ATTRS.format(kind='PURE_ELEMWISE')} {{
    %0 = linalg.elemwise_binary {{fun = #linalg.binary_fn<add>}} ins(%a, %b : {t}, {t}) outs(%out : {t}) -> {t}
    return %0 : {t}
  }}
}}
"""


def with_dynamic_rows(ir, rows):
    """The same group with its leading (row) dim `rows` dynamic: every type
    `tensor<rows x ...>` spelled `tensor<? x ...>`, and every tensor.empty of
    such a type sized by `tensor.dim` of the first argument (`rows` must be a
    number no other dim of the group uses)."""
    import re
    out = ir.replace(f"<{rows}x", "<?x")
    m = re.search(r"func\.func @\w+\((%[\w]+): (tensor<[^>]*>)", out)
    arg, ty = m.group(1), m.group(2)
    out = out.replace("tensor.empty() : tensor<?x", "tensor.empty(%rows_) : tensor<?x")
    j = out.index("{\n", m.end()) + 2  # the body's first line
    return out[:j] + f"    %c0_ = arith.constant 0 : index\n    %rows_ = tensor.dim {arg}, %c0_ : {ty}\n" + out[j:]


def rmsnorm_quant(rows=8192, cols=4096, eps=1e-6, batch=None):
    """RMSNorm (structure of compile-rms-norm-fp32-split-n.mlir:5-47) followed by
    dynamic per-token int8 quantisation with explicit rounding
    (nearbyint -> clamp +-127 -> cast), so the CPU lowering's truncating
    fptosi and the declared RINT cast agree."""
    lead = [batch, rows // batch] if batch else [rows]  # [B, S, H] when batched
    X, G = _t(lead + [cols], "bf16"), _t([cols], "bf16")
    XF, GF, RF = _t(lead + [cols], "f32"), _t([cols], "f32"), _t(lead, "f32")
    Q = _t(lead + [cols], "i8")
    rdim, gdims = len(lead), ", ".join(str(i) for i in range(len(lead)))
    e = f"{eps:.9e}"
    return f"""module {{
  func.func @rmsnorm_quant(%x: {X}, %gamma: {G}, %q: {Q}, %scale: {RF}) -> ({Q}, {RF})
      {_ATTRS.format(kind='LAST_AXIS_PBR')} {{
    %zero = arith.constant 0.000000e+00 : f32
    %cols = arith.constant {float(cols):.6e} : f32
    %eps = arith.constant {e} : f32
    %qmax = arith.constant 1.270000e+02 : f32
    %qmin = arith.constant -1.270000e+02 : f32
    %e0 = tensor.empty() : {XF}
    %xf = hfusion.cast {{round_mode = #hfusion.round_mode<rint>}} ins(%x : {X}) outs(%e0 : {XF}) -> {XF}
    %e1 = tensor.empty() : {XF}
    %sq = linalg.elemwise_binary {{fun = #linalg.binary_fn<mul>}} ins(%xf, %xf : {XF}, {XF}) outs(%e1 : {XF}) -> {XF}
    %e2 = tensor.empty() : {RF}
    %i2 = linalg.fill ins(%zero : f32) outs(%e2 : {RF}) -> {RF}
    %ss = linalg.reduce {{arith.addf}} ins(%sq : {XF}) outs(%i2 : {RF}) dimensions = [{rdim}]
    %e3 = tensor.empty() : {RF}
    %mean = linalg.elemwise_binary {{fun = #linalg.binary_fn<div>}} ins(%ss, %cols : {RF}, f32) outs(%e3 : {RF}) -> {RF}
    %e4 = tensor.empty() : {RF}
    %ms = linalg.elemwise_binary {{fun = #linalg.binary_fn<add>}} ins(%mean, %eps : {RF}, f32) outs(%e4 : {RF}) -> {RF}
    %e5 = tensor.empty() : {RF}
    %rt = hfusion.elemwise_unary {{fun = #hfusion.unary_fn<sqrt>}} ins(%ms : {RF}) outs(%e5 : {RF}) -> {RF}
    %e6 = tensor.empty() : {RF}
    %inv = hfusion.elemwise_unary {{fun = #hfusion.unary_fn<rec>}} ins(%rt : {RF}) outs(%e6 : {RF}) -> {RF}
    %e7 = tensor.empty() : {XF}
    %binv = linalg.broadcast ins(%inv : {RF}) outs(%e7 : {XF}) dimensions = [{rdim}]
    %e8 = tensor.empty() : {XF}
    %y1 = linalg.elemwise_binary {{fun = #linalg.binary_fn<mul>}} ins(%xf, %binv : {XF}, {XF}) outs(%e8 : {XF}) -> {XF}
    %e9 = tensor.empty() : {GF}
    %gf = hfusion.cast {{round_mode = #hfusion.round_mode<rint>}} ins(%gamma : {G}) outs(%e9 : {GF}) -> {GF}
    %e10 = tensor.empty() : {XF}
    %bg = linalg.broadcast ins(%gf : {GF}) outs(%e10 : {XF}) dimensions = [{gdims}]
    %e11 = tensor.empty() : {XF}
    %y = linalg.elemwise_binary {{fun = #linalg.binary_fn<mul>}} ins(%y1, %bg : {XF}, {XF}) outs(%e11 : {XF}) -> {XF}
    %e12 = tensor.empty() : {XF}
    %ay = linalg.elemwise_unary {{fun = #linalg.unary_fn<abs>}} ins(%y : {XF}) outs(%e12 : {XF}) -> {XF}
    %e13 = tensor.empty() : {RF}
    %i13 = linalg.fill ins(%zero : f32) outs(%e13 : {RF}) -> {RF}
    %amax = linalg.reduce {{arith.maximumf}} ins(%ay : {XF}) outs(%i13 : {RF}) dimensions = [{rdim}]
    %sc = linalg.elemwise_binary {{fun = #linalg.binary_fn<div>}} ins(%amax, %qmax : {RF}, f32) outs(%scale : {RF}) -> {RF}
    %e14 = tensor.empty() : {XF}
    %bsc = linalg.broadcast ins(%sc : {RF}) outs(%e14 : {XF}) dimensions = [{rdim}]
    %e15 = tensor.empty() : {XF}
    %ys = linalg.elemwise_binary {{fun = #linalg.binary_fn<div>}} ins(%y, %bsc : {XF}, {XF}) outs(%e15 : {XF}) -> {XF}
    %e16 = tensor.empty() : {XF}
    %r = hfusion.elemwise_unary {{fun = #hfusion.unary_fn<nearbyint>}} ins(%ys : {XF}) outs(%e16 : {XF}) -> {XF}
    %e17 = tensor.empty() : {XF}
    %c1 = hfusion.elemwise_binary {{fun = #hfusion.binary_fn<minf>}} ins(%r, %qmax : {XF}, f32) outs(%e17 : {XF}) -> {XF}
    %e18 = tensor.empty() : {XF}
    %c2 = hfusion.elemwise_binary {{fun = #hfusion.binary_fn<maxf>}} ins(%c1, %qmin : {XF}, f32) outs(%e18 : {XF}) -> {XF}
    %qv = hfusion.cast {{round_mode = #hfusion.round_mode<rint>}} ins(%c2 : {XF}) outs(%q : {Q}) -> {Q}
    return %qv, %sc : {Q}, {RF}
  }}
}}
"""


def safe_softmax(rows=4096, cols=32768):
    """Safe softmax (structure of bishengir/test/Dialect/HFusion/regbase/
    Normalize/hfusion-normalize-reduction-ops.mlir:262-277 with a maximumf
    reduce) and a final f32 -> bf16 cast (round to nearest even)."""
    X, R, O = _t([rows, cols], "f32"), _t([rows], "f32"), _t([rows, cols], "bf16")
    return f"""module {{
  func.func @safe_softmax(%x: {X}, %out: {O}) -> {O}
      {_ATTRS.format(kind='LAST_AXIS_PBR')} {{
    %zero = arith.constant 0.000000e+00 : f32
    %ninf = arith.constant 0xFF800000 : f32
    %e0 = tensor.empty() : {R}
    %i0 = linalg.fill ins(%ninf : f32) outs(%e0 : {R}) -> {R}
    %m = linalg.reduce {{arith.maximumf}} ins(%x : {X}) outs(%i0 : {R}) dimensions = [1]
    %e1 = tensor.empty() : {X}
    %bm = linalg.broadcast ins(%m : {R}) outs(%e1 : {X}) dimensions = [1]
    %e2 = tensor.empty() : {X}
    %d = linalg.elemwise_binary {{fun = #linalg.binary_fn<sub>}} ins(%x, %bm : {X}, {X}) outs(%e2 : {X}) -> {X}
    %e3 = tensor.empty() : {X}
    %ex = linalg.elemwise_unary {{fun = #linalg.unary_fn<exp>}} ins(%d : {X}) outs(%e3 : {X}) -> {X}
    %e4 = tensor.empty() : {R}
    %i4 = linalg.fill ins(%zero : f32) outs(%e4 : {R}) -> {R}
    %s = linalg.reduce {{arith.addf}} ins(%ex : {X}) outs(%i4 : {R}) dimensions = [1]
    %e5 = tensor.empty() : {X}
    %bs = linalg.broadcast ins(%s : {R}) outs(%e5 : {X}) dimensions = [1]
    %e6 = tensor.empty() : {X}
    %p = linalg.elemwise_binary {{fun = #linalg.binary_fn<div>}} ins(%ex, %bs : {X}, {X}) outs(%e6 : {X}) -> {X}
    %o = hfusion.cast {{round_mode = #hfusion.round_mode<rint>}} ins(%p : {X}) outs(%out : {O}) -> {O}
    return %o : {O}
  }}
}}
"""


def argmax(rows=256, cols=152064, index_type="i32", kind="max"):
    """reduce_with_index <max> (or <min>) over the last axis, init (-inf, 0)
    (+inf for <min>) as in bishengir/test/Dialect/HFusion/canonicalize.mlir:231-237."""
    X, V, I = _t([rows, cols], "f32"), _t([rows], "f32"), _t([rows], index_type)
    return f"""module {{
  func.func @argmax(%x: {X}, %val: {V}, %idx: {I}) -> ({V}, {I})
      {_ATTRS.format(kind='LAST_AXIS_PBR')} {{
    %c0 = arith.constant 0 : {index_type}
    %ninf = arith.constant {'0xFF800000' if kind == 'max' else '0x7F800000'} : f32
    %v0 = linalg.fill ins(%ninf : f32) outs(%val : {V}) -> {V}
    %i0 = linalg.fill ins(%c0 : {index_type}) outs(%idx : {I}) -> {I}
    %r:2 = hfusion.reduce_with_index {{tie_break_left = true}} <{kind}> ins(%x : {X}) outs(%v0, %i0 : {V}, {I}) dimensions = [1] -> {V}, {I}
    return %r#0, %r#1 : {V}, {I}
  }}
}}
"""


def w8a8_dequant(m=4096, n=4096, k=4096, b_layout="nk"):
    """W8A8 contraction (hivm.hir.matmul, B in the [N, K] weight layout, or
    [K, N] with b_layout="kn" through linalg.matmul) with the per-token x
    per-channel dequant epilogue in IR order:
    bf16((sitofp(C) * s_tok[m]) * s_ch[n])."""
    A, B = _t([m, k], "i8"), (_t([n, k], "i8") if b_layout == "nk" else _t([k, n], "i8"))
    mm = "linalg.matmul_transpose_b" if b_layout == "nk" else "linalg.matmul"
    C, CF, O = _t([m, n], "i32"), _t([m, n], "f32"), _t([m, n], "bf16")
    ST, SC = _t([m], "f32"), _t([n], "f32")
    return f"""module {{
  func.func @w8a8_dequant(%a: {A}, %b: {B}, %s_tok: {ST}, %s_ch: {SC}, %out: {O}) -> {O}
      {_ATTRS.format(kind='SINGLE_CUBE')} {{
    %c0 = arith.constant 0 : i32
    %e0 = tensor.empty() : {C}
    %acc0 = linalg.fill ins(%c0 : i32) outs(%e0 : {C}) -> {C}
    %acc = {mm} ins(%a, %b : {A}, {B}) outs(%acc0 : {C}) -> {C}
    %e1 = tensor.empty() : {CF}
    %cf = hfusion.cast {{round_mode = #hfusion.round_mode<rint>}} ins(%acc : {C}) outs(%e1 : {CF}) -> {CF}
    %e2 = tensor.empty() : {CF}
    %bt = linalg.broadcast ins(%s_tok : {ST}) outs(%e2 : {CF}) dimensions = [1]
    %e3 = tensor.empty() : {CF}
    %t = linalg.elemwise_binary {{fun = #linalg.binary_fn<mul>}} ins(%cf, %bt : {CF}, {CF}) outs(%e3 : {CF}) -> {CF}
    %e4 = tensor.empty() : {CF}
    %bc = linalg.broadcast ins(%s_ch : {SC}) outs(%e4 : {CF}) dimensions = [0]
    %e5 = tensor.empty() : {CF}
    %u = linalg.elemwise_binary {{fun = #linalg.binary_fn<mul>}} ins(%t, %bc : {CF}, {CF}) outs(%e5 : {CF}) -> {CF}
    %o = hfusion.cast {{round_mode = #hfusion.round_mode<rint>}} ins(%u : {CF}) outs(%out : {O}) -> {O}
    return %o : {O}
  }}
}}
"""


def mm_i8(m=4096, n=4096, k=4096):
    """int8 x int8 -> int32 contraction (B in the [N, K] weight layout) with no
    epilogue: the exact accumulator is the group's output."""
    A, B, C = _t([m, k], "i8"), _t([n, k], "i8"), _t([m, n], "i32")
    return f"""module {{
  func.func @mm_i8(%a: {A}, %b: {B}, %c: {C}) -> {C}
      {_ATTRS.format(kind='SINGLE_CUBE')} {{
    %c0 = arith.constant 0 : i32
    %acc0 = linalg.fill ins(%c0 : i32) outs(%c : {C}) -> {C}
    %acc = linalg.matmul_transpose_b ins(%a, %b : {A}, {B}) outs(%acc0 : {C}) -> {C}
    return %acc : {C}
  }}
}}
"""


def hivm_matmul(m, n, k, elem="f16", out="f16", bias=None, descale=None, descale_mode=None, a_t=False, b_t=False,
                name="hivm_matmul"):
    """hivm.hir.matmul on global memrefs (HIVMMacroOps.td:410-446), written like
    bishengir/test/Dialect/HIVM/IR/ops.mlir:135-167: C = descale * (A*B + bias)
    with optional bias [n], descale [n] (per channel) or [1] (per tensor), and
    optional a_transpose / b_transpose."""
    gm = ", #hivm.address_space<gm>"
    mr = lambda shape, e: "memref<" + "".join(f"{d}x" for d in shape) + e + gm + ">"
    A = mr([k, m] if a_t else [m, k], elem)
    B = mr([n, k] if b_t else [k, n], elem)
    C = mr([m, n], out)
    args = [f"%A_gm: {A}", f"%B_gm: {B}"]
    extra = []
    if bias:
        args.append(f"%bias_gm: {mr([n], bias)}")
        extra.append(f"bias = %bias_gm : {mr([n], bias)}")
    if descale:
        dshape = [n] if descale_mode == "DescalePerChannel" else [1]
        args.append(f"%descale_gm: {mr(dshape, descale)}")
        extra.append(f"descale = %descale_gm : {mr(dshape, descale)}")
    if a_t:
        extra.append("a_transpose")
    if b_t:
        extra.append("b_transpose")
    extra.append(f"descale_mode = #hivm.descale_mode<{descale_mode or 'DescaleNull'}>")
    args.append(f"%res_gm: {C}")
    tail = "\n       ".join(extra)
    return f"""module {{
  func.func @{name}({", ".join(args)}) {{
    hivm.hir.matmul
       ins(%A_gm, %B_gm : {A}, {B})
       outs(%res_gm : {C})
       {tail}
    return
  }}
}}
"""


def bf16_mmad(m=4096, n=4096, k=4096, b_layout="nk", elem="bf16"):
    """bf16 (or f16) contraction -> f32 with an output cast back to the input
    type; B in the [N, K] weight layout (linalg.matmul_transpose_b) or, with
    b_layout="kn", [K, N] (linalg.matmul)."""
    A = _t([m, k], elem)
    B = _t([n, k], elem) if b_layout == "nk" else _t([k, n], elem)
    mm = "linalg.matmul_transpose_b" if b_layout == "nk" else "linalg.matmul"
    C, O = _t([m, n], "f32"), _t([m, n], elem)
    return f"""module {{
  func.func @bf16_mmad(%a: {A}, %b: {B}, %out: {O}) -> {O}
      {_ATTRS.format(kind='SINGLE_CUBE')} {{
    %c0 = arith.constant 0.000000e+00 : f32
    %e0 = tensor.empty() : {C}
    %acc0 = linalg.fill ins(%c0 : f32) outs(%e0 : {C}) -> {C}
    %acc = {mm} ins(%a, %b : {A}, {B}) outs(%acc0 : {C}) -> {C}
    %o = hfusion.cast {{round_mode = #hfusion.round_mode<rint>}} ins(%acc : {C}) outs(%out : {O}) -> {O}
    return %o : {O}
  }}
}}
"""


# The headline configurations (BASELINE configs[0..4]).
CONFIGS = {
    "vec_add": dict(fn=vec_add, kw=dict(n=1 << 24)),
    "rmsnorm_quant": dict(fn=rmsnorm_quant, kw=dict(rows=8192, cols=4096, eps=1e-6)),
    "safe_softmax": dict(fn=safe_softmax, kw=dict(rows=4096, cols=32768)),
    "argmax": dict(fn=argmax, kw=dict(rows=256, cols=152064)),
    "w8a8_dequant": dict(fn=w8a8_dequant, kw=dict(m=4096, n=4096, k=4096)),
}


_HOST = "attributes {hacc.function_kind = #hacc.function_kind<HOST>}"


def gemm_rmsnorm_quant(m=4096, n=4096, k=4096, alpha=1.0 / 4096):
    """An un-fused host function (no fusion kind): W8A8 contraction, scale,
    RMSNorm over the output rows and dynamic int8 quantisation.  The fusion
    front-end splits it into a MIX_CV group (contraction + dequant epilogue)
    and a LAST_AXIS_PBR group (norm + quant), joined by a workspace tensor."""
    A, B, C = _t([m, k], "i8"), _t([n, k], "i8"), _t([m, n], "i32")
    XF, RF, GF, G, Q = _t([m, n], "f32"), _t([m], "f32"), _t([n], "f32"), _t([n], "bf16"), _t([m, n], "i8")
    return f"""module {{
  func.func @gemm_rmsnorm_quant(%a: {A}, %b: {B}, %gamma: {G}, %q: {Q}, %scale: {RF}) -> ({Q}, {RF})
      {_HOST} {{
    %c0 = arith.constant 0 : i32
    %alpha = arith.constant {alpha:.9e} : f32
    %zero = arith.constant 0.000000e+00 : f32
    %cols = arith.constant {float(n):.6e} : f32
    %eps = arith.constant 9.999999970e-07 : f32
    %qmax = arith.constant 1.270000e+02 : f32
    %qmin = arith.constant -1.270000e+02 : f32
    %e0 = tensor.empty() : {C}
    %acc0 = linalg.fill ins(%c0 : i32) outs(%e0 : {C}) -> {C}
    %acc = linalg.matmul_transpose_b ins(%a, %b : {A}, {B}) outs(%acc0 : {C}) -> {C}
    %e1 = tensor.empty() : {XF}
    %cf = hfusion.cast {{round_mode = #hfusion.round_mode<rint>}} ins(%acc : {C}) outs(%e1 : {XF}) -> {XF}
    %e2 = tensor.empty() : {XF}
    %x = linalg.elemwise_binary {{fun = #linalg.binary_fn<mul>}} ins(%cf, %alpha : {XF}, f32) outs(%e2 : {XF}) -> {XF}
    %e3 = tensor.empty() : {XF}
    %sq = linalg.elemwise_binary {{fun = #linalg.binary_fn<mul>}} ins(%x, %x : {XF}, {XF}) outs(%e3 : {XF}) -> {XF}
    %e4 = tensor.empty() : {RF}
    %i4 = linalg.fill ins(%zero : f32) outs(%e4 : {RF}) -> {RF}
    %ss = linalg.reduce {{arith.addf}} ins(%sq : {XF}) outs(%i4 : {RF}) dimensions = [1]
    %e5 = tensor.empty() : {RF}
    %mean = linalg.elemwise_binary {{fun = #linalg.binary_fn<div>}} ins(%ss, %cols : {RF}, f32) outs(%e5 : {RF}) -> {RF}
    %e6 = tensor.empty() : {RF}
    %ms = linalg.elemwise_binary {{fun = #linalg.binary_fn<add>}} ins(%mean, %eps : {RF}, f32) outs(%e6 : {RF}) -> {RF}
    %e7 = tensor.empty() : {RF}
    %rt = hfusion.elemwise_unary {{fun = #hfusion.unary_fn<sqrt>}} ins(%ms : {RF}) outs(%e7 : {RF}) -> {RF}
    %e8 = tensor.empty() : {RF}
    %inv = hfusion.elemwise_unary {{fun = #hfusion.unary_fn<rec>}} ins(%rt : {RF}) outs(%e8 : {RF}) -> {RF}
    %e9 = tensor.empty() : {XF}
    %binv = linalg.broadcast ins(%inv : {RF}) outs(%e9 : {XF}) dimensions = [1]
    %e10 = tensor.empty() : {XF}
    %y1 = linalg.elemwise_binary {{fun = #linalg.binary_fn<mul>}} ins(%x, %binv : {XF}, {XF}) outs(%e10 : {XF}) -> {XF}
    %e11 = tensor.empty() : {GF}
    %gf = hfusion.cast {{round_mode = #hfusion.round_mode<rint>}} ins(%gamma : {G}) outs(%e11 : {GF}) -> {GF}
    %e12 = tensor.empty() : {XF}
    %bg = linalg.broadcast ins(%gf : {GF}) outs(%e12 : {XF}) dimensions = [0]
    %e13 = tensor.empty() : {XF}
    %y = linalg.elemwise_binary {{fun = #linalg.binary_fn<mul>}} ins(%y1, %bg : {XF}, {XF}) outs(%e13 : {XF}) -> {XF}
    %e14 = tensor.empty() : {XF}
    %ay = linalg.elemwise_unary {{fun = #linalg.unary_fn<abs>}} ins(%y : {XF}) outs(%e14 : {XF}) -> {XF}
    %e15 = tensor.empty() : {RF}
    %i15 = linalg.fill ins(%zero : f32) outs(%e15 : {RF}) -> {RF}
    %amax = linalg.reduce {{arith.maximumf}} ins(%ay : {XF}) outs(%i15 : {RF}) dimensions = [1]
    %sc = linalg.elemwise_binary {{fun = #linalg.binary_fn<div>}} ins(%amax, %qmax : {RF}, f32) outs(%scale : {RF}) -> {RF}
    %e16 = tensor.empty() : {XF}
    %bsc = linalg.broadcast ins(%sc : {RF}) outs(%e16 : {XF}) dimensions = [1]
    %e17 = tensor.empty() : {XF}
    %ys = linalg.elemwise_binary {{fun = #linalg.binary_fn<div>}} ins(%y, %bsc : {XF}, {XF}) outs(%e17 : {XF}) -> {XF}
    %e18 = tensor.empty() : {XF}
    %r = hfusion.elemwise_unary {{fun = #hfusion.unary_fn<nearbyint>}} ins(%ys : {XF}) outs(%e18 : {XF}) -> {XF}
    %e19 = tensor.empty() : {XF}
    %c1 = hfusion.elemwise_binary {{fun = #hfusion.binary_fn<minf>}} ins(%r, %qmax : {XF}, f32) outs(%e19 : {XF}) -> {XF}
    %e20 = tensor.empty() : {XF}
    %c2 = hfusion.elemwise_binary {{fun = #hfusion.binary_fn<maxf>}} ins(%c1, %qmin : {XF}, f32) outs(%e20 : {XF}) -> {XF}
    %qv = hfusion.cast {{round_mode = #hfusion.round_mode<rint>}} ins(%c2 : {XF}) outs(%q : {Q}) -> {Q}
    return %qv, %sc : {Q}, {RF}
  }}
}}
"""


def scores_softmax(m=1024, n=4096, k=128, scale=0.08838834764831845):
    """An un-fused host function: bf16 scores = Q·Kᵀ·scale and a row softmax
    written to bf16.  Split into a MIX_CV group (contraction + scale) and a
    LAST_AXIS_PBR group (softmax) joined by a workspace tensor."""
    QT, KT, S = _t([m, k], "bf16"), _t([n, k], "bf16"), _t([m, n], "f32")
    R, O = _t([m], "f32"), _t([m, n], "bf16")
    return f"""module {{
  func.func @scores_softmax(%qm: {QT}, %km: {KT}, %p: {O}) -> {O}
      {_HOST} {{
    %zero = arith.constant 0.000000e+00 : f32
    %ninf = arith.constant 0xFF800000 : f32
    %sc = arith.constant {scale:.9e} : f32
    %e0 = tensor.empty() : {S}
    %acc0 = linalg.fill ins(%zero : f32) outs(%e0 : {S}) -> {S}
    %acc = linalg.matmul_transpose_b ins(%qm, %km : {QT}, {KT}) outs(%acc0 : {S}) -> {S}
    %e1 = tensor.empty() : {S}
    %x = linalg.elemwise_binary {{fun = #linalg.binary_fn<mul>}} ins(%acc, %sc : {S}, f32) outs(%e1 : {S}) -> {S}
    %e2 = tensor.empty() : {R}
    %i2 = linalg.fill ins(%ninf : f32) outs(%e2 : {R}) -> {R}
    %m = linalg.reduce {{arith.maximumf}} ins(%x : {S}) outs(%i2 : {R}) dimensions = [1]
    %e3 = tensor.empty() : {S}
    %bm = linalg.broadcast ins(%m : {R}) outs(%e3 : {S}) dimensions = [1]
    %e4 = tensor.empty() : {S}
    %d = linalg.elemwise_binary {{fun = #linalg.binary_fn<sub>}} ins(%x, %bm : {S}, {S}) outs(%e4 : {S}) -> {S}
    %e5 = tensor.empty() : {S}
    %ex = linalg.elemwise_unary {{fun = #linalg.unary_fn<exp>}} ins(%d : {S}) outs(%e5 : {S}) -> {S}
    %e6 = tensor.empty() : {R}
    %i6 = linalg.fill ins(%zero : f32) outs(%e6 : {R}) -> {R}
    %s = linalg.reduce {{arith.addf}} ins(%ex : {S}) outs(%i6 : {R}) dimensions = [1]
    %e7 = tensor.empty() : {S}
    %bs = linalg.broadcast ins(%s : {R}) outs(%e7 : {S}) dimensions = [1]
    %e8 = tensor.empty() : {S}
    %pr = linalg.elemwise_binary {{fun = #linalg.binary_fn<div>}} ins(%ex, %bs : {S}, {S}) outs(%e8 : {S}) -> {S}
    %o = hfusion.cast {{round_mode = #hfusion.round_mode<rint>}} ins(%pr : {S}) outs(%p : {O}) -> {O}
    return %o : {O}
  }}
}}
"""


def exp_cumsum_scale(rows=64, cols=1000):
    """An un-fused host function with a cumulative sum between two
    elementwise ops: y = cumsum(exp(x), dim 1) * w.  The front-end outlines
    the scan as a kernel of its own between the two elementwise groups."""
    X = _t([rows, cols], "f32")
    return f"""module {{
  func.func @exp_cumsum_scale(%x: {X}, %w: {X}) -> {X}
      {_HOST} {{
    %e0 = tensor.empty() : {X}
    %a = linalg.elemwise_unary {{fun = #linalg.unary_fn<exp>}} ins(%x : {X}) outs(%e0 : {X}) -> {X}
    %c = hfusion.cumsum %a : {X} cum_dims = [1] reverse = false -> {X}
    %e1 = tensor.empty() : {X}
    %b = linalg.elemwise_binary {{fun = #linalg.binary_fn<mul>}} ins(%c, %w : {X}, {X}) outs(%e1 : {X}) -> {X}
    return %b : {X}
  }}
}}
"""


def matmul_mx(m=4096, n=4096, k=4096, fa="e4m3", fb="e4m3", via="fp8", init=None, out="f32", name="matmul_mx"):
    """Block-scaled fp8 / fp4 contraction (hfusion.matmul_mx, HFusionOps.td:1233-1291):
    C = init + (A * 2^(sa-127)) x (B * 2^(sb-127)), A [M, K], B [K, N],
    e8m0 scales sa [M, K/32] and sb [N, K/32] (ui8); fp4 operands are
    [M, K/2] and [K/2, N] bytes.  `via` is how the fp8
    operands arrive: typed ("fp8"), as bytes through hfusion.bitcast
    ("bitcast", the form of the reference's conversion tests), or as bytes
    with lhsFormat / rhsFormat ("format").  init None accumulates onto a
    tensor.empty (zero); a number fills the accumulator first.  out "bf16"
    adds a cast epilogue."""
    # fp4 ("e2m1", format 3): two values per byte along K, carried as bytes
    # bitcast to f8E5M2, as in matmul-mx-format.mlir's fp4 case
    ty = {"e4m3": "f8E4M3FN", "e5m2": "f8E5M2", "e2m1": "f8E5M2"}
    code = {"e5m2": 1, "e4m3": 2, "e2m1": 3}
    if (fa == "e2m1") != (fb == "e2m1") or (fa == "e2m1" and via == "fp8"):
        raise ValueError("fp4 operands come in pairs, as bytes with a format")
    ka, kb = (k // 2, k // 2) if fa == "e2m1" else (k, k)
    FA, FB = _t([m, ka], ty[fa]), _t([kb, n], ty[fb])
    IA, IB = _t([m, ka], "i8"), _t([kb, n], "i8")
    SA, SB = _t([m, k // 32], "ui8"), _t([n, k // 32], "ui8")
    C, O = _t([m, n], "f32"), _t([m, n], out)
    pa, pb = (IA, IB) if via in ("bitcast", "format") else (FA, FB)
    body = []
    if via == "bitcast":
        body += [f"%ea = tensor.empty() : {FA}",
                 f"%a8 = hfusion.bitcast ins(%a : {IA}) outs(%ea : {FA}) -> {FA}",
                 f"%eb = tensor.empty() : {FB}",
                 f"%b8 = hfusion.bitcast ins(%b : {IB}) outs(%eb : {FB}) -> {FB}"]
        xa, xb, ta, tb = "%a8", "%b8", FA, FB
    else:
        xa, xb, ta, tb = "%a", "%b", pa, pb
    body.append(f"%e0 = tensor.empty() : {C}")
    acc = "%e0"
    if init is not None:
        body += [f"%cinit = arith.constant {float(init):e} : f32",
                 f"%acc0 = linalg.fill ins(%cinit : f32) outs(%e0 : {C}) -> {C}"]
        acc = "%acc0"
    attrs = f" {{lhsFormat = {code[fa]} : i32, rhsFormat = {code[fb]} : i32}}" if via != "fp8" else ""
    body.append(f"%c = hfusion.matmul_mx{attrs} ins({xa}, {xb}, %sa, %sb : {ta}, {tb}, {SA}, {SB}) outs({acc} : {C}) -> {C}")
    res, rty = "%c", C
    if out != "f32":
        body += [f"%e1 = tensor.empty() : {O}",
                 f"%o = hfusion.cast {{round_mode = #hfusion.round_mode<rint>}} ins(%c : {C}) outs(%e1 : {O}) -> {O}"]
        res, rty = "%o", O
    body.append(f"return {res} : {rty}")
    lines = "\n".join("    " + x for x in body)
    return f"""module {{
  func.func @{name}(%a: {pa}, %b: {pb}, %sa: {SA}, %sb: {SB}) -> {rty}
      {_ATTRS.format(kind='SINGLE_CUBE')} {{
{lines}
  }}
}}
"""


def transpose_cast(rows=4096, cols=8192, src="bf16", dst="f32"):
    """PURE_ELEMWISE group with a transpose: out[j, i] = cast(x[i, j])
    (linalg.transpose permutation [1, 0] fused with hfusion.cast)."""
    X, XT, O = _t([rows, cols], src), _t([cols, rows], src), _t([cols, rows], dst)
    return f"""module {{
  func.func @transpose_cast(%x: {X}, %o: {O}) -> {O}
      {_ATTRS.format(kind='PURE_ELEMWISE')} {{
    %e = tensor.empty() : {XT}
    %t = linalg.transpose ins(%x : {X}) outs(%e : {XT}) permutation = [1, 0]
    %r = hfusion.cast {{round_mode = #hfusion.round_mode<rint>}} ins(%t : {XT}) outs(%o : {O}) -> {O}
    return %r : {O}
  }}
}}
"""
