"""Every HFusion group the tests compile: the product groups of
`hfusion_mi355x.catalog` plus the parity cases -- reduced and ragged sizes of
the headline workloads, one module per op family of the generic lowering
(cast round modes, math functions, scans, gathers, histograms, ANY_PBR
columns, transposes, fused programs), random generic chains, and groups with
dynamic dims.  `__graft_entry__.build()` compiles them all ahead of time so
the GPU tests load prebuilt code objects.
"""
from hfusion_mi355x import catalog as _product
from hfusion_mi355x import groups as g
from hfusion_mi355x.runtime import DynamicGroup

_T = g._t
_ATTRS = g._ATTRS


def cast_modes(n=4096):
    """One module, one group per (target type, round mode, saturate) pair."""
    X = _T([n], "f32")
    funcs = []
    modes = ["rint", "round", "floor", "ceil", "trunc", "odd"]
    for m in modes:
        for tgt, sat in (("i8", True), ("i8", False), ("i32", False), ("bf16", False), ("f16", False)):
            O = _T([n], tgt)
            name = f"cast_{tgt}_{m}" + ("_sat" if sat else "")
            satattr = ", enable_saturate = true" if sat else ""
            funcs.append(f"""  func.func @{name}(%x: {X}, %o: {O}) -> {O}
      {_ATTRS.format(kind='PURE_ELEMWISE')} {{
    %r = hfusion.cast {{round_mode = #hfusion.round_mode<{m}>{satattr}}} ins(%x : {X}) outs(%o : {O}) -> {O}
    return %r : {O}
  }}""")
    # integer -> float round modes and same-type float rounding
    I = _T([n], "i32")
    for m in modes:
        funcs.append(f"""  func.func @cast_i32_f32_{m}(%x: {I}, %o: {X}) -> {X}
      {_ATTRS.format(kind='PURE_ELEMWISE')} {{
    %r = hfusion.cast {{round_mode = #hfusion.round_mode<{m}>}} ins(%x : {I}) outs(%o : {X}) -> {X}
    return %r : {X}
  }}""")
        funcs.append(f"""  func.func @cast_f32_f32_{m}(%x: {X}, %o: {X}) -> {X}
      {_ATTRS.format(kind='PURE_ELEMWISE')} {{
    %r = hfusion.cast {{round_mode = #hfusion.round_mode<{m}>}} ins(%x : {X}) outs(%o : {X}) -> {X}
    return %r : {X}
  }}""")
    return "module {\n" + "\n".join(funcs) + "\n}\n"


def eltwise_mix(rows=64, cols=1000):
    """ANY_PB group: row and column broadcasts, compare/select, unary math,
    maximumf, an i1 output and a bf16 output."""
    X, C, R = _T([rows, cols], "f32"), _T([cols], "f32"), _T([rows], "f32")
    B, O, M = _T([rows, cols], "bf16"), _T([rows, cols], "f32"), _T([rows, cols], "i1")
    return f"""module {{
  func.func @eltwise_mix(%x: {X}, %b: {C}, %s: {R}, %y: {B}, %mask: {M}) -> ({B}, {M})
      {_ATTRS.format(kind='ANY_PB')} {{
    %half = arith.constant 5.000000e-01 : f32
    %e0 = tensor.empty() : {O}
    %bb = linalg.broadcast ins(%b : {C}) outs(%e0 : {O}) dimensions = [0]
    %e1 = tensor.empty() : {O}
    %bs = linalg.broadcast ins(%s : {R}) outs(%e1 : {O}) dimensions = [1]
    %gt = hfusion.compare {{compare_fn = #hfusion.compare_fn<vgt>}} ins(%x, %bb : {O}, {O}) outs(%mask : {M}) -> {M}
    %e2 = tensor.empty() : {O}
    %ex = linalg.elemwise_unary {{fun = #linalg.unary_fn<exp>}} ins(%x : {O}) outs(%e2 : {O}) -> {O}
    %e3 = tensor.empty() : {O}
    %t = linalg.elemwise_binary {{fun = #linalg.binary_fn<mul>}} ins(%ex, %bs : {O}, {O}) outs(%e3 : {O}) -> {O}
    %e4 = tensor.empty() : {O}
    %ng = linalg.elemwise_unary {{fun = #linalg.unary_fn<negf>}} ins(%x : {O}) outs(%e4 : {O}) -> {O}
    %e5 = tensor.empty() : {O}
    %sel = hfusion.select ins(%gt, %t, %ng : {M}, {O}, {O}) outs(%e5 : {O}) -> {O}
    %e6 = tensor.empty() : {O}
    %mx = hfusion.elemwise_binary {{fun = #hfusion.binary_fn<maxf>}} ins(%sel, %half : {O}, f32) outs(%e6 : {O}) -> {O}
    %e7 = tensor.empty() : {O}
    %sq = hfusion.elemwise_unary {{fun = #hfusion.unary_fn<sqrt>}} ins(%mx : {O}) outs(%e7 : {O}) -> {O}
    %r = hfusion.cast {{round_mode = #hfusion.round_mode<rint>}} ins(%sq : {O}) outs(%y : {B}) -> {B}
    return %r, %gt : {B}, {M}
  }}
}}
"""


def layernorm(rows=64, cols=2048, eps=1e-5):
    """LAST_AXIS_PBR group with two dependent sum reductions (mean, variance),
    a column broadcast of weight and bias and an f32 row output (the mean)."""
    X, W, R = _T([rows, cols], "f32"), _T([cols], "f32"), _T([rows], "f32")
    return f"""module {{
  func.func @layernorm(%x: {X}, %w: {W}, %bias: {W}, %y: {X}, %mu: {R}) -> ({X}, {R})
      {_ATTRS.format(kind='LAST_AXIS_PBR')} {{
    %zero = arith.constant 0.000000e+00 : f32
    %n = arith.constant {float(cols):.6e} : f32
    %eps = arith.constant {eps:.9e} : f32
    %e0 = tensor.empty() : {R}
    %f0 = linalg.fill ins(%zero : f32) outs(%e0 : {R}) -> {R}
    %s = linalg.reduce {{arith.addf}} ins(%x : {X}) outs(%f0 : {R}) dimensions = [1]
    %m = linalg.elemwise_binary {{fun = #linalg.binary_fn<div>}} ins(%s, %n : {R}, f32) outs(%mu : {R}) -> {R}
    %e1 = tensor.empty() : {X}
    %bm = linalg.broadcast ins(%m : {R}) outs(%e1 : {X}) dimensions = [1]
    %e2 = tensor.empty() : {X}
    %d = linalg.elemwise_binary {{fun = #linalg.binary_fn<sub>}} ins(%x, %bm : {X}, {X}) outs(%e2 : {X}) -> {X}
    %e3 = tensor.empty() : {X}
    %d2 = linalg.elemwise_binary {{fun = #linalg.binary_fn<mul>}} ins(%d, %d : {X}, {X}) outs(%e3 : {X}) -> {X}
    %e4 = tensor.empty() : {R}
    %f4 = linalg.fill ins(%zero : f32) outs(%e4 : {R}) -> {R}
    %v = linalg.reduce {{arith.addf}} ins(%d2 : {X}) outs(%f4 : {R}) dimensions = [1]
    %e5 = tensor.empty() : {R}
    %vm = linalg.elemwise_binary {{fun = #linalg.binary_fn<div>}} ins(%v, %n : {R}, f32) outs(%e5 : {R}) -> {R}
    %e6 = tensor.empty() : {R}
    %ve = linalg.elemwise_binary {{fun = #linalg.binary_fn<add>}} ins(%vm, %eps : {R}, f32) outs(%e6 : {R}) -> {R}
    %e7 = tensor.empty() : {R}
    %rs = hfusion.elemwise_unary {{fun = #hfusion.unary_fn<rsqrt>}} ins(%ve : {R}) outs(%e7 : {R}) -> {R}
    %e8 = tensor.empty() : {X}
    %br = linalg.broadcast ins(%rs : {R}) outs(%e8 : {X}) dimensions = [1]
    %e9 = tensor.empty() : {X}
    %nx = linalg.elemwise_binary {{fun = #linalg.binary_fn<mul>}} ins(%d, %br : {X}, {X}) outs(%e9 : {X}) -> {X}
    %e10 = tensor.empty() : {X}
    %bw = linalg.broadcast ins(%w : {W}) outs(%e10 : {X}) dimensions = [0]
    %e11 = tensor.empty() : {X}
    %wx = linalg.elemwise_binary {{fun = #linalg.binary_fn<mul>}} ins(%nx, %bw : {X}, {X}) outs(%e11 : {X}) -> {X}
    %e12 = tensor.empty() : {X}
    %bb = linalg.broadcast ins(%bias : {W}) outs(%e12 : {X}) dimensions = [0]
    %o = linalg.elemwise_binary {{fun = #linalg.binary_fn<add>}} ins(%wx, %bb : {X}, {X}) outs(%y : {X}) -> {X}
    return %o, %m : {X}, {R}
  }}
}}
"""


# elementwise functions of the HFusion region builder (HFusionOps.cpp:434-640)
# that the headline groups do not use: (function, dialect) per unary/binary op
MATH_UNARY = [("tan", "hfusion"), ("acos", "hfusion"), ("acosh", "hfusion"), ("asin", "hfusion"),
              ("asinh", "hfusion"), ("atan", "hfusion"), ("atanh", "hfusion"), ("sinh", "hfusion"),
              ("cosh", "hfusion"), ("lgamma", "hfusion"), ("ilogb", "hfusion"), ("tanh", "hfusion"),
              ("sin", "hfusion"), ("cos", "hfusion"), ("erf", "hfusion"), ("log2", "hfusion"),
              ("log10", "hfusion"), ("log1p", "hfusion"), ("exp2", "hfusion"), ("expm1", "hfusion"),
              ("rsqrt", "hfusion"), ("log", "linalg")]
MATH_BINARY = ["atan2", "ldexp", "divfhp", "powf", "copysign", "mod"]
INT_BINARY = [("powi", "i32"), ("powi", "i16"), ("ceildivui", "i32"), ("modui", "i32"), ("ceildivui", "i8")]


def math_fns(n=4096):
    """One module, one PURE_ELEMWISE group per elementwise function (f32
    unary and binary, integer binary on several widths) plus an operand
    `bitcast` type_fn (i32 bits read as f32)."""
    X = _T([n], "f32")
    funcs = []
    for fn, dia in MATH_UNARY:
        attr = f"#{dia}.unary_fn<{fn}>"
        funcs.append(f"""  func.func @u_{fn}(%x: {X}, %o: {X}) -> {X}
      {_ATTRS.format(kind='PURE_ELEMWISE')} {{
    %r = {dia}.elemwise_unary {{fun = {attr}}} ins(%x : {X}) outs(%o : {X}) -> {X}
    return %r : {X}
  }}""")
    for fn in MATH_BINARY:
        funcs.append(f"""  func.func @b_{fn}(%x: {X}, %y: {X}, %o: {X}) -> {X}
      {_ATTRS.format(kind='PURE_ELEMWISE')} {{
    %r = hfusion.elemwise_binary {{fun = #hfusion.binary_fn<{fn}>}} ins(%x, %y : {X}, {X}) outs(%o : {X}) -> {X}
    return %r : {X}
  }}""")
    for fn, t in INT_BINARY:
        I = _T([n], t)
        funcs.append(f"""  func.func @i_{fn}_{t}(%x: {I}, %y: {I}, %o: {I}) -> {I}
      {_ATTRS.format(kind='PURE_ELEMWISE')} {{
    %r = hfusion.elemwise_binary {{fun = #hfusion.binary_fn<{fn}>}} ins(%x, %y : {I}, {I}) outs(%o : {I}) -> {I}
    return %r : {I}
  }}""")
    I = _T([n], "i32")
    funcs.append(f"""  func.func @bitcast_add(%x: {I}, %y: {I}, %o: {X}) -> {X}
      {_ATTRS.format(kind='PURE_ELEMWISE')} {{
    %r = linalg.elemwise_binary {{fun = #linalg.binary_fn<add>, cast = #linalg.type_fn<bitcast>}} ins(%x, %y : {I}, {I}) outs(%o : {X}) -> {X}
    return %r : {X}
  }}""")
    return "module {\n" + "\n".join(funcs) + "\n}\n"


FP_OPS = [("isinf", "f32"), ("isnan", "f32"), ("isfinite", "f32"), ("isinf", "bf16"), ("isnan", "f16"),
          ("nextafter", "f32"), ("nextafter", "f16"), ("hypot", "f32"), ("hypot3", "f32"), ("hypot", "f16"),
          ("erfinv", "f32"), ("erfinv", "f16"), ("bitcast", "f32"), ("signbit", "f32"), ("signbit", "f16"),
          ("signbit8", "f32"), ("cylbesseli0", "f32"), ("cylbesseli0", "f16")]


def fp_ops(n=4096):
    """One module, one group per HFusion float op without outs (predicates,
    nextafter, hypot with 2 and 3 operands, erfinv, signbit, cyl_bessel_i0) and hfusion.bitcast."""
    funcs = []
    for op, t in FP_OPS:
        X, B = _T([n], t), _T([n], "i1")
        name = f"{op}_{t}"
        attrs = _ATTRS.format(kind='PURE_ELEMWISE')
        if op in ("isinf", "isnan", "isfinite"):
            body = f"%r = hfusion.{op} %x : {X} -> {B}\n    return %r : {B}"
            sig = f"(%x: {X}) -> {B}"
        elif op == "nextafter":
            body = f"%r = hfusion.nextafter %x, %y : {X}, {X} -> {X}\n    return %r : {X}"
            sig = f"(%x: {X}, %y: {X}) -> {X}"
        elif op == "hypot":
            body = f"%r = hfusion.hypot %x, %y : {X}, {X} -> {X}\n    return %r : {X}"
            sig = f"(%x: {X}, %y: {X}) -> {X}"
        elif op == "hypot3":
            body = f"%r = hfusion.hypot %x, %y, %z : {X}, {X}, {X} -> {X}\n    return %r : {X}"
            sig = f"(%x: {X}, %y: {X}, %z: {X}) -> {X}"
        elif op in ("signbit", "signbit8"):
            # generic op form, as the reference's own tests write it
            R = B if op == "signbit" else _T([n], "i8")
            body = f'%r = "hfusion.signbit"(%x) : ({X}) -> {R}\n    return %r : {R}'
            sig = f"(%x: {X}) -> {R}"
        elif op == "cylbesseli0":
            body = f"%r = hfusion.cyl_bessel_i0 %x : {X} -> {X}\n    return %r : {X}"
            sig = f"(%x: {X}) -> {X}"
        elif op == "erfinv":
            body = f"%r = hfusion.erfinv %x : {X} -> {X}\n    return %r : {X}"
            sig = f"(%x: {X}) -> {X}"
        else:
            I = _T([n], "i32")
            body = f"%r = hfusion.bitcast ins(%x : {I}) outs(%o : {X}) -> {X}\n    return %r : {X}"
            sig = f"(%x: {I}, %o: {X}) -> {X}"
        funcs.append(f"""  func.func @{name}{sig}
      {attrs} {{
    {body}
  }}""")
    return "module {\n" + "\n".join(funcs) + "\n}\n"


# (name, op, elem in, elem out, shape, dim, reverse, extra attr)
SCAN_OPS = [("cumsum_f32_d1", "cumsum", "f32", "f32", [64, 1000], 1, False, ""),
            ("cumsum_f32_d0_rev", "cumsum", "f32", "f32", [64, 1000], 0, True, ""),
            ("cumprod_f32", "cumprod", "f32", "f32", [32, 64], 1, False, ""),
            ("cumprod_bf16_rev", "cumprod", "bf16", "bf16", [16, 256], 1, True, ""),
            ("cummax_f32", "cummax", "f32", "f32", [64, 512], 1, False, ""),
            ("cummin_f32_num", "cummin", "f32", "f32", [64, 512], 0, False, "{propagate_nan = false} "),
            ("cumsum_i32_i64", "cumsum", "i32", "i64", [4096], 0, False, ""),
            ("cumprod_i16", "cumprod", "i16", "i16", [8, 300], 1, False, ""),
            ("cummax_i8_rev", "cummax", "i8", "i8", [64, 100], 1, True, "")]


def scan_ops():
    """One module, one group per cumulative op (cumsum/cumprod/cummax/cummin)
    over several types, dims and directions."""
    funcs = []
    for name, op, ie, oe, shape, dim, rev, extra in SCAN_OPS:
        X, O = _T(shape, ie), _T(shape, oe)
        funcs.append(f"""  func.func @{name}(%x: {X}) -> {O}
      {_ATTRS.format(kind='ANY_PBR')} {{
    %r = hfusion.{op} %x {extra}: {X} cum_dims = [{dim}] reverse = {str(rev).lower()} -> {O}
    return %r : {O}
  }}""")
    return "module {\n" + "\n".join(funcs) + "\n}\n"


# (name, input elem, input shape, bins, count elem, mask elem or None)
HIST_OPS = [("hist_i32", "i32", [100000], 64, "i32", None),
            ("hist_mask_i64", "i32", [300, 700], 10000, "i64", "i1"),
            ("hist_i8_wrap", "i8", [5000], 16, "i8", None)]
INTERLEAVE_OPS = [("deint_f32_c0", "f32", 0), ("deint_f32_c1", "f32", 1), ("deint_bf16_all", "bf16", -1),
                  ("inter_f32", "f32", None), ("inter_i8", "i8", None)]


def misc_ops():
    """histogram (LDS and global bin paths, optional mask, wrapping counts)
    and (de)interleave along the last dim."""
    funcs = []
    for name, ie, shape, bins, ce, me in HIST_OPS:
        X, O = _T(shape, ie), _T([bins], ce)
        if me:
            M = _T(shape, me)
            funcs.append(f"""  func.func @{name}(%x: {X}, %m: {M}) -> {O}
      {_ATTRS.format(kind='ANY_PBR')} {{
    %r = hfusion.histogram %x, {bins}, %m : {X}, {M} -> {O}
    return %r : {O}
  }}""")
        else:
            funcs.append(f"""  func.func @{name}(%x: {X}) -> {O}
      {_ATTRS.format(kind='ANY_PBR')} {{
    %r = hfusion.histogram %x, {bins} : {X} -> {O}
    return %r : {O}
  }}""")
    for name, e, ch in INTERLEAVE_OPS:
        if ch is None:
            X, O = _T([64, 500], e), _T([64, 1000], e)
            funcs.append(f"""  func.func @{name}(%a: {X}, %b: {X}) -> {O}
      {_ATTRS.format(kind='PURE_ELEMWISE')} {{
    %r = hfusion.interleave %a, %b : {X}, {X} -> {O}
    return %r : {O}
  }}""")
        elif ch == -1:
            X, O = _T([64, 1000], e), _T([64, 500], e)
            funcs.append(f"""  func.func @{name}(%x: {X}) -> ({O}, {O})
      {_ATTRS.format(kind='PURE_ELEMWISE')} {{
    %r:2 = hfusion.deinterleave %x channel<all> : {X} -> {O}, {O}
    return %r#0, %r#1 : {O}, {O}
  }}""")
        else:
            X, O = _T([64, 1000], e), _T([64, 500], e)
            funcs.append(f"""  func.func @{name}(%x: {X}) -> {O}
      {_ATTRS.format(kind='PURE_ELEMWISE')} {{
    %r = hfusion.deinterleave %x channel<{ch}> : {X} -> {O}
    return %r : {O}
  }}""")
    # flip, mulext / mulextui, arange
    for e in ("f32", "bf16"):
        X = _T([64, 1000], e)
        funcs.append(f"""  func.func @flip_{e}(%x: {X}) -> {X}
      {_ATTRS.format(kind='PURE_ELEMWISE')} {{
    %r = hfusion.flip %x : {X} flip_axis = 1 -> {X}
    return %r : {X}
  }}""")
    for op in ("mulext", "mulextui"):
        for e in ("i8", "i32", "i64"):
            X = _T([4096], e)
            funcs.append(f"""  func.func @{op}_{e}(%a: {X}, %b: {X}) -> ({X}, {X})
      {_ATTRS.format(kind='PURE_ELEMWISE')} {{
    %lo, %hi = hfusion.{op} %a, %b : {X}
    return %lo, %hi : {X}, {X}
  }}""")
    for e in ("i32", "f32"):
        O = _T([48, 130], e)
        funcs.append(f"""  func.func @arange_{e}(%o: {O}, %off: index) -> {O}
      {_ATTRS.format(kind='PURE_ELEMWISE')} {{
    %s0 = arith.constant 1000 : index
    %s1 = arith.constant -3 : index
    %r = hfusion.arange offset[%off] strides[%s0, %s1] outs(%o : {O}) -> {O}
    return %r : {O}
  }}""")
    return "module {\n" + "\n".join(funcs) + "\n}\n"


# (name, src elem, src shape, index elem, index shape, axis)
GATHER_OPS = [("gather_f16_ax1", "f16", [5, 6], "i32", [5, 3], 1),
              ("gather_f32_ax1", "f32", [64, 1000], "i32", [64, 100], 1),
              ("gather_bf16_ax0", "bf16", [100, 32], "i64", [50, 32], 0)]


def gather_ops():
    """hfusion.gather along axis 1 and 0, i32 and i64 indices, the init
    (fallback for out-of-range indices) passed as the outs argument."""
    funcs = []
    for name, se, ss, ie, ish, ax in GATHER_OPS:
        S, I, O = _T(ss, se), _T(ish, ie), _T(ish, se)
        funcs.append(f"""  func.func @{name}(%src: {S}, %idx: {I}, %init: {O}) -> {O}
      {_ATTRS.format(kind='PURE_ELEMWISE')} {{
    %r = hfusion.gather {{operandSegmentSizes = array<i32: 2, 1>}} ins(%src, %idx : {S}, {I}) outs(%init : {O}) axis = {ax} -> {O}
    return %r : {O}
  }}""")
    return "module {\n" + "\n".join(funcs) + "\n}\n"


MISC_EXTRA = (["flip_f32", "flip_bf16"] + [f"{op}_{e}" for op in ("mulext", "mulextui") for e in ("i8", "i32", "i64")]
              + ["arange_i32", "arange_f32"])


def memref_chain(n=4096):
    """Destination-style ops on memrefs with no SSA results: the second op
    reads the buffer the first one wrote; both written buffers are results."""
    M = f"memref<{n}xf32>"
    return f"""module {{
  func.func @memref_chain(%x: {M}, %tmp: {M}, %y: {M})
      {_ATTRS.format(kind='PURE_ELEMWISE')} {{
    hfusion.elemwise_unary {{fun = #hfusion.unary_fn<sqrt>}} ins(%x : {M}) outs(%tmp : {M})
    linalg.elemwise_binary {{fun = #linalg.binary_fn<add>}} ins(%tmp, %x : {M}, {M}) outs(%y : {M})
    return
  }}
}}
"""


def reshape_chain():
    """Elementwise ops joined by expand_shape / collapse_shape views: the
    group runs over the shared flat index."""
    A, B3 = _T([128, 256], "f32"), _T([32, 4, 256], "f32")
    return f"""module {{
  func.func @reshape_chain(%a: {A}, %b: {A}, %c: {B3}) -> {A}
      {_ATTRS.format(kind='PURE_ELEMWISE')} {{
    %e0 = tensor.empty() : {A}
    %s = linalg.elemwise_binary {{fun = #linalg.binary_fn<add>}} ins(%a, %b : {A}, {A}) outs(%e0 : {A}) -> {A}
    %x = tensor.expand_shape %s [[0, 1], [2]] output_shape [32, 4, 256] : {A} into {B3}
    %e1 = tensor.empty() : {B3}
    %m = linalg.elemwise_binary {{fun = #linalg.binary_fn<mul>}} ins(%x, %c : {B3}, {B3}) outs(%e1 : {B3}) -> {B3}
    %y = tensor.collapse_shape %m [[0, 1], [2]] : {B3} into {A}
    %e2 = tensor.empty() : {A}
    %r = linalg.elemwise_unary {{fun = #linalg.unary_fn<abs>}} ins(%y : {A}) outs(%e2 : {A}) -> {A}
    return %r : {A}
  }}
}}
"""


def generic_ops():
    """linalg.generic with a region of scalar arith / math ops: a row bias
    (map (d0, d1) -> (d1)), a column scale ((d0, d1) -> (d0)), a captured
    scalar constant and scalar argument, compare/select, f16 <-> f32 casts
    and integer ops."""
    X, B, XT = _T([64, 1000], "f32"), _T([1000], "f32"), _T([64], "f32")
    H, I = _T([64, 1000], "f16"), _T([64, 1000], "i32")
    M = _T([64, 1000], "i1")
    return f"""#id = affine_map<(d0, d1) -> (d0, d1)>
#row = affine_map<(d0, d1) -> (d1)>
#col = affine_map<(d0, d1) -> (d0)>
module {{
  func.func @generic_bias_act(%x: {X}, %b: {B}, %xt: {XT}, %s: f32, %o: {X}) -> {X}
      {_ATTRS.format(kind='ANY_PB')} {{
    %c05 = arith.constant 5.000000e-01 : f32
    %r = linalg.generic {{indexing_maps = [#id, #row, #col, #id], iterator_types = ["parallel", "parallel"]}}
        ins(%x, %b, %xt : {X}, {B}, {XT}) outs(%o : {X}) {{
    ^bb0(%in: f32, %bias: f32, %t: f32, %out: f32):
      %0 = arith.addf %in, %bias : f32
      %1 = arith.mulf %0, %c05 : f32
      %2 = math.tanh %1 : f32
      %3 = arith.cmpf ogt, %0, %t : f32
      %4 = arith.mulf %t, %s : f32
      %5 = arith.select %3, %2, %4 : f32
      %c1 = arith.constant 1.000000e+00 : f32
      %6 = arith.maximumf %5, %c1 : f32
      %7 = math.exp %0 : f32
      %8 = arith.divf %7, %6 : f32
      linalg.yield %8 : f32
    }} -> {X}
    return %r : {X}
  }}
  func.func @generic_f16_int(%h: {H}, %i: {I}, %o: {H}, %m: {M}) -> ({H}, {M})
      {_ATTRS.format(kind='PURE_ELEMWISE')} {{
    %r = linalg.generic {{indexing_maps = [affine_map<(d0, d1) -> (d0, d1)>, affine_map<(d0, d1) -> (d0, d1)>, affine_map<(d0, d1) -> (d0, d1)>], iterator_types = ["parallel", "parallel"]}}
        ins(%h, %i : {H}, {I}) outs(%o : {H}) {{
    ^bb0(%a: f16, %n: i32, %out: f16):
      %0 = arith.extf %a : f16 to f32
      %1 = arith.sitofp %n : i32 to f32
      %2 = arith.mulf %0, %1 : f32
      %3 = arith.truncf %2 : f32 to f16
      %4 = arith.addf %3, %a : f16
      linalg.yield %4 : f16
    }} -> {H}
    %q = linalg.generic {{indexing_maps = [#id, #id], iterator_types = ["parallel", "parallel"]}}
        ins(%i : {I}) outs(%m : {M}) {{
    ^bb0(%n: i32, %out: i1):
      %c3 = arith.constant 3 : i32
      %0 = arith.remsi %n, %c3 : i32
      %1 = arith.shli %n, %c3 : i32
      %2 = arith.xori %0, %1 : i32
      %c0 = arith.constant 0 : i32
      %3 = arith.cmpi slt, %2, %c0 : i32
      linalg.yield %3 : i1
    }} -> {M}
    return %r, %q : {H}, {M}
  }}
}}
"""


def fuzz_generic(count=12, seed=20261201, shape=(32, 257)):
    """Seeded random elementwise groups: linalg.generic regions over f32 / f16
    / i32 operands (a row-broadcast operand among them) built only from
    exactly rounded ops (add, sub, mul, div, max/min, abs, neg, sqrt,
    compare + select, extf/truncf, sitofp), so every result is bit-exact
    against the oracle."""
    import random
    rnd = random.Random(seed)
    r, c = shape
    funcs = []
    fops = ["arith.addf", "arith.subf", "arith.mulf", "arith.divf", "arith.maximumf", "arith.minimumf"]
    for n in range(count):
        ft = rnd.choice(["f32", "f16"])
        X, B, I, O = _T([r, c], ft), _T([c], ft), _T([r, c], "i32"), _T([r, c], ft)
        body, vals, k = [], ["%a", "%b", "%bb"], 0

        def new(stmt):
            nonlocal k
            nm = f"%v{k}"
            k += 1
            body.append(f"      {nm} = {stmt}")
            return nm
        vals.append(new(f"arith.sitofp %n : i32 to {ft}"))
        for _ in range(rnd.randint(3, 7)):
            kind = rnd.random()
            x, y = rnd.choice(vals), rnd.choice(vals)
            if kind < 0.55:
                vals.append(new(f"{rnd.choice(fops)} {x}, {y} : {ft}"))
            elif kind < 0.7:
                vals.append(new(f"{rnd.choice(['math.absf', 'arith.negf', 'math.sqrt'])} {x} : {ft}"))
            elif kind < 0.85:
                cnd = new(f"arith.cmpf {rnd.choice(['olt', 'oge', 'une', 'ugt'])}, {x}, {y} : {ft}")
                vals.append(new(f"arith.select {cnd}, {x}, {rnd.choice(vals)} : {ft}"))
            elif ft == "f16":
                e = new(f"arith.extf {x} : f16 to f32")
                m = new(f"arith.mulf {e}, {e} : f32")
                vals.append(new(f"arith.truncf {m} : f32 to f16"))
            else:
                vals.append(new(f"arith.addf {x}, {x} : {ft}"))
        body.append(f"      linalg.yield {vals[-1]} : {ft}")
        region = "\n".join(body)
        funcs.append(f"""  func.func @fuzz{n}(%x: {X}, %bias: {B}, %i: {I}, %o: {O}) -> {O}
      {_ATTRS.format(kind='ANY_PB')} {{
    %r = linalg.generic {{indexing_maps = [affine_map<(d0, d1) -> (d0, d1)>, affine_map<(d0, d1) -> (d1)>, affine_map<(d0, d1) -> (d0, d1)>, affine_map<(d0, d1) -> (d0, d1)>], iterator_types = ["parallel", "parallel"]}}
        ins(%x, %bias, %i : {X}, {B}, {I}) outs(%o : {O}) {{
    ^bb0(%a: {ft}, %bb: {ft}, %n: i32, %out: {ft}):
      %b = arith.addf %a, %bb : {ft}
{region}
    }} -> {O}
    return %r : {O}
  }}""")
    return "module {\n" + "\n".join(funcs) + "\n}\n"


def fuzz_rows(count=8, seed=20261202):
    """Seeded random LAST_AXIS_PBR groups from named ops: an elementwise chain
    with a row-broadcast operand, a max or min row reduction, its broadcast
    back into a second chain, results both the row values and the reduction.
    Exactly rounded, order-free ops only, so results are bit-exact."""
    import random
    rnd = random.Random(seed)
    funcs = []
    for n in range(count):
        r, c = rnd.choice([(64, 1000), (13, 4096), (256, 96), (7, 33000)])
        X, B, R = _T([r, c], "f32"), _T([c], "f32"), _T([r], "f32")
        lines, k = [], 0

        def ew(op, ins):
            nonlocal k
            k += 1
            e, v = f"%e{k}", f"%v{k}"
            fam = "linalg" if op in ("add", "sub", "mul", "div", "max_signed", "min_signed", "abs", "negf") else "hfusion"
            if op in ("abs", "negf", "sqrt"):
                attr = f"#{'linalg' if fam == 'linalg' else 'hfusion'}.unary_fn<{op}>"
                kind = f"{fam}.elemwise_unary"
                tys = X
            else:
                attr = f"#linalg.binary_fn<{op}>" if fam == "linalg" else f"#hfusion.binary_fn<{op}>"
                kind = f"{fam}.elemwise_binary"
                tys = ", ".join([X] * len(ins))
            lines.append(f"    {e} = tensor.empty() : {X}")
            lines.append(f"    {v} = {kind} {{fun = {attr}}} ins({', '.join(ins)} : {tys}) outs({e} : {X}) -> {X}")
            return v
        lines.append(f"    %eb = tensor.empty() : {X}")
        lines.append(f"    %bb = linalg.broadcast ins(%b : {B}) outs(%eb : {X}) dimensions = [0]")
        vals = ["%x", "%bb"]
        for _ in range(rnd.randint(2, 4)):
            op = rnd.choice(["add", "sub", "mul", "max_signed", "min_signed", "abs", "negf"])
            vals.append(ew(op, [rnd.choice(vals)] if op in ("abs", "negf") else [rnd.choice(vals), rnd.choice(vals)]))
        red = rnd.choice(["maximumf", "minimumf"])
        init = "0xFF800000" if red == "maximumf" else "0x7F800000"
        lines.append(f"    %init = arith.constant {init} : f32")
        lines.append(f"    %f = linalg.fill ins(%init : f32) outs(%m : {R}) -> {R}")
        lines.append(f"    %red = linalg.reduce {{arith.{red}}} ins({vals[-1]} : {X}) outs(%f : {R}) dimensions = [1]")
        lines.append(f"    %er = tensor.empty() : {X}")
        lines.append(f"    %rb = linalg.broadcast ins(%red : {R}) outs(%er : {X}) dimensions = [1]")
        vals.append("%rb")
        for _ in range(rnd.randint(1, 3)):
            op = rnd.choice(["sub", "add", "mul", "max_signed", "abs"])
            vals.append(ew(op, [rnd.choice(vals[-3:])] if op == "abs" else [rnd.choice(vals[-3:]), rnd.choice(vals)]))
        body = "\n".join(lines)
        funcs.append(f"""  func.func @frow{n}(%x: {X}, %b: {B}, %m: {R}) -> ({X}, {R})
      {_ATTRS.format(kind='LAST_AXIS_PBR')} {{
{body}
    return {vals[-1]}, %red : {X}, {R}
  }}""")
    return "module {\n" + "\n".join(funcs) + "\n}\n"


def generic_reduce():
    """linalg.generic row reductions: max of x*w (exact) and sum of
    x*w (a float sum: the row program's order differs from the serial loop)."""
    X, W, R = _T([64, 1000], "f32"), _T([1000], "f32"), _T([64], "f32")
    funcs = []
    for name, comb, init in (("gred_max", "arith.maximumf", "0xFF800000"), ("gred_sum", "arith.addf", "0.000000e+00")):
        funcs.append(f"""  func.func @{name}(%x: {X}, %w: {W}, %o: {R}) -> {R}
      {_ATTRS.format(kind='LAST_AXIS_PBR')} {{
    %init = arith.constant {init} : f32
    %f = linalg.fill ins(%init : f32) outs(%o : {R}) -> {R}
    %r = linalg.generic {{indexing_maps = [#in, #row, #out], iterator_types = ["parallel", "reduction"]}}
        ins(%x, %w : {X}, {W}) outs(%f : {R}) {{
    ^bb0(%a: f32, %b: f32, %acc: f32):
      %p = arith.mulf %a, %b : f32
      %m = {comb} %p, %acc : f32
      linalg.yield %m : f32
    }} -> {R}
    return %r : {R}
  }}""")
    return ("#in = affine_map<(d0, d1) -> (d0, d1)>\n#row = affine_map<(d0, d1) -> (d1)>\n"
            "#out = affine_map<(d0, d1) -> (d0)>\nmodule {\n" + "\n".join(funcs) + "\n}\n")


def reduce_ops(rows=48, cols=3000):
    """Row reductions with each f32 combiner and an i32 sum (exact)."""
    X, R, XI, RI = _T([rows, cols], "f32"), _T([rows], "f32"), _T([rows, cols], "i32"), _T([rows], "i32")
    return f"""module {{
  func.func @reduce_ops(%x: {X}, %xi: {XI}, %mx: {R}, %mn: {R}, %mxn: {R}, %si: {RI}) -> ({R}, {R}, {R}, {RI})
      {_ATTRS.format(kind='LAST_AXIS_PBR')} {{
    %ninf = arith.constant 0xFF800000 : f32
    %pinf = arith.constant 0x7F800000 : f32
    %c0 = arith.constant 0 : i32
    %f0 = linalg.fill ins(%ninf : f32) outs(%mx : {R}) -> {R}
    %a = linalg.reduce {{arith.maximumf}} ins(%x : {X}) outs(%f0 : {R}) dimensions = [1]
    %f1 = linalg.fill ins(%pinf : f32) outs(%mn : {R}) -> {R}
    %b = linalg.reduce {{arith.minimumf}} ins(%x : {X}) outs(%f1 : {R}) dimensions = [1]
    %f2 = linalg.fill ins(%ninf : f32) outs(%mxn : {R}) -> {R}
    %c = linalg.reduce {{arith.maxnumf}} ins(%x : {X}) outs(%f2 : {R}) dimensions = [1]
    %f3 = linalg.fill ins(%c0 : i32) outs(%si : {RI}) -> {RI}
    %d = linalg.reduce {{arith.addi}} ins(%xi : {XI}) outs(%f3 : {RI}) dimensions = [1]
    return %a, %b, %c, %d : {R}, {R}, {R}, {RI}
  }}
}}
"""


def quant_ties(rows=64, cols=1024):
    """nearbyint(x / s[row]) with f32 output: the dynamic-quantisation
    rounding, checked on quotients placed on and next to half-integers."""
    X, R = _T([rows, cols], "f32"), _T([rows], "f32")
    return f"""module {{
  func.func @quant_ties(%x: {X}, %s: {R}, %o: {X}, %mx: {R}) -> ({X}, {R})
      {_ATTRS.format(kind='LAST_AXIS_PBR')} {{
    %ninf = arith.constant 0xFF800000 : f32
    %f = linalg.fill ins(%ninf : f32) outs(%mx : {R}) -> {R}
    %m = linalg.reduce {{arith.maximumf}} ins(%x : {X}) outs(%f : {R}) dimensions = [1]
    %e0 = tensor.empty() : {X}
    %bs = linalg.broadcast ins(%s : {R}) outs(%e0 : {X}) dimensions = [1]
    %e1 = tensor.empty() : {X}
    %q = linalg.elemwise_binary {{fun = #linalg.binary_fn<div>}} ins(%x, %bs : {X}, {X}) outs(%e1 : {X}) -> {X}
    %r = hfusion.elemwise_unary {{fun = #hfusion.unary_fn<nearbyint>}} ins(%q : {X}) outs(%o : {X}) -> {X}
    return %r, %m : {X}, {R}
  }}
}}
"""


FP8_TYPES = {"e4m3": "f8E4M3FN", "e5m2": "f8E5M2"}


def quant_i8_ties(rows=64, cols=1024, lo=-127, hi=127, name="quant_i8_ties"):
    """(int8)clamp(nearbyint(x / s[row]), lo, hi): the int8 dynamic-quant tail
    on its own (with a row max beside it, so the group is a row program),
    for quotients on and next to half-integers and beyond the clamp bounds."""
    X, R, Q = _T([rows, cols], "f32"), _T([rows], "f32"), _T([rows, cols], "i8")
    return f"""module {{
  func.func @{name}(%x: {X}, %s: {R}, %q: {Q}, %mx: {R}) -> ({Q}, {R})
      {_ATTRS.format(kind='LAST_AXIS_PBR')} {{
    %ninf = arith.constant 0xFF800000 : f32
    %f = linalg.fill ins(%ninf : f32) outs(%mx : {R}) -> {R}
    %m = linalg.reduce {{arith.maximumf}} ins(%x : {X}) outs(%f : {R}) dimensions = [1]
    %hi = arith.constant {float(hi):.6e} : f32
    %lo = arith.constant {float(lo):.6e} : f32
    %e0 = tensor.empty() : {X}
    %bs = linalg.broadcast ins(%s : {R}) outs(%e0 : {X}) dimensions = [1]
    %e1 = tensor.empty() : {X}
    %d = linalg.elemwise_binary {{fun = #linalg.binary_fn<div>}} ins(%x, %bs : {X}, {X}) outs(%e1 : {X}) -> {X}
    %e2 = tensor.empty() : {X}
    %r = hfusion.elemwise_unary {{fun = #hfusion.unary_fn<nearbyint>}} ins(%d : {X}) outs(%e2 : {X}) -> {X}
    %e3 = tensor.empty() : {X}
    %c1 = hfusion.elemwise_binary {{fun = #hfusion.binary_fn<minf>}} ins(%r, %hi : {X}, f32) outs(%e3 : {X}) -> {X}
    %e4 = tensor.empty() : {X}
    %c2 = hfusion.elemwise_binary {{fun = #hfusion.binary_fn<maxf>}} ins(%c1, %lo : {X}, f32) outs(%e4 : {X}) -> {X}
    %o = hfusion.cast {{round_mode = #hfusion.round_mode<rint>}} ins(%c2 : {X}) outs(%q : {Q}) -> {Q}
    return %o, %m : {Q}, {R}
  }}
}}
"""


def cast_fp8(n=4096):
    """fp8 casts: f32 -> f8E4M3FN / f8E5M2 under every round mode, with and
    without saturation; fp8 -> f32; f16 <-> f8E5M2 through f32 (the form of
    hfusion-normalize-casting-ops.mlir:321-339); and f32 -> i16 / i8 casts whose
    result carries annotation.mark {overflow_mode = "saturate"}
    (hfusion-normalize-casting-ops.mlir:53-74)."""
    X, H = _T([n], "f32"), _T([n], "f16")
    funcs = []
    for short, ty in FP8_TYPES.items():
        O = _T([n], ty)
        for m in ["rint", "round", "floor", "ceil", "trunc", "odd"]:
            for sat in (False, True):
                satattr = ", enable_saturate = true" if sat else ""
                funcs.append(f"""  func.func @cast_{short}_{m}{"_sat" if sat else ""}(%x: {X}, %o: {O}) -> {O}
      {_ATTRS.format(kind='PURE_ELEMWISE')} {{
    %r = hfusion.cast {{round_mode = #hfusion.round_mode<{m}>{satattr}}} ins(%x : {X}) outs(%o : {O}) -> {O}
    return %r : {O}
  }}""")
        funcs.append(f"""  func.func @dec_{short}(%x: {O}, %o: {X}) -> {X}
      {_ATTRS.format(kind='PURE_ELEMWISE')} {{
    %r = hfusion.cast {{round_mode = #hfusion.round_mode<rint>}} ins(%x : {O}) outs(%o : {X}) -> {X}
    return %r : {X}
  }}""")
    E = _T([n], "f8E5M2")
    funcs.append(f"""  func.func @f16_to_e5m2(%x: {H}, %o: {E}) -> {E}
      {_ATTRS.format(kind='PURE_ELEMWISE')} {{
    %e = tensor.empty() : {X}
    %t = hfusion.cast {{round_mode = #hfusion.round_mode<rint>}} ins(%x : {H}) outs(%e : {X}) -> {X}
    %r = hfusion.cast {{enable_overflow = true, enable_saturate = false, round_mode = #hfusion.round_mode<rint>}} ins(%t : {X}) outs(%o : {E}) -> {E}
    return %r : {E}
  }}""")
    funcs.append(f"""  func.func @e5m2_to_f16(%x: {E}, %o: {H}) -> {H}
      {_ATTRS.format(kind='PURE_ELEMWISE')} {{
    %e = tensor.empty() : {X}
    %t = hfusion.cast {{round_mode = #hfusion.round_mode<rint>}} ins(%x : {E}) outs(%e : {X}) -> {X}
    %r = hfusion.cast {{round_mode = #hfusion.round_mode<rint>}} ins(%t : {X}) outs(%o : {H}) -> {H}
    return %r : {H}
  }}""")
    for it in ("i16", "i8"):
        O = _T([n], it)
        funcs.append(f"""  func.func @ovf_{it}_trunc(%x: {X}, %o: {O}) -> {O}
      {_ATTRS.format(kind='PURE_ELEMWISE')} {{
    %r = hfusion.cast {{enable_overflow = true, round_mode = #hfusion.round_mode<trunc>}} ins(%x : {X}) outs(%o : {O}) -> {O}
    annotation.mark %r {{overflow_mode = "saturate"}} : {O}
    return %r : {O}
  }}""")
    return "module {\n" + "\n".join(funcs) + "\n}\n"


def fp8_quant(rows=64, cols=4096):
    """Dynamic per-token fp8 quantisation (the fp8 counterpart of the int8
    group): scale = max|x| / 448, q = f8E4M3FN(x / scale) with round to
    nearest even and saturation."""
    X, R = _T([rows, cols], "bf16"), _T([rows], "f32")
    XF, Q = _T([rows, cols], "f32"), _T([rows, cols], "f8E4M3FN")
    return f"""module {{
  func.func @fp8_quant(%x: {X}, %q: {Q}, %scale: {R}) -> ({Q}, {R})
      {_ATTRS.format(kind='LAST_AXIS_PBR')} {{
    %zero = arith.constant 0.000000e+00 : f32
    %fmax = arith.constant 4.480000e+02 : f32
    %e0 = tensor.empty() : {XF}
    %xf = hfusion.cast {{round_mode = #hfusion.round_mode<rint>}} ins(%x : {X}) outs(%e0 : {XF}) -> {XF}
    %e1 = tensor.empty() : {XF}
    %ax = linalg.elemwise_unary {{fun = #linalg.unary_fn<abs>}} ins(%xf : {XF}) outs(%e1 : {XF}) -> {XF}
    %e2 = tensor.empty() : {R}
    %i0 = linalg.fill ins(%zero : f32) outs(%e2 : {R}) -> {R}
    %amax = linalg.reduce {{arith.maximumf}} ins(%ax : {XF}) outs(%i0 : {R}) dimensions = [1]
    %e3 = tensor.empty() : {R}
    %sc = linalg.elemwise_binary {{fun = #linalg.binary_fn<div>}} ins(%amax, %fmax : {R}, f32) outs(%scale : {R}) -> {R}
    %e4 = tensor.empty() : {XF}
    %bs = linalg.broadcast ins(%sc : {R}) outs(%e4 : {XF}) dimensions = [1]
    %e5 = tensor.empty() : {XF}
    %y = linalg.elemwise_binary {{fun = #linalg.binary_fn<div>}} ins(%xf, %bs : {XF}, {XF}) outs(%e5 : {XF}) -> {XF}
    %qq = hfusion.cast {{round_mode = #hfusion.round_mode<rint>, enable_saturate = true}} ins(%y : {XF}) outs(%q : {Q}) -> {Q}
    return %qq, %sc : {Q}, {R}
  }}
}}
"""



# ------------------------------------------------------------ ANY_PBR / rank-N
def any_pbr_ops():
    """Reductions over a non-last axis (ANY_PBR: FusibleHelper.cpp:63-64),
    reduce_with_index along a middle / first axis, and rank-3 last-axis
    groups, one function each."""
    f = []
    # sum of squares over the middle axis of [8, 64, 100], scaled
    X, O = _T([8, 64, 100], "f32"), _T([8, 100], "f32")
    f.append(f"""  func.func @sumsq_mid(%x: {X}, %o: {O}) -> {O}
      {_ATTRS.format(kind='ANY_PBR')} {{
    %z = arith.constant 0.000000e+00 : f32
    %h = arith.constant 5.000000e-01 : f32
    %e0 = tensor.empty() : {X}
    %sq = linalg.elemwise_binary {{fun = #linalg.binary_fn<mul>}} ins(%x, %x : {X}, {X}) outs(%e0 : {X}) -> {X}
    %e1 = tensor.empty() : {O}
    %i = linalg.fill ins(%z : f32) outs(%e1 : {O}) -> {O}
    %s = linalg.reduce {{arith.addf}} ins(%sq : {X}) outs(%i : {O}) dimensions = [1]
    %r = linalg.elemwise_binary {{fun = #linalg.binary_fn<mul>}} ins(%s, %h : {O}, f32) outs(%o : {O}) -> {O}
    return %r : {O}
  }}""")
    # softmax along the first axis of [512, 1000] -> bf16
    X, R, B = _T([512, 1000], "f32"), _T([1000], "f32"), _T([512, 1000], "bf16")
    f.append(f"""  func.func @softmax_d0(%x: {X}, %o: {B}) -> {B}
      {_ATTRS.format(kind='ANY_PBR')} {{
    %ninf = arith.constant 0xFF800000 : f32
    %z = arith.constant 0.000000e+00 : f32
    %e0 = tensor.empty() : {R}
    %f0 = linalg.fill ins(%ninf : f32) outs(%e0 : {R}) -> {R}
    %m = linalg.reduce {{arith.maximumf}} ins(%x : {X}) outs(%f0 : {R}) dimensions = [0]
    %e1 = tensor.empty() : {X}
    %bm = linalg.broadcast ins(%m : {R}) outs(%e1 : {X}) dimensions = [0]
    %e2 = tensor.empty() : {X}
    %d = linalg.elemwise_binary {{fun = #linalg.binary_fn<sub>}} ins(%x, %bm : {X}, {X}) outs(%e2 : {X}) -> {X}
    %e3 = tensor.empty() : {X}
    %ex = linalg.elemwise_unary {{fun = #linalg.unary_fn<exp>}} ins(%d : {X}) outs(%e3 : {X}) -> {X}
    %e4 = tensor.empty() : {R}
    %f1 = linalg.fill ins(%z : f32) outs(%e4 : {R}) -> {R}
    %s = linalg.reduce {{arith.addf}} ins(%ex : {X}) outs(%f1 : {R}) dimensions = [0]
    %e5 = tensor.empty() : {X}
    %bs = linalg.broadcast ins(%s : {R}) outs(%e5 : {X}) dimensions = [0]
    %e6 = tensor.empty() : {X}
    %q = linalg.elemwise_binary {{fun = #linalg.binary_fn<div>}} ins(%ex, %bs : {X}, {X}) outs(%e6 : {X}) -> {X}
    %r = hfusion.cast {{round_mode = #hfusion.round_mode<rint>}} ins(%q : {X}) outs(%o : {B}) -> {B}
    return %r : {B}
  }}""")
    # argmax along the middle axis of [16, 300, 40]
    X, V, I = _T([16, 300, 40], "f32"), _T([16, 40], "f32"), _T([16, 40], "i32")
    f.append(f"""  func.func @argmax_mid(%x: {X}, %val: {V}, %idx: {I}) -> ({V}, {I})
      {_ATTRS.format(kind='ANY_PBR')} {{
    %c0 = arith.constant 0 : i32
    %ninf = arith.constant 0xFF800000 : f32
    %v0 = linalg.fill ins(%ninf : f32) outs(%val : {V}) -> {V}
    %i0 = linalg.fill ins(%c0 : i32) outs(%idx : {I}) -> {I}
    %r:2 = hfusion.reduce_with_index {{tie_break_left = true}} <max> ins(%x : {X}) outs(%v0, %i0 : {V}, {I}) dimensions = [1] -> {V}, {I}
    return %r#0, %r#1 : {V}, {I}
  }}""")
    # argmin along the first axis of an i32 [1000, 64], i64 indices
    X, V, I = _T([1000, 64], "i32"), _T([64], "i32"), _T([64], "i64")
    f.append(f"""  func.func @argmin_d0_i32(%x: {X}, %val: {V}, %idx: {I}) -> ({V}, {I})
      {_ATTRS.format(kind='ANY_PBR')} {{
    %c0 = arith.constant 0 : i64
    %big = arith.constant 2147483647 : i32
    %v0 = linalg.fill ins(%big : i32) outs(%val : {V}) -> {V}
    %i0 = linalg.fill ins(%c0 : i64) outs(%idx : {I}) -> {I}
    %r:2 = hfusion.reduce_with_index <min> ins(%x : {X}) outs(%v0, %i0 : {V}, {I}) dimensions = [0] -> {V}, {I}
    return %r#0, %r#1 : {V}, {I}
  }}""")
    # argmax over the last axis of exp(x) (fused producer: not the split-row kernel)
    X, V, I = _T([64, 777], "f32"), _T([64], "f32"), _T([64], "i32")
    f.append(f"""  func.func @argmax_fused(%x: {X}, %val: {V}, %idx: {I}) -> ({V}, {I})
      {_ATTRS.format(kind='LAST_AXIS_PBR')} {{
    %c0 = arith.constant 0 : i32
    %ninf = arith.constant 0xFF800000 : f32
    %e = tensor.empty() : {X}
    %n = linalg.elemwise_unary {{fun = #linalg.unary_fn<negf>}} ins(%x : {X}) outs(%e : {X}) -> {X}
    %v0 = linalg.fill ins(%ninf : f32) outs(%val : {V}) -> {V}
    %i0 = linalg.fill ins(%c0 : i32) outs(%idx : {I}) -> {I}
    %r:2 = hfusion.reduce_with_index <max> ins(%n : {X}) outs(%v0, %i0 : {V}, {I}) dimensions = [1] -> {V}, {I}
    return %r#0, %r#1 : {V}, {I}
  }}""")
    # rank-3 last-axis sum of [8, 64, 100]
    X, O = _T([8, 64, 100], "f32"), _T([8, 64], "f32")
    f.append(f"""  func.func @sum_rank3_last(%x: {X}, %o: {O}) -> {O}
      {_ATTRS.format(kind='LAST_AXIS_PBR')} {{
    %z = arith.constant 0.000000e+00 : f32
    %i = linalg.fill ins(%z : f32) outs(%o : {O}) -> {O}
    %s = linalg.reduce {{arith.addf}} ins(%x : {X}) outs(%i : {O}) dimensions = [2]
    return %s : {O}
  }}""")
    # rank-3 last-axis max with a [S, C] operand broadcast along the batch
    # dim: no row layout fits, the column program takes it
    X, Bv, O = _T([4, 16, 256], "f32"), _T([16, 256], "f32"), _T([4, 16], "f32")
    f.append(f"""  func.func @max_bias_rank3(%x: {X}, %b: {Bv}, %o: {O}) -> {O}
      {_ATTRS.format(kind='LAST_AXIS_PBR')} {{
    %ninf = arith.constant 0xFF800000 : f32
    %e0 = tensor.empty() : {X}
    %bb = linalg.broadcast ins(%b : {Bv}) outs(%e0 : {X}) dimensions = [0]
    %e1 = tensor.empty() : {X}
    %a = linalg.elemwise_binary {{fun = #linalg.binary_fn<add>}} ins(%x, %bb : {X}, {X}) outs(%e1 : {X}) -> {X}
    %i = linalg.fill ins(%ninf : f32) outs(%o : {O}) -> {O}
    %m = linalg.reduce {{arith.maximumf}} ins(%a : {X}) outs(%i : {O}) dimensions = [2]
    return %m : {O}
  }}""")
    # i32 sum over the first two axes of [6, 50, 33] (one collapsed reduced dim)
    X, O = _T([6, 50, 33], "i32"), _T([33], "i32")
    f.append(f"""  func.func @isum_d01(%x: {X}, %o: {O}) -> {O}
      {_ATTRS.format(kind='ANY_PBR')} {{
    %c0 = arith.constant 0 : i32
    %i = linalg.fill ins(%c0 : i32) outs(%o : {O}) -> {O}
    %s = linalg.reduce {{arith.addi}} ins(%x : {X}) outs(%i : {O}) dimensions = [0, 1]
    return %s : {O}
  }}""")
    return "module {\n" + "\n".join(f) + "\n}\n"


ANY_PBR_OPS = ["sumsq_mid", "softmax_d0", "argmax_mid", "argmin_d0_i32", "argmax_fused", "sum_rank3_last",
               "max_bias_rank3", "isum_d01"]


def transpose_ops():
    """Groups with linalg.transpose: 2-D and 3-D permutations fused with
    casts and binary ops, a transpose applied after an elementwise op, a
    permutation that only moves unit dims (a reshape), ragged tile edges."""
    f = []
    X, XT, O = _T([300, 200], "bf16"), _T([200, 300], "bf16"), _T([200, 300], "f32")
    f.append(f"""  func.func @tr2d_cast(%x: {X}, %o: {O}) -> {O}
      {_ATTRS.format(kind='PURE_ELEMWISE')} {{
    %e = tensor.empty() : {XT}
    %t = linalg.transpose ins(%x : {X}) outs(%e : {XT}) permutation = [1, 0]
    %r = hfusion.cast {{round_mode = #hfusion.round_mode<rint>}} ins(%t : {XT}) outs(%o : {O}) -> {O}
    return %r : {O}
  }}""")
    X, XT, Y, O = _T([8, 96, 130], "f32"), _T([8, 130, 96], "f32"), _T([8, 130, 96], "f32"), _T([8, 130, 96], "bf16")
    f.append(f"""  func.func @tr3d_add(%x: {X}, %y: {Y}, %o: {O}) -> {O}
      {_ATTRS.format(kind='PURE_ELEMWISE')} {{
    %e0 = tensor.empty() : {X}
    %s = hfusion.elemwise_unary {{fun = #hfusion.unary_fn<sqrt>}} ins(%x : {X}) outs(%e0 : {X}) -> {X}
    %e1 = tensor.empty() : {XT}
    %t = linalg.transpose ins(%s : {X}) outs(%e1 : {XT}) permutation = [0, 2, 1]
    %e2 = tensor.empty() : {Y}
    %a = linalg.elemwise_binary {{fun = #linalg.binary_fn<add>}} ins(%t, %y : {XT}, {Y}) outs(%e2 : {Y}) -> {Y}
    %r = hfusion.cast {{round_mode = #hfusion.round_mode<rint>}} ins(%a : {Y}) outs(%o : {O}) -> {O}
    return %r : {O}
  }}""")
    X, XT, O = _T([16, 33, 64], "i8"), _T([64, 16, 33], "i8"), _T([64, 16, 33], "i32")
    f.append(f"""  func.func @tr3d_rot_i8(%x: {X}, %o: {O}) -> {O}
      {_ATTRS.format(kind='PURE_ELEMWISE')} {{
    %e = tensor.empty() : {XT}
    %t = linalg.transpose ins(%x : {X}) outs(%e : {XT}) permutation = [2, 0, 1]
    %r = hfusion.cast {{round_mode = #hfusion.round_mode<rint>}} ins(%t : {XT}) outs(%o : {O}) -> {O}
    return %r : {O}
  }}""")
    X, XT, O = _T([4, 1, 100], "f32"), _T([4, 100, 1], "f32"), _T([4, 100, 1], "f32")
    f.append(f"""  func.func @tr_unit(%x: {X}, %o: {O}) -> {O}
      {_ATTRS.format(kind='PURE_ELEMWISE')} {{
    %e = tensor.empty() : {XT}
    %t = linalg.transpose ins(%x : {X}) outs(%e : {XT}) permutation = [0, 2, 1]
    %r = linalg.elemwise_unary {{fun = #linalg.unary_fn<abs>}} ins(%t : {XT}) outs(%o : {O}) -> {O}
    return %r : {O}
  }}""")
    return "module {\n" + "\n".join(f) + "\n}\n"


TRANSPOSE_OPS = ["tr2d_cast", "tr3d_add", "tr3d_rot_i8", "tr_unit"]

# hfusion.sort cases: (name, elem, shape, descending); the shapes of
# bishengir/test/Dialect/HFusion/test_sort.mlir (6, 4x4, 2x3x4 descending),
# ragged and power-of-two rows, one element per row, the longest row (16384)
SORT_OPS = [("sort_1d_asc", "f32", [6], False), ("sort_2d_asc", "f32", [4, 4], False),
            ("sort_3d_desc", "f32", [2, 3, 4], True), ("sort_f32_asc", "f32", [64, 1000], False),
            ("sort_f32_desc", "f32", [37, 77], True), ("sort_bf16_asc", "bf16", [16, 4096], False),
            ("sort_f16_desc", "f16", [8, 333], True), ("sort_i8_asc", "i8", [33, 100], False),
            ("sort_i16_desc", "i16", [5, 2048], True), ("sort_i32_asc", "i32", [3, 16384], False),
            ("sort_i32_desc", "i32", [50, 3], True), ("sort_f32_len1", "f32", [100, 1], False)]


def neg_sort_scale(rows=37, cols=300):
    """An un-fused host function y = 2 * sort(-x) (descending) along the last
    axis: the front-end outlines the sort as a kernel of its own between two
    elementwise groups."""
    X = _T([rows, cols], "f32")
    return f"""module {{
  func.func @neg_sort_scale(%x: {X}) -> {X}
      attributes {{hacc.function_kind = #hacc.function_kind<HOST>}} {{
    %e0 = tensor.empty() : {X}
    %a = linalg.elemwise_unary {{fun = #linalg.unary_fn<negf>}} ins(%x : {X}) outs(%e0 : {X}) -> {X}
    %s = hfusion.sort ins(%a : {X}) descending = true sort_axis = 1 -> {X}
    %c = arith.constant 2.000000e+00 : f32
    %e1 = tensor.empty() : {X}
    %b = linalg.elemwise_binary {{fun = #linalg.binary_fn<mul>}} ins(%s, %c : {X}, f32) outs(%e1 : {X}) -> {X}
    return %b : {X}
  }}
}}
"""


def sort_ops():
    """One module, one group per hfusion.sort case."""
    funcs = []
    for name, elem, shape, desc in SORT_OPS:
        X = _T(shape, elem)
        funcs.append(f"""  func.func @{name}(%x: {X}) -> {X}
      {_ATTRS.format(kind='ANY_PB')} {{
    %r = hfusion.sort ins(%x : {X}) descending = {str(desc).lower()} sort_axis = {len(shape) - 1} -> {X}
    return %r : {X}
  }}""")
    return "module {\n" + "\n".join(funcs) + "\n}\n"


def sigmoid_grad_sums(b=24, s=512, h=16, w=12, name="sig_sums"):
    """The model-derived LAST_AXIS_PBR group of
    bishengir/test/Dialect/HFusion/hfusion-pipeline.mlir:56-125 at its shape
    [24, 512, 16, 12] (parametrised): a sigmoid-gradient chain in bf16 over
    row-broadcast [B, S, 1, 1] operands collapsed to [B, S], four f32 row sums
    over the trailing [H, W] (two of them through a collapse to [B, S, H*W]),
    two results expanded back to [B, S, 1, 1] and cast to bf16."""
    X, XB = _T([b, s, h, w], "bf16"), _T([b, s, 1, 1], "bf16")
    XF, XC = _T([b, s, h, w], "f32"), _T([b, s, h * w], "f32")
    RB, R2, R4, R4B = _T([b, s], "bf16"), _T([b, s], "f32"), _T([b, s, 1, 1], "f32"), _T([b, s, 1, 1], "bf16")
    XI = _T([b, s, h, w], "i64")
    mul = "linalg.elemwise_binary {fun = #linalg.binary_fn<mul>}"
    add = "linalg.elemwise_binary {fun = #linalg.binary_fn<add>}"
    rint = "hfusion.cast {round_mode = #hfusion.round_mode<rint>}"
    red = "linalg.reduce ins({x} : {t}) outs(%zs : {R2}) dimensions = {d}\n      (%in: f32, %init: f32) {{\n        %q = arith.addf %in, %init : f32\n        linalg.yield %q : f32\n      }}"
    return f"""module {{
  func.func @{name}(%a0: {X}, %a1: {X}, %a2: {XB}, %a3: {XB}, %a4: {XF}) -> ({R2}, {R2}, {R4}, {R4}, {R4B}, {R4B})
      {_ATTRS.format(kind='LAST_AXIS_PBR')} {{
    %one_t = arith.constant dense<1> : tensor<i64>
    %one_i = arith.constant 1 : i64
    %one = arith.constant 1.000000e+00 : bf16
    %zero = arith.constant 0.000000e+00 : f32
    %e = tensor.empty() : {X}
    %c2 = tensor.collapse_shape %a2 [[0], [1, 2, 3]] : {XB} into {RB}
    %b2 = linalg.broadcast ins(%c2 : {RB}) outs(%e : {X}) dimensions = [2, 3]
    %m1 = {mul} ins(%a1, %b2 : {X}, {X}) outs(%e : {X}) -> {X}
    %c3 = tensor.collapse_shape %a3 [[0], [1, 2, 3]] : {XB} into {RB}
    %b3 = linalg.broadcast ins(%c3 : {RB}) outs(%e : {X}) dimensions = [2, 3]
    %ei = tensor.empty() : {XI}
    %fi = linalg.fill ins(%one_i : i64) outs(%ei : {XI}) -> {XI}
    %ones = hfusion.cast {{round_mode = #hfusion.round_mode<trunc>}} ins(%fi : {XI}) outs(%e : {X}) -> {X}
    %m5 = {mul} ins(%b3, %ones : {X}, {X}) outs(%e : {X}) -> {X}
    %z = {add} ins(%m1, %m5 : {X}, {X}) outs(%e : {X}) -> {X}
    %nz = linalg.elemwise_unary {{fun = #linalg.unary_fn<negf>}} ins(%z : {X}) outs(%e : {X}) -> {X}
    %ex = linalg.elemwise_unary {{fun = #linalg.unary_fn<exp>}} ins(%nz : {X}) outs(%e : {X}) -> {X}
    %den = {add} ins(%ex, %one : {X}, bf16) outs(%e : {X}) -> {X}
    %sig = linalg.elemwise_binary {{fun = #linalg.binary_fn<div>}} ins(%one, %den : bf16, {X}) outs(%e : {X}) -> {X}
    %one_f = arith.sitofp %one_t : tensor<i64> to tensor<bf16>
    %bone = linalg.broadcast ins(%one_f : tensor<bf16>) outs(%e : {X}) dimensions = [0, 1, 2, 3]
    %s12 = {mul} ins(%sig, %ones : {X}, {X}) outs(%e : {X}) -> {X}
    %s13 = linalg.elemwise_binary {{fun = #linalg.binary_fn<sub>}} ins(%bone, %s12 : {X}, {X}) outs(%e : {X}) -> {X}
    %s14 = {mul} ins(%z, %s13 : {X}, {X}) outs(%e : {X}) -> {X}
    %s15 = {mul} ins(%ones, %ones : {X}, {X}) outs(%e : {X}) -> {X}
    %s16 = {add} ins(%s14, %s15 : {X}, {X}) outs(%e : {X}) -> {X}
    %s17 = {mul} ins(%sig, %s16 : {X}, {X}) outs(%e : {X}) -> {X}
    %s18 = {mul} ins(%a0, %s17 : {X}, {X}) outs(%e : {X}) -> {X}
    %s19 = {mul} ins(%s18, %b2 : {X}, {X}) outs(%e : {X}) -> {X}
    %ef = tensor.empty() : {XF}
    %f21 = {rint} ins(%s19 : {X}) outs(%ef : {XF}) -> {XF}
    %f22 = {mul} ins(%f21, %a4 : {XF}, {XF}) outs(%ef : {XF}) -> {XF}
    %k22 = tensor.collapse_shape %f22 [[0], [1], [2, 3]] : {XF} into {XC}
    %er = tensor.empty() : {R2}
    %zs = linalg.fill ins(%zero : f32) outs(%er : {R2}) -> {R2}
    %r0 = {red.format(x="%k22", t=XC, R2=R2, d="[2]")}
    %k21 = tensor.collapse_shape %f21 [[0], [1], [2, 3]] : {XF} into {XC}
    %r1 = {red.format(x="%k21", t=XC, R2=R2, d="[2]")}
    %p25 = {mul} ins(%s18, %a1 : {X}, {X}) outs(%e : {X}) -> {X}
    %f26 = {rint} ins(%p25 : {X}) outs(%ef : {XF}) -> {XF}
    %r2 = {red.format(x="%f26", t=XF, R2=R2, d="[2, 3]")}
    %x2 = tensor.expand_shape %r2 [[0], [1, 2, 3]] output_shape [{b}, {s}, 1, 1] : {R2} into {R4}
    %f27 = {rint} ins(%s18 : {X}) outs(%ef : {XF}) -> {XF}
    %r3 = {red.format(x="%f27", t=XF, R2=R2, d="[2, 3]")}
    %x3 = tensor.expand_shape %r3 [[0], [1, 2, 3]] output_shape [{b}, {s}, 1, 1] : {R2} into {R4}
    %eb = tensor.empty() : {R4B}
    %o4 = {rint} ins(%x2 : {R4}) outs(%eb : {R4B}) -> {R4B}
    %o5 = {rint} ins(%x3 : {R4}) outs(%eb : {R4B}) -> {R4B}
    return %r0, %r1, %x2, %x3, %o4, %o5 : {R2}, {R2}, {R4}, {R4}, {R4B}, {R4B}
  }}
}}
"""


def reshape_transpose_ops():
    """Reshapes and transposes inside groups that reduce or broadcast (the
    reference admits both into LAST_AXIS_PBR / ANY_PBR / ANY_PB groups,
    FusibleHelper.cpp:617-629), one function each."""
    f = []
    # ANY_PB: a [R,1,1] operand collapsed to [R] and broadcast over a
    # collapsed [R, 8*64] view of x; the product expanded back to x's shape
    X, XC, Bv, BC = _T([16, 8, 64], "f32"), _T([16, 512], "f32"), _T([16, 1, 1], "f32"), _T([16], "f32")
    f.append(f"""  func.func @rs_bcast_pb(%x: {X}, %b: {Bv}, %o: {X}) -> {X}
      {_ATTRS.format(kind='ANY_PB')} {{
    %xc = tensor.collapse_shape %x [[0], [1, 2]] : {X} into {XC}
    %bc = tensor.collapse_shape %b [[0, 1, 2]] : {Bv} into {BC}
    %e = tensor.empty() : {XC}
    %bb = linalg.broadcast ins(%bc : {BC}) outs(%e : {XC}) dimensions = [1]
    %m = linalg.elemwise_binary {{fun = #linalg.binary_fn<mul>}} ins(%xc, %bb : {XC}, {XC}) outs(%e : {XC}) -> {XC}
    %me = tensor.expand_shape %m [[0], [1, 2]] output_shape [16, 8, 64] : {XC} into {X}
    %r = linalg.elemwise_binary {{fun = #linalg.binary_fn<sub>}} ins(%me, %x : {X}, {X}) outs(%o : {X}) -> {X}
    return %r : {X}
  }}""")
    # ANY_PBR: a sum over a collapsed middle pair of dims, expanded to [6,1,30]
    X, XC, O2, O3 = _T([6, 10, 20, 30], "f32"), _T([6, 200, 30], "f32"), _T([6, 30], "f32"), _T([6, 1, 30], "f32")
    f.append(f"""  func.func @rs_sum_mid(%x: {X}, %o: {O3}) -> {O3}
      {_ATTRS.format(kind='ANY_PBR')} {{
    %z = arith.constant 0.000000e+00 : f32
    %e = tensor.empty() : {X}
    %sq = linalg.elemwise_binary {{fun = #linalg.binary_fn<mul>}} ins(%x, %x : {X}, {X}) outs(%e : {X}) -> {X}
    %c = tensor.collapse_shape %sq [[0], [1, 2], [3]] : {X} into {XC}
    %e1 = tensor.empty() : {O2}
    %i = linalg.fill ins(%z : f32) outs(%e1 : {O2}) -> {O2}
    %s = linalg.reduce {{arith.addf}} ins(%c : {XC}) outs(%i : {O2}) dimensions = [1]
    %x3 = tensor.expand_shape %s [[0, 1], [2]] output_shape [6, 1, 30] : {O2} into {O3}
    %r = hfusion.elemwise_unary {{fun = #hfusion.unary_fn<sqrt>}} ins(%x3 : {O3}) outs(%o : {O3}) -> {O3}
    return %r : {O3}
  }}""")
    # LAST_AXIS_PBR: transpose -> mul -> row sum
    X, XT, O = _T([300, 64], "f32"), _T([64, 300], "f32"), _T([64], "f32")
    f.append(f"""  func.func @tr_mul_sum(%x: {X}, %y: {XT}, %o: {O}) -> {O}
      {_ATTRS.format(kind='LAST_AXIS_PBR')} {{
    %z = arith.constant 0.000000e+00 : f32
    %e = tensor.empty() : {XT}
    %t = linalg.transpose ins(%x : {X}) outs(%e : {XT}) permutation = [1, 0]
    %e1 = tensor.empty() : {XT}
    %m = linalg.elemwise_binary {{fun = #linalg.binary_fn<mul>}} ins(%t, %y : {XT}, {XT}) outs(%e1 : {XT}) -> {XT}
    %i = linalg.fill ins(%z : f32) outs(%o : {O}) -> {O}
    %s = linalg.reduce {{arith.addf}} ins(%m : {XT}) outs(%i : {O}) dimensions = [1]
    return %s : {O}
  }}""")
    # argmax along the last axis of a transposed bf16 tensor
    X, XT, V, I = _T([500, 40], "bf16"), _T([40, 500], "bf16"), _T([40], "bf16"), _T([40], "i32")
    f.append(f"""  func.func @tr_argmax(%x: {X}, %val: {V}, %idx: {I}) -> ({V}, {I})
      {_ATTRS.format(kind='LAST_AXIS_PBR')} {{
    %c0 = arith.constant 0 : i32
    %ninf = arith.constant 0xFF80 : bf16
    %e = tensor.empty() : {XT}
    %t = linalg.transpose ins(%x : {X}) outs(%e : {XT}) permutation = [1, 0]
    %v0 = linalg.fill ins(%ninf : bf16) outs(%val : {V}) -> {V}
    %i0 = linalg.fill ins(%c0 : i32) outs(%idx : {I}) -> {I}
    %r:2 = hfusion.reduce_with_index <max> ins(%t : {XT}) outs(%v0, %i0 : {V}, {I}) dimensions = [1] -> {V}, {I}
    return %r#0, %r#1 : {V}, {I}
  }}""")
    # a rank-3 transpose feeding a max over the middle axis, with a bias
    # broadcast along the transposed result's last axis
    X, XT, Bv, O = _T([12, 40, 70], "f32"), _T([70, 12, 40], "f32"), _T([70], "f32"), _T([70, 40], "f32")
    f.append(f"""  func.func @tr3_max_bias(%x: {X}, %b: {Bv}, %o: {O}) -> {O}
      {_ATTRS.format(kind='ANY_PBR')} {{
    %ninf = arith.constant 0xFF800000 : f32
    %e = tensor.empty() : {XT}
    %t = linalg.transpose ins(%x : {X}) outs(%e : {XT}) permutation = [2, 0, 1]
    %e1 = tensor.empty() : {XT}
    %bb = linalg.broadcast ins(%b : {Bv}) outs(%e1 : {XT}) dimensions = [1, 2]
    %e2 = tensor.empty() : {XT}
    %a = linalg.elemwise_binary {{fun = #linalg.binary_fn<add>}} ins(%t, %bb : {XT}, {XT}) outs(%e2 : {XT}) -> {XT}
    %i = linalg.fill ins(%ninf : f32) outs(%o : {O}) -> {O}
    %m = linalg.reduce {{arith.maximumf}} ins(%a : {XT}) outs(%i : {O}) dimensions = [1]
    return %m : {O}
  }}""")
    # ANY_PB: a transposed operand minus a broadcast row vector
    X, XT, Bv = _T([64, 100], "f32"), _T([100, 64], "f32"), _T([64], "f32")
    f.append(f"""  func.func @tr_bcast_sub(%x: {X}, %b: {Bv}, %o: {XT}) -> {XT}
      {_ATTRS.format(kind='ANY_PB')} {{
    %e = tensor.empty() : {XT}
    %t = linalg.transpose ins(%x : {X}) outs(%e : {XT}) permutation = [1, 0]
    %e1 = tensor.empty() : {XT}
    %bb = linalg.broadcast ins(%b : {Bv}) outs(%e1 : {XT}) dimensions = [0]
    %r = linalg.elemwise_binary {{fun = #linalg.binary_fn<sub>}} ins(%t, %bb : {XT}, {XT}) outs(%o : {XT}) -> {XT}
    return %r : {XT}
  }}""")
    return "module {\n" + "\n".join(f) + "\n}\n"


RS_TR_OPS = ["rs_bcast_pb", "rs_sum_mid", "tr_mul_sum", "tr_argmax", "tr3_max_bias", "tr_bcast_sub"]


def host_reshape_sum(b=8, h=16, w=32):
    """Un-fused host IR: exp -> collapse_shape -> row sum -> expand_shape ->
    log.  The front-end fuses it into one LAST_AXIS_PBR group whose reshapes
    the lowering resolves."""
    X, XC, R, R2 = _T([b, h, w], "f32"), _T([b, h * w], "f32"), _T([b], "f32"), _T([b, 1], "f32")
    return f"""module {{
  func.func @prog_rs_exp_sum_log(%x: {X}, %o: {R2}) -> {R2}
      attributes {{hacc.function_kind = #hacc.function_kind<HOST>}} {{
    %z = arith.constant 0.000000e+00 : f32
    %e = tensor.empty() : {X}
    %a = linalg.elemwise_unary {{fun = #linalg.unary_fn<exp>}} ins(%x : {X}) outs(%e : {X}) -> {X}
    %c = tensor.collapse_shape %a [[0], [1, 2]] : {X} into {XC}
    %e1 = tensor.empty() : {R}
    %i = linalg.fill ins(%z : f32) outs(%e1 : {R}) -> {R}
    %s = linalg.reduce {{arith.addf}} ins(%c : {XC}) outs(%i : {R}) dimensions = [1]
    %x2 = tensor.expand_shape %s [[0, 1]] output_shape [{b}, 1] : {R} into {R2}
    %r = linalg.elemwise_unary {{fun = #linalg.unary_fn<log>}} ins(%x2 : {R2}) outs(%o : {R2}) -> {R2}
    return %r : {R2}
  }}
}}
"""


def host_transpose_sum(m=300, n=64):
    """Un-fused host IR: transpose -> mul -> row sum (one fused group)."""
    X, XT, O = _T([m, n], "f32"), _T([n, m], "f32"), _T([n], "f32")
    return f"""module {{
  func.func @prog_tr_mul_sum(%x: {X}, %y: {XT}, %o: {O}) -> {O}
      attributes {{hacc.function_kind = #hacc.function_kind<HOST>}} {{
    %z = arith.constant 0.000000e+00 : f32
    %e = tensor.empty() : {XT}
    %t = linalg.transpose ins(%x : {X}) outs(%e : {XT}) permutation = [1, 0]
    %e1 = tensor.empty() : {XT}
    %m = linalg.elemwise_binary {{fun = #linalg.binary_fn<mul>}} ins(%t, %y : {XT}, {XT}) outs(%e1 : {XT}) -> {XT}
    %i = linalg.fill ins(%z : f32) outs(%o : {O}) -> {O}
    %s = linalg.reduce {{arith.addf}} ins(%m : {XT}) outs(%i : {O}) dimensions = [1]
    return %s : {O}
  }}
}}
"""


def entries():
    """name -> IR text of every group the tests run: the product groups plus
    the parity cases below."""
    e = dict(_product.entries())
    # reduced / ragged parity sizes
    e["vec_add_1m"] = g.vec_add(1 << 20)
    e["vec_add_ragged"] = g.vec_add(1001)
    e["vec_add_i16"] = g.vec_add(16, dtype="i16")
    e["rmsnorm_quant_ragged"] = g.rmsnorm_quant(13, 1000)
    e["rmsnorm_quant_w2048"] = g.rmsnorm_quant(96, 2048)
    # a nonzero init of the sum of squares (the kernel's first lane and its
    # fallback walk start from it)
    e["rmsnorm_quant_init"] = g.rmsnorm_quant(256, 4096).replace(
        "%i2 = linalg.fill ins(%zero", "%i2 = linalg.fill ins(%sinit").replace(
        "%zero = arith.constant", "%sinit = arith.constant 3.000000e-01 : f32\n    %zero = arith.constant", 1)
    e["rmsnorm_quant_w3072"] = g.rmsnorm_quant(64, 3072)
    e["safe_softmax_64"] = g.safe_softmax(64, 32768)
    e["safe_softmax_ragged"] = g.safe_softmax(33, 1000)
    e["argmax_16"] = g.argmax(16, 152064)
    e["argmax_ragged"] = g.argmax(5, 1001)
    e["argmax_i64"] = g.argmax(8, 4096, index_type="i64")
    e["argmin_ragged"] = g.argmax(9, 5001, kind="min")
    e["argmax_tall"] = g.argmax(2048, 33797)
    e["w8a8_512"] = g.w8a8_dequant(512, 512, 512)
    e["w8a8_ragged"] = g.w8a8_dequant(300, 200, 160)
    e["w8a8_ragged_dma"] = g.w8a8_dequant(300, 200, 192)
    e["w8a8_ragged_dma128"] = g.w8a8_dequant(300, 200, 384)
    e["w8a8_kn"] = g.w8a8_dequant(320, 256, 128, b_layout="kn")
    e["w8a8_kn_ragged"] = g.w8a8_dequant(300, 208, 384, b_layout="kn")
    e["w8a8_kn_wide"] = g.w8a8_dequant(264, 784, 256, b_layout="kn")
    e["w8a8_kn_dma64"] = g.w8a8_dequant(300, 208, 192, b_layout="kn")
    e["w8a8_kn_tiny"] = g.w8a8_dequant(1, 16, 128, b_layout="kn")
    # hfusion.matmul_mx: typed fp8, bytes through hfusion.bitcast, bytes with
    # lhsFormat / rhsFormat; ragged M and N; a fill init and a bf16 epilogue
    e["mx_e4m3"] = g.matmul_mx(256, 256, 256, name="mx_e4m3")
    e["mx_e5m2_bitcast"] = g.matmul_mx(300, 208, 384, fa="e5m2", fb="e4m3", via="bitcast", init=0.5, name="mx_e5m2_bitcast")
    e["mx_format_bf16"] = g.matmul_mx(264, 784, 256, fa="e4m3", fb="e5m2", via="format", out="bf16", name="mx_format_bf16")
    e["mx_e5m2"] = g.matmul_mx(128, 128, 128, fa="e5m2", fb="e5m2", name="mx_e5m2")
    # fp4 (e2m1, format 3): bytes holding two values along K, bitcast to
    # f8E5M2 as in matmul-mx-format.mlir, or with the formats alone
    e["mx_fp4_256"] = g.matmul_mx(256, 256, 512, fa="e2m1", fb="e2m1", via="bitcast", name="mx_fp4_256")
    e["mx_fp4_ragged"] = g.matmul_mx(300, 208, 768, fa="e2m1", fb="e2m1", via="format", init=0.5, name="mx_fp4_ragged")
    e["mx_fp4_bf16"] = g.matmul_mx(264, 784, 256, fa="e2m1", fb="e2m1", via="bitcast", out="bf16", name="mx_fp4_bf16")
    # the same through scaled bf16 operands and the bf16 matrix core (mx_exact=1)
    for n in ("mx_e4m3", "mx_e5m2_bitcast", "mx_format_bf16", "mx_e5m2", "mx_fp8"):
        e[n + "_exact"] = e[n]
    e["bf16_mmad_ragged"] = g.bf16_mmad(200, 136, 96)
    e["bf16_mmad_ragged128"] = g.bf16_mmad(200, 136, 192)
    # B [K, N] through the ring (16-bit transposing reads), bf16 and f16
    e["bf16_mmad_kn"] = g.bf16_mmad(256, 256, 128, b_layout="kn")
    e["bf16_mmad_kn_ragged"] = g.bf16_mmad(200, 136, 192, b_layout="kn")
    e["f16_mmad_kn"] = g.bf16_mmad(264, 520, 320, b_layout="kn", elem="f16")
    e["bf16_mmad_kn_tiny"] = g.bf16_mmad(3, 8, 64, b_layout="kn")
    e["mm_i8_full"] = g.mm_i8(4096, 4096, 4096)
    # hivm.hir.matmul forms of bishengir/test/Dialect/HIVM/IR/ops.mlir (16x16 f16) and wider
    e["hivm_mm_f16_null"] = g.hivm_matmul(16, 16, 16)
    e["hivm_mm_f16_bias_pc"] = g.hivm_matmul(16, 16, 16, bias="f16", descale="f16", descale_mode="DescalePerChannel")
    e["hivm_mm_f16_bias_pt_t"] = g.hivm_matmul(16, 16, 16, bias="f16", descale="f16", descale_mode="DescalePerTensor",
                                               a_t=True, b_t=True)
    e["hivm_mm_i8_pc"] = g.hivm_matmul(300, 200, 192, elem="i8", out="bf16", bias="i32", descale="f32",
                                       descale_mode="DescalePerChannel", b_t=True)
    e["hivm_mm_i8_pt_i8out"] = g.hivm_matmul(256, 320, 128, elem="i8", out="i8", descale="f32",
                                             descale_mode="DescalePerTensor", b_t=True)
    e["hivm_mm_bf16_at"] = g.hivm_matmul(160, 96, 64, elem="bf16", out="f32", bias="f32", a_t=True)
    # A [K, M] staged K-major on the ring, with B [N, K] or [K, N]
    e["hivm_mm_i8_at"] = g.hivm_matmul(272, 320, 256, elem="i8", out="bf16", descale="f32",
                                       descale_mode="DescalePerChannel", a_t=True, b_t=True)
    e["hivm_mm_i8_at_kn"] = g.hivm_matmul(256, 208, 384, elem="i8", out="bf16", descale="f32",
                                          descale_mode="DescalePerTensor", a_t=True)
    e["hivm_mm_bf16_at_bt"] = g.hivm_matmul(200, 136, 128, elem="bf16", out="f32", a_t=True, b_t=True)
    e["hivm_mm_f16_at_bt"] = g.hivm_matmul(152, 264, 192, elem="f16", out="f16", a_t=True, b_t=True)
    e["mm_i8_ragged"] = g.mm_i8(300, 200, 192)
    e["bf16_mmad_256"] = g.bf16_mmad(256, 256, 256)
    e["cast_modes"] = cast_modes(4096)
    e["eltwise_mix"] = eltwise_mix(64, 1000)
    e["layernorm"] = layernorm(64, 2048)
    e["reduce_ops"] = reduce_ops(48, 3000)
    e["math_fns"] = math_fns(4096)
    e["fp_ops"] = fp_ops(4096)
    e["scan_ops"] = scan_ops()
    e["misc_ops"] = misc_ops()
    e["gather_ops"] = gather_ops()
    e["memref_chain"] = memref_chain(4096)
    e["reshape_chain"] = reshape_chain()
    e["generic_ops"] = generic_ops()
    e["fuzz_generic"] = fuzz_generic()
    e["fuzz_rows"] = fuzz_rows()
    e["generic_reduce"] = generic_reduce()
    e["any_pbr_ops"] = any_pbr_ops()
    e["transpose_ops"] = transpose_ops()
    e["sig_sums"] = sigmoid_grad_sums()
    e["sig_sums_small"] = sigmoid_grad_sums(3, 40, 4, 6, name="sig_sums_small")
    e["rs_tr_ops"] = reshape_transpose_ops()
    e["prog_rs_exp_sum_log"] = host_reshape_sum()
    e["prog_tr_mul_sum"] = host_transpose_sum()
    e["sort_ops"] = sort_ops()
    e["prog_neg_sort_scale"] = neg_sort_scale()
    # dynamic row counts (compiled per size: DynamicGroup / option dyn=...)
    e["rmsnorm_quant_dyn"] = g.with_dynamic_rows(g.rmsnorm_quant(7919, 4096), 7919)
    e["softmax_dyn"] = g.with_dynamic_rows(g.safe_softmax(7919, 1000), 7919)
    e["vec_add_dyn"] = g.with_dynamic_rows(g.vec_add(7919), 7919)
    # one kernel for every row count (compiler option dyn=runtime)
    e["rmsnorm_quant_dyn_rt"] = e["rmsnorm_quant_dyn"]
    e["softmax_dyn_rt"] = e["softmax_dyn"]
    e["eltwise_mix_dyn_rt"] = g.with_dynamic_rows(eltwise_mix(67, 1000), 67)
    e["w8a8_dyn_rt"] = g.with_dynamic_rows(g.w8a8_dequant(333, 512, 512), 333)
    e["argmax_dyn_rt"] = g.with_dynamic_rows(g.argmax(333, 50000), 333)
    e["mx_fp4_dyn_rt"] = g.with_dynamic_rows(g.matmul_mx(333, 256, 512, fa="e2m1", fb="e2m1", via="bitcast",
                                                         name="mx_fp4_dyn"), 333)
    e["rmsnorm_quant_rank3"] = g.rmsnorm_quant(256, 1024, batch=4)
    # the same groups through the one-wave-per-row kernel (hf_rmsq.h, the
    # default for the widths it takes), named for it ...
    for n in ("rmsnorm_quant", "rmsnorm_quant_256", "rmsnorm_quant_rank3", "rmsnorm_quant_ragged"):
        e[n + "_rmsq"] = e[n]
    # ... through the generic row program (option rmsq_kernel=0) ...
    for n in ("rmsnorm_quant", "rmsnorm_quant_256", "rmsnorm_quant_rank3"):
        e[n + "_rowprog"] = e[n]
    # ... and through the opt-in chain-wave kernel (hf_rmsn.h)
    for n in ("rmsnorm_quant", "rmsnorm_quant_256", "rmsnorm_quant_rank3"):
        e[n + "_rmsn"] = e[n]
    e["rank0"] = """module {
  func.func @rank0(%a: tensor<f32>, %b: tensor<f32>) -> tensor<f32>
      """ + _ATTRS.format(kind='PURE_ELEMWISE') + """ {
    %e = tensor.empty() : tensor<f32>
    %r = linalg.elemwise_binary {fun = #linalg.binary_fn<mul>} ins(%a, %b : tensor<f32>, tensor<f32>) outs(%e : tensor<f32>) -> tensor<f32>
    %e2 = tensor.empty() : tensor<f32>
    %s = hfusion.elemwise_unary {fun = #hfusion.unary_fn<sqrt>} ins(%r : tensor<f32>) outs(%e2 : tensor<f32>) -> tensor<f32>
    return %s : tensor<f32>
  }
}
"""
    e["quant_ties"] = quant_ties(64, 1024)
    e["quant_i8_ties"] = quant_i8_ties(64, 1024)
    e["quant_i8_ties_m128"] = quant_i8_ties(64, 1024, lo=-128, name="quant_i8_ties_m128")
    e["quant_i8_ties_narrow"] = quant_i8_ties(64, 1000, lo=-100, hi=100, name="quant_i8_ties_narrow")
    e["cast_fp8"] = cast_fp8(4096)
    e["fp8_quant"] = fp8_quant(64, 4096)
    e["fp8_quant_ragged"] = fp8_quant(13, 1000)
    # un-fused host functions: the fusion front-end splits them into launch
    # programs of several groups
    e["prog_gemm_rmsnorm_quant"] = g.gemm_rmsnorm_quant(256, 512, 256)
    e["prog_gemm_rmsnorm_quant_ragged"] = g.gemm_rmsnorm_quant(100, 320, 192)
    e["prog_scores_softmax"] = g.scores_softmax(128, 1024, 128)
    e["prog_scores_softmax_ragged"] = g.scores_softmax(72, 1000, 64)
    e["prog_exp_cumsum_scale"] = g.exp_cumsum_scale(64, 1000)
    return e


def get(name):
    return entries()[name]


# row counts the dynamic groups are prebuilt for (the GPU tests call them with these)
DYN_ROWS = {"rmsnorm_quant_dyn": [1, 37, 300], "softmax_dyn": [5, 129], "vec_add_dyn": [1, 1000, 65537]}


def dyn_options(name, rows):
    """The specialisation option of a dynamic catalog group at `rows` rows
    (every dynamic dim of these groups is the row count)."""
    dg = DynamicGroup(get(name))
    return dg.options_for([rows] * len(dg.dims))


def options(name):
    """Compiler options a prebuilt group is built with ("" for the defaults;
    a dynamic group: its first prebuilt row count)."""
    if name in DYN_ROWS:
        return dyn_options(name, DYN_ROWS[name][0])
    if name.endswith("_rmsq"):
        return "rmsq_kernel=1"
    if name.endswith("_rowprog"):
        return "rmsq_kernel=0"
    if name.endswith("_rt"):
        return "dyn=runtime"
    if name.endswith("_exact"):
        return "mx_exact=1"
    return "rmsn_kernel=1" if name.endswith("_rmsn") else ""
