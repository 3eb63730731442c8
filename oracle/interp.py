"""hfref interpreter — executes an HFusion group IR on the CPU the way the
reference's CPU lowering does.  TEST INFRASTRUCTURE ONLY: imported by tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg, never by the product.

Restates `lower-for-cpu-runner-pipeline`
(bishengir/lib/ExecutionEngine/ExecutionEnginePipelines.cpp:39-90): every op
becomes its own loop nest over materialised buffers; scalar bodies come from
RegionBuilderHelper (bishengir/lib/Dialect/HFusion/IR/HFusionOps.cpp:434-862),
reductions fold serially from the `outs` init (convert-linalg-to-loops),
reduce_with_index uses the region of HFusionOps.cpp:1507-1595 and
linalg.matmul the upstream mul/add region with k innermost.

The IR reader here is independent of the product's C++ reader (a different
implementation of the same textual subset), so a parse mistake on one side
shows up as a parity failure.

`cast_semantics`:
  "declared" — hfusion.cast honours its round_mode / enable_saturate
               (HFusionEnums.td:122-141); this is what the MI355X kernels do.
  "cpu"      — what the CPU lowering executes: convertScalarToDtype ignores
               the round mode (f32->iN is fptosi = truncation, same-type float
               casts are math.round; HFusionOps.cpp:762-862).
"""
import ctypes
import os
import re

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
_lib = None


def lib():
    global _lib
    if _lib is None:
        path = os.path.join(HERE, "libhfref.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} not built (make -C {HERE})")
        L = ctypes.CDLL(path)
        P = ctypes.c_void_p
        I64 = ctypes.c_int64
        INT = ctypes.c_int
        sig = {
            "hfref_unary_f32": [INT, P, P, I64],
            "hfref_binary_f32": [INT, P, P, P, I64],
            "hfref_fma_f32": [P, P, P, P, I64],
            "hfref_binary_i64": [INT, P, P, P, I64, INT],
            "hfref_compare_f32": [INT, P, P, P, I64],
            "hfref_compare_i64": [INT, P, P, P, I64],
            "hfref_bf16_to_f32_n": [P, P, I64],
            "hfref_fp8_to_f32_n": [P, P, I64, INT],
            "hfref_matmul_mx": [P, P, P, P, P, I64, I64, I64, INT, INT],
            "hfref_f32_to_fp8_n": [P, P, I64, INT, INT, INT],
            "hfref_int_to_fp8_n": [P, P, I64, INT, INT, INT],
            "hfref_f32_to_bf16_n": [P, P, I64, INT],
            "hfref_f16_to_f32_n": [P, P, I64],
            "hfref_f32_to_f16_n": [P, P, I64, INT],
            "hfref_fptosi_n": [P, P, I64, INT, P],
            "hfref_f32_to_int_mode_n": [P, P, I64, INT, INT, INT],
            "hfref_int_to_f32_n": [P, P, I64, INT],
            "hfref_roundeven_n": [P, P, I64],
            "hfref_round_n": [P, P, I64],
            "hfref_reduce_f32": [INT, P, P, I64, I64],
            "hfref_reduce_i64": [INT, P, P, I64, I64, INT],
            "hfref_reduce_with_index_f32": [INT, P, P, P, P, I64, I64],
            "hfref_reduce_with_index_i64": [INT, P, P, P, P, I64, I64, INT],
            "hfref_matmul_i8_i32": [P, P, P, I64, I64, I64, INT],
            "hfref_matmul_f32": [P, P, P, I64, I64, I64, INT],
            "hfref_vecadd_f32": [P, P, P, I64],
            "hfref_rmsnorm_quant": [P, P, ctypes.c_float, P, P, I64, I64],
            "hfref_softmax_bf16": [P, P, I64, I64],
            "hfref_argmax": [P, P, P, I64, I64],
            "hfref_w8a8_dequant_rows": [P, P, P, P, P, I64, I64, I64, I64, I64],
            "hfref_memref_gather": [P, INT, INT, P],
            "hfref_memref_scatter": [P, P, INT, INT],
            "hfref_vecadd_f32_memref": [P, P, P],
            "hfref_rmsnorm_quant_memref": [P, P, ctypes.c_float, P, P],
            "hfref_softmax_bf16_memref": [P, P],
            "hfref_argmax_memref": [P, P, P],
            "hfref_w8a8_dequant_memref": [P, P, P, P, P],
            "hfref_sort_rows": [P, I64, I64, INT, INT],
        }
        for name, args in sig.items():
            f = getattr(L, name)
            f.argtypes = args
            f.restype = None
        for name in ("hfref_f32_to_bf16", "hfref_f32_to_f16", "hfref_f32_to_bf16_mode", "hfref_f32_to_f16_mode"):
            getattr(L, name).restype = ctypes.c_uint16
        L.hfref_f32_to_bf16.argtypes = [ctypes.c_float]
        L.hfref_f32_to_f16.argtypes = [ctypes.c_float]
        L.hfref_f32_to_bf16_mode.argtypes = [ctypes.c_float, INT]
        L.hfref_f32_to_f16_mode.argtypes = [ctypes.c_float, INT]
        L.hfref_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.hfref_bf16_to_f32.restype = ctypes.c_float
        L.hfref_fp4_to_f32.argtypes = [ctypes.c_uint8]
        L.hfref_fp4_to_f32.restype = ctypes.c_float
        L.hfref_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.hfref_f16_to_f32.restype = ctypes.c_float
        L.hfref_f32_to_int_mode.argtypes = [ctypes.c_float, INT, INT, INT]
        L.hfref_f32_to_int_mode.restype = ctypes.c_int64
        for name in sig:
            if name.endswith("_memref") or name.startswith("hfref_memref_") or name == "hfref_sort_rows":
                getattr(L, name).restype = ctypes.c_int
        L.hfref_int_to_f32_mode.argtypes = [ctypes.c_int64, INT]
        L.hfref_int_to_f32_mode.restype = ctypes.c_float
        L.hfref_fold_round_to_odd.argtypes = [ctypes.c_double]
        L.hfref_fold_round_to_odd.restype = ctypes.c_int64
        _lib = L
    return _lib


def ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def _contig(a, dtype=None):
    """C-contiguous array of `a` (rank 0 stays rank 0, unlike
    numpy.ascontiguousarray)."""
    a = np.asarray(a, dtype=dtype)
    return a if a.flags.c_contiguous else a.copy(order="C")


# ---------------------------------------------------------------- types
FP8 = {"f8E4M3FN": 0, "f8E5M2": 1}
NP = {"f32": np.float32, "f64": np.float64, "bf16": np.uint16, "f16": np.uint16, "f8E4M3FN": np.uint8, "f8E5M2": np.uint8,
      "i1": np.bool_,
      "i8": np.int8, "ui8": np.uint8, "i16": np.int16, "i32": np.int32, "i64": np.int64, "index": np.int64}
BITS = {"i1": 1, "i8": 8, "i16": 16, "i32": 32, "i64": 64, "index": 64}
FLOATS = ("f32", "f64", "bf16", "f16", "f8E4M3FN", "f8E5M2")
ROUND = {"rint": 0, "round": 1, "floor": 2, "ceil": 3, "trunc": 4, "odd": 5, "truncwithoverflow": 6}


class T:
    """A tensor or scalar value: numpy data + element type name."""

    def __init__(self, a, elem):
        self.a = a
        self.elem = elem


def parse_type(s):
    s = s.strip()
    m = re.fullmatch(r"(?:tensor|memref)<(.*)>", s)
    if m:
        body = _split_top(m.group(1))[0]  # memref layout / address space after the first comma
        parts = body.replace(" ", "").split("x")
        # a dynamic dim `?` is -1: its size comes from the values at run time
        return tuple(-1 if p == "?" else int(p) for p in parts[:-1]), parts[-1]
    return None, s


def to_f32(v):
    a = _contig(v.a)
    if v.elem == "f32":
        return a.astype(np.float32, copy=False)
    if v.elem == "bf16":
        out = np.empty(a.shape, np.float32)
        lib().hfref_bf16_to_f32_n(ptr(a), ptr(out), a.size)
        return out
    if v.elem == "f16":
        out = np.empty(a.shape, np.float32)
        lib().hfref_f16_to_f32_n(ptr(a), ptr(out), a.size)
        return out
    if v.elem == "f64":
        return a.astype(np.float32)
    if v.elem in FP8:
        out = np.empty(a.shape, np.float32)
        lib().hfref_fp8_to_f32_n(ptr(_contig(a, np.uint8)), ptr(out), a.size, FP8[v.elem])
        return out
    raise TypeError(v.elem)


def from_f32(f, elem, mode=0, sat=False):
    f = _contig(f, dtype=np.float32)
    if elem == "f32":
        return f
    if elem in FP8:
        out = np.empty(f.shape, np.uint8)
        lib().hfref_f32_to_fp8_n(ptr(f), ptr(out), f.size, FP8[elem], mode, int(sat))
        return out
    if elem in ("bf16", "f16"):
        out = np.empty(f.shape, np.uint16)
        getattr(lib(), "hfref_f32_to_bf16_n" if elem == "bf16" else "hfref_f32_to_f16_n")(ptr(f), ptr(out), f.size, mode)
        return out
    if elem == "f64":
        return f.astype(np.float64)
    raise TypeError(elem)


def wrap_int(a64, elem):
    if elem == "i1":
        return (a64 & 1).astype(np.bool_)
    return a64.astype(NP[elem])  # numpy astype wraps two's-complement


def bitcast(v, elem):
    """arith.bitcast — the `bitcast` type_fn of named ops: the same bits read
    as a type of the same width (HFusionOps.cpp:752-756)."""
    if v.elem == elem:
        return v
    src, dst = np.dtype(NP[v.elem]), np.dtype(NP[elem])
    if v.elem == "i1" or elem == "i1" or src.itemsize != dst.itemsize:
        raise NotImplementedError(f"bitcast {v.elem} -> {elem}")
    return T(_contig(v.a).view(dst), elem)


def convert(v, elem, unsigned=False):
    """convertScalarToDtype (upstream MLIR) — the `cast` type_fn of named ops."""
    if v.elem == elem or {v.elem, elem} <= {"i64", "index"}:
        return T(v.a, elem)
    if v.elem in FLOATS and elem in FLOATS:
        if elem == "f64":
            return T(to_f32(v).astype(np.float64) if v.elem != "f64" else v.a, elem)
        return T(from_f32(to_f32(v), elem), elem)
    if v.elem not in FLOATS and elem in FLOATS:
        a = _contig(v.a)
        if unsigned or v.elem == "i1":
            bits = BITS[v.elem]
            a64 = a.astype(np.int64) & ((1 << bits) - 1) if bits < 64 else a.astype(np.int64)
        else:
            a64 = a.astype(np.int64)
        a64 = _contig(a64)
        if elem == "f64":
            return T(a64.astype(np.float64), elem)
        f = np.empty(a64.shape, np.float32)
        lib().hfref_int_to_f32_n(ptr(a64), ptr(f), a64.size, 0)
        return T(from_f32(f, elem), elem)
    if v.elem in FLOATS and elem not in FLOATS:
        f = _contig(to_f32(v))
        if elem == "i1":
            return T(f != 0, elem)
        out = np.empty(f.shape, np.int64)
        poison = ctypes.c_int(0)
        lib().hfref_fptosi_n(ptr(f), ptr(out), f.size, BITS[elem], ctypes.byref(poison))
        return T(wrap_int(out, elem), elem)
    # int -> int
    a64 = np.asarray(v.a).astype(np.int64)
    if (unsigned or v.elem == "i1") and BITS[elem] > BITS[v.elem]:
        a64 = a64 & ((1 << BITS[v.elem]) - 1)
    return T(wrap_int(a64, elem), elem)


def declared_cast(v, elem, mode, sat, unsigned=False):
    """hfusion.cast with its declared round mode and saturation."""
    if v.elem in FLOATS and elem in FLOATS:
        f = to_f32(v)
        if v.elem == elem:
            if mode == 0:
                r = np.empty_like(f)
                lib().hfref_roundeven_n(ptr(f), ptr(r), f.size)
            else:
                out = np.empty(f.shape, np.int64)
                # round to an integral value in float: via the int rounding on exact values
                r = f.copy()
                fin = np.isfinite(f) & (np.abs(f) < 2.0 ** 23)
                tmp = _contig(f[fin])
                o = np.empty(tmp.shape, np.int64)
                lib().hfref_f32_to_int_mode_n(ptr(tmp), ptr(o), tmp.size, mode, 64, 0)
                r[fin] = o.astype(np.float32)
                r[fin & (r == 0)] = np.copysign(0.0, f[fin & (r == 0)])
            return T(from_f32(r, elem), elem)
        if elem == "f32":
            return T(f, elem)
        return T(from_f32(f, elem, mode, sat), elem)
    if v.elem in FLOATS and elem not in FLOATS:
        f = _contig(to_f32(v))
        out = np.empty(f.shape, np.int64)
        lib().hfref_f32_to_int_mode_n(ptr(f), ptr(out), f.size, mode, BITS[elem], int(sat))
        return T(wrap_int(out, elem), elem)
    if v.elem not in FLOATS and elem in FLOATS:
        a64 = _contig(np.asarray(v.a).astype(np.int64))
        if unsigned or v.elem == "i1":
            a64 = a64 & ((1 << BITS[v.elem]) - 1) if BITS[v.elem] < 64 else a64
        if elem in FP8:  # one rounding, from the exact integer
            out = np.empty(a64.shape, np.uint8)
            lib().hfref_int_to_fp8_n(ptr(a64), ptr(out), a64.size, FP8[elem], mode, int(sat))
            return T(out, elem)
        f = np.empty(a64.shape, np.float32)
        lib().hfref_int_to_f32_n(ptr(a64), ptr(f), a64.size, mode)
        return T(from_f32(f, elem), elem)
    a64 = np.asarray(v.a).astype(np.int64)
    if sat and BITS[elem] < BITS[v.elem]:
        lo, hi = -(1 << (BITS[elem] - 1)), (1 << (BITS[elem] - 1)) - 1
        a64 = np.clip(a64, lo, hi)
    return convert(T(a64, "i64"), elem, unsigned)


UNARY = {"sqrt": 0, "rsqrt": 1, "exp": 2, "exp2": 3, "log": 4, "log2": 5, "log10": 6, "log1p": 7, "expm1": 8,
         "abs": 9, "absf": 9, "negf": 10, "neg": 10, "relu": 11, "rec": 12, "reciprocal": 12, "tanh": 13,
         "sin": 14, "cos": 15, "erf": 16, "nearbyint": 17, "ceil": 18, "floor": 19, "round": 20, "square": 21,
         "trunc": 22, "tan": 23, "acos": 24, "acosh": 25, "asin": 26, "asinh": 27, "atan": 28, "atanh": 29,
         "sinh": 30, "cosh": 31, "lgamma": 32, "ilogb": 33}
BINARY_F = {"add": 0, "sub": 1, "mul": 2, "div": 3, "maxf": 4, "max_signed": 4, "minf": 5, "min_signed": 5,
            "maxnumf": 6, "minnumf": 7, "powf": 8, "mod": 9, "modui": 9, "copysign": 10, "atan2": 11,
            "ldexp": 12, "divfhp": 13}
BINARY_I = {"add": 32, "sub": 33, "mul": 34, "div": 35, "max_signed": 36, "maxsi": 36, "min_signed": 37,
            "vand": 38, "vor": 39, "vxor": 40, "shli": 41, "shrsi": 42, "shrui": 43, "mod": 44,
            "floordivsi": 45, "ceildivsi": 46, "max_unsigned": 47, "min_unsigned": 48, "powi": 49,
            "ceildivui": 50, "modui": 51}
COMPARE = {"veq": 0, "vne": 1, "vlt": 2, "vle": 3, "vgt": 4, "vge": 5}
REDUCE_F = {"arith.addf": 0, "arith.mulf": 1, "arith.maximumf": 2, "arith.minimumf": 3, "arith.maxnumf": 4,
            "arith.minnumf": 5}
REDUCE_I = {"arith.addi": 0, "arith.muli": 1, "arith.maxsi": 2, "arith.minsi": 3, "arith.andi": 4,
            "arith.ori": 5, "arith.xori": 6, "arith.maxui": 7, "arith.minui": 8}


_SINGLE = ("hfusion.cumsum", "hfusion.cumprod", "hfusion.cummax", "hfusion.cummin", "hfusion.histogram",
           "hfusion.deinterleave", "hfusion.interleave", "hfusion.flip", "hfusion.mulext", "hfusion.mulextui", "hfusion.sort")

_SORT_KIND = {"f32": 0, "f16": 1, "bf16": 2, "i8": 8, "i16": 16, "i32": 32, "i64": 64}


def _single_op(op, rest, xs, rtypes):
    """HFusion ops with their own syntax: cumulative ops, histogram and
    (de)interleave (HFusionOps.td:160-420, 637-660)."""
    shape, elem = rtypes[0]
    name = op.split(".", 1)[1]
    if name.startswith("cum"):
        # CPU meaning (cumprod: ConvertHFusionToUpstream.cpp:385-450): in index
        # order along the dim (reverse: from the end), acc_0 = x_0,
        # acc_l = acc_{l-1} (op) x_l rounded to the element type at each step
        d = int(re.search(r"cum_dims\s*=\s*\[\s*(-?\d+)", rest).group(1))
        rev = re.search(r"reverse\s*=\s*true", rest) is not None
        nan = re.search(r"propagate_nan\s*=\s*false", rest) is None
        x = convert(xs[0], elem)
        a = _contig(np.moveaxis(np.asarray(x.a), d, 0))
        order = range(a.shape[0] - 1, -1, -1) if rev else range(a.shape[0])
        out = np.empty_like(a)
        if elem in FLOATS:
            fn = {"cumsum": "add", "cumprod": "mul", "cummax": "maxf" if nan else "maxnumf",
                  "cummin": "minf" if nan else "minnumf"}[name]
        else:
            fn = {"cumsum": "add", "cumprod": "mul", "cummax": "max_signed", "cummin": "min_signed"}[name]
        acc = None
        for l in order:
            xv = T(np.array(a[l]), elem)
            acc = xv if acc is None else apply_binary(fn, acc, xv, elem, a[l].shape)
            out[l] = acc.a
        return [T(_contig(np.moveaxis(out, 0, d)), elem)]
    if name == "sort":
        # value sort along the last axis (HFusionOps.cpp:3341-3348 accepts only
        # the tail axis), as the bubble sort of hfref_sort_rows
        ax = int(re.search(r"sort_axis\s*=\s*(-?\d+)", rest).group(1))
        desc = re.search(r"descending\s*=\s*true", rest) is not None
        a = np.asarray(xs[0].a)
        if ax not in (-1, a.ndim - 1):
            raise ValueError("hfusion.sort: only the last axis can be sorted")
        if len(rtypes) != 1:
            raise ValueError("hfusion.sort: only the value result is restated (no index result)")
        out = _contig(a).copy()
        L = a.shape[-1] if a.ndim else 1
        if L > 1 and out.size:
            if lib().hfref_sort_rows(out.ctypes.data, out.size // L, L, _SORT_KIND[xs[0].elem], int(desc)) != 0:
                raise ValueError(f"hfusion.sort of {xs[0].elem}")
        return [T(out, xs[0].elem)]
    if name == "flip":
        # reverse along flip_axis (HFusionOps.td:226-245)
        m = re.search(r"flip_axis\s*=\s*(-?\d+)", rest)
        ax = int(m.group(1)) if m else -1
        return [T(_contig(np.flip(np.asarray(xs[0].a), ax)), elem)]
    if name in ("mulext", "mulextui"):
        # (2N)-bit product of sign- or zero-extended operands: low and high halves
        bits = BITS[elem]
        a, b = (np.asarray(v.a).astype(object).ravel() for v in xs)
        m = 1 << bits
        if name == "mulextui":
            a, b = [x % m for x in a], [x % m for x in b]
        prod = [int(x) * int(y) for x, y in zip(a, b)]
        wrap = lambda v: (v % m) - m if (v % m) >= m // 2 else v % m  # noqa: E731
        lo = np.array([wrap(p) for p in prod], np.int64)
        hi = np.array([wrap(p >> bits) for p in prod], np.int64)
        sh = np.shape(xs[0].a)
        return [T(wrap_int(lo.reshape(sh), elem), elem), T(wrap_int(hi.reshape(sh), elem), elem)]
    if name == "histogram":
        bins = int(re.search(r"^\s*%[\w.$-]+\s*,\s*(\d+)", rest).group(1))
        v = np.asarray(xs[0].a).astype(np.int64).ravel()
        ok = (v >= 0) & (v < bins)
        if len(xs) > 1:
            ok &= np.asarray(xs[1].a).ravel().astype(np.int64) != 0
        counts = np.bincount(v[ok], minlength=bins).astype(np.int64)
        return [T(wrap_int(counts, elem), elem)]
    if name == "deinterleave":
        m = re.search(r"channel\s*<\s*(all|-?\d+)\s*>", rest)
        ch = -1 if m.group(1) == "all" else int(m.group(1))
        a = np.asarray(xs[0].a)
        if ch == -1:
            return [T(_contig(a[..., 0::2]), elem), T(_contig(a[..., 1::2]), elem)]
        return [T(_contig(a[..., ch::2]), elem)]
    a, b = np.asarray(xs[0].a), np.asarray(xs[1].a)
    out = np.empty(a.shape[:-1] + (2 * a.shape[-1],), a.dtype)
    out[..., 0::2], out[..., 1::2] = a, b
    return [T(out, elem)]


_NON_DPS = ("hfusion.isinf", "hfusion.isnan", "hfusion.isfinite", "hfusion.nextafter", "hfusion.hypot",
            "hfusion.erfinv", "hfusion.signbit", "hfusion.cyl_bessel_i0")


def _non_dps(op, xs, shape, elem):
    """HFusion float ops without outs (HFusionOps.td:251-305, 1309-1400)."""
    f32 = np.float32
    if op in ("hfusion.isinf", "hfusion.isnan", "hfusion.isfinite"):
        f = to_f32(xs[0])
        return {"hfusion.isinf": np.isinf, "hfusion.isnan": np.isnan, "hfusion.isfinite": np.isfinite}[op](f)
    if op == "hfusion.signbit":
        # HFusionOps.td:1295, expanded in hfusion-normalize-ops.mlir:3055-3080 as
        # (bits & sign_mask) != 0 on the operand's own width
        a = _contig(xs[0].a)
        bits = a.view(np.uint32) >> 31 if xs[0].elem == "f32" else a.view(np.uint16) >> 15
        return bits.astype(np.int8 if elem == "i8" else np.bool_)
    if op == "hfusion.nextafter":
        # IEEE nextafter (Normalize.cpp:8640-8660): one ulp from x toward y
        if elem == "f32":
            return np.nextafter(xs[0].a.astype(f32), xs[1].a.astype(f32))
        h = [_contig(x.a, np.uint16).view(np.float16) for x in xs]
        return np.nextafter(h[0], h[1]).view(np.uint16)
    if op == "hfusion.hypot":
        # Normalize.cpp:8969-9330: f32 takes the scaled path, f16 the direct one
        fs = [to_f32(x) for x in xs]
        a = [np.abs(f) for f in fs]
        nan = np.zeros(shape, bool)
        inf = np.zeros(shape, bool)
        for f, ai in zip(fs, a):
            nan |= np.isnan(f)
            inf |= ai == np.inf
        with np.errstate(all="ignore"):
            if elem == "f32":
                sc = np.where(a[0] > a[1], a[0], a[1])
                for ai in a[2:]:
                    sc = np.where(sc > ai, sc, ai)
                safe = np.where(sc == 0, f32(1), sc).astype(f32)

                def term(ai):
                    q = (ai / safe).astype(f32)
                    return np.where(sc == 0, f32(0), np.where(ai == sc, f32(1), (q * q).astype(f32))).astype(f32)
                sm = (term(a[0]) + term(a[1])).astype(f32)
                for ai in a[2:]:
                    sm = (sm + term(ai)).astype(f32)
                r = (sc * np.sqrt(sm)).astype(f32)
            elif elem == "f16":
                sm = (a[0] * a[0] + a[1] * a[1]).astype(f32)
                for ai in a[2:]:
                    sm = (sm + ai * ai).astype(f32)
                r = np.sqrt(sm).astype(f32)
            else:
                raise NotImplementedError(f"hypot on {elem}")
        r[nan] = np.nan
        r[inf] = np.inf
        return from_f32(r, elem)
    if op == "hfusion.cyl_bessel_i0":
        # hfusion-normalize-ops.mlir:3586-3830 expands it as the Cephes
        # Chebyshev series of i0 (Clenshaw, Cephes `i0`); scipy.special.i0 is
        # the same published algorithm, evaluated here in float64
        # the lowering multiplies exp(|x|) * i0e(|x|) in f32
        # (Normalize.cpp:8549-8573): exp overflows from |x| = 88.72283935546875
        # (the f32 just above ln(FLT_MAX)), so the result is +inf there
        import scipy.special
        x64 = to_f32(xs[0]).astype(np.float64)
        with np.errstate(all="ignore"):
            r = scipy.special.i0(x64).astype(f32)
        r[np.isfinite(x64) & (np.abs(x64) >= 88.72283935546875)] = np.inf
        return from_f32(r, elem)
    if op == "hfusion.erfinv":
        import scipy.special
        with np.errstate(all="ignore"):
            r = scipy.special.erfinv(to_f32(xs[0]).astype(np.float64)).astype(f32)
        return from_f32(r, elem)
    raise NotImplementedError(op)


def _full(v, shape):
    return _contig(np.broadcast_to(v.a, shape))


def apply_unary(fn, x, U):
    if U in FLOATS:
        f = _contig(np.broadcast_to(to_f32(x), np.shape(x.a)))
        out = np.empty(f.shape, np.float32)
        lib().hfref_unary_f32(UNARY[fn], ptr(f), ptr(out), f.size)
        return T(from_f32(out, U), U)
    a = np.asarray(x.a).astype(np.int64)
    if fn == "relu":
        r = np.maximum(a, 0)
    elif fn == "vnot":
        r = ~a
    elif fn in ("absi", "abs"):
        r = np.abs(a)
    else:
        raise NotImplementedError(f"integer unary {fn}")
    return T(wrap_int(r, U), U)


def apply_binary(fn, x, y, U, shape):
    if U in FLOATS:
        a = _contig(np.broadcast_to(to_f32(x), shape))
        b = _contig(np.broadcast_to(to_f32(y), shape))
        out = np.empty(shape, np.float32)
        lib().hfref_binary_f32(BINARY_F[fn], ptr(a), ptr(b), ptr(out), out.size)
        return T(from_f32(out, U), U)
    a = _contig(np.broadcast_to(np.asarray(x.a).astype(np.int64), shape))
    b = _contig(np.broadcast_to(np.asarray(y.a).astype(np.int64), shape))
    out = np.empty(shape, np.int64)
    lib().hfref_binary_i64(BINARY_I[fn], ptr(a), ptr(b), ptr(out), out.size, BITS[U])
    return T(wrap_int(out, U), U)


# ---------------------------------------------------------------- parsing
_RES = re.compile(r"^\s*(%[\w.$-]+)(?::(\d+))?(?:\s*,\s*(%[\w.$-]+))*\s*=\s*([\w.]+)(.*)$")


def _statements(body):
    """Splits a function body into statements, joining multi-line regions."""
    out, cur, depth = [], "", 0
    for line in body.split("\n"):
        line = line.split("//")[0].rstrip()
        if not line.strip():
            continue
        cur = (cur + " " + line) if cur else line
        depth += line.count("{") - line.count("}") + line.count("(") - line.count(")")
        if depth <= 0:
            # a region opener on the following line belongs to this statement
            out.append(cur)
            cur, depth = "", 0
    merged = []
    for s in out:
        # generic op form `%r = "dialect.op"(%a) : (T) -> R` reads as `%r = dialect.op (%a) : ...`
        s = re.sub(r'=\s*"([\w.]+)"\s*\(', r'= \1 (', s, count=1)
        st = s.strip()
        if merged and (st.startswith("(") or st.startswith(_HIVM_CONT)):
            merged[-1] += " " + s
        else:
            merged.append(s)
    return merged


# clause keywords that continue a multi-line hivm op (HIVMMacroOps.td:432-446)
_HIVM_CONT = ("ins(", "outs(", "bias", "descale", "a_transpose", "b_transpose", "tiling_params", "block_sizes",
              "process_sizes", "swizzle_", "epilogue_p_tiles")


def _split_top(s, sep=","):
    parts, depth, cur = [], 0, ""
    for ch in s:
        if ch in "<([{":
            depth += 1
        elif ch in ">)]}":
            depth -= 1
        if ch == sep and depth == 0:
            parts.append(cur)
            cur = ""
        else:
            cur += ch
    if cur.strip():
        parts.append(cur)
    return [p.strip() for p in parts]


def _group(s, key):
    """Contents of `key(...)` with balanced parentheses."""
    i = s.find(key + "(")
    if i < 0:
        return None
    i += len(key) + 1
    depth, j = 1, i
    while depth:
        if s[j] == "(":
            depth += 1
        elif s[j] == ")":
            depth -= 1
        j += 1
    return s[i:j - 1]


def _operands(group):
    if group is None:
        return [], []
    if ":" in group:
        names, types = group.split(":", 1)
        return [n.strip() for n in names.split(",") if n.strip()], [parse_type(t) for t in _split_top(types)]
    return [n.strip() for n in group.split(",") if n.strip()], []


def _attr(s, key):
    m = re.search(key + r"\s*=\s*#[\w.]+<(\w+)>", s)
    if m:
        return m.group(1)
    m = re.search(key + r"\s*=\s*(\w+)", s)
    return m.group(1) if m else None


def parse_funcs(text):
    funcs = {}
    for m in re.finditer(r"func\.func\s+(?:private\s+)?@(\w+)\s*\(", text):
        name = m.group(1)
        i = m.end()
        depth, j = 1, i
        while depth:
            depth += {"(": 1, ")": -1}.get(text[j], 0)
            j += 1
        parts = _split_top(text[i:j - 1])
        if parts and ":" not in parts[0]:
            continue  # an external declaration `func.func private @f(f32) -> f32`
        args = []
        for a in parts:
            nm, ty = a.split(":", 1)
            args.append((nm.strip(), parse_type(ty.split("{")[0])))
        # body: first '{' after `attributes {...}` (or after the signature)
        k = j
        sig_end = text.index("{", k)
        rest = text[k:sig_end]
        if "attributes" in rest:
            d, q = 1, sig_end + 1
            while d:
                d += {"{": 1, "}": -1}.get(text[q], 0)
                q += 1
            sig_end = text.index("{", q)
        d, q = 1, sig_end + 1
        while d:
            d += {"{": 1, "}": -1}.get(text[q], 0)
            q += 1
        funcs[name] = (args, text[sig_end + 1:q - 1])
    return funcs


class Interp:
    def __init__(self, text, cast_semantics="declared"):
        self.funcs = parse_funcs(text)
        self.cast_semantics = cast_semantics
        # module-level attribute aliases (`#map = affine_map<...>`)
        self.aliases = dict(re.findall(r"^\s*(#[\w.$-]+)\s*=\s*(affine_map<.*>)\s*$", text, re.M))

    def run(self, func=None, *inputs):
        """Runs group `func` with numpy inputs (one per argument; bf16/f16
        given as uint16 bit patterns).  Returns the list of results."""
        if func is None:
            if len(self.funcs) != 1:
                raise ValueError("several functions; name one")
            func = next(iter(self.funcs))
        args, body = self.funcs[func]
        if len(inputs) != len(args):
            raise ValueError(f"@{func} takes {len(args)} arguments")
        env = {}
        self.empties = set()
        for (nm, (shape, elem)), x in zip(args, inputs):
            if shape is None:
                env[nm] = T(np.asarray(x, dtype=NP[elem]), elem)
            else:
                a = np.array(x, dtype=NP[elem], order="C")  # keeps rank 0
                if len(a.shape) != len(shape) or any(d >= 0 and d != g for d, g in zip(shape, a.shape)):
                    raise ValueError(f"{nm}: expected shape {shape}, got {a.shape}")
                env[nm] = T(a.copy(), elem)
        self.written = []
        # annotation.mark {overflow_mode = "saturate"} makes the marked value's
        # cast saturate (Normalize.cpp:4285-4301)
        self.sat_marks = set()
        for st in _statements(body):
            m = re.match(r"\s*annotation\.mark\s+(%[\w.$-]+).*overflow_mode\s*=\s*\"(\w*)\"", st)
            if m and "saturate" in m.group(2):
                self.sat_marks.add(m.group(1))
        for st in _statements(body):
            s = st.strip()
            if s.startswith("return") or s.startswith("func.return"):
                names = re.findall(r"%[\w.$#-]+", s.split(":")[0])
                # destination-style (memref) groups return what their ops wrote
                return [env[n].a for n in names] if names else [env[n].a for n in self.written]
            if s.startswith("hivm.hir.matmul"):
                self._hivm_matmul(s, env)
                continue
            if s.startswith("annotation.mark"):
                continue
            if not s.startswith("%") and "outs(" in s:
                # a destination-style op on a memref: it writes its outs
                # buffer, which later statements read under the same name
                buf = _operands(_group(s.split(None, 1)[1], "outs"))[0][0]
                self._exec(f"{buf} = {s}", env)
                if buf not in self.written:
                    self.written.append(buf)
                continue
            self._exec(s, env)
        raise ValueError("function without return")

    def _hivm_matmul(self, s, env):
        """hivm.hir.matmul (HIVMMacroOps.td:373-398): C = descale * (A*B + bias),
        written into the `outs` memref.  The reference has no CPU lowering for
        it; this is the documented formula with the accumulator of the input
        type (exact int32 for i8, serial fp32 over k for bf16/f16); an integer
        bias joins the int32 accumulator, then fp32 (RNE); a float bias is
        added in fp32; the descale (per channel [N] or per tensor [1])
        multiplies in fp32; the result rounds to C's type (RNE, saturating for
        integer C)."""
        ins, _ = _operands(_group(s, "ins"))
        outs, _ = _operands(_group(s, "outs"))
        A, B, C = env[ins[0]], env[ins[1]], env[outs[0]]
        at, bt = "a_transpose" in s, "b_transpose" in s
        a = _contig(A.a.T if at else A.a)
        M, K = a.shape
        N = C.a.shape[1]
        # the serial matmul takes B as [K, N] (bt=0) or [N, K] (bt=1)
        b = _contig(B.a)
        if A.elem == "i8":
            acc = np.zeros((M, N), np.int32)
            lib().hfref_matmul_i8_i32(ptr(a), ptr(b), ptr(acc), M, N, K, int(bt))
        else:
            acc = np.zeros((M, N), np.float32)
            lib().hfref_matmul_f32(ptr(_contig(to_f32(T(a, A.elem)))), ptr(_contig(to_f32(T(b, B.elem)))),
                                   ptr(acc), M, N, K, int(bt))
        bm = re.search(r"\bbias\s*=\s*(%[\w.$-]+)", s)
        dm = re.search(r"\bdescale\s*=\s*(%[\w.$-]+)", s)
        mode = _attr(s, "descale_mode") or ("DescalePerChannel" if dm else "DescaleNull")
        bias = env[bm.group(1)] if bm else None
        if A.elem == "i8" and bias is not None and bias.elem in BITS:
            acc = (acc.astype(np.int64) + bias.a.astype(np.int64)[None, :]).astype(np.int32)
            bias = None
        t = convert(T(acc, "i32" if A.elem == "i8" else "f32"), "f32").a
        if bias is not None:
            t = (t + to_f32(bias)[None, :]).astype(np.float32)
        if dm:
            d = to_f32(env[dm.group(1)])
            t = (t * (d[None, :] if mode == "DescalePerChannel" else d[0])).astype(np.float32)
        tf = T(_contig(t, np.float32), "f32")
        env[outs[0]] = declared_cast(tf, C.elem, 0, True) if C.elem in BITS else convert(tf, C.elem)
        self.written.append(outs[0])

    def _exec(self, s, env):
        m = re.match(r"^\s*(%[\w.$-]+)(?::(\d+))?((?:\s*,\s*%[\w.$-]+)*)\s*=\s*([\w.]+)(.*)$", s)
        if not m:
            raise ValueError(f"cannot parse statement: {s}")
        res, nres, op, rest = m.group(1), m.group(2), m.group(4), m.group(5)
        more = re.findall(r"%[\w.$-]+", m.group(3) or "")

        def get(n):
            return env[n]

        if op == "arith.constant":
            lit, ty = rest.rsplit(":", 1)
            shape, elem = parse_type(ty)
            lit = lit.strip()
            dm = re.match(r"dense<(.*)>", lit)
            if dm:
                lit = dm.group(1)
            if lit in ("true", "false"):
                val = lit == "true"
            elif lit.lower().startswith("0x") and elem in ("bf16", "f16"):
                # hex literal of a 16-bit float: its bit pattern
                arr = np.array(int(lit, 16), np.uint16)
                env[res] = T(arr if shape is None else np.broadcast_to(arr, shape).copy(), elem)
                return
            elif lit.lower().startswith("0x") and elem in FLOATS:
                bits = int(lit, 16)
                val = {"f32": lambda b: np.array([b], np.uint32).view(np.float32)[0],
                       "f64": lambda b: np.array([b], np.uint64).view(np.float64)[0]}[elem](bits)
            elif elem in FLOATS:
                val = float(lit)
            else:
                val = int(lit, 0)
            if elem in ("bf16", "f16"):
                arr = from_f32(np.array(val, np.float32), elem)
            else:
                arr = np.array(val, dtype=NP[elem])
            env[res] = T(arr if shape is None else np.broadcast_to(arr, shape).copy(), elem)
            return
        if op == "tensor.empty":
            shape, elem = parse_type(rest.split(":", 1)[1])
            if -1 in shape:
                # tensor.empty(%d0, ...): the dynamic dims in order
                dyn = iter(int(env[n].a) for n in re.findall(r"%[\w.$-]+", rest.split(":", 1)[0]))
                shape = tuple(next(dyn) if d < 0 else d for d in shape)
            env[res] = T(np.zeros(shape, NP[elem]), elem)
            self.empties.add(res)
            return
        if op == "tensor.dim":
            names = re.findall(r"%[\w.$-]+", rest)
            env[res] = T(np.int64(env[names[0]].a.shape[int(env[names[1]].a)]), "index")
            return
        if op in ("tensor.expand_shape", "tensor.collapse_shape"):
            # a row-major view with the result type after `into`
            src = re.findall(r"%[\w.$#-]+", rest)[0]
            shape, elem = parse_type(rest.rsplit("into", 1)[1])
            env[res] = T(_contig(env[src].a).reshape(shape), elem)
            return
        if op.startswith("arith.") and "ins(" not in rest:
            self._scalar_arith(res, op, rest, env)
            return
        if op in _SINGLE:
            names = re.findall(r"%[\w.$-]+", rest.split(":", 1)[0])
            rtypes = [parse_type(t) for t in _split_top(rest.rsplit("->", 1)[1] if "->" in rest else rest.rsplit(":", 1)[1])]
            outs = _single_op(op, rest, [env[n] for n in names], rtypes)
            if more:
                for nm, o in zip([res] + more, outs):
                    env[nm] = o
            elif len(outs) == 1:
                env[res] = outs[0]
            else:
                for i, o in enumerate(outs):
                    env[f"{res}#{i}"] = o
                env[res] = outs[0]
            return
        if op in _NON_DPS:
            names = re.findall(r"%[\w.$-]+", rest.split(":", 1)[0])
            shape, elem = parse_type(rest.rsplit("->", 1)[1])
            if -1 in shape:
                shape = env[names[0]].a.shape
            xs = [T(np.broadcast_to(env[n].a, shape), env[n].elem) for n in names]
            env[res] = T(_contig(_non_dps(op, xs, shape, elem)), elem)
            return
        ins, ins_t = _operands(_group(rest, "ins"))
        outs, outs_t = _operands(_group(rest, "outs"))
        if op == "linalg.generic":
            env[res] = self._generic(rest, ins, outs, env)
            return
        if op == "hfusion.gather":
            # out[p] = src[p with axis coordinate index[p]] when the index is in
            # range, else init[p] (HFusionStructuredOps.td:222-238)
            src, ix = get(ins[0]), get(ins[1])
            o = get(outs[0])
            ax = int(re.search(r"axis\s*=\s*(-?\d+)", rest).group(1))
            k = np.asarray(ix.a).astype(np.int64)
            ok = (k >= 0) & (k < np.asarray(src.a).shape[ax])
            g = np.take_along_axis(np.asarray(src.a), np.where(ok, k, 0), axis=ax)
            env[res] = T(np.where(ok, g, np.asarray(o.a)).astype(NP[o.elem]), o.elem)
            return
        if op == "hfusion.arange":
            # value at (i0, i1, ...) = offset + sum_d stride_d * i_d
            # (HFusionStructuredOps.td:163-175), converted to the element type
            o = get(outs[0])
            head = rest.split("outs(", 1)[0]
            vals = [int(np.asarray(env[n].a)) for n in re.findall(r"%[\w.$-]+", head)]
            off = vals.pop(0) if "offset[" in head else 0
            grids = np.indices(o.a.shape, dtype=np.int64)
            v = np.full(o.a.shape, off, np.int64)
            for st, g in zip(vals, grids):
                v = v + st * g
            env[res] = convert(T(v, "i64"), o.elem)
            return
        if op == "linalg.fill":
            o = get(outs[0])
            v = convert(get(ins[0]), o.elem)
            env[res] = T(np.broadcast_to(v.a, o.a.shape).copy(), o.elem)
            return
        if op == "linalg.transpose":
            # out[i_0..i_n] = in[j] with j[perm[k]] = i_k (out dim k is in dim perm[k])
            perm = [int(d) for d in re.search(r"permutation\s*=\s*\[([^\]]*)\]", rest).group(1).split(",") if d.strip()]
            x, o = get(ins[0]), get(outs[0])
            env[res] = T(_contig(np.transpose(x.a, perm)), o.elem)
            return
        if op == "linalg.broadcast":
            dims = [int(d) for d in re.search(r"dimensions\s*=\s*\[([^\]]*)\]", rest).group(1).split(",") if d.strip()]
            x, o = get(ins[0]), get(outs[0])
            a = x.a
            for d in sorted(dims):
                a = np.expand_dims(a, d)
            env[res] = T(np.broadcast_to(a, o.a.shape).copy(), o.elem)
            return
        if op == "linalg.reduce":
            self._reduce(res, rest, ins, outs, env)
            return
        if op == "hfusion.reduce_with_index":
            self._reduce_with_index(res, rest, ins, outs, env)
            return
        if op == "hfusion.matmul_mx":
            # fp8 A [M, K], B [K, N]; lhsFormat / rhsFormat (1 e5m2, 2 e4m3,
            # 3 fp4 e2m1, HFusionAttrs.td:131-137) decide over the element
            # type when present (HFusionToHIVM keeps the format when the type
            # does not match it, Matmul.cpp:62-70); fp4 packs two values per
            # byte along K (A [M, K/2], B [K/2, N] bytes); e8m0 scales
            # [M|N, K/32]
            A, B, SA, SB, Cinit = get(ins[0]), get(ins[1]), get(ins[2]), get(ins[3]), get(outs[0])

            def fmt(v, attr):
                code = re.search(attr + r"\s*=\s*(\d+)", rest)
                if code:
                    if code.group(1) not in ("1", "2", "3"):
                        raise NotImplementedError("matmul_mx operand format")
                    return {"1": 1, "2": 0, "3": 4}[code.group(1)]
                if v.elem in FP8:
                    return FP8[v.elem]
                raise NotImplementedError("matmul_mx operand format")
            fa_, fb_ = fmt(A, "lhsFormat"), fmt(B, "rhsFormat")
            M, K = A.a.shape
            N = B.a.shape[1]
            if fa_ == 4:
                K *= 2
            C = _contig(np.array(Cinit.a, np.float32, copy=True))
            byts = [_contig(v.a).view(np.uint8) for v in (A, B, SA, SB)]  # raw bytes, sign-free
            lib().hfref_matmul_mx(*(ptr(x) for x in byts), ptr(C), M, N, K, fa_, fb_)
            env[res] = T(C, "f32")
            return
        if op in ("linalg.matmul", "linalg.matmul_transpose_b"):
            A, B, Cinit = get(ins[0]), get(ins[1]), get(outs[0])
            bt = int(op.endswith("transpose_b"))
            M, K = A.a.shape
            N = Cinit.a.shape[1]
            if A.elem == "i8" and Cinit.elem == "i32":
                C = _contig(Cinit.a.copy())
                lib().hfref_matmul_i8_i32(ptr(_contig(A.a)), ptr(_contig(B.a)), ptr(C), M, N, K, bt)
            elif Cinit.elem == "f32":
                C = _contig(Cinit.a.copy())
                lib().hfref_matmul_f32(ptr(_contig(to_f32(A))), ptr(_contig(to_f32(B))), ptr(C),
                                       M, N, K, bt)
            else:
                raise NotImplementedError("matmul types")
            env[res] = T(C, Cinit.elem)
            return
        # elementwise ops
        o = get(outs[0])
        U, shape = o.elem, o.a.shape
        xs = [get(n) for n in ins]
        uns = _attr(rest, "cast") == "cast_unsigned"
        if _attr(rest, "cast") == "bitcast":
            cv = lambda v: bitcast(v, U)  # noqa: E731
        else:
            cv = lambda v: convert(v, U, uns)  # noqa: E731
        if op in ("hfusion.elemwise_unary", "linalg.elemwise_unary"):
            fn = _attr(rest, "fun") or ("sqrt" if op.startswith("hfusion") else "exp")
            r = apply_unary(fn, cv(T(np.broadcast_to(xs[0].a, shape), xs[0].elem)), U)
        elif op in ("hfusion.elemwise_binary", "linalg.elemwise_binary"):
            fn = _attr(rest, "fun") or ("vand" if op.startswith("hfusion") else "add")
            r = apply_binary(fn, cv(xs[0]), cv(xs[1]), U, shape)
        elif op == "hfusion.compare":
            fn = _attr(rest, "compare_fn") or "veq"
            a, b = xs
            if a.elem in FLOATS:
                fa = _contig(np.broadcast_to(to_f32(a), shape))
                fb = _contig(np.broadcast_to(to_f32(b), shape))
                out = np.empty(shape, np.uint8)
                lib().hfref_compare_f32(COMPARE[fn], ptr(fa), ptr(fb), ptr(out), out.size)
            else:
                ia = _contig(np.broadcast_to(a.a.astype(np.int64), shape))
                ib = _contig(np.broadcast_to(b.a.astype(np.int64), shape))
                out = np.empty(shape, np.uint8)
                lib().hfref_compare_i64(COMPARE[fn], ptr(ia), ptr(ib), ptr(out), out.size)
            r = T(out.astype(np.bool_), "i1")
        elif op == "hfusion.bitcast":
            r = bitcast(T(_contig(np.broadcast_to(xs[0].a, shape)), xs[0].elem), U)
        elif op == "hfusion.select":
            c, a, b = xs
            r = T(np.where(np.broadcast_to(c.a, shape), np.broadcast_to(a.a, shape), np.broadcast_to(b.a, shape)).astype(NP[U]), U)
        elif op == "hfusion.cast":
            mode = ROUND[_attr(rest, "round_mode") or "rint"]
            sat = (_attr(rest, "enable_saturate") == "true") or res in self.sat_marks
            x = T(np.broadcast_to(xs[0].a, shape), xs[0].elem)
            if self.cast_semantics == "cpu":
                if x.elem == U and U in FLOATS:
                    f = _contig(to_f32(x))
                    rr = np.empty_like(f)
                    lib().hfref_round_n(ptr(f), ptr(rr), f.size)
                    r = T(from_f32(rr, U), U)
                else:
                    r = convert(x, U, uns)
            else:
                r = declared_cast(x, U, mode, sat, uns or "ui2" in (_attr(rest, "unsigned_mode") or ""))
        else:
            raise NotImplementedError(f"op {op}")
        env[res] = T(_contig(np.broadcast_to(r.a, shape)).astype(NP[U], copy=False), U)

    def _generic(self, rest, ins, outs, env):
        """linalg.generic with parallel loops, identity output map and
        plain-dim input maps: the region's scalar ops evaluated over the loop
        domain, each rounded to its type (the CPU loop body of
        convert-linalg-to-loops)."""
        head, region = rest.split("{", 1)[0], rest
        attrs = rest[rest.index("{"):]
        maps_txt = re.search(r"indexing_maps\s*=\s*\[(.*?)\]\s*,\s*iterator_types", attrs, re.S)
        maps_src = maps_txt.group(1) if maps_txt else ""
        for k in sorted(self.aliases, key=len, reverse=True):
            maps_src = re.sub(re.escape(k) + r"(?![\w])", self.aliases[k], maps_src)
        maps = []
        for m in re.finditer(r"affine_map<\(([^)]*)\)\s*->\s*\(([^)]*)\)>", maps_src):
            maps.append([int(d.strip()[1:]) for d in m.group(2).split(",") if d.strip()])
        its = [t.strip().strip('"') for t in re.search(r"iterator_types\s*=\s*\[([^\]]*)\]", attrs).group(1).split(",")]
        o = env[outs[0]]
        if "reduction" in its:
            return self._generic_reduce(region, ins, outs, env, maps, its)
        dom = np.asarray(o.a).shape
        nd = len(dom)

        def place(v, mp):
            a = np.asarray(v.a)
            if a.ndim == 0:
                return T(np.broadcast_to(a, dom), v.elem)
            order = np.argsort(mp)
            a = a.transpose(order)
            sm = sorted(mp)
            full = [dom[d] if d in sm else 1 for d in range(nd)]
            return T(np.broadcast_to(a.reshape(full), dom), v.elem)
        body = region[region.index("^"):]
        hdr = re.match(r"\^\w+\(([^)]*)\)\s*:", body)
        bargs = [x.split(":")[0].strip() for x in hdr.group(1).split(",") if ":" in x]
        local = {}
        for i, nm in enumerate(bargs[:len(ins)]):
            local[nm] = place(env[ins[i]], maps[i]) if np.ndim(env[ins[i]].a) else T(np.broadcast_to(env[ins[i]].a, dom), env[ins[i]].elem)
        return self._run_region_body(body[hdr.end():], local, dom, env, o.elem)

    def _run_region_body(self, text, local, dom, env, out_elem):
        """Evaluates the statements of a linalg.generic region (after its block
        header) with the block arguments in `local`; returns the yielded
        value converted to `out_elem`."""

        def get(nm):
            if nm in local:
                return local[nm]
            v = env[nm]
            return T(np.broadcast_to(v.a, dom), v.elem)
        fb = {"arith.addf": "add", "arith.subf": "sub", "arith.mulf": "mul", "arith.divf": "div",
              "arith.maximumf": "maxf", "arith.minimumf": "minf", "arith.maxnumf": "maxnumf",
              "arith.minnumf": "minnumf", "arith.remf": "mod", "math.powf": "powf", "math.atan2": "atan2",
              "math.copysign": "copysign"}
        fu = {"arith.negf": "negf", "math.exp": "exp", "math.exp2": "exp2", "math.log": "log", "math.log2": "log2",
              "math.log10": "log10", "math.log1p": "log1p", "math.expm1": "expm1", "math.sqrt": "sqrt",
              "math.rsqrt": "rsqrt", "math.tanh": "tanh", "math.sin": "sin", "math.cos": "cos", "math.tan": "tan",
              "math.erf": "erf", "math.absf": "abs", "math.floor": "floor", "math.ceil": "ceil", "math.round": "round",
              "math.roundeven": "nearbyint", "math.trunc": "trunc", "math.atan": "atan", "math.asin": "asin",
              "math.acos": "acos", "math.sinh": "sinh", "math.cosh": "cosh", "math.asinh": "asinh",
              "math.acosh": "acosh", "math.atanh": "atanh"}
        ib = {"arith.addi": "add", "arith.subi": "sub", "arith.muli": "mul", "arith.divsi": "div", "arith.remsi": "mod",
              "arith.remui": "modui", "arith.andi": "vand", "arith.ori": "vor", "arith.xori": "vxor",
              "arith.shli": "shli", "arith.shrsi": "shrsi", "arith.shrui": "shrui", "arith.maxsi": "max_signed",
              "arith.minsi": "min_signed", "arith.maxui": "max_unsigned", "arith.minui": "min_unsigned",
              "arith.ceildivsi": "ceildivsi", "arith.floordivsi": "floordivsi", "arith.ceildivui": "ceildivui",
              "math.ipowi": "powi"}
        stmts = re.split(r"\n|(?<=[\w>)\]])\s+(?=%[\w.$-]+\s*=|linalg\.yield)", text)
        for st in stmts:
            st = re.sub(r"fastmath<[^>]*>", "", st).strip().rstrip("}").strip()
            if not st:
                continue
            if st.startswith("linalg.yield"):
                v = get(re.findall(r"%[\w.$-]+", st)[0])
                return convert(v, out_elem) if v.elem != out_elem else T(_contig(v.a), v.elem)
            m = re.match(r"(%[\w.$-]+)\s*=\s*([\w.]+)\s*(.*)$", st)
            r_, opn, tail = m.group(1), m.group(2), m.group(3)
            lhs, _, ty = tail.rpartition(":")
            to = None
            if " to " in ty:
                ty, to = ty.split(" to ")
                to = to.strip()
            ty = ty.strip()
            names = re.findall(r"%[\w.$-]+", lhs)
            xs = [get(n) for n in names]
            if opn == "arith.constant":
                lit = lhs.strip()
                if lit in ("true", "false"):
                    val = lit == "true"
                elif lit.lower().startswith("0x") and ty in FLOATS:
                    val = np.array([int(lit, 16)], np.uint32).view(np.float32)[0]
                elif ty in FLOATS:
                    val = float(lit)
                else:
                    val = int(lit, 0)
                arr = from_f32(np.array(val, np.float32), ty) if ty in ("bf16", "f16") else np.array(val, NP[ty])
                local[r_] = T(np.broadcast_to(arr, dom), ty)
            elif opn in fb:
                local[r_] = apply_binary(fb[opn], xs[0], xs[1], ty, dom)
            elif opn in fu:
                local[r_] = apply_unary(fu[opn], xs[0], ty)
            elif opn in ib:
                local[r_] = apply_binary(ib[opn], xs[0], xs[1], ty, dom)
            elif opn == "arith.select":
                local[r_] = T(np.where(np.asarray(xs[0].a), np.asarray(xs[1].a), np.asarray(xs[2].a)), xs[1].elem)
            elif opn in ("arith.cmpf", "arith.cmpi"):
                pred = lhs.strip().split(",")[0].strip()
                if opn == "arith.cmpf":
                    x, y = to_f32(xs[0]), to_f32(xs[1])
                    with np.errstate(invalid="ignore"):
                        res_ = {"oeq": x == y, "one": (x < y) | (x > y), "olt": x < y, "ole": x <= y, "ogt": x > y,
                                "oge": x >= y, "ord": (x == x) & (y == y), "ueq": ~((x < y) | (x > y)), "une": ~(x == y),
                                "ult": ~(x >= y), "ule": ~(x > y), "ugt": ~(x <= y), "uge": ~(x < y),
                                "uno": (x != x) | (y != y)}[pred]
                else:
                    x, y = np.asarray(xs[0].a).astype(np.int64), np.asarray(xs[1].a).astype(np.int64)
                    if pred[0] == "u":
                        b = BITS.get(xs[0].elem, 64)
                        msk = (1 << b) - 1 if b < 64 else -1
                        x, y = (x & msk).astype(np.uint64), (y & msk).astype(np.uint64)
                    res_ = {"eq": x == y, "ne": x != y, "slt": x < y, "sle": x <= y, "sgt": x > y, "sge": x >= y,
                            "ult": x < y, "ule": x <= y, "ugt": x > y, "uge": x >= y}[pred]
                local[r_] = T(np.asarray(res_, np.bool_), "i1")
            elif opn == "arith.bitcast":
                local[r_] = bitcast(T(_contig(xs[0].a), xs[0].elem), to)
            elif opn in ("arith.extf", "arith.truncf", "arith.sitofp", "arith.uitofp", "arith.fptosi", "arith.fptoui",
                         "arith.extsi", "arith.extui", "arith.trunci", "arith.index_cast", "arith.index_castui"):
                uns = opn in ("arith.uitofp", "arith.fptoui", "arith.extui", "arith.index_castui")
                local[r_] = convert(T(_contig(xs[0].a), xs[0].elem), to, uns)
            else:
                raise NotImplementedError(f"region op {opn}")
        raise ValueError("linalg.generic region without linalg.yield")

    def _generic_reduce(self, region, ins, outs, env, maps, its):
        """linalg.generic with reduction loops, as convert-linalg-to-loops runs
        it: for every point of the parallel dims, the reduction dims in
        increasing order, each step's region evaluated with %out = the value
        so far (initially the outs tensor)."""
        o = env[outs[0]]
        nd = len(its)
        red = [d for d in range(nd) if its[d] == "reduction"]
        # loop extents from the inputs' shapes through their maps
        ext = [None] * nd
        for nm, mp in zip(ins, maps):
            sh = np.shape(env[nm].a)
            for ax, d in enumerate(mp):
                ext[d] = sh[ax]
        for ax, d in enumerate(maps[len(ins)]):
            ext[d] = np.shape(o.a)[ax]
        if any(e is None for e in ext):
            raise NotImplementedError("linalg.generic loop without an extent")
        acc = T(np.array(o.a, copy=True), o.elem)
        omap = maps[len(ins)]
        pdom = tuple(ext[d] for d in omap)
        for idx in np.ndindex(*[ext[d] for d in red]):
            # views of the inputs at this reduction point, over the output's dims
            def slice_in(nm, mp):
                a = np.asarray(env[nm].a)
                sel, keep = [], []
                for ax, d in enumerate(mp):
                    if d in red:
                        sel.append(idx[red.index(d)])
                    else:
                        sel.append(slice(None))
                        keep.append(d)
                v = a[tuple(sel)]
                order = [keep.index(d) for d in omap if d in keep]
                v = np.transpose(v, order) if v.ndim else v
                full = [pdom[i] if omap[i] in keep else 1 for i in range(len(omap))]
                return T(np.broadcast_to(np.reshape(v, full), pdom), env[nm].elem)
            step_ins = {nm: slice_in(nm, mp) for nm, mp in zip(ins, maps)}
            acc = self._eval_region(region, ins, step_ins, acc, pdom, env)
        return acc

    def _eval_region(self, region, ins, vals, out_val, dom, env):
        """One evaluation of a linalg.generic region over `dom` with the ins
        block arguments bound to `vals` and the outs argument to `out_val`."""
        body = region[region.index("^"):]
        hdr = re.match(r"\^\w+\(([^)]*)\)\s*:", body)
        bargs = [x.split(":")[0].strip() for x in hdr.group(1).split(",") if ":" in x]
        sub = {}
        for i, nm in enumerate(bargs):
            sub[nm] = vals[ins[i]] if i < len(ins) else out_val
        return self._run_region_body(body[hdr.end():], sub, dom, env, out_val.elem)

    def _scalar_arith(self, res, op, rest, env):
        names = re.findall(r"%[\w.$-]+", rest)
        ty = rest.rsplit(":", 1)[1]
        to = None
        if " to " in ty:
            ty, to = ty.split(" to ")
        _, elem = parse_type(to or ty)
        vals = [env[n].a for n in names]
        f32 = elem == "f32"
        if op in ("arith.index_cast", "arith.index_castui", "arith.extsi", "arith.extui", "arith.trunci",
                  "arith.sitofp", "arith.uitofp", "arith.extf", "arith.truncf"):
            # scalars and tensors alike (a rank-0 tensor<i64> -> tensor<bf16>
            # gives the bf16 bit pattern of the value)
            env[res] = convert(env[names[0]], elem, unsigned=op in ("arith.index_castui", "arith.extui", "arith.uitofp"))
            return
        else:
            a = [np.float32(x) if f32 else x for x in vals]
            v = {"arith.addf": lambda: a[0] + a[1], "arith.subf": lambda: a[0] - a[1],
                 "arith.mulf": lambda: a[0] * a[1], "arith.divf": lambda: a[0] / a[1],
                 "arith.negf": lambda: -a[0], "arith.addi": lambda: a[0] + a[1],
                 "arith.subi": lambda: a[0] - a[1], "arith.muli": lambda: a[0] * a[1]}[op]()
            v = np.array(v, NP[elem])
        env[res] = T(v, elem)

    def _reduce(self, res, rest, ins, outs, env):
        dims = [int(d) for d in re.search(r"dimensions\s*=\s*\[([^\]]*)\]", rest).group(1).split(",") if d.strip()]
        comb = re.search(r"\{\s*(arith\.\w+)\s*\}", rest)
        if comb is None:
            comb = re.search(r"(arith\.\w+)\s+%", rest)
        comb = comb.group(1)
        x, init = env[ins[0]], env[outs[0]]
        if outs[0] in self.empties:
            # reducing into an uninitialised tensor.empty: start from the identity
            ident = {"arith.addf": -0.0, "arith.mulf": 1.0, "arith.maximumf": -np.inf, "arith.minimumf": np.inf,
                     "arith.maxnumf": np.nan, "arith.minnumf": np.nan}
            if x.elem == "f32":
                init = T(np.full(init.a.shape, ident[comb], np.float32), "f32")
        rank = x.a.ndim
        keep = [d for d in range(rank) if d not in dims]
        # loop nest d0..d{r-1}: for each output element the reduced indices
        # are visited in ascending lexicographic order
        xt = _contig(np.transpose(x.a, dims + keep))
        K = int(np.prod([x.a.shape[d] for d in dims]))
        N = int(np.prod([x.a.shape[d] for d in keep])) if keep else 1
        if x.elem == "f32":
            acc = _contig(init.a.astype(np.float32).reshape(N)).copy()
            lib().hfref_reduce_f32(REDUCE_F[comb], ptr(xt.reshape(K, N)), ptr(acc), K, N)
            env[res] = T(acc.reshape(init.a.shape), "f32")
        elif x.elem in ("bf16", "f16"):
            raise NotImplementedError("16-bit float reductions")
        else:
            acc = _contig(init.a.astype(np.int64).reshape(N)).copy()
            xi = _contig(xt.reshape(K, N).astype(np.int64))
            lib().hfref_reduce_i64(REDUCE_I[comb], ptr(xi), ptr(acc), K, N, BITS[x.elem])
            env[res] = T(wrap_int(acc, x.elem).reshape(init.a.shape), x.elem)

    def _reduce_with_index(self, res, rest, ins, outs, env):
        dims = [int(d) for d in re.search(r"dimensions\s*=\s*\[([^\]]*)\]", rest).group(1).split(",") if d.strip()]
        kind = re.search(r"<(\w+)>", rest.split("ins(")[0]).group(1)
        x = env[ins[0]]
        idx_in = env[ins[1]] if len(ins) > 1 else None
        v0, i0 = env[outs[0]], env[outs[1]]
        d = dims[0]
        rank = x.a.ndim
        keep = [k for k in range(rank) if k != d]
        xt = _contig(np.transpose(x.a, [d] + keep))
        K = x.a.shape[d]
        N = int(np.prod([x.a.shape[k] for k in keep])) if keep else 1
        val = _contig(v0.a.reshape(N)).copy()
        idx = _contig(i0.a.astype(np.int64).reshape(N)).copy()
        ii = None
        if idx_in is not None:
            ii = _contig(np.transpose(idx_in.a, [d] + keep).astype(np.int64).reshape(K, N))
        if x.elem in ("bf16", "f16"):
            # the region's maximumf / cmpf on 16-bit floats run on their exact
            # f32 extensions; the folded value converts back exactly
            vf = _contig(to_f32(T(val, x.elem)).astype(np.float32))
            xf = _contig(to_f32(T(xt.reshape(K, N), x.elem)).astype(np.float32))
            lib().hfref_reduce_with_index_f32({"max": 0, "min": 1}[kind], ptr(xf),
                                              ptr(ii) if ii is not None else None, ptr(vf), ptr(idx), K, N)
            val = from_f32(vf, x.elem)
        elif x.elem == "f32":
            lib().hfref_reduce_with_index_f32({"max": 0, "min": 1}[kind], ptr(xt.reshape(K, N)),
                                              ptr(ii) if ii is not None else None, ptr(val), ptr(idx), K, N)
        else:
            xi = _contig(xt.reshape(K, N).astype(np.int64))
            v64 = _contig(val.astype(np.int64))
            lib().hfref_reduce_with_index_i64({"max": 0, "min": 1, "maxui": 2, "minui": 3}[kind], ptr(xi),
                                              ptr(ii) if ii is not None else None, ptr(v64), ptr(idx), K, N, BITS[x.elem])
            val = wrap_int(v64, x.elem)
        base = res
        env[base + "#0"] = T(val.reshape(v0.a.shape), v0.elem)
        env[base + "#1"] = T(wrap_int(idx, i0.elem).reshape(i0.a.shape), i0.elem)
        env[base] = env[base + "#0"]


def run(ir_text, *inputs, func=None, cast_semantics="declared"):
    return Interp(ir_text, cast_semantics).run(func, *inputs)
