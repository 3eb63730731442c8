"""The oracle's elementwise functions of catalog module math_fns, pinned
against independent references: numpy / scipy / the math module in double
precision rounded to f32 (within a few f32 ulps: glibc's f32 functions are not
all correctly rounded), and exact closed forms for the exactly rounded ones
(ilogb, ldexp, divfhp, copysign, fmod, integer power / division, bitcast).
A function mapped to the wrong libm routine fails by orders of magnitude."""
import math

import numpy as np
import pytest
import scipy.special

import hfusion_mi355x as hf
import group_catalog as cat
from helpers import math_funcs, math_inputs, run_oracle

_D = {
    "tan": np.tan, "acos": np.arccos, "acosh": np.arccosh, "asin": np.arcsin, "asinh": np.arcsinh,
    "atan": np.arctan, "atanh": np.arctanh, "sinh": np.sinh, "cosh": np.cosh, "tanh": np.tanh,
    "sin": np.sin, "cos": np.cos, "erf": scipy.special.erf, "log2": np.log2, "log10": np.log10,
    "log1p": np.log1p, "exp2": np.exp2, "expm1": np.expm1, "log": np.log,
    "rsqrt": lambda x: 1.0 / np.sqrt(x),
    "lgamma": np.vectorize(lambda v: v if math.isnan(v) else math.inf if math.isinf(v) or (v <= 0 and v == math.floor(v))
                           else math.lgamma(v), otypes=[np.float64]),
}


def _close(got, ref, ulps):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    same_nan = np.isnan(got) == np.isnan(ref)
    fin = np.isfinite(ref) & np.isfinite(got)
    same_inf = np.where(np.isinf(ref), got == ref, True)
    tol = ulps * np.spacing(np.abs(ref).astype(np.float32)).astype(np.float64) + 1e-37
    with np.errstate(invalid="ignore"):
        ok = np.where(fin, np.abs(got - ref) <= tol, same_nan & same_inf)
    return ok


@pytest.mark.parametrize("func", [f for f in math_funcs() if f.startswith("u_")])
def test_unary_against_double(func):
    fn = func[2:]
    x, o = math_inputs(func)
    got, = run_oracle("math_fns", [x, o], func=func)
    if fn == "ilogb":
        _, e = np.frexp(x.astype(np.float64))
        ref = np.where(np.isnan(x), np.nan, np.where(x == 0, -np.inf, np.where(np.isinf(x), np.inf, e - 1.0)))
        assert np.array_equal(got, ref.astype(np.float32), equal_nan=True)
        return
    with np.errstate(all="ignore"):
        ref = _D[fn](x.astype(np.float64)).astype(np.float32)
    # lgamma near its zeros (x = 1, 2) is ill-conditioned in f32 inputs: absolute bar there
    ok = _close(got, ref, 4 if fn != "lgamma" else 8)
    if fn == "lgamma":
        ok |= np.abs(got.astype(np.float64) - ref) <= 2e-6
    bad = ~ok
    assert not bad.any(), f"{fn}: {int(bad.sum())} off, e.g. x={x[bad][:3]} got={got[bad][:3]} ref={ref[bad][:3]}"


def test_binary_exact_and_close():
    for func in ("b_atan2", "b_ldexp", "b_divfhp", "b_powf", "b_copysign", "b_mod"):
        a, b, o = math_inputs(func)
        got, = run_oracle("math_fns", [a, b, o], func=func)
        A, B = a.astype(np.float64), b.astype(np.float64)
        with np.errstate(all="ignore"):
            if func == "b_atan2":
                assert _close(got, np.arctan2(A, B).astype(np.float32), 4).all()
            elif func == "b_ldexp":
                k = np.where(np.isnan(b), 0, np.clip(b, -2**31, 2**31 - 1)).astype(np.int64)
                ref = np.ldexp(a, np.clip(k, -400, 400).astype(np.int32))  # f32 ldexp, nearest-even
                assert np.array_equal(got, ref, equal_nan=True)
            elif func == "b_divfhp":
                assert np.array_equal(got, a / b, equal_nan=True)
            elif func == "b_powf":
                assert _close(got, np.power(A, B).astype(np.float32), 4).all()
            elif func == "b_copysign":
                assert np.array_equal(got.view(np.uint32), np.copysign(a, b).view(np.uint32))
            else:
                assert np.array_equal(got, np.fmod(a, b), equal_nan=True)


@pytest.mark.parametrize("func", [f for f in math_funcs() if f.startswith("i_")])
def test_integer_binary(func):
    fn, t = func[2:].rsplit("_", 1)
    bits = {"i8": 8, "i16": 16, "i32": 32}[t]
    a, b, o = math_inputs(func)
    got, = run_oracle("math_fns", [a, b, o], func=func)
    m = 1 << bits

    def wrap(v):
        v %= m
        return v - m if v >= m // 2 else v
    ref = []
    for x, y in zip(a.tolist(), b.tolist()):
        if fn == "powi":
            r = (1 if x == 1 else (-1 if y % 2 else 1) if x == -1 else 0) if y < 0 else x ** y
        else:
            ux, uy = x % m, y % m
            r = 0 if uy == 0 else (-(-ux // uy) if fn == "ceildivui" else ux % uy)
        ref.append(wrap(r))
    assert np.array_equal(got.astype(np.int64), np.array(ref, np.int64))


def test_bitcast_operands():
    a, b, o = math_inputs("bitcast_add")
    got, = run_oracle("math_fns", [a, b, o], func="bitcast_add")
    assert np.array_equal(got, a.view(np.float32) + b.view(np.float32))


def test_math_module_lists_every_function():
    """Every function of the region builder's unary/binary enums that is not
    covered by another group is in math_fns (HFusionEnums.td:29-104)."""
    names = set(math_funcs())
    for fn in ("tan", "acos", "acosh", "asin", "asinh", "atan", "atanh", "sinh", "cosh", "lgamma", "ilogb"):
        assert f"u_{fn}" in names
    for fn in ("atan2", "ldexp", "divfhp"):
        assert f"b_{fn}" in names
    assert {"i_powi_i32", "i_ceildivui_i32", "i_modui_i32"} <= names
    assert cat.get("math_fns").count("func.func") == len(names)


# --------------------------------------------------------------------- fp_ops
from helpers import fp_funcs, fp_inputs  # noqa: E402


def _f32(x, t):
    if t == "f32":
        return x
    if t == "f16":
        return x.view(np.float16).astype(np.float32)
    return (x.astype(np.uint32) << 16).view(np.float32)


def test_fp_predicates_specials():
    x = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-40, 3.4e38, -1.0], np.float32)
    want = {"isinf": [0, 0, 1, 1, 0, 0, 0, 0], "isnan": [0, 0, 0, 0, 1, 0, 0, 0], "isfinite": [1, 1, 0, 0, 0, 1, 1, 1]}
    for op, w in want.items():
        ir = cat.fp_ops(8)
        got, = run_oracle_ir(ir, [x], f"{op}_f32")
        assert got.astype(int).tolist() == w, op


def run_oracle_ir(ir, args, func):
    from oracle import interp
    return interp.run(ir, *args, func=func)


@pytest.mark.parametrize("func", [f for f in fp_funcs() if f.startswith("nextafter")])
def test_nextafter_steps_one_ulp_toward_y(func):
    t = func.split("_")[1]
    x, y = fp_inputs(func)
    got, = run_oracle("fp_ops", [x, y], func=func)
    fx, fy, fg = _f32(x, t), _f32(y, t), _f32(got, t)
    nan = np.isnan(fx) | np.isnan(fy)
    assert np.isnan(fg[nan]).all()
    eq = ~nan & (fx == fy)
    assert np.array_equal(got[eq], y[eq])                      # x == y -> y
    m = ~nan & ~eq
    assert ((fg[m] - fx[m]) * (fy[m] - fx[m]) > 0).all()       # moved toward y
    # exactly one step: nothing representable strictly between x and the result
    xb = x.astype(np.int64) if t != "f32" else x.view(np.int32).astype(np.int64)
    gb = got.astype(np.int64) if t != "f32" else got.view(np.int32).astype(np.int64)
    sgn_bit = 0x8000 if t != "f32" else -2**31
    mag = lambda b: np.where(b < 0, b & 0x7FFFFFFF, b) if t == "f32" else b & 0x7FFF  # noqa: E731
    zero = m & (fx == 0)
    assert (mag(gb[zero]) == 1).all()                          # from zero: the smallest denormal
    nz = m & (fx != 0)
    assert (np.abs(mag(gb[nz]) - mag(xb[nz])) == 1).all()
    del sgn_bit


@pytest.mark.parametrize("func", [f for f in fp_funcs() if f.startswith("hypot")])
def test_hypot_against_double(func):
    t = func.split("_")[1]
    vs = fp_inputs(func)
    got, = run_oracle("fp_ops", vs, func=func)
    fs = [_f32(v, t).astype(np.float64) for v in vs]
    with np.errstate(all="ignore"):
        ref = np.sqrt(sum(f * f for f in fs))
        big = np.maximum.reduce([np.abs(f) for f in fs])
        ref = np.where(np.isfinite(ref) | ~np.isfinite(big), ref,
                       big * np.sqrt(sum((f / big) ** 2 for f in fs)))
    anynan = np.logical_or.reduce([np.isnan(f) for f in fs])
    anyinf = np.logical_or.reduce([np.isinf(f) for f in fs])
    ref = np.where(anyinf, np.inf, np.where(anynan, np.nan, ref))
    g = _f32(got, t).astype(np.float64)
    refr = ref.astype(np.float32) if t == "f32" else ref.astype(np.float16).astype(np.float32)
    ulps = 2 if t == "f32" else 1
    sp = np.spacing(np.abs(refr)).astype(np.float64)
    ok = np.where(np.isfinite(refr), np.abs(g - refr) <= ulps * sp, (g == refr) | (np.isnan(g) & np.isnan(refr)))
    assert ok.all(), f"{int((~ok).sum())} off"


@pytest.mark.parametrize("func", [f for f in fp_funcs() if f.startswith("erfinv")])
def test_erfinv_round_trip(func):
    t = func.split("_")[1]
    x, = fp_inputs(func)
    got, = run_oracle("fp_ops", [x], func=func)
    fx, fg = _f32(x, t).astype(np.float64), _f32(got, t).astype(np.float64)
    inside = np.abs(fx) < 0.999
    back = scipy.special.erf(fg[inside])
    tol = (1e-6 if t == "f32" else 2e-3) * np.maximum(np.abs(fx[inside]), 1e-3) + 1e-7
    assert (np.abs(back - fx[inside]) <= tol * 10).all()
    assert np.isposinf(fg[fx == 1.0]).all() and np.isneginf(fg[fx == -1.0]).all()
    assert np.isnan(fg[(np.abs(fx) > 1) | np.isnan(fx)]).all()


@pytest.mark.parametrize("func", ["signbit_f32", "signbit_f16", "signbit8_f32"])
def test_signbit_against_numpy(func):
    """hfusion.signbit (HFusionOps.td:1295), written in generic op form: the
    sign bit of every value, -0.0 and -NaN included, as numpy's signbit reads
    it from the float value."""
    x, = fp_inputs(func)
    got, = run_oracle("fp_ops", [x], func=func)
    xf = x if x.dtype == np.float32 else x.view(np.float16).astype(np.float32)
    want = np.signbit(xf)
    assert want[3] and want.sum() > 1000 and np.signbit(xf[np.isnan(xf)]).any()
    assert got.dtype == (np.int8 if func.startswith("signbit8") else np.bool_)
    assert np.array_equal(got.astype(bool), want)


def test_cyl_bessel_i0_closed_forms():
    """hfusion.cyl_bessel_i0 against what fixes i0: i0(0) = 1, evenness,
    the series sum_k (x^2/4)^k/(k!)^2 by brute force in exact rationals, the
    large-x asymptote e^x/sqrt(2 pi x), +inf from where the lowering's f32
    exp(|x|) overflows (|x| >= 88.72283935546875, the f32 just above
    ln(FLT_MAX); i0 itself would stay finite up to ~91.9), and NaN at +-inf
    (the form e^x * chbevl / sqrt(x) is inf / inf there)."""
    from fractions import Fraction
    xs = np.array([0.0, 0.5, -0.5, 1.0, 2.5, -7.0, 20.0, 60.0, 91.0, 92.0, np.inf, -np.inf, np.nan,
                   89.0, -90.0, 88.72283172607422, 88.72283935546875], np.float32)
    got, = run_oracle("fp_ops", [np.resize(xs, 4096)], func="cylbesseli0_f32")
    got = got[:len(xs)]
    assert got[0] == 1.0 and got[1] == got[2]
    for i in (1, 3, 4, 5, 6):
        q = Fraction(float(xs[i])) ** 2 / 4
        s, t = Fraction(0), Fraction(1)
        for k in range(1, 200):
            s += t
            t = t * q / (k * k)
        assert abs(float(got[i]) / float(s) - 1) < 1e-6, (xs[i], got[i], float(s))
    x = 60.0
    asym = math.exp(x) / math.sqrt(2 * math.pi * x) * (1 + 1 / (8 * x) + 9 / (2 * (8 * x) ** 2))
    assert abs(float(got[7]) / asym - 1) < 1e-5
    assert np.isinf(got[8]) and np.isinf(got[9]) and np.isnan(got[10]) and np.isnan(got[11]) and np.isnan(got[12])
    assert np.isinf(got[13]) and np.isinf(got[14]) and np.isinf(got[16])
    # the largest f32 below the threshold: exp(x) is finite, and so is i0
    assert np.float32(math.exp(88.72283172607422)) < np.inf and np.isfinite(got[15])
    asym = math.exp(88.72283172607422) / math.sqrt(2 * math.pi * 88.72283172607422)
    assert abs(float(got[15]) / asym - 1) < 2e-3


def test_bitcast_op():
    x, o = fp_inputs("bitcast_f32")
    got, = run_oracle("fp_ops", [x, o], func="bitcast_f32")
    assert np.array_equal(got.view(np.int32), x)


# ------------------------------------------------- scans, histogram, (de)interleave
from helpers import misc_inputs, scan_inputs  # noqa: E402


@pytest.mark.parametrize("spec", cat.SCAN_OPS, ids=[s[0] for s in cat.SCAN_OPS])
def test_scan_against_numpy_accumulate(spec):
    """numpy's accumulate is a left-to-right loop in the array's dtype, so it
    pins the serial order and the per-step rounding (numpy has no bf16: that
    group is pinned by test_bf16_cumprod_exact_rounding)."""
    name, op, ie, oe, shape, dim, rev, extra = spec
    if ie == "bf16":
        pytest.skip("bf16: see test_bf16_cumprod_exact_rounding")
    x, = scan_inputs(name)
    got, = run_oracle("scan_ops", [x], func=name)
    a = x.astype({"i64": np.int64}.get(oe, x.dtype))
    if rev:
        a = np.flip(a, dim)
    if op == "cumsum":
        r = np.cumsum(a, axis=dim, dtype=a.dtype)
    elif op == "cumprod":
        r = np.cumprod(a, axis=dim, dtype=a.dtype)
    elif op == "cummax":
        r = np.maximum.accumulate(a, axis=dim)
    else:
        r = (np.fmin if "propagate_nan = false" in extra else np.minimum).accumulate(a, axis=dim)
    if rev:
        r = np.flip(r, dim)
    assert np.array_equal(got, r, equal_nan=True)


def _bf16_round(v):
    """Round-half-even of the exact value v onto bf16 (8 significant bits,
    exponents down to the subnormal quantum 2^-133, overflow to inf), by
    scaling the significand and Python's half-even round() -- a restatement
    independent of the bit arithmetic the oracle uses."""
    if v == 0 or math.isinf(v) or math.isnan(v):
        return v
    m, e = math.frexp(abs(v))                  # |v| = m * 2^e, 0.5 <= m < 1
    q = max(e - 8, -133)                       # quantum: 8 bits below the leading one
    r = round(abs(v) / 2.0 ** q) * 2.0 ** q    # exact: |v| / 2^q has <= 53 bits here
    if r >= 2.0 ** 128 * (1 - 2.0 ** -9):      # at or past the rounding boundary of bf16 max
        r = math.inf
    return math.copysign(r, v)


def test_bf16_cumprod_exact_rounding():
    """cumprod over bf16 (reverse, dim 1): each step is the exact product of
    two bf16 values (at most 16 significant bits, exact in double) rounded
    half-even to bf16; recomputed here in double with an independent rounding."""
    name = "cumprod_bf16_rev"
    spec = {s[0]: s for s in cat.SCAN_OPS}[name]
    x, = scan_inputs(name)
    got, = run_oracle("scan_ops", [x], func=name)
    xf = (x.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    want = np.empty_like(xf)
    for r in range(xf.shape[0]):
        acc = None
        for c in range(xf.shape[1] - 1, -1, -1):
            acc = xf[r, c] if acc is None else _bf16_round(acc * xf[r, c])
            want[r, c] = acc
    wb = (want.astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    assert spec[6] and spec[5] == 1
    assert np.array_equal(np.asarray(got).view(np.uint16), wb)
    # the data reach products that are not representable: rounding happened
    assert (np.abs(want[:, :-1]) > 0).sum() > 1000


@pytest.mark.parametrize("spec", cat.HIST_OPS, ids=[h[0] for h in cat.HIST_OPS])
def test_histogram_counts(spec):
    name, ie, shape, bins, ce, me = spec
    args = misc_inputs(name)
    got, = run_oracle("misc_ops", args, func=name)
    v = args[0].ravel().astype(np.int64)
    keep = (v >= 0) & (v < bins)
    if me:
        keep &= args[1].ravel()
    want = np.zeros(bins, np.int64)
    for b in v[keep].tolist():
        want[b] += 1
    assert np.array_equal(got.astype(np.int64), want.astype({"i8": np.int8, "i32": np.int32, "i64": np.int64}[ce]).astype(np.int64))


def test_deinterleave_interleave_closed_form():
    for name, e, ch in cat.INTERLEAVE_OPS:
        args = misc_inputs(name)
        outs = run_oracle("misc_ops", args, func=name)
        if ch is None:
            a, b = args
            assert np.array_equal(outs[0][:, 0::2], a) and np.array_equal(outs[0][:, 1::2], b)
        elif ch == -1:
            assert np.array_equal(outs[0], args[0][:, 0::2]) and np.array_equal(outs[1], args[0][:, 1::2])
        else:
            assert np.array_equal(outs[0], args[0][:, ch::2])


from helpers import misc_extra_inputs  # noqa: E402


def test_mulext_halves_recompose_the_product():
    """lo + hi * 2^N equals the exact product of the sign- (mulext) or
    zero-extended (mulextui) operands, with lo read unsigned."""
    for name in [n for n in cat.MISC_EXTRA if n.startswith("mulext")]:
        a, b = misc_extra_inputs(name)
        lo, hi = run_oracle("misc_ops", [a, b], func=name)
        bits = a.dtype.itemsize * 8
        m = 1 << bits
        for x, y, l, h in zip(a.tolist()[:512], b.tolist()[:512], lo.tolist()[:512], hi.tolist()[:512]):
            if name.startswith("mulextui"):
                x, y = x % m, y % m
                h %= m
            assert (l % m) + h * m == x * y, (name, x, y, l, h)


def test_flip_and_arange_closed_forms():
    x, = misc_extra_inputs("flip_f32")
    got, = run_oracle("misc_ops", [x], func="flip_f32")
    assert np.array_equal(got, x[:, ::-1])
    o, off = misc_extra_inputs("arange_i32")
    got, = run_oracle("misc_ops", [o, off], func="arange_i32")
    i, j = np.meshgrid(np.arange(48), np.arange(130), indexing="ij")
    assert np.array_equal(got, (off + 1000 * i - 3 * j).astype(np.int32))


from helpers import gather_inputs  # noqa: E402


@pytest.mark.parametrize("spec", cat.GATHER_OPS, ids=[g[0] for g in cat.GATHER_OPS])
def test_gather_loop_form(spec):
    """The op description's loop (HFusionStructuredOps.td:222-238), run
    literally on the group's inputs: output[p] = src[.. k ..] for the k with
    index[p] == k, else the init value."""
    name, se, ss, ie, ish, ax = spec
    src, idx, init = gather_inputs(name)
    got, = run_oracle("gather_ops", [src, idx, init], func=name)
    want = init.copy()
    for p in np.ndindex(*ish):
        for k in range(ss[ax]):
            if idx[p] == k:
                q = list(p)
                q[ax] = k
                want[p] = src[tuple(q)]
    assert np.array_equal(got, want)


from helpers import generic_inputs  # noqa: E402


def test_generic_regions_closed_form():
    """linalg.generic regions evaluated by the oracle against numpy closed
    forms of the same scalar programs (float64 for the transcendental one)."""
    x, b, t, s, o = generic_inputs("generic_bias_act")
    got, = run_oracle("generic_ops", [x, b, t, s, o], func="generic_bias_act")
    z = x.astype(np.float64) + b
    tt = t[:, None].astype(np.float64)
    ref = np.exp(z) / np.maximum(np.where(z > tt, np.tanh(z * 0.5), tt * 0.3), 1.0)
    np.testing.assert_allclose(got, ref, rtol=2e-6)
    h, i, oh, om = generic_inputs("generic_f16_int")
    gh, gm = run_oracle("generic_ops", [h, i, oh, om], func="generic_f16_int")
    hf16 = h.view(np.float16)
    with np.errstate(all="ignore"):
        p = (hf16.astype(np.float32) * i.astype(np.float32)).astype(np.float16)
    with np.errstate(all="ignore"):
        assert np.array_equal(gh.view(np.float16), p + hf16, equal_nan=True)
    i64 = i.astype(np.int64)
    rem = np.fmod(i64, 3)
    shl = ((i64 << 3) & 0xFFFFFFFF).astype(np.uint32).view(np.int32).astype(np.int64)
    assert np.array_equal(gm, (rem ^ shl).astype(np.int32) < 0)


def test_generic_reduction_serial_loop():
    """linalg.generic reductions run by the oracle as the CPU loop nest does:
    max of x*w equals numpy's (exact); the sum equals a float32 left-to-right
    loop bit for bit."""
    rng = np.random.default_rng(5)
    x = rng.normal(size=(64, 1000)).astype(np.float32)
    w = rng.normal(size=1000).astype(np.float32)
    o = np.zeros(64, np.float32)
    mx, = run_oracle("generic_reduce", [x, w, o], func="gred_max")
    assert np.array_equal(mx, np.max(x * w, axis=1))
    sm, = run_oracle("generic_reduce", [x, w, o], func="gred_sum")
    acc = np.zeros(64, np.float32)
    for k in range(1000):
        acc = (acc + (x[:, k] * w[k]).astype(np.float32)).astype(np.float32)
    assert np.array_equal(sm, acc)
