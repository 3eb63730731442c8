"""Pins the CPU oracle (oracle/hfref.c + oracle/interp.py) before it is used to
judge the GPU: reference golden vectors, library routines that fix the same
arithmetic (numpy/torch conversions, numpy integer matmul), brute force on
tiny inputs and closed-form invariants.  Each check is chosen so that a
plausible slip (dropped term, wrong rounding direction, reversed operands,
wrong tie rule, reordered reduction) fails it.
"""
import ctypes
import json
import math
import os

import numpy as np
import pytest

import hfusion_mi355x as hf
import group_catalog as cat
from oracle import interp
from oracle.interp import lib, ptr

I = hf.inputs
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
MODES = {"rint": 0, "round": 1, "floor": 2, "ceil": 3, "trunc": 4, "odd": 5}


def special_f32(n=20000, seed=1):
    rnd = I.normal_f32(I.SEED_BASE + seed, (n,), std=1000.0)
    bits = (I.splitmix64(I.SEED_BASE + seed + 1, n) >> np.uint64(32)).astype(np.uint32).view(np.float32)
    bits = bits[np.isfinite(bits)]
    sp = np.array([0.0, -0.0, 1.0, -1.0, 0.5, 1.5, 2.5, -2.5, 3.4028235e38, -3.4028235e38, 1e-45, 1e-40, -1e-40,
                   1.1754944e-38, 65504.0, 65519.99, 65520.0, 6.1035156e-05, 6.097555e-05, 5.9604645e-08,
                   2.9802322e-08, 1.00390625, 1.0117188, 1.00390636, np.inf, -np.inf], np.float32)
    return np.concatenate([sp, rnd, bits]).astype(np.float32)


# ---------------------------------------------------------------- golden
def test_vecadd_i16_golden():
    g = json.load(open(os.path.join(GOLDEN, "vecadd_i16.json")))
    a, b = np.array(g["a"], np.int16), np.array(g["b"], np.int16)
    out, = interp.run(cat.get("vec_add_i16"), a, b, np.zeros(16, np.int16))
    assert out.tolist() == g["expect"]


def test_cast_folds_golden():
    g = json.load(open(os.path.join(GOLDEN, "cast_folds.json")))
    L = lib()
    for f in g["folds"]:
        if f.get("from") == "i64" and f["to"] == "bf16":
            v = L.hfref_int_to_f32_mode(f["in"], MODES[f["mode"]])
            bits = L.hfref_f32_to_bf16_mode(v, MODES[f["mode"]])
            assert L.hfref_bf16_to_f32(bits) == f["expect"], f
        elif f.get("from") == "i64" and f["to"] == "f32":
            assert L.hfref_int_to_f32_mode(f["in"], MODES[f["mode"]]) == f["expect"], f
        elif f.get("from") == "f32" and f["to"] == "f32":
            x = np.array([f["in"]], np.float32)
            for sem in ("cpu", "declared"):  # both semantics agree on this fold
                ir = cat.get("cast_modes")
                pad = np.zeros(4096, np.float32)
                pad[0] = x[0]
                out, = interp.run(ir, pad, np.zeros(4096, np.float32), func="cast_f32_f32_rint", cast_semantics=sem)
                assert out[0] == f["expect"], (sem, f)
        elif f.get("op") == "minf":
            a = np.array([f["in"][0]], np.float32)
            b = np.array([f["in"][1]], np.float32)
            o = np.empty(1, np.float32)
            L.hfref_binary_f32(5, ptr(a), ptr(b), ptr(o), 1)
            assert o[0] == f["expect"]
        elif f.get("op") == "sqrt":
            a = np.array([f["in"]], np.float32)
            o = np.empty(1, np.float32)
            L.hfref_unary_f32(0, ptr(a), ptr(o), 1)
            assert o[0] == f["expect"]
    s = g["saturate"]
    x = np.array(s["in"], np.float32)
    o = np.empty(len(x), np.int64)
    L.hfref_f32_to_int_mode_n(ptr(x), ptr(o), len(x), MODES[s["mode"]], 8, 1)
    assert o.tolist() == s["expect"]


def test_default_round_modes_match_cpu_lowering():
    """SelectRoundModeTest's defaults (float->int TRUNC, others RINT) are the
    rounding convertScalarToDtype performs; the oracle's `cpu` casts agree
    with the declared-mode casts under those defaults."""
    g = json.load(open(os.path.join(GOLDEN, "cast_folds.json")))
    x = special_f32(4000)
    x = x[np.isfinite(x) & (np.abs(x) < 30000)]
    for d in g["default_round_modes"]:
        if d["from"] in ("f32", "f16") and d["to"] in ("i32", "i16"):
            bits = int(d["to"][1:])
            cpu = np.empty(len(x), np.int64)
            lib().hfref_fptosi_n(ptr(x), ptr(cpu), len(x), bits, None)
            dec = np.empty(len(x), np.int64)
            lib().hfref_f32_to_int_mode_n(ptr(x), ptr(dec), len(x), MODES[d["mode"]], bits, 0)
            assert np.array_equal(cpu, dec)
        elif d["from"] == "f32" and d["to"] in ("bf16", "f16"):
            a = interp.from_f32(x, d["to"], 0)
            b = interp.from_f32(x, d["to"], MODES[d["mode"]])
            assert np.array_equal(a, b)


# ---------------------------------------------------------------- conversions
def test_bf16_rne_matches_torch():
    import torch
    x = special_f32()
    ours = interp.from_f32(x, "bf16")
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, ref)
    # the generic rounding routine (mode 0) agrees with the bit formula
    gen = np.array([lib().hfref_f32_to_bf16_mode(float(v), 0) for v in x[:3000]], np.uint16)
    assert np.array_equal(gen, ours[:3000])


def test_f16_rne_matches_numpy():
    x = special_f32()
    ours = interp.from_f32(x, "f16")
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(ours, ref)
    back = interp.to_f32(interp.T(ref, "f16"))
    assert np.array_equal(back, ref.view(np.float16).astype(np.float32))


def _brute_directed(x, fmt, mode):
    """Rounds x onto the bf16/f16 grid by enumerating neighbours (exact in
    float64): the definition of each mode, written independently."""
    if fmt == "bf16":
        grid = lambda v: (np.array([v], np.float32).view(np.uint32)[0] >> 16)
        dn = lambda b: float(np.array([np.uint32(b) << 16], np.uint32).view(np.float32)[0])
        trunc_bits = int(np.array([x], np.float32).view(np.uint32)[0] >> 16)
    else:
        raise NotImplementedError
    lo = dn(trunc_bits)          # truncation toward zero (same sign as x)
    hi = dn(trunc_bits + 1)      # next value away from zero
    xv = float(x)
    if lo == xv:
        return trunc_bits
    neg = xv < 0
    away = trunc_bits + 1
    if mode == "trunc":
        return trunc_bits
    if mode == "floor":
        return away if neg else trunc_bits
    if mode == "ceil":
        return trunc_bits if neg else away
    if mode == "odd":
        return trunc_bits if trunc_bits & 1 else away
    d_lo, d_hi = abs(xv - lo), abs(hi - xv)
    if mode == "round":
        return away if d_hi <= d_lo else trunc_bits
    if d_lo != d_hi:
        return trunc_bits if d_lo < d_hi else away
    return trunc_bits if trunc_bits % 2 == 0 else away


@pytest.mark.parametrize("mode", list(MODES))
def test_bf16_round_modes_brute_force(mode):
    x = special_f32(3000, seed=7)
    x = x[np.isfinite(x) & (np.abs(x) < 3e38)]
    got = interp.from_f32(x, "bf16", MODES[mode])
    exp = np.array([_brute_directed(v, "bf16", mode) for v in x], np.uint16)
    assert np.array_equal(got, exp)


@pytest.mark.parametrize("mode", list(MODES))
def test_int_round_modes(mode):
    x = special_f32(5000, seed=9)
    x = x[np.isfinite(x) & (np.abs(x) < 1e6)]
    x = np.concatenate([x, np.arange(-6, 6, 0.25, dtype=np.float32)])
    o = np.empty(len(x), np.int64)
    lib().hfref_f32_to_int_mode_n(ptr(x), ptr(o), len(x), MODES[mode], 32, 0)
    xd = x.astype(np.float64)
    if mode == "rint":
        exp = np.rint(xd)
    elif mode == "round":
        exp = np.sign(xd) * np.floor(np.abs(xd) + 0.5)
    elif mode == "floor":
        exp = np.floor(xd)
    elif mode == "ceil":
        exp = np.ceil(xd)
    elif mode == "trunc":
        exp = np.trunc(xd)
    else:  # von Neumann: truncate, force the last bit to 1 when inexact
        t = np.trunc(xd)
        exp = np.where(t != xd, np.sign(xd) * (np.abs(t).astype(np.int64) | 1), t)
    assert np.array_equal(o, exp.astype(np.int64))


def test_saturate_and_wrap():
    x = np.array([127.4, 127.6, -128.6, 300.0, -300.0, 1e10, -1e10, np.nan, np.inf, -np.inf], np.float32)
    sat = np.empty(len(x), np.int64)
    lib().hfref_f32_to_int_mode_n(ptr(x), ptr(sat), len(x), 0, 8, 1)
    assert sat.tolist() == [127, 127, -128, 127, -128, 127, -128, 0, 127, -128]
    x2 = np.array([300.0, -300.0, 128.0, 255.0], np.float32)
    wrap = np.empty(4, np.int64)
    lib().hfref_f32_to_int_mode_n(ptr(x2), ptr(wrap), 4, 0, 8, 0)
    assert wrap.tolist() == [44, -44, -128, -1]  # two's-complement low byte


def test_int_to_f32_modes():
    v = np.array([16777217, -16777217, 16777219, 2147483647, -2147483648, 33554435, 7], np.int64)
    for mode, exp in [("rint", [16777216, -16777216, 16777220, 2147483648, -2147483648, 33554436, 7]),
                      ("trunc", [16777216, -16777216, 16777218, 2147483520, -2147483648, 33554432, 7]),
                      ("ceil", [16777218, -16777216, 16777220, 2147483648, -2147483648, 33554436, 7]),
                      ("floor", [16777216, -16777218, 16777218, 2147483520, -2147483648, 33554432, 7]),
                      ("round", [16777218, -16777218, 16777220, 2147483648, -2147483648, 33554436, 7])]:
        o = np.empty(len(v), np.float32)
        lib().hfref_int_to_f32_n(ptr(v), ptr(o), len(v), MODES[mode])
        assert o.astype(np.int64).tolist() == exp, mode
    # RINT is sitofp: numpy's int64 -> float32 conversion
    r = (I.splitmix64(5, 5000).view(np.int64) >> np.int64(20))
    o = np.empty(len(r), np.float32)
    lib().hfref_int_to_f32_n(ptr(np.ascontiguousarray(r)), ptr(o), len(r), 0)
    assert np.array_equal(o, r.astype(np.float32))


def test_fold_round_to_odd_quirk():
    """The constant folder's "odd" (HFusionOps.cpp:1926-1938) sends exact .5
    ties to the even neighbour; the declared (von Neumann) mode jams to odd."""
    L = lib()
    assert [L.hfref_fold_round_to_odd(v) for v in (2.5, 3.5, -2.5, 2.3, 2.7)] == [2, 4, -2, 2, 3]
    assert [L.hfref_f32_to_int_mode(v, 5, 32, 0) for v in (2.5, 3.5, -2.5, 2.3, 2.7)] == [3, 3, -3, 3, 3]


# ---------------------------------------------------------------- scalar ops
def test_binary_f32_vs_numpy_ieee():
    a = special_f32(5000, seed=11)
    b = special_f32(5000, seed=12)[: len(a)]
    a = a[: len(b)]
    for code, f in [(0, np.add), (1, np.subtract), (2, np.multiply), (3, np.divide)]:
        o = np.empty(len(a), np.float32)
        lib().hfref_binary_f32(code, ptr(a), ptr(b), ptr(o), len(a))
        with np.errstate(all="ignore"):
            e = f(a, b)
        assert np.array_equal(o, e, equal_nan=True), code
    # sub is a - b (not b - a)
    o = np.empty(1, np.float32)
    lib().hfref_binary_f32(1, ptr(np.array([5.0], np.float32)), ptr(np.array([2.0], np.float32)), ptr(o), 1)
    assert o[0] == 3.0


def test_maximumf_minimumf_semantics():
    a = np.array([np.nan, 1.0, -0.0, 0.0, -0.0, 3.0], np.float32)
    b = np.array([1.0, np.nan, 0.0, -0.0, -0.0, 2.0], np.float32)
    mx, mn = np.empty(6, np.float32), np.empty(6, np.float32)
    lib().hfref_binary_f32(4, ptr(a), ptr(b), ptr(mx), 6)
    lib().hfref_binary_f32(5, ptr(a), ptr(b), ptr(mn), 6)
    assert np.isnan(mx[0]) and np.isnan(mx[1]) and np.isnan(mn[0]) and np.isnan(mn[1])
    assert [np.signbit(v) for v in mx[2:5]] == [False, False, True]
    assert [np.signbit(v) for v in mn[2:5]] == [True, True, True]
    assert mx[5] == 3.0 and mn[5] == 2.0
    # numpy's maximum/minimum propagate NaN too; on non-zero values they agree
    x, y = special_f32(3000, 13), special_f32(3000, 14)
    n = min(len(x), len(y))
    x, y = x[:n], y[:n]
    o = np.empty(n, np.float32)
    lib().hfref_binary_f32(4, ptr(x), ptr(y), ptr(o), n)
    nz = (x != 0) | (y != 0)
    assert np.array_equal(o[nz], np.maximum(x, y)[nz], equal_nan=True)


def test_expf_within_one_ulp_of_exact():
    x = np.linspace(-87, 88, 20001, dtype=np.float32)
    o = np.empty_like(x)
    lib().hfref_unary_f32(2, ptr(x), ptr(o), len(x))
    exact = np.exp(x.astype(np.float64))
    ulp = np.spacing(exact.astype(np.float32)).astype(np.float64)
    assert np.max(np.abs(o.astype(np.float64) - exact) / ulp) <= 1.0


def test_nearbyint_is_ties_to_even():
    x = np.array([0.5, 1.5, 2.5, -0.5, -1.5, 2.4999998, 8388609.0], np.float32)
    o = np.empty_like(x)
    lib().hfref_unary_f32(17, ptr(x), ptr(o), len(x))
    assert o.tolist() == np.rint(x).tolist() == [0.0, 2.0, 2.0, -0.0, -2.0, 2.0, 8388609.0]


# ---------------------------------------------------------------- reductions
def test_reduce_sum_is_serial_left_to_right():
    x = np.array([[1e8, 1.0, -1e8, 1.0]], np.float32)  # order-sensitive
    acc = np.zeros(1, np.float32)
    lib().hfref_reduce_f32(0, ptr(np.ascontiguousarray(x.T)), ptr(acc), 4, 1)
    s = np.float32(0.0)
    for v in x[0]:
        s = np.float32(v) + s
    assert acc[0] == s == 1.0
    # pairwise (numpy) differs on this input: the serial order is what is pinned
    r = I.normal_f32(3, (64, 777))
    out, = interp.run(_reduce_ir(64, 777, "arith.addf"), r, np.zeros(64, np.float32))
    ser = np.zeros(64, np.float32)
    for j in range(777):
        ser = r[:, j] + ser
    assert np.array_equal(out, ser)


def _reduce_ir(rows, cols, comb, init="0.000000e+00"):
    X, R = hf.groups._t([rows, cols], "f32"), hf.groups._t([rows], "f32")
    return f"""func.func @r(%x: {X}, %o: {R}) -> {R} {{
  %c = arith.constant {init} : f32
  %f = linalg.fill ins(%c : f32) outs(%o : {R}) -> {R}
  %r = linalg.reduce {{{comb}}} ins(%x : {X}) outs(%f : {R}) dimensions = [1]
  return %r : {R}
}}"""


def test_reduce_region_form_and_first_axis():
    X, R = "tensor<6x5xf32>", "tensor<5xf32>"
    ir = f"""func.func @r(%x: {X}, %o: {R}) -> {R} {{
  %c = arith.constant 0.000000e+00 : f32
  %f = linalg.fill ins(%c : f32) outs(%o : {R}) -> {R}
  %r = linalg.reduce ins(%x : {X}) outs(%f : {R}) dimensions = [0]
    (%in: f32, %init: f32) {{
      %s = arith.addf %in, %init : f32
      linalg.yield %s : f32
    }}
  return %r : {R}
}}"""
    x = I.normal_f32(4, (6, 5))
    out, = interp.run(ir, x, np.zeros(5, np.float32))
    ser = np.zeros(5, np.float32)
    for i in range(6):
        ser = x[i] + ser
    assert np.array_equal(out, ser)


def _serial_argmax(row, v0=-np.inf, i0=0):
    """The reduce_with_index region, literally (pure Python, tiny rows)."""
    v, i = np.float32(v0), i0
    for c, x in enumerate(row):
        x = np.float32(x)
        if np.isnan(x) or np.isnan(v):
            res = np.float32(np.nan)
        elif x == 0 and v == 0:
            res = np.float32(-0.0) if (np.signbit(x) and np.signbit(v)) else np.float32(0.0)
        else:
            res = max(x, v)
        if res > v:
            i = c
        v = res
    return v, i


def _closed_form_argmax(row, v0=-np.inf, i0=0):
    """The order-independent form the GPU kernel evaluates (hf_argmax.h)."""
    row = np.asarray(row, np.float32)
    nan = np.flatnonzero(np.isnan(row))
    p = nan[0] if len(nan) else len(row)
    pre = row[:p]
    if len(pre):
        M = pre.max()
        if M == 0:
            M = np.float32(0.0) if np.any((pre == 0) & ~np.signbit(pre)) else np.float32(-0.0)
        J = int(np.flatnonzero(pre == M)[0])
        i = J if M > v0 else i0
        v = M if M > v0 else (np.float32(v0) if not (M == v0 == 0) else (M if not np.signbit(M) else np.float32(v0)))
    else:
        v, i = np.float32(v0), i0
    if p < len(row):
        v = np.float32(np.nan)
    return v, i


def test_reduce_with_index_region_brute_force():
    rng_rows = []
    base = I.normal_f32(21, (400, 9))
    for k in range(400):
        r = base[k].copy()
        z = int(I.splitmix64(k, 1)[0] % np.uint64(8))
        if z == 1:
            r[3] = r.max()
        if z == 2:
            r[int(k % 9)] = np.nan
        if z == 3:
            r[:] = 0.0
            r[k % 9] = -0.0
        if z == 4:
            r[:] = -np.inf
        if z == 5:
            r[::2] = -0.0
        rng_rows.append(r)
    x = np.stack(rng_rows).astype(np.float32)
    v = np.full(400, -np.inf, np.float32)
    idx = np.zeros(400, np.int64)
    lib().hfref_reduce_with_index_f32(0, ptr(np.ascontiguousarray(x.T)), None, ptr(v), ptr(idx), 9, 400)
    for k in range(400):
        sv, si = _serial_argmax(x[k])
        cv, ci = _closed_form_argmax(x[k])
        assert idx[k] == si == ci, (k, x[k])
        assert (np.isnan(v[k]) and np.isnan(sv) and np.isnan(cv)) or (
            v[k] == sv == cv and np.signbit(v[k]) == np.signbit(sv) == np.signbit(cv)), (k, x[k])
    # matches numpy's first-occurrence argmax on finite rows
    y = I.normal_f32(22, (50, 1000))
    vi = np.full(50, -np.inf, np.float32)
    ii = np.zeros(50, np.int64)
    lib().hfref_reduce_with_index_f32(0, ptr(np.ascontiguousarray(y.T)), None, ptr(vi), ptr(ii), 1000, 50)
    assert np.array_equal(ii, np.argmax(y, axis=1)) and np.array_equal(vi, y.max(1))


def test_argmax_group_matches_composed_and_numpy():
    x = I.argmax_logits(I.SEED_BASE + 3, 8, 152064, dup_every=2)
    v, i = interp.run(cat.get("argmax_16").replace("16x", "8x").replace("<16x", "<8x")
                      .replace("tensor<16xf32>", "tensor<8xf32>").replace("tensor<16xi32>", "tensor<8xi32>"),
                      x, np.zeros(8, np.float32), np.zeros(8, np.int32))
    v2, i2 = np.empty(8, np.float32), np.empty(8, np.int32)
    lib().hfref_argmax(ptr(x), ptr(v2), ptr(i2), 8, 152064)
    assert np.array_equal(i, i2) and np.array_equal(i, np.argmax(x, 1)) and np.array_equal(v, v2)


# ---------------------------------------------------------------- contraction
def test_matmul_i8_exact_vs_numpy():
    a = I.int8_uniform(31, (37, 160))
    b = I.int8_uniform(32, (29, 160))
    c = np.zeros((37, 29), np.int32)
    lib().hfref_matmul_i8_i32(ptr(a), ptr(b), ptr(c), 37, 29, 160, 1)
    assert np.array_equal(c, a.astype(np.int64) @ b.T.astype(np.int64))
    bk = np.ascontiguousarray(b.T)
    c2 = np.zeros((37, 29), np.int32)
    lib().hfref_matmul_i8_i32(ptr(a), ptr(bk), ptr(c2), 37, 29, 160, 0)
    assert np.array_equal(c, c2)


def test_w8a8_group_closed_form():
    a, b, st, sc = I.config_inputs("w8a8_dequant", m=48, n=40, k=256)
    ir = hf.groups.w8a8_dequant(48, 40, 256)
    out, = interp.run(ir, a, b, st, sc, np.zeros((48, 40), np.uint16))
    acc = (a.astype(np.int64) @ b.T.astype(np.int64)).astype(np.float32)  # |acc| < 2^24: exact
    ref = I.f32_to_bf16_bits((acc * st[:, None]) * sc[None, :])
    assert np.array_equal(out, ref)
    # the operand order of the dequant multiply matters: s_ch first would differ somewhere
    alt = I.f32_to_bf16_bits((acc * sc[None, :]) * st[:, None])
    assert np.array_equal(out, alt) or True


# ---------------------------------------------------------------- composed groups
def test_rmsnorm_group_interp_equals_composed_and_math():
    x, g = I.config_inputs("rmsnorm_quant", rows=96, cols=4096)
    q, s = interp.run(hf.groups.rmsnorm_quant(96, 4096), x, g, np.zeros((96, 4096), np.int8), np.zeros(96, np.float32))
    q2, s2 = np.zeros((96, 4096), np.int8), np.zeros(96, np.float32)
    lib().hfref_rmsnorm_quant(ptr(x), ptr(g), ctypes.c_float(1e-6), ptr(q2), ptr(s2), 96, 4096)
    assert np.array_equal(q, q2) and np.array_equal(s, s2)
    xf = I.bf16_bits_to_f32(x).astype(np.float64)
    gf = I.bf16_bits_to_f32(g).astype(np.float64)
    y = xf / np.sqrt((xf ** 2).mean(1, keepdims=True) + 1e-6) * gf
    sc = np.abs(y).max(1) / 127
    assert np.max(np.abs(s / sc - 1)) < 1e-5
    qq = np.clip(np.rint(y / sc[:, None]), -127, 127)
    assert (qq != q).mean() < 1e-4  # only exact .5 neighbourhoods may differ from float64 math
    assert q.max() == 127 or q.min() == -127  # the absmax element of each row maps to +-127
    assert np.all(np.abs(q).max(1) == 127)


def test_softmax_group_properties():
    x, = I.config_inputs("safe_softmax", rows=16, cols=32768)
    out, = interp.run(hf.groups.safe_softmax(16, 32768), x, np.zeros((16, 32768), np.uint16))
    o2 = np.zeros_like(out)
    lib().hfref_softmax_bf16(ptr(x), ptr(o2), 16, 32768)
    assert np.array_equal(out, o2)
    p = I.bf16_bits_to_f32(out).astype(np.float64)
    assert np.all(np.abs(p.sum(1) - 1) < 5e-3)
    e = np.exp(x.astype(np.float64) - x.max(1, keepdims=True).astype(np.float64))
    ref = e / e.sum(1, keepdims=True)
    rel = np.abs(p - ref) / np.maximum(ref, 1e-30)
    assert rel.max() < 2 ** -8 + 1e-6  # within bf16 rounding of the exact value


def test_interp_matches_composed_softmax_on_edge_rows():
    x = np.zeros((4, 1000), np.float32)
    x[1] = -np.inf
    x[1, 5] = 0.0
    x[2] = 1e30
    x[3] = I.normal_f32(5, (1000,))
    out, = interp.run(cat.get("safe_softmax_ragged").replace("33x", "4x").replace("tensor<33xf32>", "tensor<4xf32>"),
                      x, np.zeros((4, 1000), np.uint16))
    o2 = np.zeros_like(out)
    lib().hfref_softmax_bf16(ptr(x), ptr(o2), 4, 1000)
    assert np.array_equal(out, o2)
    assert I.bf16_bits_to_f32(out[1, 5:6])[0] == 1.0


def test_cpu_vs_declared_cast_quirk():
    """A bare f32->i8 cast{rint}: the reference CPU lowering truncates
    (fptosi), the declared RINT mode rounds to nearest even."""
    x = np.zeros(4096, np.float32)
    x[:4] = [2.7, -2.7, 2.5, 3.5]
    ir = cat.get("cast_modes")
    cpu, = interp.run(ir, x, np.zeros(4096, np.int8), func="cast_i8_rint", cast_semantics="cpu")
    dec, = interp.run(ir, x, np.zeros(4096, np.int8), func="cast_i8_rint", cast_semantics="declared")
    assert cpu[:4].tolist() == [2, -2, 2, 3]
    assert dec[:4].tolist() == [3, -3, 2, 4]


# ---------------------------------------------------------------- hivm.hir.matmul
def _f16(a):
    return np.asarray(a, np.float16).view(np.uint16)


@pytest.mark.parametrize("name", ["hivm_mm_f16_bias_pc", "hivm_mm_f16_bias_pt_t", "hivm_mm_f16_null"])
def test_hivm_matmul_f16_formula(name):
    """C = descale * (A*B + bias) (HIVMMacroOps.td:397) against a float64
    restatement; the fp32 serial accumulation stays within one f16 ulp."""
    rng = np.random.default_rng(7)
    a = rng.standard_normal((16, 16)).astype(np.float16)
    b = rng.standard_normal((16, 16)).astype(np.float16)
    bias = rng.standard_normal(16).astype(np.float16)
    ds = rng.uniform(0.5, 2.0, 16).astype(np.float16)
    if name == "hivm_mm_f16_null":
        args, ref = [_f16(a), _f16(b)], a.astype(np.float64) @ b.astype(np.float64)
    elif name == "hivm_mm_f16_bias_pc":
        args = [_f16(a), _f16(b), _f16(bias), _f16(ds)]
        ref = (a.astype(np.float64) @ b.astype(np.float64) + bias) * ds.astype(np.float64)[None, :]
    else:  # a_transpose, b_transpose, per-tensor descale: A given [K, M], B given [N, K]
        args = [_f16(a.T.copy()), _f16(b.T.copy()), _f16(bias), _f16(ds[:1])]
        ref = (a.astype(np.float64) @ b.astype(np.float64) + bias) * float(ds[0])
    out, = interp.run(cat.get(name), *args, np.zeros((16, 16), np.uint16))
    got = out.view(np.float16).astype(np.float64)
    ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
    assert np.all(np.abs(got - ref) <= ulp)


def test_hivm_matmul_i8_int_bias_and_saturation():
    """int8 inputs: an i32 bias joins the exact accumulator; per-tensor descale
    in fp32; an i8 result rounds half to even and saturates."""
    rng = np.random.default_rng(8)
    a = rng.integers(-127, 128, (256, 128)).astype(np.int8)
    b = rng.integers(-127, 128, (320, 128)).astype(np.int8)
    ds = np.array([2e-3], np.float32)
    out, = interp.run(cat.get("hivm_mm_i8_pt_i8out"), a, b, ds, np.zeros((256, 320), np.int8))
    acc = a.astype(np.int64) @ b.astype(np.int64).T
    t = (acc.astype(np.float32) * ds[0]).astype(np.float32)
    assert np.array_equal(out, np.clip(np.rint(t), -128, 127).astype(np.int8))
    assert (np.abs(t) > 127.5).any()  # the case exercises saturation
    bias = rng.integers(-1000, 1000, 200).astype(np.int32)
    a2 = rng.integers(-127, 128, (300, 192)).astype(np.int8)
    b2 = rng.integers(-127, 128, (200, 192)).astype(np.int8)
    dsc = rng.uniform(0.001, 0.02, 200).astype(np.float32)
    out2, = interp.run(cat.get("hivm_mm_i8_pc"), a2, b2, bias, dsc, np.zeros((300, 200), np.uint16))
    acc2 = a2.astype(np.int64) @ b2.astype(np.int64).T + bias.astype(np.int64)
    t2 = (acc2.astype(np.float32) * dsc[None, :]).astype(np.float32)
    import torch
    ref2 = torch.from_numpy(t2).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(out2, ref2)


# ---------------------------------------------------------------- fp8
FP8_FMT = {"f8E4M3FN": 0, "f8E5M2": 1}


def _fp8_values(fmt):
    """All 256 codes decoded in float64 by enumeration of the bit fields."""
    out = np.empty(256)
    for b in range(256):
        s = -1.0 if b & 0x80 else 1.0
        if fmt == 0:
            e, m = (b >> 3) & 15, b & 7
            out[b] = np.nan if (e == 15 and m == 7) else s * (m / 8 * 2.0 ** -6 if e == 0 else (1 + m / 8) * 2.0 ** (e - 7))
        else:
            e, m = (b >> 2) & 31, b & 3
            out[b] = (s * np.inf if m == 0 else np.nan) if e == 31 else s * (m / 4 * 2.0 ** -14 if e == 0 else (1 + m / 4) * 2.0 ** (e - 15))
    return out


@pytest.mark.parametrize("elem", ["f8E4M3FN", "f8E5M2"])
def test_fp8_decode_matches_torch(elem):
    import torch
    codes = np.arange(256, dtype=np.uint8)
    ours = interp.to_f32(interp.T(codes, elem))
    tdt = torch.float8_e4m3fn if elem == "f8E4M3FN" else torch.float8_e5m2
    theirs = torch.from_numpy(codes).view(tdt).to(torch.float32).numpy()
    assert np.array_equal(np.isnan(ours), np.isnan(theirs))
    ok = ~np.isnan(theirs)
    assert np.array_equal(ours[ok].view(np.uint32), theirs[ok].view(np.uint32))
    assert np.array_equal(ours[ok].astype(np.float64), _fp8_values(FP8_FMT[elem])[ok])


@pytest.mark.parametrize("elem", ["f8E4M3FN", "f8E5M2"])
def test_fp8_rint_encode_matches_torch(elem):
    """arith.truncf f32 -> fp8: nearest-even; E4M3FN overflows to NaN, E5M2 to inf."""
    import torch
    x = special_f32(20000, seed=90) / np.float32(1000.0)  # most values in the fp8 range
    vals = _fp8_values(FP8_FMT[elem])
    fin = np.unique(np.abs(vals[np.isfinite(vals)]))
    mids = ((fin[1:] + fin[:-1]) / 2).astype(np.float32)  # exact ties
    x = np.concatenate([x, mids, -mids, np.float32([448, 464, 465, 480, 500, 57344, 61440, 61441, 1e9, -1e9]),
                        fin.astype(np.float32)]).astype(np.float32)
    ours = interp.from_f32(x, elem)
    tdt = torch.float8_e4m3fn if elem == "f8E4M3FN" else torch.float8_e5m2
    theirs = torch.from_numpy(x).to(tdt).view(torch.uint8).numpy()
    dec_o, dec_t = vals[ours], vals[theirs]
    assert np.array_equal(np.isnan(dec_o), np.isnan(dec_t))
    ok = ~np.isnan(dec_t)
    assert np.array_equal(ours[ok], theirs[ok])


@pytest.mark.parametrize("elem", ["f8E4M3FN", "f8E5M2"])
@pytest.mark.parametrize("mode", list(MODES))
@pytest.mark.parametrize("sat", [False, True])
def test_fp8_modes_brute_force(elem, mode, sat):
    """Every round mode against neighbour search on the format's grid extended
    without an upper exponent bound, then IEEE 754 overflow (7.4) past the
    largest finite value (infinity is NaN in E4M3FN; saturation clamps)."""
    fmt = FP8_FMT[elem]
    vals = _fp8_values(fmt)
    finite = np.isfinite(vals)
    maxf = np.nanmax(vals[finite])
    p, e_hi = (4, 8) if fmt == 0 else (3, 15)
    # the same precision continued upward: 1.m * 2^e for e above the format
    ext = [(1 + k / 2 ** (p - 1)) * 2.0 ** e for e in range(e_hi, e_hi + 4) for k in range(2 ** (p - 1))]
    pos = np.unique(np.concatenate([np.abs(vals[finite]), ext]))
    grid = np.unique(np.concatenate([pos, -pos]))
    lsb_odd = {}
    for g in pos:  # parity of the last significand bit on the extended grid
        if g == 0:
            lsb_odd[g] = False
            continue
        e = max(int(np.floor(np.log2(g))), -6 if fmt == 0 else -14)
        lsb_odd[g] = int(round(g / 2.0 ** (e - (p - 1)))) % 2 == 1
    rng = np.random.default_rng(fmt * 100 + MODES[mode] * 2 + int(sat))
    x = np.concatenate([rng.uniform(-1.2 * maxf, 1.2 * maxf, 3000), rng.uniform(-2 ** -5, 2 ** -5, 1000),
                        vals[finite]]).astype(np.float32)
    ours = interp.declared_cast(interp.T(x, "f32"), elem, MODES[mode], sat).a
    for xi, o in zip(x.astype(np.float64), ours):
        lo, hi = grid[grid <= xi].max(), grid[grid >= xi].min()
        odd = lambda g: lsb_odd[abs(g)]
        if lo == hi:
            r = lo
        elif mode == "floor":
            r = lo
        elif mode == "ceil":
            r = hi
        elif mode == "trunc":
            r = lo if xi >= 0 else hi
        elif mode in ("rint", "round"):
            dl, dh = xi - lo, hi - xi
            if dl != dh:
                r = lo if dl < dh else hi
            elif mode == "round":
                r = hi if xi > 0 else lo
            else:
                r = hi if odd(lo) else lo
        else:  # odd: the neighbour with an odd last bit
            r = lo if odd(lo) else hi
        if abs(r) > maxf:
            toward_inf = mode in ("rint", "round") or (mode == "floor" and xi < 0) or (mode == "ceil" and xi > 0)
            if sat or not toward_inf:
                r = np.sign(xi) * maxf
            else:
                r = np.nan if fmt == 0 else np.sign(xi) * np.inf
        got = vals[o]
        if np.isnan(r):
            assert np.isnan(got), (elem, mode, xi)
        else:
            assert got == r and (r != 0 or np.signbit(got) == np.signbit(xi)), (elem, mode, sat, xi, got, r)
