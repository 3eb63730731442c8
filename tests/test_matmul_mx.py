"""hfusion.matmul_mx, the block-scaled fp8 contraction (HFusionOps.td:1233-1291):
the oracle pinned on the CPU against a plain fp8 matmul (unit scales), against
a literal restatement of the reference's K = 32 decomposition
(HFusionOps.cpp:3590-3790), against exact power-of-two scaling and the NaN
scale; the lowering's limits; then the HIP kernel on the matrix core's scaled
MFMA against the oracle (GPU)."""
import numpy as np
import pytest

import hfusion_mi355x as hf
import group_catalog as cat
from helpers import run_gpu, run_oracle, bf16_ulp_diff
from oracle import interp
from oracle.interp import lib, ptr

FMT = {"e4m3": 0, "e5m2": 1}
TY = {"e4m3": "f8E4M3FN", "e5m2": "f8E5M2"}


def note(msg):
    print(f"[case] {msg}", flush=True)


def fp8_bytes(rng, shape, fmt):
    """Random fp8 codes of every finite value (NaN / inf codes excluded)."""
    v = rng.integers(0, 256, shape).astype(np.uint8)
    bad = (v & 0x7F) == 0x7F if fmt == "e4m3" else (v & 0x7C) == 0x7C
    v[bad] &= 0xF3 if fmt == "e5m2" else 0xF7
    return v


def decode(v, fmt):
    return interp.to_f32(interp.T(np.asarray(v, np.uint8), TY[fmt]))


def mx_ir(m, n, k, fa, fb, kb=None):
    kb = kb if kb is not None else k // 32
    A, B = f"tensor<{m}x{k}x{TY[fa]}>", f"tensor<{k}x{n}x{TY[fb]}>"
    SA, SB, C = f"tensor<{m}x{kb}xui8>", f"tensor<{n}x{kb}xui8>", f"tensor<{m}x{n}xf32>"
    return f"""module {{
  func.func @mx(%a: {A}, %b: {B}, %sa: {SA}, %sb: {SB}) -> {C}
      {cat._ATTRS.format(kind='SINGLE_CUBE')} {{
    %e = tensor.empty() : {C}
    %c = hfusion.matmul_mx ins(%a, %b, %sa, %sb : {A}, {B}, {SA}, {SB}) outs(%e : {C}) -> {C}
    return %c : {C}
  }}
}}
"""


def oracle_mx(a, b, sa, sb, fa, fb):
    m, k = a.shape
    return interp.run(mx_ir(m, b.shape[1], k, fa, fb, sa.shape[1]), a, b, sa, sb)[0]


def mx_case(rng, m, n, k, fa, fb, spread=8):
    a, b = fp8_bytes(rng, (m, k), fa), fp8_bytes(rng, (k, n), fb)
    sa = rng.integers(127 - spread, 128 + spread, (m, -(-k // 32))).astype(np.uint8)
    sb = rng.integers(127 - spread, 128 + spread, (n, -(-k // 32))).astype(np.uint8)
    return a, b, sa, sb


def abs_products(a, b, sa, sb, fa, fb):
    """sum_k |A'[m, k] B'[k, n]| of the scaled operands (float64): the scale
    of each output's rounding error."""
    k = a.shape[1]
    x = decode(a, fa).astype(np.float64) * np.exp2(np.repeat(sa.astype(np.float64) - 127, 32, axis=1)[:, :k])
    y = decode(b, fb).astype(np.float64) * np.exp2(np.repeat(sb.astype(np.float64) - 127, 32, axis=1)[:, :k]).T
    return np.abs(x) @ np.abs(y), x @ y


@pytest.mark.parametrize("fa,fb", [("e4m3", "e4m3"), ("e5m2", "e4m3"), ("e4m3", "e5m2"), ("e5m2", "e5m2")])
def test_oracle_mx_unit_scales_is_the_fp8_matmul(fa, fb):
    # every scale 2^0: the linalg.matmul region over the fp8 values widened to f32
    rng = np.random.default_rng(1)
    a, b, _, _ = mx_case(rng, 9, 13, 96, fa, fb)
    sa, sb = np.full((9, 3), 127, np.uint8), np.full((13, 3), 127, np.uint8)
    got = oracle_mx(a, b, sa, sb, fa, fb)
    want = np.zeros((9, 13), np.float32)
    lib().hfref_matmul_f32(ptr(np.ascontiguousarray(decode(a, fa))), ptr(np.ascontiguousarray(decode(b, fb))), ptr(want),
                           9, 13, 96, 0)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def decomposition_k32(a, b, sa, sb, fa, fb):
    """The reference's software path for K = 32, step by step in numpy:
    fp8 -> f16 (rint), scale -> u16 << 7 -> bitcast bf16 -> f32 -> f16, f16
    multiply by the broadcast scale, then linalg.matmul's f32 region (extf,
    mulf, addf serially over k from the init)."""
    def scale_f16(s):
        bf = (s.astype(np.uint16) << np.uint16(7)).astype(np.uint32) << np.uint32(16)
        return bf.view(np.float32).astype(np.float16)
    xa = decode(a, fa).astype(np.float16) * np.repeat(scale_f16(sa), 32, axis=1)
    xb = decode(b, fb).astype(np.float16) * np.repeat(scale_f16(sb), 32, axis=1).T
    acc = np.zeros((a.shape[0], b.shape[1]), np.float32)
    for kk in range(a.shape[1]):
        acc = acc + (xa[:, kk:kk + 1].astype(np.float32) * xb[kk:kk + 1, :].astype(np.float32))
    return acc


@pytest.mark.parametrize("fa,fb", [("e4m3", "e4m3"), ("e5m2", "e4m3"), ("e4m3", "e5m2"), ("e5m2", "e5m2")])
def test_oracle_mx_is_the_reference_decomposition_at_k32(fa, fb):
    # scales where the decomposition's f16 steps are exact: every scaled
    # operand inside f16's range and above its smallest subnormal
    rng = np.random.default_rng(2)
    a, b, _, _ = mx_case(rng, 16, 24, 32, fa, fb)
    lo = {"e4m3": 117, "e5m2": 122}
    hi = {"e4m3": 132, "e5m2": 127}
    sa = rng.integers(lo[fa], hi[fa] + 1, (16, 1)).astype(np.uint8)
    sb = rng.integers(lo[fb], hi[fb] + 1, (24, 1)).astype(np.uint8)
    got = oracle_mx(a, b, sa, sb, fa, fb)
    with np.errstate(over="ignore", invalid="ignore"):
        want = decomposition_k32(a, b, sa, sb, fa, fb)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_oracle_mx_power_of_two_scaling_and_nan_scale():
    rng = np.random.default_rng(3)
    a, b, sa, sb = mx_case(rng, 8, 16, 128, "e4m3", "e4m3", spread=3)
    base = oracle_mx(a, b, sa, sb, "e4m3", "e4m3")
    # raising every A scale by d multiplies every scaled operand, every
    # product and every partial sum by 2^d exactly
    for d in (-5, 4):
        got = oracle_mx(a, b, (sa.astype(int) + d).astype(np.uint8), sb, "e4m3", "e4m3")
        assert np.array_equal(got, np.ldexp(base, d).astype(np.float32)), d
    # e8m0 255 is NaN (OCP MX, the matrix core): row 3 and column 5 of the
    # result become NaN.  The reference decomposition reads 255 as +inf
    # instead (HFusionOps.cpp:3590+: ui8 << 7 bitcast to bf16), so this case
    # is parity unpinned against the reference and pins the oracle only.
    sa2, sb2 = sa.copy(), sb.copy()
    sa2[3, 2] = 255
    sb2[5, 0] = 255
    got = oracle_mx(a, b, sa2, sb2, "e4m3", "e4m3")
    nan = np.zeros_like(got, bool)
    nan[3, :] = True
    nan[:, 5] = True
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan], base[~nan])


def test_oracle_mx_reference_test_shapes():
    """The shapes of bishengir/test/Conversion/HFusionToHIVM/matmul-mx-format.mlir
    (4x8 by 8x16, one scale per row: K = 8 is one block): against exact
    float64 arithmetic (the f32 sum of 8 exact products)."""
    rng = np.random.default_rng(4)
    for fa, fb in (("e4m3", "e4m3"), ("e5m2", "e5m2")):
        a, b, sa, sb = mx_case(rng, 4, 16, 8, fa, fb, spread=4)
        got = oracle_mx(a, b, sa, sb, fa, fb)
        mag, exact = abs_products(a, b, sa, sb, fa, fb)
        assert np.all(np.abs(got - exact) <= 8 * 2.0 ** -24 * mag + 1e-30)


def test_matmul_mx_lowering_limits():
    base = cat.get("mx_e4m3")

    def ir(m, n, k, extra_attr=""):
        text = hf.groups.matmul_mx(m, n, k, via="format" if extra_attr else "fp8")
        return text.replace("lhsFormat = 2", extra_attr) if extra_attr else text
    for text, msg in ((ir(64, 64, 96), "multiple of 128"), (ir(64, 72, 128), "N must be a multiple of 16"),
                      (ir(64, 64, 128, "lhsFormat = 3"), "fp4"), (ir(64, 64, 128, "lhsFormat = 12"), "valid lhsFormat"),
                      (hf.groups.matmul_mx(64, 64, 128, fa="e2m1", fb="e2m1", via="format"), "multiple of 256")):
        with pytest.raises(hf.CompileError, match=msg):
            hf.compile(text, options="emit=hip")
    with pytest.raises(hf.CompileError, match="fp4"):
        hf.compile(cat.get("mx_fp4_256"), options="emit=hip;mx_exact=1")
    assert "mmad_mx<7," in open(hf.compile(cat.get("mx_fp4_256"), options="emit=hip").source).read()
    # ui8 only as matmul_mx scales
    bad = """module {
  func.func @f(%x: tensor<8x8xui8>) -> tensor<8x8xi32>
      """ + cat._ATTRS.format(kind='PURE_ELEMWISE') + """ {
    %e = tensor.empty() : tensor<8x8xi32>
    %c = hfusion.cast {round_mode = #hfusion.round_mode<rint>} ins(%x : tensor<8x8xui8>) outs(%e : tensor<8x8xi32>) -> tensor<8x8xi32>
    return %c : tensor<8x8xi32>
  }
}
"""
    with pytest.raises(hf.CompileError, match="ui8"):
        hf.compile(bad, options="emit=hip")
    assert "mmad_mx" in open(hf.compile(base, options="emit=hip").source).read()


# ---- fp4 (e2m1, format 3): two values per byte along K, the even k in the
# low nibble (the reference library's fp4x2_e2m1_t, LocalMmadMx.cpp:131-133)
E2M1 = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], np.float64)  # OCP MX, magnitudes of codes 0-7


def fp4_decode(nib):
    nib = np.asarray(nib, np.uint8)
    return np.where(nib & 8, -1.0, 1.0) * E2M1[nib & 7]


def fp4_case(rng, m, n, k, spread=8):
    """Random e2m1 codes (every code is a number) packed two per byte:
    A [m, k/2], B [k/2, n] bytes, and the unpacked codes [m, k], [k, n]."""
    ca = rng.integers(0, 16, (m, k)).astype(np.uint8)
    cb = rng.integers(0, 16, (k, n)).astype(np.uint8)
    a = (ca[:, 0::2] | (ca[:, 1::2] << 4)).astype(np.uint8)
    b = (cb[0::2, :] | (cb[1::2, :] << 4)).astype(np.uint8)
    sa = rng.integers(127 - spread, 128 + spread, (m, k // 32)).astype(np.uint8)
    sb = rng.integers(127 - spread, 128 + spread, (n, k // 32)).astype(np.uint8)
    return a, b, sa, sb, ca, cb


def fp4_products(ca, cb, sa, sb):
    k = ca.shape[1]
    x = fp4_decode(ca) * np.exp2(np.repeat(sa.astype(np.float64) - 127, 32, axis=1)[:, :k])
    y = fp4_decode(cb) * np.exp2(np.repeat(sb.astype(np.float64) - 127, 32, axis=1)[:, :k]).T
    return np.abs(x) @ np.abs(y), x @ y


def oracle_fp4(a, b, sa, sb, m, n, k):
    text = hf.groups.matmul_mx(m, n, k, fa="e2m1", fb="e2m1", via="bitcast")
    return interp.run(text, a, b, sa, sb)[0]


def test_oracle_fp4_values():
    # the 16 e2m1 codes: sign, 2 exponent bits (bias 1), 1 mantissa bit
    got = np.array([lib().hfref_fp4_to_f32(v) for v in range(16)], np.float64)
    assert np.array_equal(got, fp4_decode(np.arange(16)))
    assert np.array_equal(np.signbit(got), np.arange(16) >= 8)


def test_oracle_mx_fp4_exact_and_packing():
    rng = np.random.default_rng(5)
    m, n, k = 12, 20, 256
    a, b, sa, sb, ca, cb = fp4_case(rng, m, n, k, spread=0)
    # unit scales: every product a multiple of 1/4 below 36, every partial
    # sum below 2^14: the f32 serial sum is the exact (float64) product
    got = oracle_fp4(a, b, sa, sb, m, n, k)
    _, exact = fp4_products(ca, cb, sa, sb)
    assert np.array_equal(got.astype(np.float64), exact)
    # the nibble order: one nonzero code at an odd k picks B's row k
    a1 = np.zeros_like(a)
    a1[3, 7] = 0x20                       # k = 15 (high nibble of byte 7): 1.0
    got = oracle_fp4(a1, b, sa, sb, m, n, k)
    assert np.array_equal(got[3].astype(np.float64), fp4_decode(cb[15]))
    assert not got[np.arange(m) != 3].any()
    # scales: raising A's block scales by d scales every product by 2^d
    a, b, sa, sb, ca, cb = fp4_case(rng, m, n, k, spread=3)
    base = oracle_fp4(a, b, sa, sb, m, n, k)
    got = oracle_fp4(a, b, (sa.astype(int) + 4).astype(np.uint8), sb, m, n, k)
    assert np.array_equal(got, np.ldexp(base, 4).astype(np.float32))
    mag, exact = fp4_products(ca, cb, sa, sb)
    assert np.all(np.abs(base - exact) <= k * 2.0 ** -24 * mag + 1e-30)


# The matrix core's fp8 dot product over 64 k (scaled or not: the unscaled
# 16-k fp8 instruction lands on the same values) is not the f32 serial sum:
# measured on gfx950 it is within 4.3e-4 of sum|products| of the exact value
# on 1024 random 32x32x64 blocks with scales spread over 2^-7 .. 2^7, and
# within 2.6e-4 of the oracle in the cases below.  The bar is
# |gpu - oracle| <= 2^-11 * sum_k |A'B'| per element (the scaled operands
# A', B'); it does not meet a 1e-5 relative bar.
TOL = 2.0 ** -11
# mx_exact=1: the operands scaled into bf16 exactly, products exact on the
# bf16 matrix core, sums in f32: the difference to the oracle's serial f32
# sum is of the order of f32 rounding
TOL_EXACT = 2.0 ** -17

GPU_CASES = {"mx_e4m3": (256, 256, 256, "e4m3", "e4m3", None, "f32"),
             "mx_e5m2_bitcast": (300, 208, 384, "e5m2", "e4m3", 0.5, "f32"),
             "mx_format_bf16": (264, 784, 256, "e4m3", "e5m2", None, "bf16"),
             "mx_e5m2": (128, 128, 128, "e5m2", "e5m2", None, "f32")}


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(GPU_CASES) + sorted(n + "_exact" for n in GPU_CASES))
def test_matmul_mx_gpu(gpu, name):
    base = name[:-len("_exact")] if name.endswith("_exact") else name
    tol = TOL_EXACT if name.endswith("_exact") else TOL
    m, n, k, fa, fb, init, out = GPU_CASES[base]
    note(f"{name} {m}x{n}x{k} {fa}x{fb} init={init} out={out}")
    rng = np.random.default_rng(sum(map(ord, base)))
    a, b, sa, sb = mx_case(rng, m, n, k, fa, fb)
    got, = run_gpu(name, [a, b, sa, sb], gpu)
    want, = run_oracle(base, [a, b, sa, sb])
    mag, _ = abs_products(a, b, sa, sb, fa, fb)
    if out == "f32":
        err = np.abs(got.astype(np.float64) - want) / np.maximum(mag, 1e-30)
        print(f"[err] {name}: max |gpu - oracle| / sum|A'B'| = {err.max():.3e}", flush=True)
        assert np.all(np.abs(got.astype(np.float64) - want) <= tol * mag + 1e-30)
    else:
        # bf16 of values within the bar: one bf16 ulp beyond the f32 bar
        gf = (got.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
        wf = (want.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
        assert np.all(np.abs(gf - wf) <= tol * mag + 2.0 ** -7 * np.abs(wf) + 1e-30)


# fp4 on the scaled matrix core (format code 4): the bar is measured below
# (printed as [err]) and set with margin
TOL_FP4 = 2.0 ** -17
FP4_CASES = {"mx_fp4_256": (256, 256, 512, None, "f32"), "mx_fp4_ragged": (300, 208, 768, 0.5, "f32"),
             "mx_fp4_bf16": (264, 784, 256, None, "bf16")}


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(FP4_CASES))
def test_matmul_mx_fp4_gpu(gpu, name):
    m, n, k, init, out = FP4_CASES[name]
    note(f"{name} {m}x{n}x{k} fp4 init={init} out={out}")
    rng = np.random.default_rng(sum(map(ord, name)))
    a, b, sa, sb, ca, cb = fp4_case(rng, m, n, k)
    got, = run_gpu(name, [a, b, sa, sb], gpu)
    want, = run_oracle(name, [a, b, sa, sb])
    mag, _ = fp4_products(ca, cb, sa, sb)
    if out == "f32":
        err = np.abs(got.astype(np.float64) - want) / np.maximum(mag, 1e-30)
        print(f"[err] {name}: max |gpu - oracle| / sum|A'B'| = {err.max():.3e}", flush=True)
        assert np.all(np.abs(got.astype(np.float64) - want) <= TOL_FP4 * mag + 1e-30)
    else:
        gf = (got.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
        wf = (want.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
        assert np.all(np.abs(gf - wf) <= TOL_FP4 * mag + 2.0 ** -7 * np.abs(wf) + 1e-30)


@pytest.mark.gpu
@pytest.mark.parametrize("exact", [False, True])
def test_mx_fp8_full_sampled(gpu, exact):
    """The 4096^3 product group (e4m3 x e4m3, scales around 2^0): 16 rows
    spread over every tile row against the oracle run on those rows."""
    note(f"mx_fp8 4096^3, 16 sampled rows, exact={exact}")
    rng = np.random.default_rng(99)
    m = n = k = 4096
    a, b, sa, sb = mx_case(rng, m, n, k, "e4m3", "e4m3", spread=6)
    import hfusion_mi355x as hfm
    grp = hfm.compile(hfm.catalog.get("mx_fp8"), options="mx_exact=1" if exact else "", require_cached=True).load()
    from helpers import to_dev, to_host
    got = to_host(grp(*(to_dev(x, p["elem"], gpu) for x, p in zip((a, b, sa, sb), grp.meta["params"]))), "f32")
    rows = np.arange(7, m, m // 16)
    want = np.zeros((len(rows), n), np.float32)
    ar, sar = np.ascontiguousarray(a[rows]), np.ascontiguousarray(sa[rows])
    lib().hfref_matmul_mx(ptr(ar), ptr(np.ascontiguousarray(b)), ptr(sar), ptr(np.ascontiguousarray(sb)), ptr(want),
                          len(rows), n, k, 0, 0)
    mag, _ = abs_products(ar, b, sar, sb, "e4m3", "e4m3")
    err = np.abs(got[rows].astype(np.float64) - want) / np.maximum(mag, 1e-30)
    print(f"[err] mx_fp8 exact={exact}: max |gpu - oracle| / sum|A'B'| = {err.max():.3e}", flush=True)
    assert np.all(np.abs(got[rows].astype(np.float64) - want) <= (TOL_EXACT if exact else TOL) * mag + 1e-30)


@pytest.mark.gpu
def test_matmul_mx_fp4_nan_scales(gpu):
    """fp4 has no NaN or infinity codes; an e8m0 scale of 255 (NaN) on one A
    row block and one B column block makes that row and column NaN, as in
    the oracle; the rest within the bar."""
    name = "mx_fp4_256"
    m, n, k, _, _ = FP4_CASES[name]
    note(name + " NaN scales")
    rng = np.random.default_rng(23)
    a, b, sa, sb, ca, cb = fp4_case(rng, m, n, k)
    sa[5, 3] = 255
    sb[9, 14] = 255
    got, = run_gpu(name, [a, b, sa, sb], gpu)
    want, = run_oracle(name, [a, b, sa, sb])
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.isnan(want[5]).all() and np.isnan(want[:, 9]).all()
    ok = ~np.isnan(want)
    with np.errstate(invalid="ignore"):
        mag, _ = fp4_products(ca, cb, sa, sb)
    assert np.all(np.abs(got[ok].astype(np.float64) - want[ok]) <= TOL_FP4 * mag[ok] + 1e-30)


@pytest.mark.gpu
def test_mx_fp4_full_sampled(gpu):
    """The 4096^3 (logical) fp4 group: 16 rows spread over every tile row
    against the oracle run on those rows."""
    note("mx_fp4 4096^3, 16 sampled rows")
    rng = np.random.default_rng(98)
    m = n = k = 4096
    a, b, sa, sb, ca, cb = fp4_case(rng, m, n, k, spread=6)
    import hfusion_mi355x as hfm
    grp = hfm.compile(hfm.catalog.get("mx_fp4"), require_cached=True).load()
    from helpers import to_dev, to_host
    got = to_host(grp(*(to_dev(x, p["elem"], gpu) for x, p in zip((a, b, sa, sb), grp.meta["params"]))), "f32")
    rows = np.arange(7, m, m // 16)
    want = np.zeros((len(rows), n), np.float32)
    ar, sar = np.ascontiguousarray(a[rows]), np.ascontiguousarray(sa[rows])
    lib().hfref_matmul_mx(ptr(ar), ptr(np.ascontiguousarray(b)), ptr(sar), ptr(np.ascontiguousarray(sb)), ptr(want),
                          len(rows), n, k, 4, 4)
    mag, _ = fp4_products(ca[rows], cb, sar, sb)
    err = np.abs(got[rows].astype(np.float64) - want) / np.maximum(mag, 1e-30)
    print(f"[err] mx_fp4: max |gpu - oracle| / sum|A'B'| = {err.max():.3e}", flush=True)
    assert np.all(np.abs(got[rows].astype(np.float64) - want) <= TOL_FP4 * mag + 1e-30)


@pytest.mark.gpu
def test_matmul_mx_gpu_special_values(gpu):
    """NaN and infinity through the matrix core: an e8m0 scale of 255 (NaN)
    on one A row and one B column, fp8 NaN codes in another row, and e5m2
    infinities (same sign in one column, opposite signs in another); the
    NaN / inf pattern of the result must be the oracle's, the rest within the
    bar."""
    name = "mx_e5m2"
    m, n, k, fa, fb, _, _ = GPU_CASES[name]
    note(name + " special values")
    rng = np.random.default_rng(17)
    a, b, sa, sb = mx_case(rng, m, n, k, fa, fb)
    sa[5, 1] = 255                    # row 5: NaN
    sb[9, 2] = 255                    # column 9: NaN
    a[11, 40] = 0x7F                  # e5m2 NaN code: row 11 NaN
    b[:, 20] &= 0x7F                  # column 20: non-negative, one +inf
    b[3, 20] = 0x7C
    a[:, 3] = 0x3C                    # every row multiplies it by +1.0
    b[:, 30] &= 0x7F                  # column 30: +inf and -inf -> NaN
    b[3, 30], b[4, 30] = 0x7C, 0xFC
    a[:, 4] = 0x3C
    got, = run_gpu(name, [a, b, sa, sb], gpu)
    want, = run_oracle(name, [a, b, sa, sb])
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(np.isinf(got), np.isinf(want)) and np.array_equal(got[np.isinf(got)], want[np.isinf(want)])
    ok = np.isfinite(want)
    with np.errstate(invalid="ignore", over="ignore"):
        mag, _ = abs_products(a, b, sa, sb, fa, fb)
    assert np.all(np.abs(got[ok].astype(np.float64) - want[ok]) <= TOL * mag[ok] + 1e-30)
